"""The library (through the C ABI) against the golden fixtures in tests/golden: attention within
max-abs 1e-4 and rel-L2 1e-5 of the stored outputs with the pages bit-exact, RoPE and RMSNorm
bit-exact, the linear within the attention tolerance."""

import numpy as np
import pytest
import torch

from cases import rel_l2
from gpu_checks import MAX_ABS, REL_L2, bits, dev, say
from golden_fixtures import load, meta, names
from nanollvm_amd import Attention, Context, KvCacheArena, Linear, RMSNorm, RotaryEmbedding

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = Context(0)
    yield c
    c.close()


@pytest.mark.parametrize("name", names("attention"))
def test_golden_attention(ctx, name):
    fx = load(name)
    hq, hkv, d = int(fx["hq"]), int(fx["hkv"]), int(fx["d"])
    say(f"golden {name}: {str(fx['note'])}")
    paged = "k_cache" in fx
    if paged:
        nb, bs = fx["k_cache"].shape[:2]
        arena = KvCacheArena(ctx, 1, nb, bs, hkv, d)
        arena.write(0, 0, fx["k_cache"])
        arena.write(0, 1, fx["v_cache"])
    else:
        arena = KvCacheArena(ctx, 1, 2, 256, hkv, d)
    try:
        ctx.set(**meta(fx))
        ctx.bind_kv_cache(arena)
        attn = Attention(hq, d, float(fx["scale"]), hkv, int(fx["window"]), 0)
        out = attn.forward(dev(fx["q"]), dev(fx["k"]), dev(fx["v"]), ctx)
        ctx.sync()
        got = out.cpu().numpy()
        err = float(np.max(np.abs(got - fx["out"])))
        rl2 = rel_l2(got, fx["out"])
        say(f"golden {name}: max_abs={err:.3e} rel_l2={rl2:.3e}")
        assert err <= MAX_ABS and rl2 <= REL_L2, (err, rl2)
        if paged:
            assert np.array_equal(bits(arena.get_key_cache(0)), bits(fx["k_cache_out"]))
            assert np.array_equal(bits(arena.get_value_cache(0)), bits(fx["v_cache_out"]))
        else:
            assert np.all(arena.get_key_cache(0) == 0)  # no slots: nothing stored
    finally:
        ctx.clear()
        arena.close()


def test_golden_rope(ctx):
    fx = load("ref_rope_d8")
    rope = RotaryEmbedding(ctx, int(fx["head_size"]), int(fx["head_size"]), int(fx["max_pos"]),
                           float(fx["base"]))
    try:
        pos = fx["positions"]
        T = len(pos)
        ctx.set(True, [0, T], [0, T], T, T, None, None, None, None, positions=pos)
        qo, ko = rope.forward(pos, dev(fx["q"]), dev(fx["k"]), ctx)
        ctx.sync()
        assert np.array_equal(bits(qo.cpu().numpy()), bits(fx["q_out"]))
        assert np.array_equal(bits(ko.cpu().numpy()), bits(fx["k_out"]))
    finally:
        ctx.clear()
        rope.close()


def test_golden_rms_norm(ctx):
    fx = load("rms_norm_rows")
    eps = float(fx["eps"])
    for tag, w, one_plus in (("weightless", None, False), ("weight", fx["weight"], False),
                             ("one_plus", fx["weight"], True)):
        norm = RMSNorm(None if w is None else dev(w), eps, one_plus)
        got = norm.forward(dev(fx["x"]), ctx).cpu().numpy()
        assert np.array_equal(bits(got), bits(fx["out_" + tag])), tag


def test_golden_linear(ctx):
    fx = load("linear_small")
    got = Linear(dev(fx["w"]), dev(fx["b"])).forward(dev(fx["x"]), ctx).cpu().numpy()
    err = float(np.max(np.abs(got - fx["y"])))
    assert err <= MAX_ABS and rel_l2(got, fx["y"]) <= REL_L2, err
