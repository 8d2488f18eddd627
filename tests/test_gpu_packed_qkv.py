"""nva_qkv_norm_rope_attention_forward: q, k, v read in place from the packed qkv_proj output
[T, (Hq + 2 Hkv) * d] (Qwen3ForCausalLM.java:210-214 splits it with Ops.splitLast).

Bar: bit-identical to nva_norm_rope_attention_forward on the split tensors (output, rotated q
and k, every page byte); one full-size case is also checked against the oracle chain."""

import numpy as np
import pytest
import torch

from cases import Case, rel_l2, small_cases
from gpu_checks import MAX_ABS, REL_L2, bits, dev, say
from nanollvm_amd import Attention, Context, KvCacheArena, RMSNorm, RotaryEmbedding
from nanollvm_amd import workloads as W
from oracle import oracle as O

pytestmark = pytest.mark.gpu

EPS = 1e-6


@pytest.fixture(scope="module")
def ctx():
    c = Context(0)
    yield c
    c.close()


def run(ctx, case, rope, norms, packed):
    """One forward through the split or the packed entry on a fresh arena; returns the output,
    rotated q and k, and the pages."""
    wl = case.wl
    if case.paged:
        arena = KvCacheArena(ctx, 1, wl.num_blocks, wl.block_size, wl.hkv, wl.d)
        arena.write(0, 0, case.k_cache)
        arena.write(0, 1, case.v_cache)
    else:
        arena = KvCacheArena(ctx, 1, 2, 16, wl.hkv, wl.d)
    try:
        ctx.set(**wl.meta.context_args())
        ctx.bind_kv_cache(arena)
        attn = Attention(wl.hq, wl.d, wl.scale, wl.hkv, wl.window, 0)
        T = wl.tokens
        q_out = torch.empty((T, wl.hq, wl.d), dtype=torch.float32, device="cuda")
        k_out = torch.empty((T, wl.hkv, wl.d), dtype=torch.float32, device="cuda")
        qn, kn, vn = norms
        if packed:
            qkv = np.concatenate([case.q.reshape(T, -1), case.k.reshape(T, -1),
                                  case.v.reshape(T, -1)], axis=1)
            out = attn.forward_packed_qkv(rope, wl.meta.positions, dev(qkv), ctx, q_norm=qn,
                                          k_norm=kn, v_norm=vn, q_out=q_out, k_out=k_out)
        else:
            out = attn.forward_with_norm_rope(rope, wl.meta.positions, dev(case.q),
                                              dev(case.k), dev(case.v), ctx, q_norm=qn,
                                              k_norm=kn, v_norm=vn, q_out=q_out, k_out=k_out)
        ctx.sync()
        pages = (arena.get_key_cache(0), arena.get_value_cache(0)) if case.paged else None
        return out.cpu().numpy(), q_out.cpu().numpy(), k_out.cpu().numpy(), pages
    finally:
        ctx.clear()
        arena.close()


def compare(ctx, case, name, mode, theta=1e4, max_pos=512):
    wl = case.wl
    say(f"packed qkv {name} {mode}: tokens={wl.tokens} hq={wl.hq} hkv={wl.hkv} d={wl.d}")
    rng = np.random.default_rng(wl.d + len(mode))
    table = O.rope_table(wl.d, max_pos, theta)
    rope = RotaryEmbedding(ctx, wl.d, wl.d, max_pos, theta, cos_sin=table)
    try:
        if mode == "none":
            norms = (None, None, None)
        else:
            qw = dev((1.0 + 0.1 * rng.standard_normal(wl.d)).astype(np.float32))
            kw = dev((1.0 + 0.1 * rng.standard_normal(wl.d)).astype(np.float32))
            one_plus = mode == "gemma3"
            norms = (RMSNorm(qw, EPS, one_plus), RMSNorm(kw, EPS, one_plus),
                     RMSNorm.weightless(EPS) if mode == "gemma4" else None)
        split = run(ctx, case, rope, norms, packed=False)
        packed = run(ctx, case, rope, norms, packed=True)
    finally:
        rope.close()
    assert np.all(np.isfinite(split[0]))
    for what, a, b in (("out", split[0], packed[0]), ("rotated q", split[1], packed[1]),
                       ("rotated k", split[2], packed[2])):
        assert np.array_equal(bits(a), bits(b)), f"{what} differs between packed and split"
    if case.paged:
        assert np.array_equal(bits(split[3][0]), bits(packed[3][0])), "K pages differ"
        assert np.array_equal(bits(split[3][1]), bits(packed[3][1])), "V pages differ"
    return packed


SMALL = small_cases()


@pytest.mark.parametrize("name", sorted(SMALL))
@pytest.mark.parametrize("mode", ["none", "qwen3", "gemma3", "gemma4"])
def test_packed_matches_split_small(ctx, name, mode):
    compare(ctx, Case(SMALL[name], seed=17), name, mode)


def test_packed_dense_prefill_d4(ctx):
    """Head dim 4 takes the per-token form of the store kernel; dense prefill then needs the
    packed v copied out as contiguous rows."""
    wl = W.build("dense d4", [(0, 16), (0, 5)], is_prefill=True, hq=8, hkv=8, d=4, scale=1.0,
                 paged=False)
    compare(ctx, Case(wl, seed=3), "dense d4", "none")


def test_packed_qwen3_prefill_full_size_vs_oracle(ctx):
    """Qwen3-0.6B varlen prefill with the prefix hit, q/k norms: packed == split, and the
    packed output within the attention tolerance of the oracle chain."""
    wl = W.qwen3_prefill()
    case = Case(wl, seed=0)
    q0, k0 = case.q.copy(), case.k.copy()
    out, qr_got, kr_got, pages = compare(ctx, case, "qwen3 prefill", "qwen3",
                                         theta=wl.rope_theta, max_pos=wl.max_pos)
    rng = np.random.default_rng(wl.d + len("qwen3"))
    qw = (1.0 + 0.1 * rng.standard_normal(wl.d)).astype(np.float32)
    kw = (1.0 + 0.1 * rng.standard_normal(wl.d)).astype(np.float32)
    nq = O.rms_norm(q0.reshape(-1, wl.d), qw, EPS, False).reshape(q0.shape)
    nk = O.rms_norm(k0.reshape(-1, wl.d), kw, EPS, False).reshape(k0.shape)
    qr, kr = O.rope_forward(O.rope_table(wl.d, wl.max_pos, wl.rope_theta), wl.meta.positions,
                            nq, nk)
    assert np.array_equal(bits(qr_got), bits(qr)) and np.array_equal(bits(kr_got), bits(kr))
    case.q, case.k = qr, kr
    want, kc, vc = case.oracle(threads=8)
    err = float(np.max(np.abs(out - want)))
    rl2 = rel_l2(out, want)
    say(f"packed qwen3 prefill vs oracle: max_abs={err:.3e} rel_l2={rl2:.3e}")
    assert err <= MAX_ABS and rl2 <= REL_L2, (err, rl2)
    assert np.array_equal(bits(pages[0]), bits(kc)) and np.array_equal(bits(pages[1]), bits(vc))
