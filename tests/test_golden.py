"""The golden fixtures (tests/golden, written by tests/golden/make_golden.py): the oracle must
reproduce every stored output bit for bit, and the stored attention outputs must sit within
1e-5 of the float64 closed form.  Together they pin the oracle against silent change."""

import numpy as np
import pytest

from golden_fixtures import load, meta, names, oracle_attention
from oracle import oracle as O


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_fixtures_exist():
    assert len(names()) >= 7


@pytest.mark.parametrize("name", names("attention"))
def test_attention_fixture(name):
    fx = load(name)
    out, kc, vc = oracle_attention(fx)
    assert np.array_equal(bits(out), bits(fx["out"]))
    if "k_cache_out" in fx:
        assert np.array_equal(bits(kc), bits(fx["k_cache_out"]))
        assert np.array_equal(bits(vc), bits(fx["v_cache_out"]))
        m = meta(fx)
        ref = O.attention_fp64(int(fx["hq"]), int(fx["d"]), float(fx["scale"]), int(fx["hkv"]),
                               is_prefill=m["is_prefill"], q=fx["q"], k=fx["k"], v=fx["v"],
                               cu_q=m.get("cu_seqlens_q"), cu_k=m.get("cu_seqlens_k"),
                               context_lens=m.get("context_lens"),
                               block_tables=m.get("block_tables"), k_cache=kc, v_cache=vc,
                               sliding_window=int(fx["window"]))
        assert np.max(np.abs(ref - fx["out"])) <= 1e-5


def test_rope_fixture():
    fx = load("ref_rope_d8")
    table = O.rope_table(int(fx["head_size"]), int(fx["max_pos"]), float(fx["base"]))
    assert np.array_equal(bits(table), bits(fx["table"]))
    qr, kr = O.rope_forward(table, fx["positions"], fx["q"], fx["k"])
    assert np.array_equal(bits(qr), bits(fx["q_out"])) and np.array_equal(bits(kr), bits(fx["k_out"]))


def test_rms_norm_fixture():
    fx = load("rms_norm_rows")
    eps = float(fx["eps"])
    for tag, w, one_plus in (("weightless", None, False), ("weight", fx["weight"], False),
                             ("one_plus", fx["weight"], True)):
        assert np.array_equal(bits(O.rms_norm(fx["x"], w, eps, one_plus)), bits(fx["out_" + tag]))


def test_linear_fixture():
    fx = load("linear_small")
    assert np.array_equal(bits(O.linear(fx["x"], fx["w"], fx["b"])), bits(fx["y"]))
