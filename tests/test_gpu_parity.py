"""Parity of the HIP path (through the C ABI) with the CPU oracle.

Bar: attention outputs within max-abs 1e-4 and rel-L2 1e-5 of the oracle; K/V page contents
(every slot, including untouched NaN-filled ones) and rotated q/k bit-exact."""

import sys

import numpy as np
import pytest
import torch

from cases import Case, rel_l2, small_cases
from gpu_checks import MAX_ABS, REL_L2, bits, check_attention, dev, load_arena, say
from nanollvm_amd import Attention, Context, KvCacheArena, RotaryEmbedding
from nanollvm_amd import workloads as W
from oracle import oracle as O

pytestmark = pytest.mark.gpu



@pytest.fixture(scope="module")
def ctx():
    c = Context(0)
    yield c
    c.close()


SMALL = small_cases()


@pytest.mark.parametrize("name", sorted(SMALL))
def test_small_cases(ctx, name):
    check_attention(ctx, Case(SMALL[name], seed=31), name)


def test_reference_causal_prefill_case(ctx):
    """T/CoreUnitTest.java:1462-1471: filledRamp q=k=v [16,8,4], Attention(8,4,1f,8,0), arena of
    2 blocks x 256, dense prefill (no slots, no tables); tolerance 1e-5."""
    say("reference causal prefill d=4")
    q = O.filled_ramp(16, 8, 4)
    arena = KvCacheArena(ctx, 1, 2, 256, 8, 4)
    try:
        ctx.set(True, [0, 16], [0, 16], 16, 16, None, None, None, [0])
        ctx.bind_kv_cache(arena)
        out = Attention(8, 4, 1.0, 8, 0, 0).forward(dev(q), dev(q), dev(q), ctx)
        ctx.sync()
        want = O.attention_forward(8, 4, 1.0, 8, is_prefill=True, q=q, k=q, v=q, cu_q=[0, 16],
                                   cu_k=[0, 16], k_cache=np.zeros((2, 256, 8, 4), np.float32),
                                   v_cache=np.zeros((2, 256, 8, 4), np.float32))
        assert np.max(np.abs(out.cpu().numpy() - want)) < 1e-5
        assert np.all(arena.get_key_cache(0) == 0)  # no slots -> no store
    finally:
        ctx.clear()
        arena.close()


def test_reference_rotary_case_bit_exact(ctx):
    """T/CoreUnitTest.java:1487-1505: RoPE d=8, maxPos 128, base 1e4, 64 tokens, 8q/4k heads."""
    say("reference rotary d=8")
    table = O.rope_table(8, 128, 1e4)
    rope = RotaryEmbedding(ctx, 8, 8, 128, 1e4)  # table built by the library itself
    try:
        q = O.filled_ramp(64, 8, 8)
        k = O.filled_ramp(64, 4, 8)
        pos = np.arange(64, dtype=np.float32)
        ctx.set(True, [0, 64], [0, 64], 64, 64, None, None, None, None, positions=pos)
        qo, ko = rope.forward(pos, dev(q), dev(k), ctx)
        ctx.sync()
        wq, wk = O.rope_forward(table, pos, q, k)
        assert np.array_equal(bits(qo.cpu().numpy()), bits(wq))
        assert np.array_equal(bits(ko.cpu().numpy()), bits(wk))
    finally:
        ctx.clear()
        rope.close()


def test_rope_qwen_table_bit_exact(ctx):
    say("rope qwen table theta 1e6")
    table = O.rope_table(128, 40960, 1e6)
    rope = RotaryEmbedding(ctx, 128, 128, 40960, 1e6, cos_sin=table)
    try:
        rng = np.random.default_rng(4)
        T = 300
        pos = rng.integers(0, 40960, T).astype(np.float32)
        q = rng.standard_normal((T, 16, 128), dtype=np.float32)
        k = rng.standard_normal((T, 8, 128), dtype=np.float32)
        ctx.set(True, [0, T], [0, T], T, T, None, None, None, None, positions=pos)
        qo, ko = rope.forward(pos, dev(q), dev(k), ctx)
        ctx.sync()
        wq, wk = O.rope_forward(table, pos, q, k)
        assert np.array_equal(bits(qo.cpu().numpy()), bits(wq))
        assert np.array_equal(bits(ko.cpu().numpy()), bits(wk))
        # Out-of-range position: IllegalArgumentException, nothing enqueued.
        bad = pos.copy()
        bad[7] = 40960
        with pytest.raises(ValueError):
            rope.forward(bad, dev(q), dev(k), ctx)
    finally:
        ctx.clear()
        rope.close()


def test_library_table_matches_oracle_table(ctx):
    """The library's own table builder equals the oracle's (same float/double steps)."""
    say("rope table builder")
    table = O.rope_table(64, 2048, 1e4)
    rope = RotaryEmbedding(ctx, 64, 64, 2048, 1e4)
    try:
        pos = np.arange(2048, dtype=np.float32)
        x = np.ones((2048, 1, 64), np.float32)
        x[:, :, 32:] = 0.0   # rotated = (cos, sin) rows exactly
        ctx.set(True, [0, 2048], [0, 2048], 2048, 2048, None, None, None, None, positions=pos)
        qo, _ = rope.forward(pos, dev(x), dev(x), ctx)
        ctx.sync()
        assert np.array_equal(bits(qo.cpu().numpy()[:, 0, :]), bits(table))
    finally:
        ctx.clear()
        rope.close()


@pytest.mark.parametrize("name", ["prefill_cache", "decode_gqa", "prefill_dense"])
def test_fused_rope_attention(ctx, name):
    wl = SMALL[name]
    table = O.rope_table(wl.d, 512, 1e4)
    rope = RotaryEmbedding(ctx, wl.d, wl.d, 512, 1e4, cos_sin=table)
    try:
        check_attention(ctx, Case(wl, seed=41), "fused " + name, fused_rope=(rope, table))
    finally:
        rope.close()


def test_qwen3_decode_small_full_size(ctx):
    check_attention(ctx, Case(W.qwen3_decode_small(), seed=0), "qwen3 decode B=8")


def test_qwen3_prefill_full_size_fused(ctx):
    wl = W.qwen3_prefill()
    table = O.rope_table(128, wl.max_pos, wl.rope_theta)
    rope = RotaryEmbedding(ctx, 128, 128, wl.max_pos, wl.rope_theta, cos_sin=table)
    try:
        check_attention(ctx, Case(wl, seed=0), "qwen3 prefill 512/1024/1536/2048",
                        fused_rope=(rope, table))
    finally:
        rope.close()


@pytest.mark.parametrize("local", [True, False])
def test_gemma3_decode_full_size(ctx, local):
    check_attention(ctx, Case(W.gemma3_decode(local=local), seed=0),
                    f"gemma3 decode {'local' if local else 'global'}")


def test_qwen3_4b_mixed_reduced_contexts(ctx):
    """Mixed prefill chunks + qLen=1 rows in one launch at the Qwen3-4B head shape; contexts
    reduced 4-8x so the CPU oracle finishes in seconds."""
    wl = W.qwen3_4b_mixed(chunks=4, chunk=256, prior_hi=1024, rows=16, ctx_lo=512, ctx_hi=2048)
    check_attention(ctx, Case(wl, seed=0), "qwen3-4b mixed (reduced)")


@pytest.mark.parametrize("hq,window", [(4, 512), (4, 0), (8, 512)])
def test_gemma_prefill_d256_mfma(ctx, hq, window):
    """Gemma-shaped varlen prefill on the MFMA kernel at head_dim 256 (Gemma3-270M: 4 q heads /
    1 kv head; Gemma 4 sliding layers: 8 / 1), scale 1/16, with a prefix-cache hit, a mid-page
    chunk start and sequences longer than the 512-token window."""
    rng = np.random.default_rng(17 + hq + window)
    wl = W.build("gemma prefill d256", [(0, 700), (512, 300), (37, 129)], is_prefill=True,
                 hq=hq, hkv=1, d=256, scale=W.GEMMA_SCALE, window=window, rng=rng)
    check_attention(ctx, Case(wl, seed=5), f"gemma prefill d=256 hq={hq} W={window}")
