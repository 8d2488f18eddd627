"""Edge behaviour of the reference on the GPU, through the C ABI, against the oracle.

* storeKvCache skips negative slots (Attention.java:230-234).  Decode and prefill-with-cache
  steps with -1 slots mixed in store only the other rows: every page byte, NaN-filled unused
  slots included, equals the oracle's pages; the attention reads the old page contents at the
  skipped tokens' positions, as the reference does, and matches the oracle.  Checked on the
  plain store and on the fused RoPE + store kernel.
* gatherKvCache leaves zero rows for negative slots (Attention.java:207-211): a shared-KV dense
  prefill with -1 slots attends over zero K/V rows there, as the oracle does.
* RotaryEmbedding.apply rounds positions with Math.round (Norms.java:317-322): fractional
  positions (x.5, -0.5, 15.4, 0.49999997, NaN, maxPos - 0.51) through the fused norm + RoPE +
  attention entry give rotated q/k bit-identical to the oracle's; a position that rounds to
  maxPos or to -1 fails with IllegalArgumentException before any work (pages untouched).
* The library's own table builder (nva_rope_create_theta, Norms.java:183-204) at the Qwen3-0.6B
  table (d = 128, theta 1e6, maxPos 40960) and the Gemma3 local table (d = 256, theta 1e4,
  maxPos 32768) equals the oracle's table bit for bit.  The table is read back exactly by
  rotating rows [1, ..., 1, 0, ..., 0]: o[i] = 1*c - 0*s = c and o[h+i] = 0*c + 1*s = s.
"""

import numpy as np
import pytest
import torch

from cases import Case, rel_l2
from gpu_checks import MAX_ABS, REL_L2, bits, check_attention, dev, say
from nanollvm_amd import (Attention, Context, IllegalArgumentException, KvCacheArena, RMSNorm,
                          RotaryEmbedding)
from nanollvm_amd import workloads as W
from oracle import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = Context(0)
    yield c
    c.close()


def skip_slots(case, idx, seed):
    """Sets the slots of tokens ``idx`` to -1 and gives their would-be page rows seeded finite
    values (the reference then attends over those old contents)."""
    wl, rng = case.wl, np.random.default_rng(seed)
    m = wl.meta
    slots = m.slot_mapping.copy()
    kc = case.k_cache.reshape(-1, wl.hkv, wl.d)
    vc = case.v_cache.reshape(-1, wl.hkv, wl.d)
    kc[slots[idx]] = rng.standard_normal((len(idx), wl.hkv, wl.d), dtype=np.float32)
    vc[slots[idx]] = rng.standard_normal((len(idx), wl.hkv, wl.d), dtype=np.float32)
    slots[idx] = -1
    m.slot_mapping = slots


def decode_case():
    rng = np.random.default_rng(21)
    ctxs = [1, 2, 15, 16, 17, 40, 63, 64, 65, 100, 257, 300]
    wl = W.build("decode, -1 slots", [(c - 1, 1) for c in ctxs], is_prefill=False, hq=8, hkv=2,
                 d=64, scale=0.125, rng=rng, block_size=16)
    case = Case(wl, seed=21)
    skip_slots(case, np.array([0, 3, 4, 9, 11]), 5)
    return case


def prefill_case():
    rng = np.random.default_rng(22)
    wl = W.build("prefill with cache, -1 slots", [(32, 20), (0, 40), (5, 11), (47, 1), (16, 70)],
                 is_prefill=True, hq=8, hkv=2, d=64, scale=0.125, rng=rng, block_size=16)
    case = Case(wl, seed=22)
    T = wl.tokens
    skip_slots(case, np.array([0, 1, 19, 20, 45, 60, 71, T - 1]), 6)
    return case


@pytest.mark.parametrize("make", [decode_case, prefill_case], ids=["decode", "prefill"])
def test_store_skips_negative_slots(ctx, make):
    case = make()
    assert (case.wl.meta.slot_mapping < 0).sum() >= 5
    check_attention(ctx, case, f"{case.wl.name} (store kernel)")


@pytest.mark.parametrize("make", [decode_case, prefill_case], ids=["decode", "prefill"])
def test_fused_rope_store_skips_negative_slots(ctx, make):
    case = make()
    table = O.rope_table(case.wl.d, 4096, 1e6)
    rope = RotaryEmbedding(ctx, case.wl.d, case.wl.d, 4096, 1e6, cos_sin=table)
    try:
        check_attention(ctx, case, f"{case.wl.name} (fused RoPE + store)",
                        fused_rope=(rope, table))
    finally:
        rope.close()


def test_shared_kv_gather_zero_rows_for_negative_slots(ctx):
    hq, hkv, d, bs = 4, 2, 32, 16
    rng = np.random.default_rng(23)
    wl = W.build("shared dense, -1 slots", [(0, 40), (0, 70), (0, 3)], is_prefill=True, hq=hq,
                 hkv=hkv, d=d, scale=0.2, rng=rng, block_size=bs)
    m = wl.meta
    slots = m.slot_mapping.copy()
    slots[[0, 5, 39, 40, 41, 100, 112]] = -1
    say(f"shared dense prefill with {int((slots < 0).sum())} negative slots (gather)")
    arena = KvCacheArena(ctx, 2, wl.num_blocks, bs, hkv, head_dims=[d, d],
                         allocate=[True, False])
    kc = rng.standard_normal((wl.num_blocks, bs, hkv, d)).astype(np.float32)
    vc = rng.standard_normal((wl.num_blocks, bs, hkv, d)).astype(np.float32)
    arena.write(0, 0, kc)
    arena.write(0, 1, vc)
    try:
        args = m.context_args()
        args.update(block_tables=None, slot_mapping=slots)
        ctx.set(**args)
        ctx.bind_kv_cache(arena)
        q = rng.standard_normal((wl.tokens, hq, d)).astype(np.float32)
        out = Attention(hq, d, 0.2, hkv, 0, kv_layer_index=0, write_kv=False).forward(
            dev(q), None, None, ctx)
        ctx.sync()
        want = O.attention_forward(hq, d, 0.2, hkv, is_prefill=True, q=q, cu_q=m.cu_seqlens_q,
                                   cu_k=m.cu_seqlens_k, slot_mapping=slots, k_cache=kc.copy(),
                                   v_cache=vc.copy(), write_kv=False, threads=4)
        # The closed form: the gathered rows are zero at negative slots.
        kg = np.where((slots < 0)[:, None, None], 0.0,
                      kc.reshape(-1, hkv, d)[np.maximum(slots, 0)]).astype(np.float32)
        vg = np.where((slots < 0)[:, None, None], 0.0,
                      vc.reshape(-1, hkv, d)[np.maximum(slots, 0)]).astype(np.float32)
        dense = O.attention_forward(hq, d, 0.2, hkv, is_prefill=True, q=q, k=kg, v=vg,
                                    cu_q=m.cu_seqlens_q, cu_k=m.cu_seqlens_k, threads=4)
        assert np.array_equal(bits(want), bits(dense)), "oracle gather differs from zero rows"
        got = out.cpu().numpy()
        err = float(np.max(np.abs(got - want)))
        rl2 = rel_l2(got, want)
        say(f"shared gather with -1 slots: max_abs={err:.3e} rel_l2={rl2:.3e}")
        assert err <= MAX_ABS and rl2 <= REL_L2, (err, rl2)
        assert np.array_equal(bits(arena.get_key_cache(0)), bits(kc))
        assert np.array_equal(bits(arena.get_value_cache(0)), bits(vc))
    finally:
        ctx.clear()
        arena.close()


MAX_POS = 40960
FRACTIONAL = [2.5, -0.5, 15.4, 0.49999997, float("nan"), MAX_POS - 0.51, 7.5, 1e-45, 100.5,
              3.4999998]


def fractional_case():
    rng = np.random.default_rng(24)
    n = len(FRACTIONAL)
    wl = W.build("decode, fractional positions", [(c - 1, 1) for c in rng.integers(1, 400, n)],
                 is_prefill=False, hq=16, hkv=8, d=128, scale=W.QWEN_SCALE, rng=rng)
    return wl, Case(wl, seed=24)


def test_fractional_positions_round_like_java(ctx):
    wl, case = fractional_case()
    pos = np.array(FRACTIONAL, np.float32)
    want_pos = [O.java_round(x) for x in pos]
    assert want_pos == [3, 0, 15, 0, 0, MAX_POS - 1, 8, 0, 101, 3], want_pos
    say(f"fractional positions {pos.tolist()} -> {want_pos}")
    rng = np.random.default_rng(25)
    qw = dev(rng.standard_normal(wl.d).astype(np.float32))
    kw = dev(rng.standard_normal(wl.d).astype(np.float32))
    table = O.rope_table(wl.d, MAX_POS, 1e6)
    rope = RotaryEmbedding(ctx, wl.d, wl.d, MAX_POS, 1e6, cos_sin=table)
    arena = KvCacheArena(ctx, 1, wl.num_blocks, wl.block_size, wl.hkv, wl.d)
    arena.write(0, 0, case.k_cache)
    arena.write(0, 1, case.v_cache)
    try:
        ctx.set(**wl.meta.context_args())
        ctx.bind_kv_cache(arena)
        q_out = torch.empty(case.q.shape, device="cuda")
        k_out = torch.empty(case.k.shape, device="cuda")
        attn = Attention(wl.hq, wl.d, wl.scale, wl.hkv)
        out = attn.forward_with_norm_rope(rope, pos, dev(case.q), dev(case.k), dev(case.v), ctx,
                                          q_norm=RMSNorm(qw, 1e-6), k_norm=RMSNorm(kw, 1e-6),
                                          q_out=q_out, k_out=k_out)
        ctx.sync()
        nq = O.rms_norm(case.q.reshape(-1, wl.d), qw.cpu().numpy(), 1e-6).reshape(case.q.shape)
        nk = O.rms_norm(case.k.reshape(-1, wl.d), kw.cpu().numpy(), 1e-6).reshape(case.k.shape)
        qr, kr = O.rope_forward(table, pos, nq, nk)
        qr2, kr2 = O.rope_forward(table, np.array(want_pos, np.float32), nq, nk)
        assert np.array_equal(bits(qr), bits(qr2)) and np.array_equal(bits(kr), bits(kr2))
        assert np.array_equal(bits(q_out.cpu().numpy()), bits(qr)), "rotated q differs"
        assert np.array_equal(bits(k_out.cpu().numpy()), bits(kr)), "rotated k differs"
        case.q, case.k = qr, kr
        want, kc, vc = case.oracle(threads=8)
        got = out.cpu().numpy()
        err = float(np.max(np.abs(got - want)))
        say(f"fractional positions: max_abs={err:.3e}")
        assert err <= MAX_ABS and rel_l2(got, want) <= REL_L2
        assert np.array_equal(bits(arena.get_key_cache(0)), bits(kc))
        assert np.array_equal(bits(arena.get_value_cache(0)), bits(vc))
    finally:
        ctx.clear()
        arena.close()
        rope.close()


@pytest.mark.parametrize("bad", [MAX_POS - 0.5, -0.51, float(MAX_POS)], ids=str)
def test_position_out_of_range_after_rounding(ctx, bad):
    wl, case = fractional_case()
    pos = np.array(FRACTIONAL, np.float32)
    pos[4] = bad
    table = O.rope_table(wl.d, MAX_POS, 1e6)
    rope = RotaryEmbedding(ctx, wl.d, wl.d, MAX_POS, 1e6, cos_sin=table)
    arena = KvCacheArena(ctx, 1, wl.num_blocks, wl.block_size, wl.hkv, wl.d)
    arena.write(0, 0, case.k_cache)
    arena.write(0, 1, case.v_cache)
    try:
        ctx.set(**wl.meta.context_args())
        ctx.bind_kv_cache(arena)
        with pytest.raises(IllegalArgumentException, match="out of range"):
            Attention(wl.hq, wl.d, wl.scale, wl.hkv).forward_with_norm_rope(
                rope, pos, dev(case.q), dev(case.k), dev(case.v), ctx)
        ctx.sync()
        assert np.array_equal(bits(arena.get_key_cache(0)), bits(case.k_cache))
        assert np.array_equal(bits(arena.get_value_cache(0)), bits(case.v_cache))
    finally:
        ctx.clear()
        arena.close()
        rope.close()


@pytest.mark.parametrize("d,theta,max_pos", [(128, 1e6, 40960), (256, 1e4, 32768)],
                         ids=["qwen3-0.6b", "gemma3-local"])
def test_library_table_builder_bit_exact(ctx, d, theta, max_pos):
    say(f"library RoPE table d={d} theta={theta:g} maxPos={max_pos}")
    rope = RotaryEmbedding(ctx, d, d, max_pos, theta)  # built by nva_rope_create_theta
    try:
        pos = np.arange(max_pos, dtype=np.float32)
        ctx.set(True, [0, max_pos], [0, max_pos], max_pos, max_pos, positions=pos)
        x = torch.zeros((max_pos, 1, d), device="cuda")
        x[:, :, : d // 2] = 1.0
        q_rot, k_rot = rope.forward(None, x, x.clone(), ctx)
        ctx.sync()
        got = q_rot.cpu().numpy().reshape(max_pos, d)
        want = O.rope_table(d, max_pos, theta)
        assert np.array_equal(bits(got), bits(want)), (
            f"{int((bits(got) != bits(want)).sum())} table entries differ")
        assert np.array_equal(bits(k_rot.cpu().numpy().reshape(max_pos, d)), bits(want))
    finally:
        ctx.clear()
        rope.close()
