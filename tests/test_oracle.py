"""Pins the CPU oracle: closed forms, an independent float64 textbook restatement, special cases
with known answers, the reference's own (self-consistency) tests re-expressed, and planted
mistakes that each must fail at least one of these checks."""

import math

import numpy as np
import pytest

from cases import Case, rel_l2, small_cases
from nanollvm_amd import workloads as W
from oracle import oracle as O

CASES = small_cases()


# ------------------------------------------------------------------------------ Math.round

def test_java_round_matches_floor_half_up():
    vals = np.array([0.0, 0.49999997, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, -0.49999997, 7.0, 1e9,
                     3e9, -3e9, 40959.5, 1.0000001], np.float32)
    for x in vals:
        want = math.floor(float(x) + 0.5)
        want = max(-2**31, min(2**31 - 1, want))
        assert O.java_round(x) == want, x
    assert O.java_round(np.float32(np.nan)) == 0


# ------------------------------------------------------------------------------ RoPE table

@pytest.mark.parametrize("d,base", [(8, 1e4), (128, 1e6), (256, 1e4), (4, 10.0)])
def test_rope_inv_freq_matches_double_formula(d, base):
    inv = O.rope_inv_freq(d, d, base)
    b = float(np.float32(base))
    want = np.array([np.float32(1.0 / math.pow(b, (2.0 * i) / d)) for i in range(d // 2)],
                    np.float32)
    assert np.array_equal(inv.view(np.uint32), want.view(np.uint32))


def test_rope_inv_freq_rejects_partial_rotary():
    with pytest.raises(ValueError):
        O.rope_inv_freq(8, 4, 1e4)


@pytest.mark.parametrize("d,max_pos,base", [(8, 128, 1e4), (128, 300, 1e6)])
def test_rope_table_matches_python_libm(d, max_pos, base):
    t = O.rope_table(d, max_pos, base)
    inv = O.rope_inv_freq(d, d, base)
    half = d // 2
    for pos in range(0, max_pos, 7):
        for i in range(half):
            ang = float(np.float32(np.float32(pos) * inv[i]))
            assert t[pos, i] == np.float32(math.cos(ang))
            assert t[pos, half + i] == np.float32(math.sin(ang))
    assert np.all(t[0, :half] == 1.0) and np.all(t[0, half:] == 0.0)


# ------------------------------------------------------------------------------ RoPE apply

def _rope_np32(table, positions, x):
    pos = np.array([O.java_round(p) for p in positions])
    half = x.shape[-1] // 2
    c = table[pos][:, None, :half]
    s = table[pos][:, None, half:]
    x1, x2 = x[..., :half], x[..., half:]
    return np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], axis=-1).astype(np.float32)


def test_rope_forward_bit_exact_and_close_to_fp64():
    rng = np.random.default_rng(3)
    table = O.rope_table(128, 4096, 1e6)
    T = 37
    pos = rng.integers(0, 4096, T).astype(np.float32)
    q = rng.standard_normal((T, 16, 128), dtype=np.float32)
    k = rng.standard_normal((T, 8, 128), dtype=np.float32)
    qo, ko = O.rope_forward(table, pos, q, k)
    assert np.array_equal(qo.view(np.uint32), _rope_np32(table, pos, q).view(np.uint32))
    assert np.array_equal(ko.view(np.uint32), _rope_np32(table, pos, k).view(np.uint32))
    assert np.max(np.abs(qo - O.rope_fp64(table, pos, q))) < 1e-5
    # Rotation keeps the norm of every (i, i+half) pair.
    half = 64
    n_in = q[..., :half] ** 2 + q[..., half:] ** 2
    n_out = qo[..., :half].astype(np.float64) ** 2 + qo[..., half:].astype(np.float64) ** 2
    assert np.max(np.abs(n_in - n_out) / np.maximum(n_in, 1e-3)) < 1e-5


def test_rope_position_zero_is_identity():
    table = O.rope_table(16, 8, 1e4)
    q = np.random.default_rng(0).standard_normal((2, 3, 16), dtype=np.float32)
    qo, ko = O.rope_forward(table, np.zeros(2, np.float32), q, q[:, :1])
    assert np.array_equal(qo, q) and np.array_equal(ko, q[:, :1])


def test_rope_out_of_range_position_raises():
    table = O.rope_table(8, 16, 1e4)
    q = np.zeros((2, 1, 8), np.float32)
    with pytest.raises(ValueError):
        O.rope_forward(table, np.array([0, 16], np.float32), q, q)
    with pytest.raises(ValueError):
        O.rope_forward(table, np.array([-0.6, 1], np.float32), q, q)
    O.rope_forward(table, np.array([-0.5, 15.4], np.float32), q, q)  # rounds to 0 and 15


def test_rope_planted_sign_mistake_is_caught():
    table = O.rope_table(32, 64, 1e4)
    rng = np.random.default_rng(1)
    pos = rng.integers(1, 64, 5).astype(np.float32)
    q = rng.standard_normal((5, 2, 32), dtype=np.float32)
    qo, _ = O.rope_forward(table, pos, q, q, mutation=O.MUT_ROPE_SIGN)
    assert np.max(np.abs(qo - O.rope_fp64(table, pos, q))) > 1e-2


def test_reference_rotary_parallel_case():
    """T/CoreUnitTest.java:1487-1505: d=8, maxPos 128, base 1e4, 64 tokens, 8 q / 4 k heads."""
    table = O.rope_table(8, 128, 1e4)
    pos = np.arange(64, dtype=np.float32)
    q = O.filled_ramp(64, 8, 8)
    k = O.filled_ramp(64, 4, 8)
    qo, ko = O.rope_forward(table, pos, q, k)
    assert np.array_equal(qo, _rope_np32(table, pos, q))
    assert np.array_equal(ko, _rope_np32(table, pos, k))


# ------------------------------------------------------------------------------ store

def test_store_closed_form_and_negative_slots():
    rng = np.random.default_rng(2)
    kc = np.full((4, 4, 2, 8), np.nan, np.float32)
    vc = kc.copy()
    k = rng.standard_normal((5, 2, 8), dtype=np.float32)
    v = rng.standard_normal((5, 2, 8), dtype=np.float32)
    slots = np.array([3, -1, 15, 0, -7], np.int32)
    O.store_kv(k, v, slots, kc, vc)
    flat_k = kc.reshape(16, 2, 8)
    flat_v = vc.reshape(16, 2, 8)
    for i, s in enumerate(slots):
        if s >= 0:
            assert np.array_equal(flat_k[s], k[i]) and np.array_equal(flat_v[s], v[i])
    untouched = [s for s in range(16) if s not in (3, 15, 0)]
    assert np.all(np.isnan(flat_k[untouched])) and np.all(np.isnan(flat_v[untouched]))


# ------------------------------------------------------------------------------ attention

@pytest.mark.parametrize("name", sorted(CASES))
def test_attention_matches_fp64_textbook(name):
    c = Case(CASES[name], seed=11)
    out, kc, vc = c.oracle()
    ref = c.fp64(kc, vc)
    assert np.all(np.isfinite(out))
    assert np.max(np.abs(out - ref)) < 2e-6, name
    assert rel_l2(out, ref) < 1e-6


@pytest.mark.parametrize("name", sorted(CASES))
def test_attention_store_is_bit_exact(name):
    c = Case(CASES[name], seed=12)
    _, kc, vc = c.oracle()
    if kc is None:
        return
    m = c.wl.meta
    flat_k = kc.reshape(-1, c.wl.hkv, c.wl.d)
    flat_v = vc.reshape(-1, c.wl.hkv, c.wl.d)
    assert np.array_equal(flat_k[m.slot_mapping], c.k)
    assert np.array_equal(flat_v[m.slot_mapping], c.v)
    touched = set(m.slot_mapping.tolist()) | set(c.wl.prior_slots().tolist())
    others = np.array([s for s in range(flat_k.shape[0]) if s not in touched])
    if len(others):
        assert np.all(np.isnan(flat_k[others]))


@pytest.mark.parametrize("kernels", [8, 16])
def test_scalar_and_vector_kernel_semantics_agree(kernels):
    """T/CoreUnitTest.java:656-745 tolerance style: backends agree within 1e-5."""
    c = Case(CASES["prefill_cache"], seed=13)
    a, _, _ = c.oracle(kernels=0)
    b, _, _ = c.oracle(kernels=kernels)
    assert np.max(np.abs(a - b)) < 1e-5


def test_reference_causal_prefill_parallel_case():
    """T/CoreUnitTest.java:1462-1471 with 546-584: filledRamp q/k/v [16, 8, 4], Attention(8, 4,
    1f, 8, 0), one 2-block arena of block size 256, dense prefill; threads 2 == sequential."""
    q = O.filled_ramp(16, 8, 4)
    kc = np.zeros((2, 256, 8, 4), np.float32)
    vc = kc.copy()
    args = dict(is_prefill=True, q=q, k=q, v=q, cu_q=[0, 16], cu_k=[0, 16], k_cache=kc,
                v_cache=vc)
    seq = O.attention_forward(8, 4, 1.0, 8, threads=1, **args)
    par = O.attention_forward(8, 4, 1.0, 8, threads=2, **args)
    assert np.array_equal(seq, par)
    ref = O.attention_fp64(8, 4, 1.0, 8, is_prefill=True, q=q, k=q, v=q, cu_q=[0, 16],
                           cu_k=[0, 16])
    assert np.max(np.abs(seq - ref)) < 1e-5


def test_parallel_split_is_bit_identical_on_paged_cases():
    c = Case(CASES["prefill_cache"], seed=14)
    a, _, _ = c.oracle(threads=1)
    b, _, _ = c.oracle(threads=3)
    assert np.array_equal(a, b)


# Special cases with closed-form answers.

def _single(q_len, k_len, hq, hkv, d, keys, vals, window=0, scale=0.3, q=None):
    rng = np.random.default_rng(5)
    q = rng.standard_normal((q_len, hq, d), dtype=np.float32) if q is None else q
    bs = 8
    pages = -(-k_len // bs)
    kc = np.zeros((pages, bs, hkv, d), np.float32)
    vc = kc.copy()
    kc.reshape(-1, hkv, d)[:k_len] = keys
    vc.reshape(-1, hkv, d)[:k_len] = vals
    tables = np.arange(pages, dtype=np.int32)[None, :]
    return O.attention_forward(hq, d, scale, hkv, is_prefill=True, q=q, cu_q=[0, q_len],
                               cu_k=[0, k_len], block_tables=tables, k_cache=kc, v_cache=vc,
                               sliding_window=window), q


def test_single_key_returns_v():
    rng = np.random.default_rng(6)
    v = rng.standard_normal((1, 2, 8), dtype=np.float32)
    out, _ = _single(1, 1, 4, 2, 8, rng.standard_normal((1, 2, 8), dtype=np.float32), v)
    for h in range(4):
        assert np.allclose(out[0, h], v[0, h // 2], atol=1e-7)


def test_identical_keys_average_visible_values():
    rng = np.random.default_rng(7)
    n = 150
    key = rng.standard_normal((1, 1, 16), dtype=np.float32)
    keys = np.repeat(key, n, axis=0)
    vals = rng.standard_normal((n, 1, 16), dtype=np.float32)
    out, _ = _single(n, n, 2, 1, 16, keys, vals)
    for qi in (0, 63, 64, 149):
        want = vals[:qi + 1, 0].astype(np.float64).mean(0)
        assert np.max(np.abs(out[qi, 0] - want)) < 1e-5


def test_window_one_returns_own_value():
    rng = np.random.default_rng(8)
    n = 70
    vals = rng.standard_normal((n, 1, 8), dtype=np.float32)
    out, _ = _single(n, n, 1, 1, 8, rng.standard_normal((n, 1, 8), dtype=np.float32), vals,
                     window=1)
    assert np.allclose(out[:, 0], vals[:, 0], atol=1e-7)


@pytest.mark.parametrize("rep", [2, 3, 5, 7])
def test_mha_equals_gqa_with_duplicated_kv(rep):
    # Query head h reads KV head h // rep (Attention.java:152-171): with every KV head repeated
    # rep times in place, multi-head attention gives the same rows.  The GPU's odd ratios (the
    # 40 / 8 and 28 / 4 head shapes) are checked against this oracle.
    rng = np.random.default_rng(9 + rep)
    n = 90
    keys = rng.standard_normal((n, 2, 16), dtype=np.float32)
    vals = rng.standard_normal((n, 2, 16), dtype=np.float32)
    gqa, q = _single(n, n, 2 * rep, 2, 16, keys, vals)
    mha, _ = _single(n, n, 2 * rep, 2 * rep, 16, np.repeat(keys, rep, axis=1),
                     np.repeat(vals, rep, axis=1), q=q)
    assert np.max(np.abs(gqa - mha)) < 1e-6


def test_wide_window_equals_no_window():
    rng = np.random.default_rng(10)
    n = 80
    keys = rng.standard_normal((n, 1, 8), dtype=np.float32)
    vals = rng.standard_normal((n, 1, 8), dtype=np.float32)
    a, q = _single(n, n, 2, 1, 8, keys, vals, window=0)
    b, _ = _single(n, n, 2, 1, 8, keys, vals, window=n, q=q)
    assert np.array_equal(a, b)


def test_qlen1_prefill_equals_decode():
    wl = W.build("d", [(70, 1), (15, 1)], is_prefill=False, hq=4, hkv=2, d=16, scale=0.25,
                 rng=np.random.default_rng(3), block_size=16)
    c = Case(wl, seed=1)
    dec, _, _ = c.oracle()
    m = wl.meta
    pre = O.attention_forward(4, 16, 0.25, 2, is_prefill=True, q=c.q, k=c.k, v=c.v,
                              cu_q=[0, 1, 2], cu_k=[0, 71, 87], slot_mapping=m.slot_mapping,
                              block_tables=m.block_tables, k_cache=c.k_cache.copy(),
                              v_cache=c.v_cache.copy())
    assert np.array_equal(dec, pre)


def test_empty_context_gives_zero():
    out = O.attention_forward(2, 8, 1.0, 1, is_prefill=False, q=np.ones((1, 2, 8), np.float32),
                              context_lens=[0], block_tables=[[0]],
                              k_cache=np.zeros((1, 4, 1, 8), np.float32),
                              v_cache=np.zeros((1, 4, 1, 8), np.float32))
    assert np.all(out == 0)


def test_dispatch_errors():
    q = np.zeros((2, 2, 8), np.float32)
    with pytest.raises(TypeError):
        O.attention_forward(2, 8, 1.0, 1, is_prefill=True, q=q, cu_q=[0, 2], cu_k=[0, 2],
                            has_arena=False)
    with pytest.raises(RuntimeError):
        O.attention_forward(2, 8, 1.0, 1, is_prefill=True, q=q, cu_q=[0, 2], cu_k=[0, 2],
                            write_kv=False, k_cache=np.zeros((1, 4, 1, 8), np.float32),
                            v_cache=np.zeros((1, 4, 1, 8), np.float32))


# Planted mistakes: each must fail at least one of the checks above.

def _checks_pass(mutation) -> bool:
    for name in ("decode_gqa", "decode_mqa_window", "prefill_dense", "prefill_cache",
                 "prefill_cache_window"):
        c = Case(CASES[name], seed=21)
        out, kc, vc = c.oracle(mutation=mutation)
        ref = c.fp64(kc, vc)
        if not np.all(np.isfinite(out)) or np.max(np.abs(out - ref)) >= 2e-6:
            return False
    return True


def test_checks_pass_unmutated():
    assert _checks_pass(O.MUT_NONE)


@pytest.mark.parametrize("mutation", [O.MUT_DROP_SCALE, O.MUT_KVH_MODULO, O.MUT_CAUSAL_OFF1,
                                      O.MUT_WINDOW_OFF1, O.MUT_NO_RESCALE])
def test_planted_mistake_is_caught(mutation):
    assert not _checks_pass(mutation)
