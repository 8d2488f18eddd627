"""Pins the oracle's shared-KV branch (Attention.attendFromCache / gatherKvCache,
layers/Attention.java:176-216): a layer that does not write K/V reads the producer layer's
pages.  Checked against the float64 textbook form over the rows the branch must read, and
against closed forms (no page is written; negative slots gather zero rows)."""

import dataclasses

import numpy as np
import pytest

from nanollvm_amd import workloads as W
from oracle import oracle as O


def _pages(wl, rng):
    shape = (wl.num_blocks, wl.block_size, wl.hkv, wl.d)
    return (rng.standard_normal(shape).astype(np.float32),
            rng.standard_normal(shape).astype(np.float32))


@pytest.mark.parametrize("is_prefill", [False, True])
def test_shared_paged_reads_producer_pages_without_writing(is_prefill):
    rng = np.random.default_rng(2)
    seqs = [(c - 1, 1) for c in (5, 17, 40)] if not is_prefill else [(16, 9), (0, 20), (3, 7)]
    wl = W.build("shared", seqs, is_prefill=is_prefill, hq=4, hkv=2, d=16, scale=0.25, rng=rng,
                 block_size=16)
    kc, vc = _pages(wl, rng)
    kc0, vc0 = kc.copy(), vc.copy()
    m = wl.meta
    q = rng.standard_normal((wl.tokens, 4, 16)).astype(np.float32)
    junk = np.full((wl.tokens, 2, 16), 1e6, np.float32)  # the caller's k/v are never read
    out = O.attention_forward(4, 16, 0.25, 2, is_prefill=is_prefill, q=q, k=junk, v=junk,
                              cu_q=m.cu_seqlens_q, cu_k=m.cu_seqlens_k,
                              slot_mapping=m.slot_mapping, context_lens=m.context_lens,
                              block_tables=m.block_tables, k_cache=kc, v_cache=vc,
                              write_kv=False)
    assert np.array_equal(kc, kc0) and np.array_equal(vc, vc0)
    want = O.attention_fp64(4, 16, 0.25, 2, is_prefill=is_prefill, q=q, cu_q=m.cu_seqlens_q,
                            cu_k=m.cu_seqlens_k, context_lens=m.context_lens,
                            block_tables=m.block_tables, k_cache=kc, v_cache=vc)
    assert np.max(np.abs(out - want)) < 2e-6


def test_shared_dense_prefill_gathers_slots():
    rng = np.random.default_rng(3)
    wl = W.build("shared dense", [(0, 9), (0, 20)], is_prefill=True, hq=4, hkv=1, d=8,
                 scale=0.3, rng=rng, block_size=16)
    kc, vc = _pages(wl, rng)
    m = wl.meta
    slots = m.slot_mapping.copy()
    slots[[2, 15]] = -1  # padding: gathers zero rows
    q = rng.standard_normal((wl.tokens, 4, 8)).astype(np.float32)
    out = O.attention_forward(4, 8, 0.3, 1, is_prefill=True, q=q, cu_q=m.cu_seqlens_q,
                              cu_k=m.cu_seqlens_k, slot_mapping=slots, k_cache=kc, v_cache=vc,
                              write_kv=False)
    flat_k = kc.reshape(-1, 1, 8)
    flat_v = vc.reshape(-1, 1, 8)
    gk = np.where((slots >= 0)[:, None, None], flat_k[np.maximum(slots, 0)], 0.0)
    gv = np.where((slots >= 0)[:, None, None], flat_v[np.maximum(slots, 0)], 0.0)
    want = O.attention_fp64(4, 8, 0.3, 1, is_prefill=True, q=q, k=gk.astype(np.float32),
                            v=gv.astype(np.float32), cu_q=m.cu_seqlens_q, cu_k=m.cu_seqlens_k)
    assert np.max(np.abs(out - want)) < 2e-6
