"""Seeded attention cases shared by the CPU oracle tests and the GPU parity tests."""

from __future__ import annotations

import numpy as np

from nanollvm_amd import workloads as W
from oracle import oracle as O


class Case:
    """A workload plus seeded q/k/v and pre-step page contents (unused slots NaN)."""

    def __init__(self, wl: W.Workload, seed: int = 0, fill_nan: bool = True):
        self.wl = wl
        rng = np.random.default_rng(seed + 1000)
        T = wl.tokens
        self.q = rng.standard_normal((T, wl.hq, wl.d), dtype=np.float32)
        self.k = rng.standard_normal((T, wl.hkv, wl.d), dtype=np.float32)
        self.v = rng.standard_normal((T, wl.hkv, wl.d), dtype=np.float32)
        self.paged = wl.tables is not None
        if self.paged:
            shape = (wl.num_blocks, wl.block_size, wl.hkv, wl.d)
            fill = np.nan if fill_nan else 0.0
            self.k_cache = np.full(shape, fill, np.float32)
            self.v_cache = np.full(shape, fill, np.float32)
            prior = wl.prior_slots()
            kc = self.k_cache.reshape(-1, wl.hkv, wl.d)
            vc = self.v_cache.reshape(-1, wl.hkv, wl.d)
            kc[prior] = rng.standard_normal((len(prior), wl.hkv, wl.d), dtype=np.float32)
            vc[prior] = rng.standard_normal((len(prior), wl.hkv, wl.d), dtype=np.float32)
        else:
            self.k_cache = self.v_cache = None

    def oracle(self, threads=1, kernels=0, mutation=0, store=True):
        """Oracle Attention.forward: returns (out, k_cache_after, v_cache_after)."""
        m = self.wl.meta
        kc = None if self.k_cache is None else self.k_cache.copy()
        vc = None if self.v_cache is None else self.v_cache.copy()
        out = O.attention_forward(
            self.wl.hq, self.wl.d, self.wl.scale, self.wl.hkv, is_prefill=m.is_prefill,
            q=self.q, k=self.k, v=self.v, cu_q=m.cu_seqlens_q, cu_k=m.cu_seqlens_k,
            slot_mapping=m.slot_mapping if store else None, context_lens=m.context_lens,
            block_tables=m.block_tables, k_cache=kc, v_cache=vc,
            sliding_window=self.wl.window, threads=threads, kernels=kernels, mutation=mutation)
        return out, kc, vc

    def fp64(self, k_cache, v_cache):
        m = self.wl.meta
        return O.attention_fp64(
            self.wl.hq, self.wl.d, self.wl.scale, self.wl.hkv, is_prefill=m.is_prefill, q=self.q,
            k=self.k, v=self.v, cu_q=m.cu_seqlens_q, cu_k=m.cu_seqlens_k,
            context_lens=m.context_lens, block_tables=m.block_tables, k_cache=k_cache,
            v_cache=v_cache, sliding_window=self.wl.window)


def rel_l2(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    den = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (den if den > 0 else 1.0))


def small_cases():
    """Small seeded cases covering every branch of Attention.forward."""
    rng = np.random.default_rng(7)
    cases = {}
    # Decode, GQA 2:1, fragmented small pages, contexts crossing page edges.
    ctx = [1, 2, 15, 16, 17, 40, 63, 64, 65, 100]
    cases["decode_gqa"] = W.build("decode gqa", [(c - 1, 1) for c in ctx], is_prefill=False,
                                  hq=4, hkv=2, d=16, scale=0.25, rng=rng, block_size=16)
    # Decode, MQA 4:1 with sliding window 7.
    cases["decode_mqa_window"] = W.build("decode mqa w7", [(c - 1, 1) for c in ctx],
                                         is_prefill=False, hq=4, hkv=1, d=32, scale=0.17,
                                         window=7, rng=rng, block_size=16)
    # Dense prefill (no tables, no slots): prefillDense.
    cases["prefill_dense"] = W.build("prefill dense", [(0, 5), (0, 33), (0, 1), (0, 70)],
                                     is_prefill=True, hq=4, hkv=2, d=16, scale=0.25, rng=rng,
                                     paged=False)
    # Prefill with cache: prefix hits (full pages), mid-page chunk starts, qLen=1 rows.
    cases["prefill_cache"] = W.build("prefill cache",
                                     [(32, 20), (0, 40), (5, 11), (47, 1), (16, 48)],
                                     is_prefill=True, hq=8, hkv=2, d=16, scale=0.25, rng=rng,
                                     block_size=16)
    # Prefill with cache and a sliding window.
    cases["prefill_cache_window"] = W.build("prefill cache w9", [(20, 30), (0, 17), (3, 40)],
                                            is_prefill=True, hq=2, hkv=2, d=32, scale=0.2,
                                            window=9, rng=rng, block_size=16)
    return cases
