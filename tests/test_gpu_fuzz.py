"""Seeded random sweep of the attention path against the oracle.

Each case draws a configuration: head dim (8 .. 512), GQA ratio (1 .. 8), KV heads, page size
(1 .. 256), sliding window, decode / prefill with cache / dense prefill, and a batch of ragged
sequences (prefix hits, mid-page starts, one-query rows, empty-window edges).  A second family
draws GQA ratios 3 .. 32 that are not powers of two or exceed 8.  The bar is the path's:
attention within max-abs 1e-4 and rel-L2 1e-5 of the oracle, every page byte equal."""

import numpy as np
import pytest

from cases import Case
from gpu_checks import check_attention
from nanollvm_amd import Context
from nanollvm_amd import workloads as W

pytestmark = pytest.mark.gpu

SEEDS = list(range(48))


@pytest.fixture(scope="module")
def ctx():
    c = Context(0)
    yield c
    c.close()


def draw(seed):
    rng = np.random.default_rng(90000 + seed)
    d = int(rng.choice([8, 16, 32, 64, 128, 256, 512]))
    rep = int(rng.choice([1, 2, 4, 8]))
    hkv = int(rng.choice([1, 2, 3]))
    mode = str(rng.choice(["decode", "prefill", "dense"]))
    bs = int(rng.choice([1, 4, 16, 64, 256]))
    window = int(rng.choice([0, 0, 1, 5, 33, 300]))
    budget = 2500 if d <= 128 else 1200  # keeps the oracle quick
    nseq = int(rng.integers(1, 6))
    seqs = []
    for _ in range(nseq):
        if mode == "decode":
            seqs.append((int(rng.integers(0, budget // nseq)), 1))
        elif mode == "dense":
            seqs.append((0, int(rng.integers(1, max(2, budget // (4 * nseq))))))
        else:
            cached = int(rng.integers(0, budget // (2 * nseq)))
            seqs.append((cached, int(rng.integers(1, max(2, budget // (4 * nseq))))))
    scale = float(np.float32(1.0 / np.sqrt(d)) * np.float32(rng.uniform(0.5, 2.0)))
    wl = W.build(f"fuzz {seed}: d={d} rep={rep} hkv={hkv} {mode} bs={bs} W={window} {seqs}",
                 seqs, is_prefill=mode != "decode", hq=hkv * rep, hkv=hkv, d=d, scale=scale,
                 window=window, rng=rng, paged=mode != "dense", block_size=bs, pool_cap=40000)
    return wl


@pytest.mark.parametrize("seed", SEEDS)
def test_fuzz(ctx, seed):
    wl = draw(seed)
    check_attention(ctx, Case(wl, seed=seed), wl.name)


def draw_gqa(seed):
    """GQA ratios that are not powers of two or exceed 8 (the row kernel's 3/5/6/7-head forms,
    the MFMA row kernel up to 16 heads, two head groups per KV head above that), d 32 .. 512,
    pages that are and are not powers of two; prefill steps mix in one-query rows, so a plan
    holds MFMA tiles and rows at once."""
    rng = np.random.default_rng(91000 + seed)
    d = int(rng.choice([32, 64, 128, 128, 256, 512]))
    rep = int(rng.choice([3, 5, 6, 7, 10, 12, 16, 24, 32]))
    hkv = int(rng.choice([1, 2, 4])) if rep <= 16 else 1
    mode = str(rng.choice(["decode", "decode", "prefill"]))
    bs = int(rng.choice([16, 32, 256, 768]))
    window = int(rng.choice([0, 0, 17, 300]))
    budget = 2400 if d <= 128 else 1000
    nseq = int(rng.integers(1, 7))
    seqs = []
    for s in range(nseq):
        cached = int(rng.integers(0, budget // nseq))
        if mode == "decode" or s % 2 == 1:
            seqs.append((cached, 1))
        else:
            seqs.append((cached // 2, int(rng.integers(2, max(3, budget // (4 * nseq))))))
    scale = float(np.float32(1.0 / np.sqrt(d)) * np.float32(rng.uniform(0.5, 2.0)))
    return W.build(f"fuzz-gqa {seed}: d={d} rep={rep} hkv={hkv} {mode} bs={bs} W={window} {seqs}",
                   seqs, is_prefill=mode != "decode", hq=hkv * rep, hkv=hkv, d=d, scale=scale,
                   window=window, rng=rng, paged=True, block_size=bs, pool_cap=40000)


@pytest.mark.parametrize("seed", list(range(32)))
def test_fuzz_gqa(ctx, seed):
    wl = draw_gqa(seed)
    check_attention(ctx, Case(wl, seed=seed), wl.name)
