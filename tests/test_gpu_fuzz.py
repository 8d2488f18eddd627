"""Seeded random sweep of the attention path against the oracle.

Each case draws a configuration: head dim (8 .. 512), GQA ratio (1 .. 8), KV heads, page size
(1 .. 256), sliding window, decode / prefill with cache / dense prefill, and a batch of ragged
sequences (prefix hits, mid-page starts, one-query rows, empty-window edges).  The bar is the
path's: attention within max-abs 1e-4 and rel-L2 1e-5 of the oracle, every page byte equal."""

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
