"""Prefill steps through the per-head norm + RoPE + attention call (nva_norm_rope_attention_forward:
kernel (a) normalises, rotates and stores, then the MFMA tiles and any qLen = 1 rows run) with
no rotated-q/k output asked for, swept over shapes.

Bar: every page byte bit-exact against the oracle chain (normHeads, RoPE, Attention.forward);
attention within max-abs 1e-4 and rel-L2 1e-5 of it; and the same call with q_out/k_out given
returns the oracle's rotated q bit for bit and bit-identical attention.  A seeded sweep covers
head dims 64..512, GQA ratios 1..8, dense and paged KV with page sizes 1..256, prefix hits and
mid-page chunk starts, windows, the norm semantics of Qwen3 / Gemma 3 / Gemma 4 and RoPE alone,
and steps that mix qLen = 1 sequences (row items) into the tiles."""

import numpy as np
import pytest

from cases import Case
from gpu_checks import check_fused
from nanollvm_amd import Context
from nanollvm_amd import workloads as W

pytestmark = pytest.mark.gpu

SEEDS = list(range(32))


@pytest.fixture(scope="module")
def ctx():
    c = Context(0)
    yield c
    c.close()


def draw(seed):
    rng = np.random.default_rng(90000 + seed)
    d = int(rng.choice([64, 128, 128, 256, 512]))
    rep = int(rng.choice([1, 2, 3, 4, 8]))
    hkv = int(rng.choice([1, 2, 3]))
    paged = bool(rng.integers(0, 4) > 0)
    bs = int(rng.choice([1, 16, 64, 256])) if paged else 16
    window = int(rng.choice([0, 0, 7, 100]))
    mode = str(rng.choice(["none", "qwen3", "gemma3", "gemma4"]))
    with_row = bool(rng.integers(0, 5) == 0)
    nseq = int(rng.integers(1, 5))
    budget = 900 if d <= 128 else 400
    seqs = []
    for _ in range(nseq):
        new = int(rng.integers(2, budget // nseq + 3))
        cached = int(rng.integers(0, budget // nseq + 1)) if paged else 0
        seqs.append((cached, new))
    if with_row:
        seqs.insert(int(rng.integers(0, len(seqs) + 1)),
                    (int(rng.integers(0, 200)) if paged else 0, 1))
    scale = float(np.float32(1.0 / np.sqrt(d)) * np.float32(rng.uniform(0.5, 2.0)))
    wl = W.build(f"prefill norm+rope {seed}: d={d} rep={rep} hkv={hkv} paged={paged} bs={bs} "
                 f"W={window} {mode} {seqs}", seqs, is_prefill=True, hq=hkv * rep, hkv=hkv,
                 d=d, scale=scale, window=window, rng=rng, paged=paged, block_size=bs,
                 pool_cap=40000)
    if mode == "none":
        q_w = k_w = None
    elif mode == "gemma3":
        q_w = (0.1 * rng.standard_normal(d)).astype(np.float32)
        k_w = (0.1 * rng.standard_normal(d)).astype(np.float32)
    else:
        q_w = (1.0 + 0.1 * rng.standard_normal(d)).astype(np.float32)
        k_w = (1.0 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    return wl, mode, q_w, k_w


@pytest.mark.parametrize("seed", SEEDS)
def test_prefill_norm_rope_sweep(ctx, seed):
    wl, mode, q_w, k_w = draw(seed)
    if mode == "none":
        check_fused(ctx, Case(wl, seed=seed), wl.name, None, None, max_pos=4096, theta=1e6,
                    outputs=False, norms=False, twin=True)
    else:
        check_fused(ctx, Case(wl, seed=seed), wl.name, q_w, k_w, one_plus=mode == "gemma3",
                    v_norm=mode == "gemma4", max_pos=4096, theta=1e6, outputs=False, twin=True)


@pytest.mark.parametrize("mode", ["qwen3", "gemma3"])
def test_prefill_norm_rope_full_size(ctx, mode):
    """The Qwen3-4B prefill shape (32 q heads over 8 KV heads, d = 128), 4096 new tokens over
    four sequences with prefix hits, weighted norms."""
    rng = np.random.default_rng(5)
    seqs = [(0, 1024), (256, 1024), (1000, 1024), (3, 1024)]
    wl = W.build(f"prefill norm+rope Qwen3-4B {mode}", seqs, is_prefill=True, hq=32, hkv=8, d=128,
                 scale=W.QWEN_SCALE, rng=rng, block_size=256)
    off = 0.0 if mode == "gemma3" else 1.0
    q_w = (off + 0.1 * rng.standard_normal(128)).astype(np.float32)
    k_w = (off + 0.1 * rng.standard_normal(128)).astype(np.float32)
    check_fused(ctx, Case(wl, seed=6), wl.name, q_w, k_w, one_plus=mode == "gemma3",
                max_pos=4096, theta=1e6, outputs=False, twin=True)
