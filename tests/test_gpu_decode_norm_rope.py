"""Decode steps through the per-head norm + RoPE + attention call (nva_norm_rope_attention_forward:
one kernel normalises, rotates and stores, then the split-KV decode runs), swept over shapes.

Bar: rotated q/k and every page byte bit-exact against the oracle chain (normHeads, RoPE,
Attention.forward: storeKvCache then decode); attention within max-abs 1e-4 and rel-L2 1e-5.
A seeded sweep covers head dims 8..512, GQA ratios 1..16 (several head groups per KV head),
page sizes 1..256, windows, the norm semantics of Qwen3 / Gemma 3 / Gemma 4, with and without
the rotated outputs; a row with no visible key still has its token stored."""

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
    rng = np.random.default_rng(70000 + seed)
    d = int(rng.choice([8, 16, 32, 64, 128, 256, 512]))
    rep = int(rng.choice([1, 2, 4, 8, 16]))
    hkv = int(rng.choice([1, 2, 3]))
    bs = int(rng.choice([1, 4, 16, 64, 256]))
    window = int(rng.choice([0, 0, 1, 5, 33, 300]))
    mode = str(rng.choice(["none", "qwen3", "gemma3", "gemma4"]))
    outputs = bool(rng.integers(0, 2))
    budget = 2500 if d <= 128 else 1200
    nseq = int(rng.integers(1, 9))
    seqs = [(int(rng.integers(0, budget // nseq)), 1) for _ in range(nseq)]
    scale = float(np.float32(1.0 / np.sqrt(d)) * np.float32(rng.uniform(0.5, 2.0)))
    wl = W.build(f"decode norm+rope {seed}: d={d} rep={rep} hkv={hkv} bs={bs} W={window} "
                 f"{mode} {seqs}", seqs, is_prefill=False, hq=hkv * rep, hkv=hkv, d=d,
                 scale=scale, window=window, rng=rng, block_size=bs, pool_cap=40000)
    if mode == "none":
        q_w = k_w = None
    elif mode == "gemma3":
        q_w = (0.1 * rng.standard_normal(d)).astype(np.float32)
        k_w = (0.1 * rng.standard_normal(d)).astype(np.float32)
    else:
        q_w = (1.0 + 0.1 * rng.standard_normal(d)).astype(np.float32)
        k_w = (1.0 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    return wl, mode, q_w, k_w, outputs


@pytest.mark.parametrize("seed", SEEDS)
def test_decode_norm_rope_sweep(ctx, seed):
    wl, mode, q_w, k_w, outputs = draw(seed)
    if mode == "none":
        # No norms: nva_norm_rope_attention_forward with null norms (= nva_rope_attention_forward).
        check_fused(ctx, Case(wl, seed=seed), wl.name, None, None, max_pos=4096, theta=1e6,
                    outputs=outputs, norms=False)
    else:
        check_fused(ctx, Case(wl, seed=seed), wl.name, q_w, k_w, one_plus=mode == "gemma3",
                    v_norm=mode == "gemma4", max_pos=4096, theta=1e6, outputs=outputs)


def test_row_without_keys_still_stores(ctx):
    """A decode row whose context length is 0 attends to nothing (zero output) but its token is
    still stored (Attention.java:221-240 stores every token)."""
    rng = np.random.default_rng(11)
    wl = W.build("decode with an empty row", [(40, 1), (7, 1), (300, 1)], is_prefill=False,
                 hq=4, hkv=2, d=128, scale=W.QWEN_SCALE, rng=rng, block_size=16)
    wl.meta.context_lens[1] = 0
    q_w = (1.0 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    k_w = (1.0 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    check_fused(ctx, Case(wl, seed=12), "decode, empty row", q_w, k_w, max_pos=1024)
