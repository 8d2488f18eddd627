"""Parity of the per-head RMSNorm (standalone and fused with RoPE + store + attention) on the
GPU, through the C ABI, against the CPU oracle.

Bar: normalised, rotated q/k and every page byte bit-exact (the norm follows the reference's
scalar sumSquares order); attention outputs within max-abs 1e-4 and rel-L2 1e-5."""

import sys

import numpy as np
import pytest
import torch

from cases import Case, rel_l2, small_cases
from gpu_checks import EPS, check_fused
from nanollvm_amd import Attention, Context, KvCacheArena, RMSNorm, RotaryEmbedding
from nanollvm_amd import workloads as W
from oracle import oracle as O

pytestmark = pytest.mark.gpu

MAX_ABS = 1e-4
REL_L2 = 1e-5


def say(msg):
    print(f"[gpu] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ctx():
    c = Context(0)
    yield c
    c.close()


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("width", [3, 7, 128, 256, 1024, 4100])
@pytest.mark.parametrize("kind", ["weightless", "weight", "one_plus"])
def test_rms_norm_bit_exact(ctx, width, kind):
    say(f"rms_norm width={width} {kind}")
    rng = np.random.default_rng(width + len(kind))
    x = (rng.standard_normal((37, width)) * 3.0).astype(np.float32)
    w = None if kind == "weightless" else rng.standard_normal(width).astype(np.float32)
    norm = RMSNorm(None if w is None else dev(w), EPS, kind == "one_plus")
    got = norm.forward(dev(x), ctx)
    ctx.sync()
    want = O.rms_norm(x, w, EPS, kind == "one_plus")
    diff = bits(got.cpu().numpy()) != bits(want)
    assert not diff.any(), f"{int(diff.sum())} of {diff.size} elements differ"


def test_rms_norm_order_known_answer(ctx):
    """[4096, 1, 1, 1]: the scalar order gives sum 2^24 exactly (a pairwise or lane-split order
    gives 2^24 + 2), so the output pins the summation order on the device too."""
    x = np.zeros((1, 128), np.float32)
    x[0, :4] = [4096.0, 1.0, 1.0, 1.0]
    got = RMSNorm.weightless(0.0).forward(dev(x), ctx).cpu().numpy()
    inv = np.float32(1.0 / np.sqrt(2.0 ** 17))
    assert got[0, 1] == inv and got[0, 0] == np.float32(np.float32(4096.0) * inv)


SMALL = small_cases()


@pytest.mark.parametrize("name", ["prefill_cache", "decode_gqa", "prefill_dense",
                                  "decode_mqa_window", "prefill_cache_window"])
@pytest.mark.parametrize("mode", ["qwen3", "gemma3", "gemma4"])
def test_fused_norm_small(ctx, name, mode):
    wl = SMALL[name]
    rng = np.random.default_rng(5)
    qw = rng.standard_normal(wl.d).astype(np.float32)
    kw = rng.standard_normal(wl.d).astype(np.float32)
    check_fused(ctx, Case(wl, seed=43), f"norm {mode} {name}", qw, kw,
                one_plus=mode == "gemma3", v_norm=mode == "gemma4")


def test_fused_norm_qwen3_prefill_full_size(ctx):
    """Qwen3-0.6B varlen prefill 512/1024/1536/2048 (4 cached pages on the last sequence) with
    q_norm/k_norm weights, RoPE theta 1e6."""
    wl = W.qwen3_prefill()
    rng = np.random.default_rng(6)
    qw = (1.0 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    kw = (1.0 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    check_fused(ctx, Case(wl, seed=0), "norm qwen3 prefill", qw, kw, max_pos=wl.max_pos,
                theta=wl.rope_theta)


def test_fused_norm_qwen3_decode_full_size(ctx):
    wl = W.qwen3_decode_small()
    rng = np.random.default_rng(7)
    qw = (1.0 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    kw = (1.0 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    check_fused(ctx, Case(wl, seed=0), "norm qwen3 decode B=8", qw, kw, max_pos=wl.max_pos,
                theta=wl.rope_theta)


def test_fused_norm_gemma3_decode_full_size(ctx):
    wl = W.gemma3_decode(local=True)
    rng = np.random.default_rng(8)
    qw = (0.1 * rng.standard_normal(256)).astype(np.float32)
    kw = (0.1 * rng.standard_normal(256)).astype(np.float32)
    check_fused(ctx, Case(wl, seed=0), "norm gemma3 local decode", qw, kw, one_plus=True,
                max_pos=wl.max_pos, theta=wl.rope_theta)


@pytest.mark.parametrize("is_prefill", [True, False])
def test_fused_norm_gemma4_global_d512(ctx, is_prefill):
    """Gemma-4-text global layer shape (8 q / 1 kv heads, d = 512, scale 1; Gemma4ForCausalLM.
    java:164-197): q/k norm weights and the weightless v norm.  A 512-wide row holds two float4
    columns per lane, so its sum of squares folds 128 group sums in two chains; q, k and the
    pages must equal the oracle bit for bit."""
    rng = np.random.default_rng(9)
    seqs = [(0, 70), (33, 41), (5, 1)] if is_prefill else [(c - 1, 1) for c in (3, 64, 200, 517)]
    wl = W.build("gemma4 global d512", seqs, is_prefill=is_prefill, hq=8, hkv=1, d=512,
                 scale=1.0, rng=rng, block_size=16)
    qw = (1.0 + 0.1 * rng.standard_normal(512)).astype(np.float32)
    kw = (1.0 + 0.1 * rng.standard_normal(512)).astype(np.float32)
    check_fused(ctx, Case(wl, seed=3), f"norm gemma4 d512 prefill={is_prefill}", qw, kw,
                v_norm=True, max_pos=1024, theta=1e6)
