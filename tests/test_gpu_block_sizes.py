"""Page sizes the reference accepts beyond 256: any multiple of 256 (Config.java:60-61), so 512
(a power of two: the kernels' aligned paths) and 768 / 1280 (not: the paths that divide by the
page size).  Decode, paged prefill with a prefix hit and a mid-page chunk start, and a mixed step
(MFMA tiles plus qLen = 1 rows), through the plain attention call and through the norm + RoPE +
store call.

Bar: attention within max-abs 1e-4 and rel-L2 1e-5 of the oracle; every page byte and the
rotated q/k bit-exact."""

import numpy as np
import pytest

from cases import Case
from gpu_checks import check_attention, check_fused
from nanollvm_amd import Context
from nanollvm_amd import workloads as W

pytestmark = pytest.mark.gpu

SIZES = [512, 768, 1280]


@pytest.fixture(scope="module")
def ctx():
    c = Context(0)
    yield c
    c.close()


def workload(kind, bs, seed):
    rng = np.random.default_rng(seed)
    if kind == "decode":
        seqs = [(int(c), 1) for c in rng.integers(1, 3 * bs, size=6)]
        return W.build(f"decode bs={bs}", seqs, is_prefill=False, hq=8, hkv=4, d=128,
                       scale=W.QWEN_SCALE, rng=rng, block_size=bs)
    if kind == "prefill":
        # A full-page prefix hit, a mid-page chunk start, a short and a long new part.
        seqs = [(bs, 200), (bs // 2 + 37, 90), (0, 300), (2 * bs + 5, 1)]
        return W.build(f"paged prefill bs={bs}", seqs, is_prefill=True, hq=8, hkv=4, d=128,
                       scale=W.QWEN_SCALE, rng=rng, block_size=bs)
    # Mixed: two prefill chunks and decode rows in one step.
    seqs = [(bs + 11, 128), (0, 96)] + [(int(c), 1) for c in rng.integers(bs, 3 * bs, size=5)]
    return W.build(f"mixed bs={bs}", seqs, is_prefill=True, hq=8, hkv=2, d=128,
                   scale=W.QWEN_SCALE, rng=rng, block_size=bs)


@pytest.mark.parametrize("bs", SIZES)
@pytest.mark.parametrize("kind", ["decode", "prefill", "mixed"])
def test_attention_page_size(ctx, kind, bs):
    wl = workload(kind, bs, seed=bs + len(kind))
    check_attention(ctx, Case(wl, seed=bs), wl.name)


@pytest.mark.parametrize("bs", SIZES)
@pytest.mark.parametrize("kind", ["decode", "prefill"])
def test_norm_rope_page_size(ctx, kind, bs):
    wl = workload(kind, bs, seed=3 * bs + len(kind))
    rng = np.random.default_rng(bs)
    q_w = (1.0 + 0.1 * rng.standard_normal(wl.d)).astype(np.float32)
    k_w = (1.0 + 0.1 * rng.standard_normal(wl.d)).astype(np.float32)
    check_fused(ctx, Case(wl, seed=bs + 1), "norm+rope " + wl.name, q_w, k_w, max_pos=4096,
                theta=1e6)
