"""GQA ratios that are not powers of two (query heads per KV head 3, 5, 6, 7: Qwen3-14B has
40 query heads over 8 KV heads, Qwen2.5-7B 28 over 4) and above 8 (12, 16: the MFMA row kernel
carries up to 16 heads of a KV head), through the C ABI against the oracle: decode, paged
prefill with prefix hits and one-query rows, and dense prefill, at d = 64 and 128, page sizes
16, 256 and 768 (not a power of two: the row kernel instead of the MFMA one), with and without a
sliding window.  The bar is the path's: attention within max-abs 1e-4 and rel-L2 1e-5 of the
oracle, every page byte equal.  (Layers/Attention.java:152-171 and :328-396 take any integer
ratio: kvh = h / rep.)"""

import numpy as np
import pytest

from cases import Case
from gpu_checks import check_attention
from nanollvm_amd import Context
from nanollvm_amd import workloads as W

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    with Context(0) as c:
        yield c


CASES = [
    # (rep, hkv, d, mode, block_size, window)
    (5, 8, 128, "decode", 256, 0),     # Qwen3-14B heads
    (5, 8, 128, "prefill", 256, 0),
    (7, 4, 128, "decode", 16, 0),      # Qwen2.5-7B heads
    (7, 4, 128, "prefill", 16, 0),
    (3, 2, 64, "decode", 16, 33),
    (3, 2, 64, "prefill", 256, 33),
    (6, 1, 128, "decode", 256, 0),
    (6, 2, 64, "prefill", 16, 0),
    (5, 1, 64, "dense", 0, 0),
    (7, 2, 128, "dense", 0, 300),
    (16, 1, 128, "decode", 16, 0),
    (12, 2, 64, "decode", 256, 33),
    (16, 2, 128, "prefill", 256, 0),
    (10, 1, 128, "decode", 768, 0),
    (8, 2, 128, "decode", 768, 0),
]


@pytest.mark.parametrize("rep,hkv,d,mode,block_size,window", CASES)
def test_gqa_ratio(ctx, rep, hkv, d, mode, block_size, window):
    rng = np.random.default_rng(rep * 1000 + hkv * 100 + d)
    if mode == "decode":
        seqs = [(int(c), 1) for c in rng.integers(0, 3000, 12)]
    elif mode == "prefill":
        seqs = [(0, 300), (256, 77), (513, 1), (37, 200), (1000, 129)]
    else:
        seqs = [(0, 300), (0, 1), (0, 131)]
    wl = W.build(f"gqa {rep}:1 hkv={hkv} d={d} {mode} bs={block_size} W={window}", seqs,
                 is_prefill=mode != "decode", hq=hkv * rep, hkv=hkv, d=d,
                 scale=float(1.0 / np.sqrt(d)), window=window, rng=rng,
                 paged=mode != "dense", block_size=block_size or 16, pool_cap=1 << 20)
    check_attention(ctx, Case(wl, seed=rep + d), wl.name)
