"""Parity of the fp32 MFMA prefill kernel over its whole configuration space, against the oracle.

The prefill kernel is instantiated for head dims 64, 128, 256 and 512 and for 1, 2, 4 or 8 query
heads per workgroup (GQA ratio 1, 2, 4, 8).  Each case mixes ragged sequences: a prefix hit
(full pages), a mid-page chunk start, a two-query sequence (the smallest MFMA tile), a one-query
row (the row kernel) and lengths that leave partial query tiles and partial key tiles.  It runs
paged with small and with the default page size, and dense (prefillDense), with and without a
sliding window.  Bar: max-abs 1e-4 and rel-L2 1e-5 against the oracle; K/V pages bit-exact.
Each case also checks that the MFMA kernel really ran."""

import numpy as np
import pytest

from cases import Case
from gpu_checks import check_attention, say
from nanollvm_amd import Context
from nanollvm_amd import workloads as W

pytestmark = pytest.mark.gpu

PAGED_SEQS = [(16, 70), (5, 33), (0, 2), (9, 1), (40, 129)]
DENSE_SEQS = [(0, 70), (0, 33), (0, 2), (0, 1), (0, 129)]


@pytest.fixture(scope="module")
def ctx():
    c = Context(0)
    yield c
    c.close()


@pytest.mark.parametrize("layout", ["paged16", "paged256", "dense"])
@pytest.mark.parametrize("window", [0, 37])
@pytest.mark.parametrize("rep", [1, 2, 4, 8])
@pytest.mark.parametrize("d", [64, 128, 256, 512])
def test_mfma_prefill_matrix(ctx, d, rep, window, layout):
    hkv = 2
    hq = hkv * rep
    seed = d * 1000 + rep * 100 + window * 3 + len(layout)
    rng = np.random.default_rng(seed)
    paged = layout != "dense"
    wl = W.build(f"mfma d{d} rep{rep} w{window} {layout}",
                 PAGED_SEQS if paged else DENSE_SEQS, is_prefill=True, hq=hq, hkv=hkv, d=d,
                 scale=float(np.float32(d ** -0.5)), window=window, rng=rng, paged=paged,
                 block_size=16 if layout == "paged16" else 256)
    ctx.reset_stats()
    ctx.set_timing(True)
    try:
        check_attention(ctx, Case(wl, seed=seed), wl.name)
        launches, _ = ctx.kernel_stats("prefill")
    finally:
        ctx.set_timing(False)
    say(f"{wl.name}: prefill kernel launches={launches}")
    assert launches >= 1, "the MFMA prefill kernel did not run"


@pytest.mark.parametrize("block_size", [1, 16, 256])
@pytest.mark.parametrize("is_prefill", [False, True])
def test_long_rows_small_pages(ctx, block_size, is_prefill):
    """Rows of thousands of keys over pages of 1 and 16 tokens: a work item of the row kernel
    (or a segment of the prefill kernel) then spans many pages, up to the number whose block ids
    the kernel stages in LDS; the host caps items and segments at that."""
    rng = np.random.default_rng(block_size * 7 + int(is_prefill))
    if is_prefill:
        seqs = [(2900, 40), (0, 300), (1500, 3)]
    else:
        seqs = [(2999, 1), (1499, 1), (4999, 1), (64, 1)]
    wl = W.build(f"long rows bs{block_size} {'prefill' if is_prefill else 'decode'}", seqs,
                 is_prefill=is_prefill, hq=4, hkv=2, d=128, scale=float(np.float32(128 ** -0.5)),
                 rng=rng, block_size=block_size, pool_cap=20000)
    check_attention(ctx, Case(wl, seed=block_size + 3), wl.name)


@pytest.mark.parametrize("block_size", [32, 64, 128])
@pytest.mark.parametrize("window", [0, 45])
@pytest.mark.parametrize("d", [64, 128, 256])
def test_tile_copies_across_pages(ctx, d, block_size, window):
    """Pages of one to four 32-key tiles: a full tile inside one page is copied from one row
    base (its block id re-read only when the page changes), while the chunk's last tile and tiles
    that a window start or a mid-page chunk start moves across a page boundary take per-row
    addresses.  Ragged sequences mix both kinds in every segment; the window of 45 keys starts
    tiles off the 32-key grid."""
    rng = np.random.default_rng(d + block_size + window)
    seqs = [(block_size * 3, 150), (block_size // 2 + 7, 97), (0, 260), (5 * block_size + 3, 33)]
    wl = W.build(f"tile copies d{d} bs{block_size} w{window}", seqs, is_prefill=True, hq=4,
                 hkv=2, d=d, scale=float(np.float32(d ** -0.5)), window=window, rng=rng,
                 block_size=block_size)
    ctx.reset_stats()
    ctx.set_timing(True)
    try:
        check_attention(ctx, Case(wl, seed=d * 3 + block_size), wl.name)
        launches, _ = ctx.kernel_stats("prefill")
    finally:
        ctx.set_timing(False)
    assert launches >= 1, "the MFMA prefill kernel did not run"


@pytest.mark.parametrize("block_size,new", [(1, 2048), (4, 4096)])
def test_runs_longer_than_page_cap(ctx, block_size, new):
    """Equal runs of key tiles per slot longer than one segment may span over pages of 1 or 4
    tokens (126 pages: 3 or 15 tiles of 32 keys): the planner cuts such a run into several
    segments of the same query tile in the same slot, whichever of its two cuts it keeps (at
    2048 / 4096 new tokens over 256 slots a run is 5 / 17 tiles)."""
    rng = np.random.default_rng(block_size * 11 + new)
    seqs = [(0, new), (700, 64)]
    wl = W.build(f"page-capped runs bs{block_size}", seqs, is_prefill=True, hq=4, hkv=2, d=128,
                 scale=float(np.float32(128 ** -0.5)), rng=rng, block_size=block_size,
                 pool_cap=20000)
    ctx.reset_stats()
    ctx.set_timing(True)
    try:
        check_attention(ctx, Case(wl, seed=block_size + new), wl.name)
        launches, _ = ctx.kernel_stats("prefill")
    finally:
        ctx.set_timing(False)
    assert launches >= 1, "the MFMA prefill kernel did not run"
