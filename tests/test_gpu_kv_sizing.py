"""Sizing the device KV arena (Config.resolveNumKvcacheBlocks, llm/Config.java:93-125, with the
device's free HBM in place of the Java heap) through the C ABI: the count nva_kv_blocks_that_fit
returns for a fraction of free HBM allocates, and about twice that count fails with NVA_E_OOM
and leaves the device usable; the rest of the reference's formula (configured count, the
maxNumSeqs x maxModelLen estimate, the floor of 32, the kvHeapFraction range) holds."""

import ctypes

import numpy as np
import pytest
import torch

from gpu_checks import say
from nanollvm_amd import Context, KvCacheArena, NvaError, _native as N
from nanollvm_amd.layers import IllegalArgumentException

pytestmark = pytest.mark.gpu

# Qwen3-0.6B: 28 layers, 8 KV heads of 128 dims, 256-token pages.
LAYERS, HKV, D, BS = 28, 8, 128, 256
PER_BLOCK = 2 * BS * HKV * D * 4 * LAYERS


@pytest.fixture(scope="module")
def ctx():
    c = Context(0)
    yield c
    c.close()


def test_formula_and_allocation(ctx):
    torch.cuda.empty_cache()
    blocks, free = KvCacheArena.blocks_that_fit(ctx, LAYERS, BS, HKV, head_dim=D, fraction=0.6)
    say(f"kv sizing: free {free / 2**30:.1f} GiB, {PER_BLOCK} B per page, fraction 0.6 -> "
        f"{blocks} pages")
    assert blocks == max(32, int(free * 0.6) // PER_BLOCK)
    arena = KvCacheArena(ctx, LAYERS, blocks, BS, HKV, D)
    say(f"kv sizing: {blocks} pages allocated ({blocks * PER_BLOCK / 2**30:.1f} GiB)")
    per_page = BS * HKV * D
    page = arena.read(LAYERS - 1, 1, offset=(blocks - 1) * per_page, count=per_page)
    arena.close()
    assert not np.any(page)  # zero-filled to the last page
    with pytest.raises(NvaError) as err:
        KvCacheArena(ctx, LAYERS, 2 * blocks, BS, HKV, D)
    st = N.load().nva_status_string(N.NVA_E_OOM).decode()
    say(f"kv sizing: {2 * blocks} pages -> {err.value}")
    assert "out of memory" in str(err.value).lower() or st in str(err.value)
    # The failed allocation left nothing behind and no error pending: the same count fits again.
    again, _ = KvCacheArena.blocks_that_fit(ctx, LAYERS, BS, HKV, head_dim=D, fraction=0.6)
    assert abs(again - blocks) <= max(2, blocks // 100)
    x = torch.ones(1 << 20, device="cuda").sum()
    assert float(x) == float(1 << 20)


def test_oom_status_code(ctx):
    blocks, _ = KvCacheArena.blocks_that_fit(ctx, 1, BS, HKV, head_dim=D, fraction=1.0)
    hd = np.asarray([D], np.int32)
    h = ctypes.c_void_p()
    st = N.load().nva_kv_create(ctx.handle, 1, 2 * blocks, BS, HKV, hd.ctypes.data, None,
                                ctypes.byref(h))
    say(f"kv sizing: one layer of {2 * blocks} pages -> status {st}")
    assert st == N.NVA_E_OOM and not h.value


def test_reference_rules(ctx):
    hd = [D] * LAYERS
    # A configured count wins (Config.java:100-102).
    assert KvCacheArena.resolve_num_blocks(ctx, 77, 8, 40960, BS, HKV, hd) == 77
    # The estimate max(maxNumSeqs * ceil(maxModelLen / blockSize), 128) wins when it is smaller.
    assert KvCacheArena.resolve_num_blocks(ctx, 0, 4, 1000, BS, HKV, hd) == 128
    assert KvCacheArena.resolve_num_blocks(ctx, 0, 64, 4096, BS, HKV, hd) == 64 * 16
    # Layers without pages (shared KV) add no bytes per page.
    a, _ = KvCacheArena.blocks_that_fit(ctx, 2, BS, HKV, head_dims=[D, D], fraction=0.5)
    b, _ = KvCacheArena.blocks_that_fit(ctx, 2, BS, HKV, head_dims=[D, D],
                                        allocate=[True, False], fraction=0.5)
    assert abs(b - 2 * a) <= 2
    # The floor of 32 pages, whatever the page size.
    huge, _ = KvCacheArena.blocks_that_fit(ctx, 1, 1 << 20, 64, head_dim=4096, fraction=1e-6)
    assert huge == 32
    # kvHeapFraction must lie in (0, 1] (Config.java:66-69).
    for f in (0.0, -0.5, 1.5, float("nan")):
        with pytest.raises(IllegalArgumentException):
            KvCacheArena.blocks_that_fit(ctx, 1, BS, HKV, head_dim=D, fraction=f)
