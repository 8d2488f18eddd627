"""Edge cases of Attention.forward through the C ABI.

* q rows past the last sequence (cu_seqlens_q ends before the tensor does) stay zero, as the
  reference's fresh Tensor.zeros output leaves them (Attention.java:152-171) -- checked with an
  output buffer that held NaN just before;
* a decode row with no cached keys (context 0) gives zeros (Attention.java:393, l == 0);
* an empty batch is a no-op."""

import numpy as np
import pytest
import torch

from gpu_checks import dev, say
from nanollvm_amd import Attention, Context, KvCacheArena
from oracle import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = Context(0)
    yield c
    c.close()


def poison_allocator(shape):
    """Leaves a NaN-filled block of this size in torch's caching allocator, so that the next
    torch.empty of the same size starts out as NaN rather than zero."""
    t = torch.full(shape, float("nan"), device="cuda")
    torch.cuda.synchronize()
    del t


def test_rows_past_the_last_sequence_stay_zero(ctx):
    say("edges: uncovered rows")
    rng = np.random.default_rng(3)
    T, hq, hkv, d = 12, 4, 2, 32
    q = rng.standard_normal((T, hq, d), dtype=np.float32)
    k = rng.standard_normal((T, hkv, d), dtype=np.float32)
    v = rng.standard_normal((T, hkv, d), dtype=np.float32)
    arena = KvCacheArena(ctx, 1, 2, 16, hkv, d)
    try:
        ctx.set(True, [0, 5, 8], [0, 5, 8], 5, 5, None, None, None, None)
        ctx.bind_kv_cache(arena)
        poison_allocator((T, hq, d))
        out = Attention(hq, d, 0.2, hkv, 0, 0).forward(dev(q), dev(k), dev(v), ctx)
        ctx.sync()
        got = out.cpu().numpy()
        want = O.attention_forward(hq, d, 0.2, hkv, is_prefill=True, q=q, k=k, v=v,
                                   cu_q=[0, 5, 8], cu_k=[0, 5, 8])
        assert np.all(got[8:] == 0.0), "rows past the last sequence must be zero"
        assert np.max(np.abs(got[:8] - want[:8])) <= 1e-5
    finally:
        ctx.clear()
        arena.close()


def test_decode_row_with_empty_context_is_zero(ctx):
    say("edges: decode with context 0")
    rng = np.random.default_rng(4)
    hq, hkv, d, bs = 4, 2, 16, 16
    q = rng.standard_normal((2, hq, d), dtype=np.float32)
    arena = KvCacheArena(ctx, 1, 4, bs, hkv, d)
    kc = rng.standard_normal((4, bs, hkv, d), dtype=np.float32)
    arena.write(0, 0, kc)
    arena.write(0, 1, kc)
    try:
        # Row 0 sees 5 keys of page 2; row 1 has context 0 (no key visible).
        ctx.set(False, None, None, 0, 5, None, [5, 0], [[2], [3]], None)
        ctx.bind_kv_cache(arena)
        poison_allocator((2, hq, d))
        out = Attention(hq, d, 0.25, hkv, 0, 0).forward(dev(q), None, None, ctx)
        ctx.sync()
        got = out.cpu().numpy()
        want = O.attention_forward(hq, d, 0.25, hkv, is_prefill=False, q=q, context_lens=[5, 0],
                                   block_tables=[[2], [3]], k_cache=kc.copy(), v_cache=kc.copy())
        assert np.all(got[1] == 0.0)
        assert np.max(np.abs(got[0] - want[0])) <= 1e-5
    finally:
        ctx.clear()
        arena.close()


def test_empty_batch(ctx):
    say("edges: empty batch")
    arena = KvCacheArena(ctx, 1, 2, 16, 2, 16)
    try:
        ctx.set(True, [0], [0], 0, 0, None, None, None, None)
        ctx.bind_kv_cache(arena)
        z = torch.empty((0, 4, 16), device="cuda")
        zk = torch.empty((0, 2, 16), device="cuda")
        out = Attention(4, 16, 0.25, 2, 0, 0).forward(z, zk, zk, ctx)
        ctx.sync()
        assert tuple(out.shape) == (0, 4, 16)
    finally:
        ctx.clear()
        arena.close()
