"""Host-side metadata producers (the engine side of the boundary) against the reference's own
test and the invariants the attention kernels rely on."""

import numpy as np

import engine as E
from nanollvm_amd import workloads as W


def _prefill_once(bm, seq):
    cached = bm.can_allocate(seq)
    assert cached >= 0
    bm.allocate(seq, cached)
    seq.num_scheduled_tokens = seq.num_tokens - seq.num_cached_tokens
    bm.hash_blocks(seq)
    seq.num_cached_tokens += seq.num_scheduled_tokens
    seq.num_scheduled_tokens = 0
    return cached


def test_block_manager_prefix_cache_reference_case():
    """T/CoreUnitTest.java:368-383: 16 blocks of 4; a prompt sharing 8 tokens reuses 2 pages."""
    bm = E.BlockManager(16, 4)
    a = E.Sequence([1, 2, 3, 4, 5, 6, 7, 8, 9], 4)
    _prefill_once(bm, a)
    b = E.Sequence([1, 2, 3, 4, 5, 6, 7, 8, 10], 4)
    assert bm.can_allocate(b) == 2


def test_last_page_is_never_a_prefix_hit():
    bm = E.BlockManager(16, 4)
    a = E.Sequence([1, 2, 3, 4, 5, 6, 7, 8], 4)
    _prefill_once(bm, a)
    b = E.Sequence([1, 2, 3, 4, 5, 6, 7, 8], 4)
    assert bm.can_allocate(b) == 1


def test_prepare_prefill_with_prefix_hit_and_decode():
    bs = 4
    bm = E.BlockManager(32, bs)
    a = E.Sequence(list(range(100, 111)), bs)
    _prefill_once(bm, a)
    b = E.Sequence(list(range(100, 109)) + [7, 7, 7], bs)
    cached = bm.can_allocate(b)
    assert cached == 2
    bm.allocate(b, cached)
    b.num_scheduled_tokens = b.num_tokens - b.num_cached_tokens
    meta = E.prepare_prefill([b], bs)
    assert meta.cu_seqlens_q.tolist() == [0, 4]
    assert meta.cu_seqlens_k.tolist() == [0, 12]       # full context through the chunk end
    assert meta.positions.tolist() == [8, 9, 10, 11]
    tab = b.block_table
    want = [tab[t // bs] * bs + t % bs for t in range(8, 12)]
    assert meta.slot_mapping.tolist() == want
    assert meta.block_tables is not None and meta.block_tables[0].tolist() == tab
    # Decode: appending a token that opens a new page allocates exactly one block.
    b.num_cached_tokens += b.num_scheduled_tokens
    b.num_scheduled_tokens = 0
    b.append_token(5)
    assert bm.can_append(b)
    bm.may_append(b)
    assert len(b.block_table) == 4
    d = E.prepare_decode([a, b], bs)
    assert d.context_lens.tolist() == [11, 13]
    assert d.positions.tolist() == [10, 12]
    assert d.slot_mapping[1] == b.block_table[3] * bs + 0
    assert d.block_tables.shape == (2, 4) and d.block_tables[0, 3] == -1


def test_mid_page_chunk_slots():
    s = E.Sequence(list(range(20)), 4)
    s.block_table = [9, 3, 7, 1, 5]
    s.num_cached_tokens = 6
    s.num_scheduled_tokens = 11
    meta = E.prepare_prefill([s], 4)
    want = [s.block_table[t // 4] * 4 + t % 4 for t in range(6, 17)]
    assert meta.slot_mapping.tolist() == want


def test_hash_is_deterministic_and_chained():
    h1 = E.BlockManager.compute_hash([1, 2, 3, 4], -1)
    h2 = E.BlockManager.compute_hash([1, 2, 3, 4], -1)
    h3 = E.BlockManager.compute_hash([1, 2, 3, 4], h1)
    assert h1 == h2 and h1 != h3
    assert -2**63 <= h1 < 2**63


def test_workload_geometry():
    wl = W.qwen3_decode_large()
    pages = sum(-(-(c + n) // 256) for c, n in wl.seqs)
    assert wl.num_blocks == min(8191, int(np.ceil(1.25 * pages)))
    used = [b for t in wl.tables for b in t]
    assert len(set(used)) == len(used) and max(used) < wl.num_blocks
    assert wl.meta.context_lens.tolist() == [c + 1 for c, _ in wl.seqs]
    c2 = W.qwen3_prefill()
    assert c2.meta.cu_seqlens_q.tolist() == [0, 512, 1536, 3072, 4096]
    assert c2.meta.cu_seqlens_k.tolist() == [0, 512, 1536, 3072, 5120]
    assert c2.visible_pairs() == 3_409_920
