"""The library's step-metadata producers (nva_build_prefill_metadata / nva_build_decode_metadata,
Transformer.preparePrefill / prepareDecode) against the engine-side restatement, field by
field and exactly, over scheduler states the reference's BlockManager produces: prefix-cache
hits, chunked prefill starting mid-page, sequences without pages, decode steps that open a new
page.  Host only: no GPU."""

import numpy as np
import pytest

import engine as E
from nanollvm_amd import step as S


def same(a, b):
    if a is None or b is None:
        return a is None and b is None
    return np.array_equal(np.asarray(a), np.asarray(b))


def check_equal(got, want):
    assert got.is_prefill == want.is_prefill
    for f in ("cu_seqlens_q", "cu_seqlens_k", "slot_mapping", "context_lens", "block_tables",
              "seq_ids", "positions"):
        assert same(getattr(got, f), getattr(want, f)), f
    assert got.max_seqlen_q == want.max_seqlen_q and got.max_seqlen_k == want.max_seqlen_k


def scheduler_state(seed, bs, chunk=None):
    """Prompts with shared prefixes through the BlockManager; optionally chunked."""
    rng = np.random.default_rng(seed)
    bm = E.BlockManager(4096, bs)
    base = rng.integers(0, 1000, 600).tolist()
    seqs = []
    for i in range(int(rng.integers(1, 9))):
        share = int(rng.integers(0, 400))
        toks = base[:share] + rng.integers(0, 1000, int(rng.integers(1, 300))).tolist()
        s = E.Sequence(toks, bs)
        cached = bm.can_allocate(s)
        assert cached >= 0
        bm.allocate(s, cached)
        left = s.num_tokens - s.num_cached_tokens
        s.num_scheduled_tokens = min(left, chunk) if chunk else left
        seqs.append(s)
        # Publish the pages so later prompts can hit them (as the reference does after prefill).
        bm.hash_blocks(s)
    return bm, seqs


@pytest.mark.parametrize("seed", range(12))
@pytest.mark.parametrize("bs", [4, 16, 256, 768])
def test_prefill_matches_engine(seed, bs):
    _, seqs = scheduler_state(seed, bs, chunk=None if seed % 2 else 37)
    check_equal(S.build_prefill_metadata(seqs, bs), E.prepare_prefill(seqs, bs))


@pytest.mark.parametrize("seed", range(12))
@pytest.mark.parametrize("bs", [4, 16, 256, 768])
def test_decode_matches_engine(seed, bs):
    bm, seqs = scheduler_state(seed, bs)
    for s in seqs:
        s.num_cached_tokens += s.num_scheduled_tokens
        s.num_scheduled_tokens = 0
    rng = np.random.default_rng(seed + 100)
    for _ in range(int(rng.integers(1, 2 * bs + 2))):  # enough appends to open new pages
        for s in seqs:
            s.append_token(int(rng.integers(0, 1000)))
            bm.may_append(s)
        check_equal(S.build_decode_metadata(seqs, bs), E.prepare_decode(seqs, bs))


def test_prefill_without_prefix_attaches_no_tables_and_pageless_seq_adds_no_slots():
    bs = 4
    a = E.Sequence(list(range(10)), bs)
    a.block_table = [3, 1, 2]
    a.num_scheduled_tokens = 10
    b = E.Sequence(list(range(5)), bs)  # no pages yet
    b.num_scheduled_tokens = 5
    got = S.build_prefill_metadata([a, b], bs)
    check_equal(got, E.prepare_prefill([a, b], bs))
    assert got.block_tables is None and len(got.slot_mapping) == 10


def test_errors_where_the_reference_throws():
    bs = 4
    a = E.Sequence(list(range(10)), bs)
    a.block_table = [3, 1]          # needs 3 pages
    a.num_scheduled_tokens = 10
    with pytest.raises(S.MetadataError):
        S.build_prefill_metadata([a], bs)
    d = E.Sequence(list(range(3)), bs)  # decode with an empty table
    with pytest.raises(S.MetadataError):
        S.build_decode_metadata([d], bs)
