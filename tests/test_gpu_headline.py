"""Paged workloads at their full size, run whole through the C ABI, checked where the oracle
would otherwise need the whole pool on the host:

* the headline decode: Qwen3-0.6B attention shape (16 q / 8 kv heads, d = 128), 256 rows with
  contexts log-uniform in [128, 32768] over 8191 shuffled 256-token pages (17 GB of K/V);
* the mixed step: Qwen3-4B-like (32 q / 8 kv heads), 4 prefill chunks of 512 tokens after
  U[0, 4096] cached tokens plus 64 decode rows with contexts U[4096, 16384] (5.4 GB read).

For each:
* every query row matches the oracle (Attention.decode / prefillWithCache,
  Attention.java:263-299): the sequences are taken in batches whose pages, copied to the host
  after the step, fit in 1 GB, and the oracle runs on each batch with renumbered tables;
  max-abs and rel-L2 are taken over all rows;
* block indexing (BlockManager hands out any block ids, BlockManager.java:147-266): the same
  step over a second arena holding the same pages at permuted block ids, with the tables and
  slots renumbered to match, gives bit-identical output and stores the same bits;
* the store (Attention.storeKvCache, Attention.java:221-240): every new K and V row sits at its
  slot, bit for bit."""

import numpy as np
import pytest
import torch

from cases import rel_l2
from gpu_checks import MAX_ABS, REL_L2, arena_views, bits, fill_normal, say
from nanollvm_amd import Attention, Context, KvCacheArena
from nanollvm_amd import workloads as W
from oracle import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = Context(0)
    yield c
    c.close()


def stored_rows(arena, slots, row_floats):
    """K and V rows at the given slots, gathered on the device."""
    k, v = arena_views(arena)
    idx = torch.from_numpy(np.asarray(slots, np.int64)).cuda()
    return (k.view(-1, row_floats).index_select(0, idx).cpu().numpy(),
            v.view(-1, row_floats).index_select(0, idx).cpu().numpy())


def seq_extent(m, s):
    """(first q row, q rows, keys) of sequence s of the step."""
    if m.is_prefill:
        q0, q1 = int(m.cu_seqlens_q[s]), int(m.cu_seqlens_q[s + 1])
        return q0, q1 - q0, int(m.cu_seqlens_k[s + 1] - m.cu_seqlens_k[s])
    return s, 1, int(m.context_lens[s])


def oracle_batch(wl, arena, q, picks):
    """The oracle on sequences ``picks`` over a host copy of just their pages, with the tables
    renumbered to the copy: (q rows, output rows)."""
    m, bs, hkv, d = wl.meta, wl.block_size, wl.hkv, wl.d
    keys = [seq_extent(m, s)[2] for s in picks]
    pages = [m.block_tables[s][: (k + bs - 1) // bs] for s, k in zip(picks, keys)]
    flat = np.concatenate(pages).astype(np.int64)
    sel = torch.from_numpy(flat).cuda()
    ka, va = arena_views(arena)
    kc = ka.index_select(0, sel).cpu().numpy().reshape(len(flat), bs, hkv, d)
    vc = va.index_select(0, sel).cpu().numpy().reshape(len(flat), bs, hkv, d)
    tables = np.full((len(picks), max(len(p) for p in pages)), -1, np.int32)
    start = 0
    for i, p in enumerate(pages):
        tables[i, : len(p)] = np.arange(start, start + len(p))
        start += len(p)
    qrows = np.concatenate([np.arange(seq_extent(m, s)[0], sum(seq_extent(m, s)[:2]))
                            for s in picks])
    kw = dict(block_tables=tables, k_cache=kc, v_cache=vc, threads=16)
    if m.is_prefill:
        cu_q = np.concatenate([[0], np.cumsum([seq_extent(m, s)[1] for s in picks])])
        cu_k = np.concatenate([[0], np.cumsum(keys)])
        kw.update(cu_q=cu_q.astype(np.int32), cu_k=cu_k.astype(np.int32))
    else:
        kw.update(context_lens=np.asarray(keys, np.int32))
    want = O.attention_forward(wl.hq, d, wl.scale, hkv, is_prefill=m.is_prefill, q=q[qrows],
                               **kw)
    return qrows, want


def check_all_rows(wl, arena, q, out, name, batch_bytes=1 << 30):
    """Every query row of the step against the oracle, in batches of sequences whose K + V
    pages fit ``batch_bytes`` on the host; max-abs and rel-L2 over all rows."""
    m, bs, hkv, d = wl.meta, wl.block_size, wl.hkv, wl.d
    page_bytes = 2 * bs * hkv * d * 4
    per_batch = max(1, batch_bytes // page_bytes)
    nseq = len(wl.seqs)
    npages = [(seq_extent(m, s)[2] + bs - 1) // bs for s in range(nseq)]
    batches, cur, cur_pages = [], [], 0
    for s in range(nseq):
        if cur and cur_pages + npages[s] > per_batch:
            batches.append(cur)
            cur, cur_pages = [], 0
        cur.append(s)
        cur_pages += npages[s]
    if cur:
        batches.append(cur)
    err, num, den, rows = 0.0, 0.0, 0.0, 0
    for bi, picks in enumerate(batches):
        qrows, want = oracle_batch(wl, arena, q, picks)
        got = out[qrows]
        diff = got.astype(np.float64) - want.astype(np.float64)
        err = max(err, float(np.max(np.abs(diff))))
        num += float(np.sum(diff * diff))
        den += float(np.sum(want.astype(np.float64) ** 2))
        rows += len(qrows)
        say(f"{name}: batch {bi + 1}/{len(batches)}: {len(picks)} sequences, "
            f"{sum(npages[s] for s in picks)} pages, running max_abs={err:.3e}")
    rl2 = float(np.sqrt(num / den)) if den > 0 else 0.0
    say(f"{name}: all {rows} q rows of {nseq} sequences: max_abs={err:.3e} rel_l2={rl2:.3e}")
    assert rows == wl.tokens
    assert err <= MAX_ABS and rl2 <= REL_L2, (err, rl2)


def run_full_size(ctx, wl, name):
    m = wl.meta
    nb, bs, hkv, d, hq = wl.num_blocks, wl.block_size, wl.hkv, wl.d, wl.hq
    row = hkv * d
    say(f"{name}: {len(wl.seqs)} sequences, {wl.tokens} q rows, {nb} pages of {bs}")
    g = torch.Generator(device="cuda")
    g.manual_seed(77)
    q = torch.randn((wl.tokens, hq, d), device="cuda", generator=g)
    k = torch.randn((wl.tokens, hkv, d), device="cuda", generator=g)
    v = torch.randn((wl.tokens, hkv, d), device="cuda", generator=g)
    qh, kh, vh = q.cpu().numpy(), k.cpu().numpy(), v.cpu().numpy()

    rng = np.random.default_rng(5)
    perm = rng.permutation(nb).astype(np.int32)  # page j of arena A is page perm[j] of B
    tables_b = np.where(m.block_tables >= 0, perm[np.maximum(m.block_tables, 0)], -1)
    tables_b = tables_b.astype(np.int32)
    slots_b = (perm[m.slot_mapping // bs] * bs + m.slot_mapping % bs).astype(np.int32)

    a_arena = KvCacheArena(ctx, 1, nb, bs, hkv, d)
    b_arena = KvCacheArena(ctx, 1, nb, bs, hkv, d)
    try:
        say(f"{name}: filling arena A, copying its pages to permuted ids in B")
        fill_normal(a_arena, 1234)
        idx = torch.from_numpy(perm.astype(np.int64)).cuda()
        for ta, tb in zip(arena_views(a_arena), arena_views(b_arena)):
            tb.index_copy_(0, idx, ta)
        torch.cuda.synchronize()
        attn = Attention(hq, d, wl.scale, hkv, wl.window, 0)

        say(f"{name}: step over arena A")
        ctx.set(**m.context_args())
        ctx.bind_kv_cache(a_arena)
        out_a = attn.forward(q, k, v, ctx).cpu().numpy()
        say(f"{name}: step over arena B (permuted pages)")
        args = m.context_args()
        args.update(block_tables=tables_b, slot_mapping=slots_b)
        ctx.set(**args)
        ctx.bind_kv_cache(b_arena)
        out_b = attn.forward(q, k, v, ctx).cpu().numpy()
        ctx.clear()
        assert np.all(np.isfinite(out_a))
        assert np.array_equal(bits(out_a), bits(out_b)), "output depends on the block ids"

        for arena, slots in ((a_arena, m.slot_mapping), (b_arena, slots_b)):
            ks, vs = stored_rows(arena, slots, row)
            assert np.array_equal(bits(ks), bits(kh.reshape(-1, row))), "stored K differs"
            assert np.array_equal(bits(vs), bits(vh.reshape(-1, row))), "stored V differs"

        check_all_rows(wl, a_arena, qh, out_a, name)
    finally:
        ctx.clear()
        b_arena.close()
        a_arena.close()


def test_headline_decode_full_size(ctx):
    run_full_size(ctx, W.qwen3_decode_large(), "headline decode")


def test_mixed_step_full_size(ctx):
    run_full_size(ctx, W.qwen3_4b_mixed(), "mixed step")
