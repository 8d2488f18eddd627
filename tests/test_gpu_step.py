"""End-to-end on the GPU: the library builds and uploads the step metadata from the scheduler's
sequences (Context.prepare_prefill / prepare_decode), then the attention layer runs on it; the
result equals the oracle driven by the engine-side restatement of the same producers."""

import sys

import numpy as np
import pytest
import torch

from cases import rel_l2
from nanollvm_amd import Attention, Context, KvCacheArena
import engine as E
from oracle import oracle as O

pytestmark = pytest.mark.gpu

BS, HQ, HKV, D = 16, 4, 2, 32


def say(msg):
    print(f"[gpu] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ctx():
    c = Context(0)
    yield c
    c.close()


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_prepare_then_attend(ctx):
    rng = np.random.default_rng(77)
    bm = E.BlockManager(256, BS)
    base = rng.integers(0, 500, 200).tolist()
    seqs = []
    for i in range(6):
        toks = base[:int(rng.integers(0, 120))] + rng.integers(0, 500, int(rng.integers(1, 90))).tolist()
        s = E.Sequence(toks, BS)
        bm.allocate(s, bm.can_allocate(s))
        s.num_scheduled_tokens = min(s.num_tokens - s.num_cached_tokens, 50)
        bm.hash_blocks(s)
        seqs.append(s)
    shape = (256, BS, HKV, D)
    kc = rng.standard_normal(shape).astype(np.float32)
    vc = rng.standard_normal(shape).astype(np.float32)
    arena = KvCacheArena(ctx, 1, 256, BS, HKV, D)
    try:
        for phase in ("prefill", "decode"):
            arena.write(0, 0, kc)
            arena.write(0, 1, vc)
            if phase == "prefill":
                ctx.prepare_prefill(seqs, BS)
                meta = E.prepare_prefill(seqs, BS)
            else:
                for s in seqs:
                    s.num_cached_tokens += s.num_scheduled_tokens
                    s.num_scheduled_tokens = 0
                    s.append_token(1)
                    bm.may_append(s)
                ctx.prepare_decode(seqs, BS)
                meta = E.prepare_decode(seqs, BS)
            ctx.bind_kv_cache(arena)
            T = len(meta.positions)
            say(f"prepare {phase}: {len(seqs)} seqs, {T} tokens")
            q = rng.standard_normal((T, HQ, D)).astype(np.float32)
            k = rng.standard_normal((T, HKV, D)).astype(np.float32)
            v = rng.standard_normal((T, HKV, D)).astype(np.float32)
            out = Attention(HQ, D, 0.2, HKV).forward(torch.from_numpy(q).cuda(),
                                                     torch.from_numpy(k).cuda(),
                                                     torch.from_numpy(v).cuda(), ctx)
            ctx.sync()
            wk, wv = kc.copy(), vc.copy()
            want = O.attention_forward(HQ, D, 0.2, HKV, is_prefill=meta.is_prefill, q=q, k=k,
                                       v=v, cu_q=meta.cu_seqlens_q, cu_k=meta.cu_seqlens_k,
                                       slot_mapping=meta.slot_mapping,
                                       context_lens=meta.context_lens,
                                       block_tables=meta.block_tables, k_cache=wk, v_cache=wv,
                                       threads=4)
            got = out.cpu().numpy()
            assert np.max(np.abs(got - want)) <= 1e-4 and rel_l2(got, want) <= 1e-5
            assert np.array_equal(bits(arena.get_key_cache(0)), bits(wk))
            assert np.array_equal(bits(arena.get_value_cache(0)), bits(wv))
            ctx.clear()
    finally:
        arena.close()
