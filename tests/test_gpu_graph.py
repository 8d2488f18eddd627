"""nva_attention_forward_noalloc captured into a HIP graph (through torch.cuda.graph) and
replayed, through the C ABI.

The no-allocation entry point is the one meant for callers under graph capture: once a step's
plan is in the library's scratch array, a call launches kernels only (no allocation, no plan
copy, no memset), so its launch sequence can be captured.  Checked on a split-KV decode (store,
row kernel, merge), on one with more workgroups than the row kernel keeps resident (several
dispatch rounds), on one with 8 query heads per KV head (the MFMA row kernel), and on a mixed
prefill (MFMA tiles on the context's stream, qLen = 1 rows forked onto its second stream and
joined with events): each replay, with eager work and synchronisations between the replays,
gives output bit-identical to the eager call on the same inputs, also after the inputs the graph
reads are overwritten with new values.
"""

import ctypes

import numpy as np
import pytest
import torch

from cases import Case
from gpu_checks import bits, dev, say
from nanollvm_amd import Attention, Context, KvCacheArena, _native as N
from nanollvm_amd import workloads as W

pytestmark = pytest.mark.gpu


def noalloc(ctx, arena, attn, q, k, v, out):
    return N.load().nva_attention_forward_noalloc(
        ctx.handle, arena.handle, ctypes.byref(attn._desc), q.data_ptr(), k.data_ptr(),
        v.data_ptr(), q.shape[0], out.data_ptr())


def run_graph(case, name, replays=3):
    wl = case.wl
    say(f"graph {name}: tokens={wl.tokens} hq={wl.hq} hkv={wl.hkv} d={wl.d}")
    s = torch.cuda.Stream()
    with torch.cuda.stream(s), Context(0, stream=s) as ctx:
        arena = KvCacheArena(ctx, 1, wl.num_blocks, wl.block_size, wl.hkv, wl.d)
        arena.write(0, 0, case.k_cache)
        arena.write(0, 1, case.v_cache)
        try:
            ctx.set(**wl.meta.context_args())
            ctx.bind_kv_cache(arena)
            attn = Attention(wl.hq, wl.d, wl.scale, wl.hkv, wl.window, 0, write_kv=True)
            q, k, v = dev(case.q), dev(case.k), dev(case.v)
            out = torch.full((wl.tokens, wl.hq, wl.d), float("nan"), device="cuda")

            def eager(qq, kk, vv):
                o = torch.full_like(out, float("nan"))
                st = noalloc(ctx, arena, attn, qq, kk, vv, o)
                assert st == N.NVA_OK, N.load().nva_last_error(ctx.handle).decode()
                s.synchronize()
                res = o.cpu().numpy()
                assert np.all(np.isfinite(res))
                return res

            want = eager(q, k, v)  # also puts the step's plan into the scratch array
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=s):
                st = noalloc(ctx, arena, attn, q, k, v, out)
            assert st == N.NVA_OK, N.load().nva_last_error(ctx.handle).decode()
            s.synchronize()
            rng = np.random.default_rng(7)
            for r in range(replays):
                if r == replays - 1:
                    # New inputs in the buffers the graph reads: the replay must recompute.
                    for t in (q, k, v):
                        t.copy_(torch.from_numpy(
                            rng.standard_normal(tuple(t.shape), dtype=np.float32)).cuda())
                    s.synchronize()
                    want = eager(q, k, v)
                out.fill_(float("nan"))
                junk = torch.randn(1 << 20, device="cuda").sum()  # eager work between replays
                s.synchronize()
                g.replay()
                s.synchronize()
                got = out.cpu().numpy()
                say(f"graph {name}: replay {r}: max |got - eager| = "
                    f"{float(np.max(np.abs(got - want))):.3e} ({float(junk):.1f})")
                assert np.array_equal(bits(got), bits(want)), f"replay {r} differs from eager"
        finally:
            ctx.clear()
            arena.close()


def test_decode_step_graph_replays():
    rng = np.random.default_rng(41)
    ctxs = [int(x) for x in rng.integers(256, 1025, 8)]
    case = Case(W.build("decode 8 rows", [(c - 1, 1) for c in ctxs], is_prefill=False, hq=16,
                        hkv=8, d=128, scale=W.QWEN_SCALE, rng=rng), seed=41)
    run_graph(case, "decode 8 rows")


def test_decode_many_rows_graph_replays():
    # 1100 rows x 2 KV heads: more workgroups than the row kernel keeps resident.
    rng = np.random.default_rng(43)
    ctxs = [int(x) for x in rng.integers(1, 301, 1100)]
    ctxs[:4] = [int(x) for x in rng.integers(5000, 9001, 4)]
    case = Case(W.build("decode 1100 rows", [(c - 1, 1) for c in ctxs], is_prefill=False, hq=4,
                        hkv=2, d=64, scale=0.125, rng=rng, block_size=16, pool_cap=1 << 20),
                seed=43)
    run_graph(case, "decode 1100 rows (several dispatch rounds)", replays=4)


def test_decode_mfma_rows_graph_replays():
    # 64 query heads over 8 KV heads: the rows run on the MFMA row kernel (8 heads per
    # workgroup).
    rng = np.random.default_rng(44)
    ctxs = [int(x) for x in rng.integers(256, 3000, 24)]
    case = Case(W.build("decode 24 rows, 64 q / 8 kv heads", [(c - 1, 1) for c in ctxs],
                        is_prefill=False, hq=64, hkv=8, d=128, scale=W.QWEN_SCALE, rng=rng),
                seed=44)
    run_graph(case, "decode 24 rows, 64 q / 8 kv heads (MFMA rows)")


def test_mixed_step_graph_replays():
    rng = np.random.default_rng(42)
    seqs = [(int(p), 128) for p in rng.integers(0, 1024, 4)] + \
           [(int(c) - 1, 1) for c in rng.integers(512, 2048, 8)]
    case = Case(W.build("mixed prefill", seqs, is_prefill=True, hq=32, hkv=8, d=128,
                        scale=W.QWEN_SCALE, rng=rng), seed=42)
    run_graph(case, "mixed prefill (tiles + forked rows)")
