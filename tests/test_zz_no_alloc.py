"""nva_attention_forward_noalloc against nva_attention_forward, through the C ABI.

The no-allocation entry point runs the same kernels on the same plan with its work buffers in
the library's static device scratch array, so its output must be bit-identical to the existing
entry point's on the same inputs, and its stored K/V identical.  Checked on two calls in a row
with the second smaller (the array keeps the first call's contents), on a split-KV decode, a
mixed prefill (MFMA tiles plus qLen = 1 rows, partials from both), a windowed prefill and a
shared-KV dense prefill whose gathered rows also live in the array; and that the call leaves the
context's grow-only device buffers untouched, and rejects a call needing more than the array
holds with the number of bytes it needs.
"""

import ctypes

import numpy as np
import pytest
import torch

from cases import Case, rel_l2
from gpu_checks import bits, dev, say
from nanollvm_amd import Attention, Context, KvCacheArena, _native as N
from nanollvm_amd import workloads as W
from oracle import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = Context(0)
    yield c
    c.close()


def device_bytes(ctx):
    return ctx.kernel_stats("device_bytes")[0]


def noalloc(ctx, arena, attn, q, k, v, out):
    st = N.load().nva_attention_forward_noalloc(
        ctx.handle, arena.handle, ctypes.byref(attn._desc), q.data_ptr(),
        0 if k is None else k.data_ptr(), 0 if v is None else v.data_ptr(), q.shape[0],
        out.data_ptr())
    return st


def run_pair(case, name, shared=False):
    """The no-allocation call, then the existing entry point, on a fresh context (whose
    grow-only buffers then hold only the step metadata) and the same step: outputs and pages
    bit-identical, both within the bar of the oracle."""
    wl = case.wl
    say(f"no-alloc {name}: tokens={wl.tokens} hq={wl.hq} hkv={wl.hkv} d={wl.d} W={wl.window}")
    with Context(0) as ctx:
        arena = KvCacheArena(ctx, 1, wl.num_blocks, wl.block_size, wl.hkv, wl.d)
        arena.write(0, 0, case.k_cache)
        arena.write(0, 1, case.v_cache)
        try:
            m = wl.meta
            args = m.context_args()
            if shared:
                args["block_tables"] = None
            ctx.set(**args)
            ctx.bind_kv_cache(arena)
            attn = Attention(wl.hq, wl.d, wl.scale, wl.hkv, wl.window, 0, write_kv=not shared)
            q = dev(case.q)
            k = None if shared else dev(case.k)
            v = None if shared else dev(case.v)
            before = device_bytes(ctx)
            out_b = torch.full((wl.tokens, wl.hq, wl.d), float("nan"), device="cuda")
            st = noalloc(ctx, arena, attn, q, k, v, out_b)
            assert st == N.NVA_OK, N.load().nva_last_error(ctx.handle).decode()
            ctx.sync()
            assert device_bytes(ctx) == before, "the no-allocation call grew a context buffer"
            out_a = attn.forward(q, k, v, ctx)
            ctx.sync()
            assert device_bytes(ctx) > before, "the existing entry point allocates its buffers"
            a, b = out_a.cpu().numpy(), out_b.cpu().numpy()
            assert np.all(np.isfinite(a))
            say(f"no-alloc {name}: max |a - b| = {float(np.max(np.abs(a - b))):.3e}")
            assert np.array_equal(bits(a), bits(b)), "outputs differ"
            if shared:
                want = O.attention_forward(wl.hq, wl.d, wl.scale, wl.hkv, is_prefill=True,
                                           q=case.q, cu_q=m.cu_seqlens_q, cu_k=m.cu_seqlens_k,
                                           slot_mapping=m.slot_mapping,
                                           k_cache=case.k_cache.copy(),
                                           v_cache=case.v_cache.copy(), write_kv=False,
                                           threads=8)
                kc, vc = case.k_cache, case.v_cache
            else:
                want, kc, vc = case.oracle(threads=8)
            err = float(np.max(np.abs(b - want)))
            say(f"no-alloc {name}: vs oracle max_abs={err:.3e}")
            assert err <= 1e-4 and rel_l2(b, want) <= 1e-5
            assert np.array_equal(bits(arena.get_key_cache(0)), bits(kc)), "K pages differ"
            assert np.array_equal(bits(arena.get_value_cache(0)), bits(vc)), "V pages differ"
            return b
        finally:
            ctx.clear()
            arena.close()


def decode_case(rows, seed):
    rng = np.random.default_rng(seed)
    ctxs = [int(x) for x in rng.integers(1, 6000, rows)]
    return Case(W.build(f"decode {rows} rows", [(c - 1, 1) for c in ctxs], is_prefill=False,
                        hq=16, hkv=8, d=128, scale=W.QWEN_SCALE, rng=rng), seed=seed)


def mixed_case(seed, scale_down=1):
    rng = np.random.default_rng(seed)
    seqs = [(int(p), 512 // scale_down) for p in rng.integers(0, 4096, 4)] + \
           [(int(c) - 1, 1) for c in rng.integers(1024, 8192, 16 // scale_down)]
    return Case(W.build("mixed prefill", seqs, is_prefill=True, hq=32, hkv=8, d=128,
                        scale=W.QWEN_SCALE, rng=rng), seed=seed)


def test_decode_two_calls_second_smaller():
    run_pair(decode_case(64, 31), "decode 64 rows")
    run_pair(decode_case(5, 32), "decode 5 rows (smaller, after the larger)")


def test_mixed_prefill_two_calls_second_smaller():
    run_pair(mixed_case(33), "mixed prefill")
    run_pair(mixed_case(34, scale_down=4), "mixed prefill (smaller)")


def test_windowed_prefill():
    rng = np.random.default_rng(35)
    wl = W.build("gemma3 local prefill", [(0, 300), (256, 200), (7, 1)], is_prefill=True, hq=4,
                 hkv=1, d=256, scale=W.GEMMA_SCALE, window=512, rng=rng)
    run_pair(Case(wl, seed=35), "windowed prefill d=256")


def test_shared_kv_gather_in_scratch():
    rng = np.random.default_rng(36)
    wl = W.build("shared dense", [(0, 300), (0, 77), (0, 1)], is_prefill=True, hq=8, hkv=2,
                 d=128, scale=0.1, rng=rng)
    case = Case(wl, seed=36)
    case.k_cache = rng.standard_normal(case.k_cache.shape, dtype=np.float32)
    case.v_cache = rng.standard_normal(case.v_cache.shape, dtype=np.float32)
    run_pair(case, "shared-KV dense prefill (gather)", shared=True)


def test_plan_copy_skipped_only_for_the_same_plan():
    """Two steps with different plans at the same offset, then the first again: every call
    matches the existing entry point (a stale plan left in the array would not)."""
    a, b = decode_case(40, 37), decode_case(41, 38)
    run_pair(a, "decode A")
    run_pair(b, "decode B")
    run_pair(a, "decode A again")


def test_rejects_more_than_the_scratch_holds(ctx):
    """Gathered K/V rows of 65536 tokens x 8 KV heads x 128 floats x 2 = 512 MiB > 128 MiB:
    the call fails before any kernel with the bytes it needs; inputs are real, full-size
    buffers."""
    T, hq, hkv, d, bs = 65536, 8, 8, 128, 256
    nb = T // bs
    arena = KvCacheArena(ctx, 1, nb, bs, hkv, d)
    try:
        slots = np.arange(T, dtype=np.int32)
        ctx.set(True, [0, T], [0, T], T, T, slot_mapping=slots)
        ctx.bind_kv_cache(arena)
        q = torch.zeros((T, hq, d), device="cuda")
        out = torch.zeros((T, hq, d), device="cuda")
        attn = Attention(hq, d, 0.1, hkv, 0, 0, write_kv=False)
        st = noalloc(ctx, arena, attn, q, None, None, out)
        msg = N.load().nva_last_error(ctx.handle).decode()
        say(f"no-alloc oversize: status {st}: {msg}")
        assert st == N.NVA_E_ARG
        assert "no-allocation" in msg and str(2 * T * hkv * d * 4 + 16) in msg
    finally:
        ctx.clear()
        arena.close()


def test_plan_reuse_in_one_step_alternating_configurations():
    """One context and one step, two attention configurations with different plans at the same
    offset of the array (no window, and a 512-token window): A, A, B, A, B, B.  The repeated
    calls take the branch that skips the plan copy; every call matches nva_attention_forward bit
    for bit (a stale plan left in the array would not)."""
    case = decode_case(64, 39)
    wl = case.wl
    # The calls read the pages without storing: put the step's own K/V rows in them first (the
    # case leaves unused slots NaN, which would make every output NaN and the comparison empty).
    kc, vc = case.k_cache.copy(), case.v_cache.copy()
    kc.reshape(-1, wl.hkv, wl.d)[wl.meta.slot_mapping] = case.k
    vc.reshape(-1, wl.hkv, wl.d)[wl.meta.slot_mapping] = case.v
    with Context(0) as ctx:
        arena = KvCacheArena(ctx, 1, wl.num_blocks, wl.block_size, wl.hkv, wl.d)
        arena.write(0, 0, kc)
        arena.write(0, 1, vc)
        try:
            ctx.set(**wl.meta.context_args())
            ctx.bind_kv_cache(arena)
            q = dev(case.q)
            layers = {"A": Attention(wl.hq, wl.d, wl.scale, wl.hkv, 0, 0, write_kv=False),
                      "B": Attention(wl.hq, wl.d, wl.scale, wl.hkv, 512, 0, write_kv=False)}
            want = {n: a.forward(q, None, None, ctx).cpu().numpy() for n, a in layers.items()}
            assert all(np.all(np.isfinite(w)) for w in want.values())
            assert not np.array_equal(want["A"], want["B"])
            for n in "AABABB":
                out = torch.full((wl.tokens, wl.hq, wl.d), float("nan"), device="cuda")
                st = noalloc(ctx, arena, layers[n], q, None, None, out)
                assert st == N.NVA_OK, N.load().nva_last_error(ctx.handle).decode()
                got = out.cpu().numpy()
                say(f"no-alloc alternating {n}: max |got - want| = "
                    f"{float(np.max(np.abs(got - want[n]))):.3e}")
                assert np.array_equal(bits(got), bits(want[n])), f"call {n} differs"
        finally:
            ctx.clear()
            arena.close()


def test_capture_needs_the_plan_in_the_array():
    """Under stream capture, a call whose plan is not in the array fails before it records
    anything (the replayed graph leaves the pages untouched); after one eager call the same call
    captures, and its replay matches nva_attention_forward bit for bit."""
    case = decode_case(48, 40)
    wl = case.wl
    s = torch.cuda.Stream()
    with torch.cuda.stream(s), Context(0, stream=s) as ctx:
        arena = KvCacheArena(ctx, 1, wl.num_blocks, wl.block_size, wl.hkv, wl.d)
        arena.write(0, 0, case.k_cache)
        arena.write(0, 1, case.v_cache)
        try:
            ctx.set(**wl.meta.context_args())
            ctx.bind_kv_cache(arena)
            attn = Attention(wl.hq, wl.d, wl.scale, wl.hkv, 0, 0, write_kv=True)
            q, k, v = dev(case.q), dev(case.k), dev(case.v)
            out = torch.full((wl.tokens, wl.hq, wl.d), float("nan"), device="cuda")
            # Another configuration's plan goes into the array first.
            other = Attention(wl.hq, wl.d, wl.scale, wl.hkv, 300, 0, write_kv=False)
            junk = torch.empty_like(out)
            assert noalloc(ctx, arena, other, q, None, None, junk) == N.NVA_OK
            s.synchronize()
            k_before = arena.get_key_cache(0).copy()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=s):
                junk.mul_(1.0)  # keeps the graph non-empty
                st = noalloc(ctx, arena, attn, q, k, v, out)
            msg = N.load().nva_last_error(ctx.handle).decode()
            say(f"no-alloc capture with a stale plan: status {st}: {msg}")
            assert st == N.NVA_E_ARG and "capture" in msg
            g.replay()
            s.synchronize()
            assert np.array_equal(bits(arena.get_key_cache(0)), bits(k_before)), \
                "the rejected call recorded the store"
            # One eager call puts the plan in the array; then capture works.
            assert noalloc(ctx, arena, attn, q, k, v, out) == N.NVA_OK
            s.synchronize()
            want = attn.forward(q, k, v, ctx).cpu().numpy()
            assert np.all(np.isfinite(want))
            g2 = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g2, stream=s):
                st = noalloc(ctx, arena, attn, q, k, v, out)
            assert st == N.NVA_OK, N.load().nva_last_error(ctx.handle).decode()
            for r in range(2):
                out.fill_(float("nan"))
                s.synchronize()
                g2.replay()
                s.synchronize()
                got = out.cpu().numpy()
                say(f"no-alloc capture replay {r}: max |got - want| = "
                    f"{float(np.max(np.abs(got - want))):.3e}")
                assert np.array_equal(bits(got), bits(want)), f"replay {r} differs"
        finally:
            ctx.clear()
            arena.close()
