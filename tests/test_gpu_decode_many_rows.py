"""Split-KV decode steps with more workgroups than the GPU holds at once (the row kernel's grid
then runs in several dispatch rounds, its longest work items first).

Checked through the C ABI: against the oracle (max-abs 1e-4, rel-L2 1e-5, K/V pages bit-exact)
at page sizes 16 and 256, with split and unsplit rows in one step; and bit-identical outputs
over repeated calls on one context, with a small decode (one dispatch round) between them.  The
graph replays of the same kind of step through the no-allocation entry point are in
test_gpu_graph.py.  Every case has at least 2200 workgroups: above the 1024 (4 per CU) the row
kernel keeps resident at these shapes, and above 8 per CU.
"""

import numpy as np
import pytest

from cases import Case
from gpu_checks import bits, check_attention, dev, load_arena, say
from nanollvm_amd import Attention, Context
from nanollvm_amd import workloads as W

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    with Context(0) as c:
        yield c


def many_rows(seed, rows, hq, hkv, d, block_size, long_rows=4):
    """`rows` decode rows of 1..300 keys plus a few of 5000..9000 (split into chunks)."""
    rng = np.random.default_rng(seed)
    ctxs = [int(x) for x in rng.integers(1, 301, rows)]
    ctxs[:long_rows] = [int(x) for x in rng.integers(5000, 9001, long_rows)]
    rng.shuffle(ctxs)
    scale = 1.0 / np.sqrt(d)
    return W.build(f"decode {rows} rows d={d}", [(c - 1, 1) for c in ctxs], is_prefill=False,
                   hq=hq, hkv=hkv, d=d, scale=scale, rng=rng, block_size=block_size,
                   pool_cap=1 << 20)


@pytest.mark.parametrize("hq,hkv,d,block_size,rows", [
    (4, 2, 64, 16, 1100),     # 2 units per row
    (16, 8, 128, 256, 300),   # Qwen3-0.6B heads: 8 units per row
])
def test_many_units_against_oracle(ctx, hq, hkv, d, block_size, rows):
    wl = many_rows(3, rows, hq, hkv, d, block_size)
    check_attention(ctx, Case(wl, seed=3), f"many-row decode d={d} bs={block_size}")


def test_repeated_calls_bit_identical(ctx):
    big = Case(many_rows(5, 1100, 4, 2, 64, 16), seed=5)
    rng = np.random.default_rng(6)
    small = Case(W.build("decode 8 rows", [(int(c) - 1, 1) for c in rng.integers(20, 200, 8)],
                         is_prefill=False, hq=4, hkv=2, d=64, scale=0.125, rng=rng,
                         block_size=16), seed=6)

    def run(case):
        wl = case.wl
        arena = load_arena(ctx, case)
        try:
            ctx.set(**wl.meta.context_args())
            ctx.bind_kv_cache(arena)
            attn = Attention(wl.hq, wl.d, wl.scale, wl.hkv, wl.window, 0)
            out = attn.forward(dev(case.q), dev(case.k), dev(case.v), ctx)
            ctx.sync()
            return out.cpu().numpy()
        finally:
            ctx.clear()
            arena.close()

    first = run(big)
    small_first = run(small)
    assert np.all(np.isfinite(first)) and np.all(np.isfinite(small_first))
    for r in range(3):
        got = run(big)
        say(f"many-row decode repeat {r}: max |got - first| = "
            f"{float(np.max(np.abs(got - first))):.3e}")
        assert np.array_equal(bits(got), bits(first)), f"call {r + 2} differs from the first"
        got_small = run(small)
        assert np.array_equal(bits(got_small), bits(small_first)), "small decode differs"


@pytest.mark.parametrize("hq,hkv,d", [(16, 8, 128), (8, 4, 128), (4, 2, 128), (40, 8, 128),
                                      (28, 4, 128), (10, 2, 128), (32, 8, 64), (14, 2, 64)])
def test_decode_bit_identical_under_every_xcd_offset(ctx, hq, hkv, d):
    """At 2, 4 or 8 KV heads and d = 64 or 128 the decode launch rotates which KV head each workgroup
    reads by the XCD the store kernel's last workgroup ran on (workgroups go to the 8 XCDs in
    turn, continuing across launches), with the row kernel (2 heads per KV head) and the MFMA
    row kernel (5 and 7).  Calls preceded by 0..7 one-workgroup kernels start on every XCD
    offset, so both rotations run; every output must be bit-identical to the first, and the
    first is checked against the oracle."""
    import torch
    rng = np.random.default_rng(11 + hq)
    case = Case(W.build(f"decode 64 rows, {hq} q / {hkv} KV heads, d={d}",
                        [(int(c) - 1, 1) for c in rng.integers(100, 3000, 64)],
                        is_prefill=False, hq=hq, hkv=hkv, d=d, scale=float(1.0 / np.sqrt(d)),
                        rng=rng, block_size=256, pool_cap=1 << 16), seed=11)
    check_attention(ctx, case, f"decode {hq} q / {hkv} KV heads, d={d}")
    wl = case.wl
    arena = load_arena(ctx, case)
    tiny = torch.zeros(1, device="cuda")
    try:
        ctx.set(**wl.meta.context_args())
        ctx.bind_kv_cache(arena)
        attn = Attention(wl.hq, wl.d, wl.scale, wl.hkv, wl.window, 0)
        q, k, v = dev(case.q), dev(case.k), dev(case.v)
        first = None
        for shift in range(8):
            for _ in range(shift):
                tiny.add_(1.0)  # one workgroup
            out = attn.forward(q, k, v, ctx)
            ctx.sync()
            got = out.cpu().numpy()
            if first is None:
                assert np.all(np.isfinite(got))
                first = got
            else:
                assert np.array_equal(bits(got), bits(first)), f"offset {shift} differs"
        say("decode bit-identical after 0..7 one-workgroup launches")
    finally:
        ctx.clear()
        arena.close()
