"""o_proj (Linear.Row -> Ops.linear) on fp32 MFMA through the C ABI, against the oracle's
restatement of the reference's gemv at decode shapes, and against float64 at the full prefill
shapes.  Bar: max-abs 1e-4 and rel-L2 1e-5, the path's floating-point tolerance.

The library's kernels by shape: the weight-streaming GEMV up to 8 rows, 32 x 32 blocks (K over
eight waves, K slices plus the reduce) while the blocks fit one per CU, 128 x 64 tiles (K slices
when the tiles leave CUs idle) above."""

import sys

import numpy as np
import pytest
import torch

from cases import rel_l2
from nanollvm_amd import Context, Linear, UnsupportedShapeError
from oracle import oracle as O

pytestmark = pytest.mark.gpu

MAX_ABS = 1e-4
REL_L2 = 1e-5


def say(msg):
    print(f"[gpu] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ctx():
    c = Context(0)
    yield c
    c.close()


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def data(rows, inf, outf, bias, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, inf)).astype(np.float32)
    w = (rng.standard_normal((outf, inf)) / np.sqrt(inf)).astype(np.float32)
    b = rng.standard_normal(outf).astype(np.float32) if bias else None
    return x, w, b


def run(ctx, x, w, b):
    lin = Linear(dev(w), None if b is None else dev(b))
    y = lin.forward(dev(x), ctx)
    ctx.sync()
    return y.cpu().numpy()


def check(got, want, name):
    err = float(np.max(np.abs(got - want)))
    rl2 = rel_l2(got, want)
    say(f"{name}: max_abs={err:.3e} rel_l2={rl2:.3e}")
    assert np.all(np.isfinite(got))
    assert err <= MAX_ABS and rl2 <= REL_L2, (err, rl2)


@pytest.mark.parametrize("rows,inf,outf,bias", [
    (1, 2048, 1024, False),    # one decode row, Qwen3-0.6B o_proj
    (8, 2048, 1024, True),     # 8-row decode batch
    (2, 4096, 2560, True),     # GEMV path, Qwen3-4B o_proj
    (3, 260, 200, False),      # GEMV path, rows short of its 4-row form, ragged N and K
    (5, 1028, 7, True),        # GEMV path, 8-row form, fewer columns than one workgroup
    (9, 260, 200, True),       # GEMV path, 16-row form
    (16, 2048, 1024, True),    # GEMV path, its largest row count
    (17, 260, 200, True),      # first row count past the GEMV path (32 x 32 blocks)
    (37, 260, 200, True),      # ragged M, N, K (K % 32 != 0)
    (33, 2048, 1000, True),    # 16 x 16 blocks: ragged M and N
    (100, 2052, 300, False),   # 16 x 16 blocks: ragged M, N and K (K % 32 == 4)
    (128, 2048, 1024, True),   # 16 x 16 blocks, two per CU (128-row decode batch)
    (64, 1028, 1024, True),    # 16 x 16 blocks, K of 1028: the last wave's range 4 k long
    (24, 8192, 256, False),    # 32 K slices of one 32-k stage per wave
    (130, 2048, 1024, False),  # M tail past one 128-row tile
    (256, 2048, 1024, True),   # 256-row decode batch: 256 blocks, one per CU
    (384, 2048, 1024, True),   # more blocks than CUs: 128 x 64 tiles, K slices plus the reduce
    (384, 1028, 1000, True),   # tiles: interior and edge tiles side by side, ragged N and K
    (300, 4100, 520, False),   # tiles: M and N tails, K % 32 == 4 (a ragged last K tile)
    (1000, 100, 70, True),     # tiles: one K tile, ragged (K = 100), N shorter than a tile
    (517, 36, 4100, False),    # tiles: K = 36 (one full K tile and a 4-wide one), N tail of 4
])
def test_linear_matches_oracle(ctx, rows, inf, outf, bias):
    x, w, b = data(rows, inf, outf, bias, rows + inf)
    check(run(ctx, x, w, b), O.linear(x, w, b), f"linear {rows}x{inf}->{outf} bias={bias}")


@pytest.mark.parametrize("rows,inf,outf", [(4096, 2048, 1024), (512, 4096, 2560),
                                           (2100, 4096, 2560), (4000, 2048, 1000),
                                           (8192, 2048, 1024)])
def test_linear_full_prefill_shapes_fp64(ctx, rows, inf, outf):
    """Qwen3-0.6B o_proj over the 4096-token prefill, and Qwen3-4B-like o_projs (2100 rows: more
    tiles than two per CU, and an M tail of 52 rows); M and N tails at a full grid (4000 x 1000:
    a 32-row band and a 40-column tile) and two rounds of tiles (8192 rows)."""
    x, w, b = data(rows, inf, outf, True, 3)
    want = x.astype(np.float64) @ w.astype(np.float64).T + b
    check(run(ctx, x, w, b), want, f"linear {rows}x{inf}->{outf} vs fp64")


def test_reference_linear_cases(ctx):
    # T/CoreUnitTest.java:296-300 (identity) and :432-471 (rows 4, in 64, out 32)
    y = run(ctx, np.array([[2.0, 3.0, 0.0, 0.0]], np.float32),
            np.array([[1, 0, 0, 0], [0, 1, 0, 0]], np.float32), None)
    assert abs(y[0, 0] - 2.0) < 1e-5 and abs(y[0, 1] - 3.0) < 1e-5
    x = ((np.arange(4 * 64) % 7) * np.float32(0.1)).astype(np.float32).reshape(4, 64)
    w = (((np.arange(32 * 64) * 3) % 11) * np.float32(0.05)).astype(np.float32).reshape(32, 64)
    assert np.max(np.abs(run(ctx, x, w, None) - O.linear(x, w))) <= 1e-4


def test_linear_rejects_unaligned_width(ctx):
    x, w, _ = data(3, 6, 5, False, 1)
    with pytest.raises(UnsupportedShapeError):
        run(ctx, x, w, None)


def test_linear_repeatable_bit_for_bit(ctx):
    """The same call twice gives the same bits (no atomics, fixed slice order), on the tiled,
    block and GEMV kernels."""
    for rows, inf, outf in ((4096, 2048, 1024), (1024, 2048, 1024), (256, 2048, 1024), (5, 2048, 1024)):
        x, w, b = data(rows, inf, outf, True, 11)
        a1, a2 = run(ctx, x, w, b), run(ctx, x, w, b)
        say(f"linear {rows}x{inf}->{outf}: repeat identical={np.array_equal(a1, a2)}")
        assert np.array_equal(a1.view(np.uint32), a2.view(np.uint32))


@pytest.mark.parametrize("seed", range(12))
def test_linear_fuzz_fp64(ctx, seed):
    """Random shapes across the four kernels and their edges (GEMV forms, 32 x 32 blocks with K
    slices, 128 x 64 tiles with slices, ragged M / N / K tails, grids that do and do not divide
    into XCD rectangles), with and without bias, against a float64 product on the device."""
    rng = np.random.default_rng(1000 + seed)
    rows = int(rng.choice([int(rng.integers(1, 9)), int(rng.integers(9, 300)),
                           int(rng.integers(300, 5000))]))
    inf = 4 * int(rng.integers(1, 1100))
    outf = int(rng.integers(1, 3000))
    bias = bool(rng.integers(0, 2))
    x, w, b = data(rows, inf, outf, bias, 77 + seed)
    got = run(ctx, x, w, b)
    want = torch.from_numpy(x).cuda().double() @ torch.from_numpy(w).cuda().double().T.contiguous()
    if b is not None:
        want = want + torch.from_numpy(b).cuda().double()
    check(got, want.cpu().numpy(), f"linear fuzz {seed}: {rows}x{inf}->{outf} bias={bias}")
