"""Pins the oracle's Ops.linear (y = x W^T + b over the sequential runtime's gemv panels):
float64 form within the first-order error bound of a sequential fp32 sum, the reference's own
linear tests re-expressed, planted mistakes."""

import numpy as np
import pytest

from oracle import oracle as O


@pytest.mark.parametrize("rows,inf,outf", [(1, 64, 32), (4, 96, 24), (7, 2048, 37), (3, 128, 256)])
@pytest.mark.parametrize("bias", [False, True])
def test_linear_matches_fp64(rows, inf, outf, bias):
    rng = np.random.default_rng(rows * 1000 + inf)
    x = rng.standard_normal((rows, inf)).astype(np.float32)
    w = (0.05 * rng.standard_normal((outf, inf))).astype(np.float32)
    b = rng.standard_normal(outf).astype(np.float32) if bias else None
    got = O.linear(x, w, b)
    want = x.astype(np.float64) @ w.astype(np.float64).T + (0.0 if b is None else b)
    # First-order bound of a sequential fp32 sum of in + 1 terms: (in + 1) * 2^-24 * sum|term|.
    mag = np.abs(x.astype(np.float64)) @ np.abs(w.astype(np.float64)).T
    if b is not None:
        mag = mag + np.abs(b)
    bound = (inf + 1) * 2.0 ** -24 * mag
    assert np.all(np.abs(got - want) <= bound)
    # and, far inside that bound, the typical (random-walk) error
    assert np.max(np.abs(got - want) / mag) < 1e-5


def test_reference_identity_case():
    # T/CoreUnitTest.java:296-300
    y = O.linear(np.array([[2.0, 3.0]], np.float32), np.array([[1, 0], [0, 1]], np.float32))
    assert abs(y[0, 0] - 2.0) < 1e-5 and abs(y[0, 1] - 3.0) < 1e-5


def test_reference_vector_linear_matches_scalar_sum():
    # T/CoreUnitTest.java:432-471: x[i] = i % 7 * 0.1, w[i] = i * 3 % 11 * 0.05
    rows, inf, outf = 4, 64, 32
    x = (np.arange(rows * inf) % 7).astype(np.float32) * np.float32(0.1)
    w = ((np.arange(outf * inf) * 3) % 11).astype(np.float32) * np.float32(0.05)
    x = x.reshape(rows, inf)
    w = w.reshape(outf, inf)
    for mode in (0, 8, 16):
        y = O.linear(x, w, mode=mode)
        for r in range(rows):
            for o in range(outf):
                e = np.float32(0.0)
                for i in range(inf):
                    e = np.float32(e + np.float32(x[r, i] * w[o, i]))
                assert abs(y[r, o] - e) <= 1e-4


def test_reference_gemv_scalar_vs_vector_with_bias():
    # T/CoreUnitTest.java:705-728 (in 96, out 24) and :473-502 (rows 3, in 128, out 256)
    for rows, inf, outf, fx, fw, fb in ((1, 96, 24, (11, 0.04), (3, 17, 0.02), 0.01),
                                        (3, 128, 256, (9, 0.07), (5, 13, 0.03), None)):
        x = ((np.arange(rows * inf) % fx[0]) * np.float32(fx[1])).astype(np.float32)
        w = (((np.arange(outf * inf) * fw[0]) % fw[1]) * np.float32(fw[2])).astype(np.float32)
        b = (np.arange(outf) * np.float32(fb)).astype(np.float32) if fb else \
            ((np.arange(outf) % 5) * np.float32(0.01)).astype(np.float32)
        ys = O.linear(x.reshape(rows, inf), w.reshape(outf, inf), b)
        for lanes in (8, 16):
            yv = O.linear(x.reshape(rows, inf), w.reshape(outf, inf), b, mode=lanes)
            assert np.max(np.abs(ys - yv)) <= 1e-4


def _checks(mutation):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, 40)).astype(np.float32)
    w = rng.standard_normal((40, 40)).astype(np.float32)
    b = rng.standard_normal(40).astype(np.float32)
    got = O.linear(x, w, b, mutation=mutation)
    want = x.astype(np.float64) @ w.astype(np.float64).T + b
    return bool(np.max(np.abs(got - want)) < 1e-4)


def test_checks_pass_unmutated():
    assert _checks(O.MUT_NONE)


@pytest.mark.parametrize("mutation", [O.MUT_LIN_TRANSPOSE, O.MUT_LIN_NO_BIAS])
def test_planted_linear_mistake_is_caught(mutation):
    assert not _checks(mutation)
