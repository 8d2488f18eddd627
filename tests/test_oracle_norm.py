"""Pins the oracle's RMSNorm (Ops.rmsNorm, tensor/Ops.java:444-500, with the scalar
sumSquares order of ScalarFloatKernels.java:55-70): a float64 textbook form, a hand-derived
known answer that fixes the summation order, exact scale invariance, the reference's own tests
re-expressed, and planted mistakes that must each fail one of these checks."""

import numpy as np
import pytest

from oracle import oracle as O


def _rows(rng, rows, width, scale=1.0):
    return (rng.standard_normal((rows, width)) * scale).astype(np.float32)


@pytest.mark.parametrize("width", [4, 7, 64, 128, 256, 1024])
@pytest.mark.parametrize("kind", ["weightless", "weight", "one_plus"])
def test_rms_norm_matches_fp64_textbook(width, kind):
    rng = np.random.default_rng(width)
    x = _rows(rng, 33, width, 3.0)
    w = None if kind == "weightless" else rng.standard_normal(width).astype(np.float32)
    got = O.rms_norm(x, w, 1e-6, kind == "one_plus")
    want = O.rms_norm_fp64(x, w, 1e-6, kind == "one_plus")
    err = np.abs(got - want) / np.maximum(np.abs(want), 1e-3)
    assert err.max() < 2e-6, err.max()


def test_scalar_sum_order_known_answer():
    # 4096^2 = 2^24.  In the scalar order the group sum is ((2^24 + 1) + 1) + 1 and each + 1 is a
    # tie between 2^24 and 2^24 + 2 that rounds to the even 2^24, so the sum is exactly 2^24.
    # A pairwise tree adds (2^24 + 1) -> 2^24 and 1 + 1 = 2 first, giving 2^24 + 2.
    x = np.zeros(128, np.float32)
    x[:4] = [4096.0, 1.0, 1.0, 1.0]
    assert O.sum_squares(x) == 2.0 ** 24
    assert O.sum_squares(x, mutation=O.MUT_NORM_PAIRWISE) == 2.0 ** 24 + 2
    # The 8-lane Vector API backend holds the four values in separate lanes and reduces them
    # after the loop: the same 2^24 + 2, i.e. the Java result depends on the host backend.
    assert O.sum_squares(x, mode=8) == 2.0 ** 24 + 2
    # Through the norm: var = 2^24 / 128 = 2^17, inv = (float)(1 / sqrt(2^17)).
    y = O.rms_norm(x[None], None, 0.0)[0]
    inv = np.float32(1.0 / np.sqrt(2.0 ** 17))
    assert y[0] == np.float32(np.float32(4096.0) * inv)
    assert y[1] == inv


def test_scale_invariance_is_exact_without_eps():
    rng = np.random.default_rng(3)
    x = _rows(rng, 16, 128)
    w = rng.standard_normal(128).astype(np.float32)
    a = O.rms_norm(x, w, 0.0)
    b = O.rms_norm(x * np.float32(2.0), w, 0.0)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_reference_add_rms_norm_values():
    # T/CoreUnitTest.java:332-349: summed rows [1.5, 1.5] and [4, 4] with weight [1, 1].
    x = np.array([[1.5, 1.5], [4.0, 4.0]], np.float32)
    out = O.rms_norm(x, np.ones(2, np.float32), 1e-6)
    assert np.allclose(out, 1.0, atol=1e-5)
    # The weightless form (RMSNorm.weightless, :352-365) gives the same values.
    assert np.allclose(O.rms_norm(x, None, 1e-6), out, atol=1e-5)


def test_reference_gemma_one_plus_weight():
    # T/CoreUnitTest.java:1047-1056: onePlusWeight with w = [0, 0.5] equals the plain norm
    # (weight [1, 1]) times (1 + w).
    x = np.array([[1.0, -1.0], [2.0, 0.0]], np.float32)
    w = np.array([0.0, 0.5], np.float32)
    out = O.rms_norm(x, w, 1e-6, True)
    plain = O.rms_norm(x, np.ones(2, np.float32), 1e-6)
    assert out[0, 0] != 0.0
    assert abs(out[0, 0] - plain[0, 0] * 1.0) < 1e-5
    assert abs(out[0, 1] - plain[0, 1] * 1.5) < 1e-5


def test_reference_scalar_vector_sum_squares_agree():
    # T/CoreUnitTest.java:660-675: a[i] = 0.1 i, scalar and vector sumSquares within 1e-3;
    # the exact value is 0.01 * sum(i^2, i < 64) = 853.44.
    a = (np.arange(64, dtype=np.float32) * np.float32(0.1)).astype(np.float32)
    s = O.sum_squares(a)
    for lanes in (8, 16):
        assert abs(s - O.sum_squares(a, mode=lanes)) <= 1e-3
    assert abs(s - 853.44) < 1e-3


def _checks(mutation):
    """Runs every check above against the oracle with a planted mistake; True if all pass."""
    rng = np.random.default_rng(11)
    ok = True
    x = _rows(rng, 8, 128, 1e-3)
    w = rng.standard_normal(128).astype(np.float32)
    for kind in ("weightless", "weight", "one_plus"):
        ww = None if kind == "weightless" else w
        got = O.rms_norm(x, ww, 1e-6, kind == "one_plus", mutation=mutation)
        want = O.rms_norm_fp64(x, ww, 1e-6, kind == "one_plus")
        ok &= bool((np.abs(got - want) / np.maximum(np.abs(want), 1e-3)).max() < 2e-6)
    z = np.zeros(128, np.float32)
    z[:4] = [4096.0, 1.0, 1.0, 1.0]
    ok &= O.sum_squares(z, mutation=mutation) == 2.0 ** 24
    g = O.rms_norm(np.array([[1.0, -1.0]], np.float32), np.array([0.0, 0.5], np.float32), 1e-6,
                   True, mutation=mutation)
    p = O.rms_norm(np.array([[1.0, -1.0]], np.float32), np.ones(2, np.float32), 1e-6,
                   mutation=mutation)
    ok &= bool(abs(g[0, 1] - p[0, 1] * 1.5) < 1e-5)
    return ok


def test_checks_pass_unmutated():
    assert _checks(O.MUT_NONE)


@pytest.mark.parametrize("mutation", [O.MUT_NORM_NO_EPS, O.MUT_NORM_DIV_N1,
                                      O.MUT_NORM_PAIRWISE, O.MUT_NORM_NO_ONE])
def test_planted_norm_mistake_is_caught(mutation):
    assert not _checks(mutation)
