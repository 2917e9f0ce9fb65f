"""The node kernel's logarithm (the per-step Nernst potential), through the host build
of the same source (hx_fastmath_log): error in ulps against numpy's log, which is
correctly rounded to well under an ulp, over the concentration ratios a Nernst term sees
(co / ci from 1e-3 to 1e9) and over the whole normal range; exact at powers of two times
the reduction's edges; refusal of arguments outside the positive normal range."""
import ctypes

import numpy as np
import pytest

from heliox_amd import lib


def fast_log(x):
    x = np.ascontiguousarray(x, np.float64)
    y = np.empty_like(x)
    P = ctypes.POINTER(ctypes.c_double)
    rc = lib().hx_fastmath_log(x.ctypes.data_as(P), y.ctypes.data_as(P), x.size)
    return rc, y


def ulps(got, ref):
    return np.abs(got - ref) / np.spacing(np.abs(ref))


def test_nernst_ratio_range():
    rng = np.random.default_rng(3)
    x = 10.0 ** rng.uniform(-3, 9, 400_000)
    rc, y = fast_log(x)
    assert rc == 0
    ref = np.log(x)
    keep = np.abs(ref) > 1e-3            # relative error is measured away from ln x = 0
    err = ulps(y[keep], ref[keep])
    print(f"max {err.max():.2f} ulp, mean {err.mean():.3f}")
    assert err.max() <= 3.0
    # near x = 1 the absolute error is what reaches the potential: below 2 ulp of 1
    near = x[np.abs(x - 1) < 0.1]
    rc, yn = fast_log(near)
    assert np.max(np.abs(yn - np.log(near))) <= 2 * np.spacing(1.0)


def test_whole_normal_range_and_reduction_edges():
    rng = np.random.default_rng(4)
    x = np.ldexp(rng.uniform(0.5, 1.0, 200_000), rng.integers(-1021, 1024, 200_000))
    edges = np.ldexp(np.array([0.5, np.sqrt(0.5), np.nextafter(np.sqrt(0.5), 1), 1.0, np.sqrt(2.0), 2.0]),
                     np.repeat(np.arange(-1000, 1001, 250), 6).reshape(-1, 6)).ravel()
    x = np.concatenate([x, edges, [np.finfo(float).tiny, np.finfo(float).max]])
    x = x[np.isfinite(x) & (x >= np.finfo(float).tiny)]
    rc, y = fast_log(x)
    assert rc == 0
    ref = np.log(x)
    keep = np.abs(ref) > 1e-3
    assert ulps(y[keep], ref[keep]).max() <= 3.0
    rc, y1 = fast_log(np.array([1.0, 2.0, 0.5]))
    assert y1[0] == 0.0 and abs(y1[1] - np.log(2.0)) <= np.spacing(np.log(2.0))


@pytest.mark.parametrize("bad", [0.0, -1.0, 1e-310, np.inf, np.nan])
def test_refuses_outside_positive_normals(bad):
    rc, _ = fast_log(np.array([1.0, bad]))
    assert rc == -1
