"""Parity metric and tolerances shared by the tests.

The north-star tolerance is "1e-5 relative (forward), 1e-4 relative
(backward), fp32". Relative error of a tensor x against a reference r is
measured norm-wise:

    rel_err(x, r) = max_i |x_i - r_i| / max_i |r_i|

Elementwise |x_i - r_i| / |r_i| is not used as the gate because reference
entries near zero (an LSE that happens to be ~0, a dQ entry produced by
heavy cancellation) make it meaningless; it is reported in messages only.
"""
import numpy as np

FWD_RTOL = 1e-5
BWD_RTOL = 1e-4


def rel_err(x, r) -> float:
    x = np.asarray(x, dtype=np.float64)
    r = np.asarray(r, dtype=np.float64)
    assert x.shape == r.shape, (x.shape, r.shape)
    if not np.all(np.isfinite(x)):
        return float("inf")
    denom = np.max(np.abs(r)) if r.size else 0.0
    num = np.max(np.abs(x - r)) if r.size else 0.0
    return float(num / denom) if denom > 0 else float(num)


def assert_close(name: str, x, r, rtol: float) -> float:
    e = rel_err(x, r)
    assert e <= rtol, f"{name}: rel_err {e:.3e} > {rtol:.0e}"
    return e
