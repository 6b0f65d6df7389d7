"""The floating-point parity bar for this build: max-abs / rel error within 1e-2.

    max|got - want| <= TOL * max|want|      (max-abs error, relative to the tensor's scale)
    mean|got - want| <= TOL * mean|want|    (mean relative error)

with TOL = 1e-2 and fp32 accumulation on both sides.  Integer / byte / index
results (embedding rows, KV-cache indexing, argmax ids) are compared bit-exactly
instead.
"""
import numpy as np

TOL = 1e-2


def rel_errors(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    err = np.abs(got - want)
    return err.max() / max(np.abs(want).max(), 1e-30), err.mean() / max(np.abs(want).mean(), 1e-30)


def assert_close(got, want, tol: float = TOL, what: str = ""):
    mx, mean = rel_errors(got, want)
    assert np.isfinite(np.asarray(got, np.float64)).all(), f"{what}: non-finite values"
    assert mx <= tol and mean <= tol, f"{what}: max-abs/scale {mx:.3e}, mean-rel {mean:.3e} > {tol}"
