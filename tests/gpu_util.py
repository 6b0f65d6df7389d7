"""Small torch <-> numpy helpers for the GPU tests (bf16 travels as int16 bits)."""
import ctypes as C
import sys

import numpy as np
import torch


def dev(a: np.ndarray) -> torch.Tensor:
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(a).cuda()


def host(t: torch.Tensor) -> np.ndarray:
    a = t.detach().cpu().numpy()
    return a.view(np.uint16) if a.dtype == np.int16 else a


# Tensors whose raw pointers were handed to the library in the current test.
# Holding them here keeps temporaries such as P(dev(x)) alive until the test
# ends (otherwise torch's caching allocator hands the block to the next
# allocation while the kernel still reads it).
_KEEP: list = []


def P(t: torch.Tensor | None):
    if t is None:
        return None
    _KEEP.append(t)
    return C.c_void_p(t.data_ptr())


def release() -> None:
    _KEEP.clear()


def bf16_empty(*shape) -> torch.Tensor:
    return torch.empty(shape, dtype=torch.int16, device="cuda")


def bf16_zeros(*shape) -> torch.Tensor:
    return torch.zeros(shape, dtype=torch.int16, device="cuda")


def say(msg: str) -> None:
    """Progress line, flushed before the GPU step it names."""
    print(msg, flush=True)
    sys.stdout.flush()


def ulp_diff(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    def key(x):
        x = x.astype(np.int32)
        return np.where(x & 0x8000, -(x & 0x7FFF), x)
    return np.abs(key(a) - key(b))


def bf16_f32(a: np.ndarray) -> np.ndarray:
    return (np.asarray(a, np.uint16).astype(np.uint32) << 16).view(np.float32)


def assert_bf16_close(got: np.ndarray, want: np.ndarray, ulps: int = 2, what: str = "",
                      floor: float = 1e-3, outlier_frac: float = 0.0):
    """Element-wise: |got - want| <= ulps * ulp(|want|) + floor * max|want|.

    The absolute floor covers values near zero, where a sign change between two
    correctly rounded results is a tiny absolute difference but thousands of
    bf16 steps.  `outlier_frac` admits that fraction of elements beyond the ulp
    bound (cancellation, e.g. a*c - b*s in RoPE, magnifies a 1-ulp input
    difference), each still within 1e-2 of the tensor's scale.
    """
    g = bf16_f32(got).astype(np.float64)
    w = bf16_f32(want).astype(np.float64)
    scale = np.abs(w).max()
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(w), 1e-38))) - 7)
    allowed = ulps * ulp + floor * scale
    err = np.abs(g - w)
    bad = err > allowed
    msg = (f"{what}: {int(bad.sum())} of {bad.size} elements beyond {ulps} ulp; "
           f"worst {err.max():.3e} (scale {scale:.3e})")
    assert bad.mean() <= outlier_frac, msg
    assert err.max() <= 1e-2 * scale, msg


def assert_delta_close(x_in: np.ndarray, got: np.ndarray, want: np.ndarray, tol: float = 1e-2,
                       what: str = ""):
    """A residual layer's own contribution (out - in) matches: per element
    |got - want| <= 2 ulp(want) + tol * max|want - x_in|, i.e. the output is
    right to its own bf16 rounding plus a small fraction of what the layer added
    (a bare delta comparison is ill-conditioned where |x_in| >> |delta|), and the
    mean error is within tol of the mean |delta|.  Prints the worst element's share
    of its allowance and the mean ratio."""
    g, w, x = (bf16_f32(a).astype(np.float64) for a in (got, want, x_in))
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(w), 1e-38))) - 7)
    allowed = 2 * ulp + tol * np.abs(w - x).max()
    err = np.abs(g - w)
    bad = err > allowed
    mean_ratio = err.mean() / max(np.abs(w - x).mean(), 1e-30)
    print(f"  {what}: worst {float((err / allowed).max()):.2f} of its allowance, "
          f"mean error / mean |delta| {mean_ratio:.3e} (bar {tol:.0e})", flush=True)
    assert not bad.any(), f"{what}: {int(bad.sum())} elements off; worst {err.max():.3e}"
    assert mean_ratio <= tol, f"{what}: mean error {err.mean():.3e}"


def report_close(got, want, tol: float | None = None, what: str = ""):
    """tolerance.assert_close (default bar 1e-2), printing the measured errors first so a run's
    log shows each check's margin."""
    from tolerance import TOL, assert_close, rel_errors
    tol = TOL if tol is None else tol
    mx, mean = rel_errors(got, want)
    print(f"  {what}: max-abs/scale {mx:.3e}, mean-rel {mean:.3e} (bar {tol:.0e})", flush=True)
    assert_close(got, want, tol=tol, what=what)


def e2e_tol(noise: float) -> float:
    """Tolerance for 32-layer end-to-end results: the 1e-2 bar or 2x the stack's own
    summation-order noise floor, whichever is larger."""
    return max(1e-2, 2.0 * noise)


def check_token(tok: int, want_logits: np.ndarray, got_logits: np.ndarray, noise: float):
    """tok is the first maximum of the GPU's own logits, and the oracle's argmax unless the
    oracle's top-2 gap is inside 2x the noise floor."""
    assert tok == int(np.argmax(got_logits))
    order = np.argsort(want_logits)
    gap = want_logits[order[-1]] - want_logits[order[-2]]
    if gap > 2 * noise * np.abs(want_logits).max():
        assert tok == int(order[-1]), (tok, int(order[-1]), gap)
