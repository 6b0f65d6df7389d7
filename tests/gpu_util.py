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


def P(t: torch.Tensor | None):
    return None if t is None else C.c_void_p(t.data_ptr())


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
