"""MI355X (gfx950) per-token Llama-3.1-8B hot path.

The product is the C-ABI library libinfengine_amd.so (include/infengine.h):
hand-written HIP kernels behind the reference engine's prefill / decode_step /
ModelWeights interface.  This package loads it with ctypes and adds thin torch
helpers (torch supplies device memory and streams).  There is no CPU or
PyTorch fallback: without the built library, importing this package fails.
"""
from ._lib import (FFN_DIM, HEAD_DIM, HIDDEN_SIZE, LIB_PATH, MAX_CONTEXT_LENGTH, NUM_KV_HEADS,
                   NUM_LAYERS, NUM_Q_HEADS, VOCAB_SIZE, IEError, ModelWeightsStruct, check,
                   last_error, lib)

__all__ = [
    "lib", "check", "last_error", "IEError", "ModelWeightsStruct", "LIB_PATH",
    "MAX_CONTEXT_LENGTH", "VOCAB_SIZE", "NUM_LAYERS", "HIDDEN_SIZE", "NUM_Q_HEADS",
    "NUM_KV_HEADS", "HEAD_DIM", "FFN_DIM",
]
