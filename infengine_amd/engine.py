"""torch-side helpers over the C-ABI: context, weights, and the per-request
buffers the reference Manager allocates (manager.cpp:38-67).

Device memory comes from torch (bf16 buffers are torch.bfloat16 tensors, whose
bits are the library's uint16 bf16); every computation runs in the library.
"""
from __future__ import annotations

import ctypes as C

import torch

from ._lib import (HIDDEN_SIZE, MAX_CONTEXT_LENGTH, VOCAB_SIZE, ModelWeightsStruct, check, lib)


def ptr(t: torch.Tensor | None) -> C.c_void_p | None:
    return None if t is None else C.c_void_p(t.data_ptr())


class _DeviceArray:
    """__cuda_array_interface__ wrapper: a zero-copy torch view of library memory."""

    def __init__(self, addr: int, shape, typestr: str):
        self.__cuda_array_interface__ = {"shape": tuple(shape), "typestr": typestr,
                                         "data": (int(addr), False), "version": 3,
                                         "strides": None}


def device_view(addr: int, shape, dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """torch tensor aliasing `addr` (device memory owned by the library)."""
    typestr = {torch.bfloat16: "<i2", torch.float32: "<f4", torch.int32: "<i4"}[dtype]
    t = torch.as_tensor(_DeviceArray(addr, shape, typestr), device="cuda")
    return t.view(dtype) if dtype == torch.bfloat16 else t


class Context:
    """ie_context on a dedicated torch stream, made torch's current stream so
    torch ops on the library's buffers are ordered with the library's kernels
    (hipGraph capture also needs a non-null stream)."""

    def __init__(self, device: int = 0, stream: torch.cuda.Stream | None = None,
                 graph: bool = True):
        torch.cuda.set_device(device)
        torch.cuda.synchronize(device)
        self.stream = stream if stream is not None else torch.cuda.Stream(device)
        torch.cuda.set_stream(self.stream)
        self.handle = C.c_void_p()
        check(lib.ie_context_create(C.byref(self.handle), device,
                                    C.c_void_p(self.stream.cuda_stream)))
        if not graph:
            check(lib.ie_context_set_graph(self.handle, 0))

    @property
    def stream_ptr(self) -> C.c_void_p:
        return C.c_void_p(self.stream.cuda_stream)

    def close(self) -> None:
        if self.handle:
            lib.ie_context_destroy(self.handle)
            self.handle = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class ModelWeights:
    """ie_model_weights (model_weights.cuh:21-34) owned by the library."""

    def __init__(self):
        self.s = ModelWeightsStruct()

    @classmethod
    def random_init(cls, seed: int = 0, std: float = 0.02) -> "ModelWeights":
        w = cls()
        check(lib.ie_model_weights_random_init(C.byref(w.s), seed, std))
        return w

    @classmethod
    def from_safetensors(cls, paths) -> "ModelWeights":
        """ModelWeights::from_safetensors (model_weights.cu:145-154): HF Llama-3.1-8B BF16
        checkpoint shards, kept BF16, in one library-owned arena."""
        w = cls()
        enc = [str(p).encode() for p in paths]
        arr = (C.c_char_p * len(enc))(*enc)
        check(lib.ie_model_weights_from_safetensors(C.byref(w.s), arr, len(enc)))
        return w

    def ref(self):
        return C.byref(self.s)

    def free(self) -> None:
        if self.s.storage:
            check(lib.ie_model_weights_free(C.byref(self.s)))

    def view(self, layer: int | None, name: str) -> torch.Tensor:
        """Zero-copy torch view of one weight tensor."""
        from ._lib import FFN_DIM, HIDDEN_SIZE as H
        shapes = {"input_layernorm": (H,), "post_attention_layernorm": (H,),
                  "w_q": (H, H), "w_k": (1024, H), "w_v": (1024, H), "w_o": (H, H),
                  "w_gate": (FFN_DIM, H), "w_up": (FFN_DIM, H), "w_down": (H, FFN_DIM),
                  "emb_lookup": (VOCAB_SIZE, H), "lm_head": (VOCAB_SIZE, H), "final_norm": (H,)}
        if layer is None:
            addr = getattr(self.s, name)
        else:
            L = self.s.layers[layer]
            if name in ("w_q", "w_k", "w_v", "w_o"):
                addr = getattr(L.transformer, name)
            elif name in ("w_gate", "w_up", "w_down"):
                addr = getattr(L.ffn_block, name)
            else:
                addr = getattr(L, name)
        return device_view(addr, shapes[name])

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def kv_cache_size() -> int:
    return int(lib.ie_kv_cache_size())


def workspace_size(max_seq_len: int) -> int:
    """manager.cpp:62-66: one workspace shared by attention and FFN."""
    return max(int(lib.ie_attn_workspace_size(max_seq_len)),
               int(lib.ie_ffn_workspace_size(max_seq_len)))


class Request:
    """The per-request device buffers of Manager::handle_request (manager.cpp:38-67)."""

    def __init__(self, ctx: Context, weights: ModelWeights, max_seq_len: int,
                 device: str = "cuda"):
        self.ctx, self.weights = ctx, weights
        L = MAX_CONTEXT_LENGTH
        self.tokens = torch.zeros(L, dtype=torch.int32, device=device)
        self.data = torch.zeros(L, HIDDEN_SIZE, dtype=torch.bfloat16, device=device)
        self.aux = torch.zeros(L, HIDDEN_SIZE, dtype=torch.bfloat16, device=device)
        self.attn = torch.zeros(L, HIDDEN_SIZE, dtype=torch.bfloat16, device=device)
        self.logits = torch.zeros(VOCAB_SIZE, dtype=torch.float32, device=device)
        self.token = torch.zeros(1, dtype=torch.int32, device=device)
        self.workspace = torch.zeros(workspace_size(max_seq_len), dtype=torch.uint8,
                                     device=device)
        self.kv = torch.zeros(kv_cache_size(), dtype=torch.uint8, device=device)

    def _args(self, seq_len: int):
        return (self.ctx.handle, self.weights.ref(), seq_len, ptr(self.tokens), ptr(self.data),
                ptr(self.aux), ptr(self.attn), ptr(self.logits), ptr(self.token),
                ptr(self.workspace), ptr(self.kv))

    def prefill(self, seq_len: int) -> int:
        return check(lib.ie_prefill(*self._args(seq_len)))

    def decode_step(self, seq_len: int) -> int:
        return check(lib.ie_decode_step(*self._args(seq_len)))

    def generate(self, prompt, max_new_tokens: int, timed_from: int | None = None,
                 eos_token: int = -1):
        """Manager::handle_request's loop (manager.cpp:60-86) without the tokenizer: prefill of
        `prompt` (host ints), then decode steps with the device-side token write-back, all in
        the library, until max_new_tokens tokens or right after eos_token (>= 0).  Returns
        (tokens, timed_ms) where timed_ms is the wall time of decode steps timed_from .. the
        last one (None when timed_from is None)."""
        import numpy as np
        ids = np.ascontiguousarray(np.asarray(prompt, dtype=np.int32))
        out = (C.c_int * max_new_tokens)()
        ms = C.c_double(0.0)
        tf = max_new_tokens if timed_from is None else timed_from
        n = check(lib.ie_generate(self.ctx.handle, self.weights.ref(),
                                  ids.ctypes.data_as(C.c_void_p), len(ids), max_new_tokens,
                                  eos_token, tf, out, ptr(self.tokens), ptr(self.data),
                                  ptr(self.aux), ptr(self.attn), ptr(self.logits), ptr(self.token),
                                  ptr(self.workspace), ptr(self.kv), C.byref(ms)))
        return list(out)[:n], (ms.value if timed_from is not None else None)

    def kv_view(self) -> torch.Tensor:
        """[layers][2][8][8192][128] bf16 view of the cache."""
        return self.kv.view(torch.bfloat16).view(32, 2, 8, MAX_CONTEXT_LENGTH, 128)
