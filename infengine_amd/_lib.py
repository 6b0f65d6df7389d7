"""ctypes binding of libinfengine_amd.so (the C-ABI declared in include/infengine.h).

The library is loaded from this package directory only; a missing library is an
ImportError, never a silent fallback.
"""
from __future__ import annotations

import ctypes as C
import pathlib

LIB_PATH = pathlib.Path(__file__).resolve().parent / "libinfengine_amd.so"

# include/infengine.h constants (config.h:5-27)
MAX_CONTEXT_LENGTH = 8192
MAX_LONG_CONTEXT = 131072
VOCAB_SIZE = 128256
NUM_LAYERS = 32
HIDDEN_SIZE = 4096
NUM_Q_HEADS = 32
NUM_KV_HEADS = 8
HEAD_DIM = 128
FFN_DIM = 14336

IE_OK = 0

_p = C.c_void_p


class TransformerBlockWeights(C.Structure):
    _fields_ = [("w_k", _p), ("w_q", _p), ("w_v", _p), ("w_o", _p)]


class FFNBlockWeights(C.Structure):
    _fields_ = [("w_up", _p), ("w_gate", _p), ("w_down", _p)]


class RoPEWeights(C.Structure):
    _fields_ = [("cos", _p), ("sin", _p)]


class Layer(C.Structure):
    _fields_ = [
        ("input_layernorm", _p),
        ("transformer", TransformerBlockWeights),
        ("post_attention_layernorm", _p),
        ("ffn_block", FFNBlockWeights),
    ]


class ModelWeightsStruct(C.Structure):
    _fields_ = [
        ("emb_lookup", _p),
        ("layers", Layer * NUM_LAYERS),
        ("final_norm", _p),
        ("lm_head", _p),
        ("rope", RoPEWeights),
        ("storage", _p),
        ("rope_rows", C.c_int),
    ]


_i, _u64, _f, _sz = C.c_int, C.c_uint64, C.c_float, C.c_size_t
_W = C.POINTER(ModelWeightsStruct)

# name -> (restype, argtypes); every entry point of include/infengine.h
SIGNATURES: dict[str, tuple] = {
    "ie_context_create": (_i, [C.POINTER(_p), _i, _p]),
    "ie_context_destroy": (_i, [_p]),
    "ie_context_stream": (_p, [_p]),
    "ie_context_set_graph": (_i, [_p, _i]),
    "ie_last_error": (C.c_char_p, []),
    "ie_attn_workspace_size": (_sz, [_i]),
    "ie_ffn_workspace_size": (_sz, [_i]),
    "ie_kv_cache_size": (_sz, []),
    "ie_prefill": (_i, [_p, _W, _i, _p, _p, _p, _p, _p, _p, _p, _p]),
    "ie_decode_step": (_i, [_p, _W, _i, _p, _p, _p, _p, _p, _p, _p, _p]),
    "ie_generate": (_i, [_p, _W, _p, _i, _i, _i, _i, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p]),
    "ie_batch_workspace_size": (_sz, [_i]),
    "ie_decode_step_batched": (_i, [_p, _W, _i, C.POINTER(_i), _p, _p, _p, _p, _p,
                                    C.POINTER(_i), _p, _p]),
    "ie_kv_page_size": (_sz, []),
    "ie_prefill_paged": (_i, [_p, _W, _i, _p, _p, _p, _p, _p, _p, _p, _p, _i, _p]),
    "ie_prefill_paged_chunk": (_i, [_p, _W, _i, _i, _p, _p, _p, _p, _p, _p, _p, _p, _i, _p]),
    "ie_kv_cache_to_pages": (_i, [_p, _p, _i, _i, _p, _i, _p]),
    "ie_decode_step_batched_paged": (_i, [_p, _W, _i, C.POINTER(_i), _p, _i, _p, _p, _p, _p,
                                          C.POINTER(_i), _p, _p, _i, _p, _i]),
    "ie_model_weights_random_init": (_i, [_W, _u64, _f]),
    "ie_model_weights_from_safetensors": (_i, [_W, C.POINTER(C.c_char_p), _i]),
    "ie_model_weights_free": (_i, [_W]),
    "ie_init_rope_buffer": (_i, [C.POINTER(_p), C.POINTER(_p)]),
    "ie_cleanup_rope_buffer": (_i, [_p, _p]),
    "ie_fill_synthetic_bf16": (_i, [_p, _sz, _u64, _u64, _f, _f, _p]),
    "ie_emblookup": (_i, [_i, _p, _p, _p, _p]),
    "ie_rmsnorm": (_i, [_i, _p, _p, _p, _p]),
    "ie_residual_add": (_i, [_i, _i, _p, _p, _p]),
    "ie_swiglu": (_i, [_i, _p, _p, _p, _p]),
    "ie_apply_rope": (_i, [_i, _i, _i, _p, _p, _p, _p, _i, _p]),
    "ie_scale_causal_softmax": (_i, [_i, _p, _p, _i, _p]),
    "ie_multiply_by_weight": (_i, [_p, _i, _i, _i, _p, _p, _p]),
    "ie_ffn": (_i, [_p, _i, _p, _p, _p, _p, _p, _p]),
    "ie_attn": (_i, [_p, _p, _p, _i, _p, _p, _p, _p, _p, _p, _p, _p, _i]),
    "ie_decode_attn": (_i, [_p, _p, _p, _i, _p, _p, _p, _p, _p, _p, _p, _p, _i]),
    "ie_lm_head": (_i, [_p, _i, _p, _p, _p]),
    "ie_sample_token_amax": (_i, [_p, _p, _p]),
    "ie_sample_argmax_rows": (_i, [_p, _i, _i, _p, _p]),
    "ie_top_p_workspace_size": (_sz, [_i, _i]),
    "ie_sample_top_p": (_i, [_p, _i, _i, _p, _f, _f, _u64, _u64, _p, _p]),
    "ie_sample_top_p_noalloc": (_i, [_p, _i, _i, _p, _f, _f, _u64, _u64, _p]),
    "ie_ffn_block_decode": (_i, [_p, _p, _p, _p, _p, _p, _p]),
    "ie_ffn_gate_up_decode": (_i, [_p, _p, _p, _p, _p, _p]),
    "ie_decoder_layer_decode": (_i, [_p, _W, _i, _i, _p, _p, _p, _p]),
    "ie_decoder_layer_prefill": (_i, [_p, _W, _i, _i, _p, _p, _p, _p, _p]),
    "ie_decoder_layer_prefill_last_row": (_i, [_p, _W, _i, _i, _p, _p, _p, _p, _p]),
    "ie_decoder_layer_batched": (_i, [_p, _W, _i, _i, C.POINTER(_i), _p, _p, _p, _p]),
    "ie_final_norm_lm_head": (_i, [_p, _i, _p, _p, _p, _p]),
    "ie_gemm_bf16": (_i, [_p, _i, _i, _i, _p, _p, _p]),
    "ie_gemm_ex": (_i, [_p, _i, _i, _i, _i, _p, _p, _p, _p]),
    "ie_attn_prefill_core": (_i, [_p, _i, _i, _p, _p, _p, _p]),
    "ie_attn_prefill_core_paged": (_i, [_p, _i, _i, _p, _p, _i, _p, _i, _p]),
    "ie_tune_gemv_waves": (_i, [_i]),
    "ie_tune_gemv_pairs_per_wave": (_i, [_i]),
    "ie_tune_gemm_schedule": (_i, [_i]),
}


class IEError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"infengine error {code}: {message}")
        self.code = code


def _load() -> C.CDLL:
    if not LIB_PATH.exists():
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python infengine_amd/build.py` "
            "(there is no fallback path)")
    lib = C.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def last_error() -> str:
    msg = lib.ie_last_error()
    return msg.decode() if msg else ""


def check(rc: int) -> int:
    """Raise IEError for a negative status; return rc (a token id for prefill/decode)."""
    if rc < 0:
        raise IEError(rc, last_error())
    return rc
