"""CPU oracle — TEST INFRASTRUCTURE ONLY.

numpy/ctypes front end of oracle/oracle.cpp, the plain C++ restatement of the
reference's per-token Llama-3.1-8B math (see the citations in oracle.cpp).
Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
it, and only as the checker; the product package never imports it.

bf16 tensors are numpy uint16 arrays holding the bit patterns.

Parity status of each function (how it is pinned, see tests/test_oracle.py):
  fill_synthetic  - statistics (mean/std) + GPU generator bit-equality
  rope_freqs      - HF transformers _compute_llama3_parameters (library)
  rope_tables     - HF llama3 parameters and HF LlamaRotaryEmbedding past 8192 positions
                    (library fixtures) + closed form cos(fp32(pos * freq)), cos^2 + sin^2 = 1
  rmsnorm         - HF LlamaRMSNorm (library) in bf16
  matmul          - float64 brute force; torch bf16 nn.functional.linear (library)
  swiglu          - torch.nn.functional.silu (library)
  apply_rope      - HF apply_rotary_pos_emb (library); pair-norm invariant
  softmax_scaled  - torch.softmax (library); rows sum to 1
  attention       - HF eager attention with repeat_kv (library, fp32)
  decoder_layer   - HF LlamaDecoderLayer (library, small config) + prefill/decode invariant
  argmax          - torch.argmax (library) incl. ties, NaN, signed zeros
  top_p           - HF TopPLogitsWarper kept set (library) + brute-force minimal prefix
"""
from __future__ import annotations

import ctypes as C
import pathlib
import subprocess

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "liboracle.so"

HIDDEN, FFN, QH, KVH, HD, VOCAB, MAXCTX, LAYERS = 4096, 14336, 32, 8, 128, 128256, 8192, 32
LONGCTX = 131072   # positions of the paged (long-context) paths and their RoPE tables


def build() -> pathlib.Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def _load() -> C.CDLL:
    if not LIB_PATH.exists():
        build()
    lib = C.CDLL(str(LIB_PATH))
    P, I, U64, F, SZ = C.c_void_p, C.c_int, C.c_uint64, C.c_float, C.c_size_t
    sig = {
        "orc_set_sum_order": (None, [I]),
        "orc_set_prob_round": (None, [I]),
        "orc_fill_synthetic": (None, [P, SZ, U64, U64, F, F]),
        "orc_tensor_id": (U64, [I, I]),
        "orc_rope_freqs": (None, [P]),
        "orc_rope_tables": (None, [I, P, P]),
        "orc_emblookup": (None, [I, P, P, P]),
        "orc_rmsnorm": (None, [I, I, P, P, P]),
        "orc_residual_add": (None, [SZ, P, P]),
        "orc_swiglu": (None, [SZ, P, P, P]),
        "orc_matmul_bf16": (None, [I, I, I, P, P, P]),
        "orc_matmul_f32": (None, [I, I, I, P, P, P]),
        "orc_apply_rope": (None, [I, I, I, I, P, P, P, P]),
        "orc_softmax_scaled": (None, [I, I, I, P, P]),
        "orc_attention": (None, [I, I, P, P, P, I, P]),
        "orc_decoder_layer": (None, [I, I, P, P, P, P, P, P, P, P, P, P, P, P, P, P, I]),
        "orc_ffn": (None, [I, P, P, P, P, P]),
        "orc_argmax": (I, [I, P]),
        "orc_top_p": (I, [I, P, F, F, U64, I, U64, P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


_lib = _load()


def _p(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle inputs must be C-contiguous"
    return a.ctypes.data


def _u16(a) -> np.ndarray:
    a = np.ascontiguousarray(a)
    assert a.dtype == np.uint16, a.dtype
    return a


class reversed_summation:
    """Context manager: every oracle dot product sums k in descending order.
    The divergence between the two orders is the fp32 rounding-noise floor."""

    def __enter__(self):
        _lib.orc_set_sum_order(1)
        return self

    def __exit__(self, *exc):
        _lib.orc_set_sum_order(0)
        return False


PROB_FP32, PROB_REFERENCE, PROB_FLASH = 0, 1, 2


class prob_rounding:
    """Context manager: the rounding point of the attention probabilities before P.V.
    PROB_FP32 (the default) keeps them in fp32; PROB_REFERENCE rounds the normalised
    probabilities to bf16 as the reference's softmax stores them (softmax.cu:105,158) before
    its A.V GEMM (attn.cu:167-204); PROB_FLASH rounds exp2((s - m) c) to bf16 against the
    running max m of 64-key tiles and divides by the sum of the rounded values at the end,
    the form of an MFMA flash attention whose P.V operand is bf16."""

    def __init__(self, mode: int):
        self.mode = mode

    def __enter__(self):
        _lib.orc_set_prob_round(self.mode)
        return self

    def __exit__(self, *exc):
        _lib.orc_set_prob_round(PROB_FP32)
        return False


# ---------------------------------------------------------------- bf16 helpers
def bf16_to_f32(a: np.ndarray) -> np.ndarray:
    return (np.asarray(a, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(a: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even; NaN stays NaN."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


# ---------------------------------------------------------------- synthetic data
def tensor_id(layer: int, field: int) -> int:
    return int(_lib.orc_tensor_id(layer, field))


LAYER_FIELDS = ("input_layernorm", "w_q", "w_k", "w_v", "w_o", "post_attention_layernorm",
                "w_gate", "w_up", "w_down")
LAYER_SHAPES = {"input_layernorm": (HIDDEN,), "w_q": (HIDDEN, HIDDEN), "w_k": (1024, HIDDEN),
                "w_v": (1024, HIDDEN), "w_o": (HIDDEN, HIDDEN), "post_attention_layernorm": (HIDDEN,),
                "w_gate": (FFN, HIDDEN), "w_up": (FFN, HIDDEN), "w_down": (HIDDEN, FFN)}


def synthetic(shape, seed: int, tid: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(shape, dtype=np.uint16)
    _lib.orc_fill_synthetic(_p(out), out.size, seed, tid, mean, std)
    return out


def layer_weights(seed: int, layer: int, std: float = 0.02) -> dict[str, np.ndarray]:
    """Weights of one layer of the synthetic model (same ids as ie_model_weights_random_init)."""
    w = {}
    for f, name in enumerate(LAYER_FIELDS):
        norm = name.endswith("layernorm")
        w[name] = synthetic(LAYER_SHAPES[name], seed, tensor_id(layer, f),
                            1.0 if norm else 0.0, 0.02 if norm else std)
    return w


def embedding(seed: int, std: float = 0.02) -> np.ndarray:
    return synthetic((VOCAB, HIDDEN), seed, 1, 0.0, std)


def final_norm(seed: int) -> np.ndarray:
    return synthetic((HIDDEN,), seed, 2, 1.0, 0.02)


def lm_head_weight(seed: int, std: float = 0.02) -> np.ndarray:
    return synthetic((VOCAB, HIDDEN), seed, 3, 0.0, std)


# ---------------------------------------------------------------- ops
def rope_freqs() -> np.ndarray:
    """The 64 fp32 Llama-3 scaled inverse frequencies the tables are built from."""
    f = np.empty(64, np.float32)
    _lib.orc_rope_freqs(_p(f))
    return f


def rope_tables(n_pos: int = MAXCTX) -> tuple[np.ndarray, np.ndarray]:
    c = np.empty((n_pos, 64), np.float32)
    s = np.empty((n_pos, 64), np.float32)
    _lib.orc_rope_tables(n_pos, _p(c), _p(s))
    return c, s


def emblookup(ids: np.ndarray, table: np.ndarray) -> np.ndarray:
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    out = np.empty((ids.size, HIDDEN), np.uint16)
    _lib.orc_emblookup(ids.size, _p(ids), _p(_u16(table)), _p(out))
    return out


def rmsnorm(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    x = _u16(x)
    cols = x.shape[-1]
    out = np.empty_like(x)
    _lib.orc_rmsnorm(x.size // cols, cols, _p(x), _p(_u16(w)), _p(out))
    return out


def residual_add(x: np.ndarray, d: np.ndarray) -> np.ndarray:
    x = _u16(x).copy()
    _lib.orc_residual_add(x.size, _p(x), _p(_u16(d)))
    return x


def swiglu(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    g, u = _u16(g), _u16(u)
    out = np.empty_like(g)
    _lib.orc_swiglu(g.size, _p(g), _p(u), _p(out))
    return out


def matmul(x: np.ndarray, w: np.ndarray, out_f32: bool = False) -> np.ndarray:
    """Y = X . W^T with fp32 accumulation (multiply_by_weight)."""
    x, w = _u16(x), _u16(w)
    k = x.shape[-1]
    m = x.size // k
    n = w.shape[0]
    assert w.shape[1] == k
    if out_f32:
        y = np.empty((m, n), np.float32)
        _lib.orc_matmul_f32(m, k, n, _p(x), _p(w), _p(y))
    else:
        y = np.empty((m, n), np.uint16)
        _lib.orc_matmul_bf16(m, k, n, _p(x), _p(w), _p(y))
    return y


def apply_rope(x: np.ndarray, start_pos: int, heads: int, seq_len: int, head_rows: int,
               cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    x = _u16(x)
    out = x.copy()
    _lib.orc_apply_rope(start_pos, heads, seq_len, head_rows, _p(np.ascontiguousarray(cos)),
                        _p(np.ascontiguousarray(sin)), _p(x), _p(out))
    return out


def softmax_scaled(x: np.ndarray, length: int, causal: bool) -> np.ndarray:
    x = _u16(x)
    out = np.empty_like(x)
    _lib.orc_softmax_scaled(x.size // length, length, int(causal), _p(x), _p(out))
    return out


def attention(q: np.ndarray, kplane: np.ndarray, vplane: np.ndarray, q_start: int,
              ctx_stride: int) -> np.ndarray:
    q = _u16(q)
    n_q = q.size // HIDDEN
    out = np.empty((n_q, HIDDEN), np.uint16)
    _lib.orc_attention(n_q, q_start, _p(q), _p(_u16(kplane)), _p(_u16(vplane)), ctx_stride,
                       _p(out))
    return out


def decoder_layer(x: np.ndarray, w: dict, start_pos: int, cos, sin, kplane: np.ndarray,
                  vplane: np.ndarray, ctx_stride: int) -> None:
    """In place on x [S, 4096] and the layer's cache planes [8, ctx_stride, 128]."""
    assert x.dtype == np.uint16 and x.flags["C_CONTIGUOUS"]
    S = x.size // HIDDEN
    _lib.orc_decoder_layer(S, start_pos, _p(x), _p(_u16(w["input_layernorm"])), _p(_u16(w["w_q"])),
                           _p(_u16(w["w_k"])), _p(_u16(w["w_v"])), _p(_u16(w["w_o"])),
                           _p(_u16(w["post_attention_layernorm"])), _p(_u16(w["w_gate"])),
                           _p(_u16(w["w_up"])), _p(_u16(w["w_down"])),
                           _p(np.ascontiguousarray(cos)), _p(np.ascontiguousarray(sin)),
                           _p(kplane), _p(vplane), ctx_stride)


def ffn(x: np.ndarray, wg, wu, wd) -> np.ndarray:
    x = _u16(x)
    S = x.size // HIDDEN
    out = np.empty((S, HIDDEN), np.uint16)
    _lib.orc_ffn(S, _p(x), _p(_u16(wg)), _p(_u16(wu)), _p(_u16(wd)), _p(out))
    return out


def argmax(logits: np.ndarray) -> int:
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    return int(_lib.orc_argmax(logits.size, _p(logits)))


def top_p(logits: np.ndarray, temperature: float, p: float, seed: int, row: int,
          step: int) -> tuple[int, dict]:
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    info = np.zeros(4, np.float64)
    tok = int(_lib.orc_top_p(logits.size, _p(logits), temperature, p, seed, row, step, _p(info)))
    return tok, {"t": info[0], "lo": info[1], "hi": info[2], "z_kept": info[3]}


class SyntheticModel:
    """The oracle's copy of ie_model_weights_random_init(seed, std): the same
    tensors, regenerated layer by layer on the host (decode.cu / prefill.cu order)."""

    def __init__(self, seed: int, std: float = 0.02, n_pos: int = LONGCTX):
        self.seed, self.std = seed, std
        self.cos, self.sin = rope_tables(n_pos)
        self._emb = None
        self._lm = None

    def embed(self, ids) -> np.ndarray:
        if self._emb is None:
            self._emb = embedding(self.seed, self.std)
        return emblookup(np.asarray(ids, np.int32), self._emb)

    def layers(self, x: np.ndarray, start_pos: int, kv: np.ndarray, n_layers: int = LAYERS):
        """Run x [S, 4096] (in place) through the layers; kv is [32, 2, 8, ctx, 128]."""
        ctx = kv.shape[3]
        for l in range(n_layers):
            w = layer_weights(self.seed, l, self.std)
            decoder_layer(x, w, start_pos, self.cos, self.sin, kv[l, 0], kv[l, 1], ctx)
        return x

    def logits(self, x_row: np.ndarray) -> np.ndarray:
        if self._lm is None:
            self._lm = lm_head_weight(self.seed, self.std)
        xn = rmsnorm(np.ascontiguousarray(x_row).reshape(1, HIDDEN), final_norm(self.seed))
        return matmul(xn, self._lm, out_f32=True)[0]

    def decode(self, token: int, pos: int, kv: np.ndarray) -> np.ndarray:
        """decode_step at seq_len = pos + 1: logits of the new token."""
        x = self.embed([token])
        self.layers(x, pos, kv)
        return self.logits(x[0])

    def prefill(self, ids, kv: np.ndarray) -> np.ndarray:
        x = self.embed(ids)
        self.layers(x, 0, kv)
        return self.logits(x[-1])
