"""Writers of Llama-3.1-8B-shaped safetensors files for the loader tests (no reference code:
the format is the published one, an 8-byte little-endian header length, a JSON header of
{name: {dtype, shape, data_offsets}} and the raw data)."""
from __future__ import annotations

import json
import pathlib
import struct

H, F, V, KV, L = 4096, 14336, 128256, 1024, 32
FIELDS = [("input_layernorm.weight", (H,)), ("self_attn.q_proj.weight", (H, H)),
          ("self_attn.k_proj.weight", (KV, H)), ("self_attn.v_proj.weight", (KV, H)),
          ("self_attn.o_proj.weight", (H, H)), ("post_attention_layernorm.weight", (H,)),
          ("mlp.gate_proj.weight", (F, H)), ("mlp.up_proj.weight", (F, H)),
          ("mlp.down_proj.weight", (H, F))]


def llama_tensors() -> list[tuple[str, tuple[int, ...]]]:
    """All 291 tensor names of a Llama-3.1-8B checkpoint with their shapes."""
    t = [("model.embed_tokens.weight", (V, H))]
    for layer in range(L):
        t += [(f"model.layers.{layer}.{n}", s) for n, s in FIELDS]
    return t + [("model.norm.weight", (H,)), ("lm_head.weight", (V, H))]


def write_header(path: pathlib.Path, entries: list[tuple[str, str, tuple[int, ...], int]],
                 metadata: bool = True, raw_header: bytes | None = None) -> tuple[int, int]:
    """entries: (name, dtype, shape, nbytes).  Writes header + a sparse data section (zeros);
    returns (data_start, data_bytes)."""
    hdr = {"__metadata__": {"format": "pt"}} if metadata else {}
    off = 0
    for name, dtype, shape, nbytes in entries:
        hdr[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [off, off + nbytes]}
        off += nbytes
    blob = raw_header if raw_header is not None else json.dumps(hdr).encode()
    blob += b" " * (-len(blob) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(blob)))
        f.write(blob)
        f.truncate(8 + len(blob) + off)
    return 8 + len(blob), off
