"""Write the committed golden fixtures under tests/golden/.

Every expected value here comes from a library routine (torch 2.10 /
transformers 5.15 as installed in the build container), never from the
reference's code: the reference's own generator (scripts/generate_test_data.py)
needs a downloaded checkpoint and its outputs are not in the tree.  The library
routines used are the ones that generator calls (torch.argmax, LlamaRMSNorm,
the Llama-3 RoPE parameters, softmax) plus HF's top-p warper for the sampler the
reference lacks.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import pathlib

import numpy as np
import torch

HERE = pathlib.Path(__file__).resolve().parent
VOCAB = 128256


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.to(torch.bfloat16).contiguous().view(torch.int16).numpy().view(np.uint16)


def argmax_cases() -> None:
    g = torch.Generator().manual_seed(42)
    rows = []
    rows.append(torch.randn(VOCAB, generator=g))                       # plain (generate_test_data.py:163-168)
    t = torch.randn(VOCAB, generator=g)
    t[5000] = t[90000] = t.max() + 1.0                                 # tie: first index wins
    rows.append(t)
    t = torch.randn(VOCAB, generator=g)
    t[77777] = float("nan")
    t[100] = float("nan")                                               # NaN beats everything, first NaN
    rows.append(t)
    t = torch.full((VOCAB,), -1.0)
    t[300] = -0.0
    t[200] = 0.0
    t[128255] = 0.0                                                     # signed zeros compare equal
    rows.append(t)
    t = torch.full((VOCAB,), float("-inf"))
    t[128255] = -1e30                                                   # max at the last index
    rows.append(t)
    logits = torch.stack(rows).float()
    expect = torch.argmax(logits, dim=-1).to(torch.int32)
    np.savez_compressed(HERE / "argmax_torch.npz", logits=logits.numpy(), expect=expect.numpy())


def rope_llama3() -> None:
    from transformers import LlamaConfig
    from transformers.modeling_rope_utils import ROPE_INIT_FUNCTIONS
    cfg = LlamaConfig(hidden_size=4096, num_attention_heads=32, num_key_value_heads=8,
                      head_dim=128, max_position_embeddings=131072,
                      rope_parameters={"rope_type": "llama3", "rope_theta": 500000.0,
                                       "factor": 8.0, "low_freq_factor": 1.0,
                                       "high_freq_factor": 4.0,
                                       "original_max_position_embeddings": 8192})
    inv_freq, _ = ROPE_INIT_FUNCTIONS["llama3"](cfg, torch.device("cpu"))
    pos = torch.tensor([0, 1, 2, 3, 100, 1000, 2047, 4095, 6000, 8191])
    ang = torch.outer(pos.double(), inv_freq.double())
    np.savez_compressed(HERE / "rope_llama3_hf.npz", inv_freq=inv_freq.numpy(),
                        positions=pos.numpy().astype(np.int32), cos=ang.cos().numpy(),
                        sin=ang.sin().numpy())


def rope_llama3_long() -> None:
    """cos/sin past the reference's 8192 positions (Llama-3.1 runs to 131072), from HF's own
    LlamaRotaryEmbedding forward: fp32 angles position * inv_freq, as the model computes them."""
    from transformers import LlamaConfig
    from transformers.models.llama.modeling_llama import LlamaRotaryEmbedding
    cfg = LlamaConfig(hidden_size=4096, num_attention_heads=32, num_key_value_heads=8,
                      head_dim=128, max_position_embeddings=131072,
                      rope_parameters={"rope_type": "llama3", "rope_theta": 500000.0,
                                       "factor": 8.0, "low_freq_factor": 1.0,
                                       "high_freq_factor": 4.0,
                                       "original_max_position_embeddings": 8192})
    rot = LlamaRotaryEmbedding(cfg)
    pos = torch.tensor([8191, 8192, 8193, 9000, 12345, 16383, 16384, 32768, 65535, 100000,
                        131071])
    cos, sin = rot(torch.zeros(1, pos.numel(), 128), pos[None, :])
    assert rot.attention_scaling == 1.0
    np.savez_compressed(HERE / "rope_llama3_hf_long.npz", positions=pos.numpy().astype(np.int32),
                        cos=cos[0, :, :64].numpy(), sin=sin[0, :, :64].numpy())


def rmsnorm_hf() -> None:
    from transformers.models.llama.modeling_llama import LlamaRMSNorm
    g = torch.Generator().manual_seed(7)
    x = (torch.randn(16, 4096, generator=g) * 2.0).to(torch.bfloat16)
    w = (1.0 + 0.02 * torch.randn(4096, generator=g)).to(torch.bfloat16)
    m = LlamaRMSNorm(4096, eps=1e-5)
    m.weight.data = w.clone()
    with torch.no_grad():
        y = m(x)
    np.savez_compressed(HERE / "rmsnorm_hf.npz", x=bf16_bits(x), w=bf16_bits(w), y=bf16_bits(y))


def top_p_hf() -> None:
    from transformers.generation.logits_process import (TemperatureLogitsWarper,
                                                        TopPLogitsWarper)
    g = torch.Generator().manual_seed(11)
    logits = torch.stack([torch.randn(VOCAB, generator=g) * 3.0,
                          torch.randn(VOCAB, generator=g) * 0.5]).float()
    scores = TemperatureLogitsWarper(0.7)(None, logits.clone())
    scores = TopPLogitsWarper(0.9)(None, scores)
    kept = torch.isfinite(scores).numpy()
    np.savez_compressed(HERE / "top_p_hf.npz", logits=logits.numpy(),
                        kept=np.packbits(kept, axis=-1), temperature=np.float32(0.7),
                        top_p=np.float32(0.9))


if __name__ == "__main__":
    argmax_cases()
    rope_llama3()
    rope_llama3_long()
    rmsnorm_hf()
    top_p_hf()
    for f in sorted(HERE.glob("*.npz")):
        print(f.name, f.stat().st_size)
