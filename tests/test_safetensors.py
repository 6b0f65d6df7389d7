"""ModelWeights::from_safetensors (model_weights.cu:14-59, 80-154): every validation error of
the loader, which all happen before any device work (so these run without a GPU), and — on the
GPU — a complete two-shard checkpoint landing field by field in the arena."""
import ctypes as C
import pathlib

import numpy as np
import pytest

from safetensors_util import H, write_header, llama_tensors

import infengine_amd as ie
from infengine_amd import IEError
from infengine_amd.engine import ModelWeights


def load(paths):
    return ModelWeights.from_safetensors(paths)


def bf16(shape):
    n = int(np.prod(shape))
    return n * 2


def full_entries():
    return [(n, "BF16", s, bf16(s)) for n, s in llama_tensors()]


def expect(paths, msg):
    with pytest.raises(IEError) as e:
        load(paths)
    assert msg in str(e.value), str(e.value)


def test_missing_file(tmp_path):
    expect([tmp_path / "nope.safetensors"], "cannot open")


def test_bad_header_json(tmp_path):
    p = tmp_path / "a.safetensors"
    write_header(p, [], raw_header=b'{"model.norm.weight": {"dtype": "BF16", ')
    expect([p], "bad header JSON")


def test_header_length_past_end(tmp_path):
    p = tmp_path / "a.safetensors"
    p.write_bytes((10**6).to_bytes(8, "little") + b"{}")
    expect([p], "header length")


def test_unknown_tensor_name(tmp_path):
    p = tmp_path / "a.safetensors"
    write_header(p, [("model.layers.0.self_attn.rotary_emb.inv_freq", "BF16", (64,), 128)])
    expect([p], "model.layers.0.self_attn.rotary_emb.inv_freq is an unknown tensor name")


def test_layer_index_out_of_range(tmp_path):
    p = tmp_path / "a.safetensors"
    write_header(p, [("model.layers.32.input_layernorm.weight", "BF16", (H,), 2 * H)])
    expect([p], "layer index out of range")


def test_wrong_dtype(tmp_path):
    p = tmp_path / "a.safetensors"
    write_header(p, [("model.norm.weight", "F16", (H,), 2 * H)])
    expect([p], "has dtype F16, expected BF16")


def test_wrong_shape(tmp_path):
    p = tmp_path / "a.safetensors"
    write_header(p, [("model.layers.3.self_attn.k_proj.weight", "BF16", (H, H), 2 * H * H)])
    expect([p], "has shape [4096, 4096], expected [1024, 4096]")


def test_byte_count_mismatch(tmp_path):
    p = tmp_path / "a.safetensors"
    write_header(p, [("model.norm.weight", "BF16", (H,), 2 * H + 2)])
    expect([p], "data bytes for 4096 bf16 elements")


def test_data_past_end_of_file(tmp_path):
    p = tmp_path / "a.safetensors"
    start, n = write_header(p, [("model.norm.weight", "BF16", (H,), 2 * H)])
    with open(p, "r+b") as f:
        f.truncate(start + n - 2)
    expect([p], "runs past the end of the file")


def test_duplicate_across_shards(tmp_path):
    a, b = tmp_path / "a.safetensors", tmp_path / "b.safetensors"
    write_header(a, [("model.norm.weight", "BF16", (H,), 2 * H)])
    write_header(b, [("model.norm.weight", "BF16", (H,), 2 * H)])
    expect([a, b], "tensor model.norm.weight appears twice")


def test_incomplete_checkpoint_names_first_missing(tmp_path):
    p = tmp_path / "a.safetensors"
    ents = [e for e in full_entries() if e[0] != "model.layers.7.mlp.up_proj.weight"]
    write_header(p, ents)
    expect([p], "missing tensor model.layers.7.mlp.up_proj.weight")


def test_no_files():
    with pytest.raises(IEError) as e:
        ie.check(ie.lib.ie_model_weights_from_safetensors(C.byref(ModelWeights().s), None, 0))
    assert "no files" in str(e.value)


# ---------------------------------------------------------------- GPU: a complete checkpoint
def _pattern(i: int, n: int) -> np.ndarray:
    rng = np.random.default_rng(1000 + i)
    return rng.integers(1, 65535, n, dtype=np.uint16)


@pytest.mark.gpu
def test_two_shard_checkpoint_lands_in_every_field(tmp_path):
    """All 291 tensors in two sparse shards; each gets a distinct 2 KiB pattern at its head and
    tail and zeros between (sparse file regions), so every name -> field mapping is checked
    without writing 16 GB."""
    import torch
    from gpu_util import host, say
    tensors = llama_tensors()
    half = len(tensors) // 2
    shards = [tensors[:half], tensors[half:]]
    paths, marks = [], {}
    for si, part in enumerate(shards):
        p = tmp_path / f"model-{si + 1:05d}-of-00002.safetensors"
        start, _ = write_header(p, [(n, "BF16", s, bf16(s)) for n, s in part])
        with open(p, "r+b") as f:
            off = start
            for n, s in part:
                i = tensors.index((n, s))
                k = min(1024, int(np.prod(s)) // 2)
                head, tail = _pattern(2 * i, k), _pattern(2 * i + 1, k)
                f.seek(off)
                f.write(head.tobytes())
                f.seek(off + bf16(s) - 2 * k)
                f.write(tail.tobytes())
                marks[n] = (s, head, tail)
                off += bf16(s)
        paths.append(p)
    say("from_safetensors: 2 sparse shards, 291 tensors")
    W = load(paths)
    try:
        from infengine_amd.engine import device_view
        for n, (s, head, tail) in marks.items():
            if n == "model.embed_tokens.weight":
                t = W.view(None, "emb_lookup")
            elif n == "lm_head.weight":
                t = W.view(None, "lm_head")
            elif n == "model.norm.weight":
                t = W.view(None, "final_norm")
            else:
                layer, sub = int(n.split(".")[2]), ".".join(n.split(".")[3:])
                field = {"input_layernorm.weight": "input_layernorm",
                         "self_attn.q_proj.weight": "w_q", "self_attn.k_proj.weight": "w_k",
                         "self_attn.v_proj.weight": "w_v", "self_attn.o_proj.weight": "w_o",
                         "post_attention_layernorm.weight": "post_attention_layernorm",
                         "mlp.gate_proj.weight": "w_gate", "mlp.up_proj.weight": "w_up",
                         "mlp.down_proj.weight": "w_down"}[sub]
                t = W.view(layer, field)
            assert tuple(t.shape) == tuple(s), n
            flat = t.reshape(-1).view(torch.int16)
            k = len(head)
            assert np.array_equal(host(flat[:k]).view(np.uint16), head), n
            assert np.array_equal(host(flat[-k:]).view(np.uint16), tail), n
            if flat.numel() > 4 * k:
                mid = flat.numel() // 2
                assert not host(flat[mid:mid + 256]).any(), n
        # RoPE tables as built by random_init (init_rope_buffer)
        R = ModelWeights.random_init(seed=0)
        for f in ("cos", "sin"):
            a = device_view(getattr(W.s.rope, f), (8192, 64), torch.float32)
            b = device_view(getattr(R.s.rope, f), (8192, 64), torch.float32)
            assert torch.equal(a, b)
        R.free()
    finally:
        W.free()
