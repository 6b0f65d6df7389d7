"""Pin the CPU oracle (oracle/) before trusting it as the GPU checker.

Each oracle function is checked against a library routine (torch / HF
transformers, the math behind the reference's generate_test_data.py), a golden
fixture written by such a routine, a closed form or an invariant — chosen so a
dropped term, wrong sign/index or transposed operand fails.  CPU only.
"""
import pathlib

import numpy as np
import pytest
import torch

import oracle as orc
from tolerance import assert_close

GOLD = pathlib.Path(__file__).resolve().parent / "golden"


def t_bf16(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)


def bits(t: torch.Tensor) -> np.ndarray:
    return t.to(torch.bfloat16).contiguous().view(torch.int16).numpy().view(np.uint16)


def ulp_diff(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Distance in bf16 units-in-the-last-place (sign-magnitude aware)."""
    def key(x):
        x = x.astype(np.int32)
        return np.where(x & 0x8000, -(x & 0x7FFF), x)
    return np.abs(key(a) - key(b))


# ---------------------------------------------------------------- bf16 + synthetic
def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32) * 10,
                        np.array([0.0, -0.0, 1e-40, -1e-40, 3.4e38, np.inf, -np.inf], np.float32)])
    ours = orc.f32_to_bf16(x)
    ref = bits(torch.from_numpy(x))
    assert np.array_equal(ours, ref)
    assert np.array_equal(orc.bf16_to_f32(ours), torch.from_numpy(x).to(torch.bfloat16).float().numpy())


def test_synthetic_is_deterministic_and_normal_shaped():
    a = orc.synthetic((1 << 20,), seed=5, tid=9, mean=0.0, std=0.02)
    b = orc.synthetic((1 << 20,), seed=5, tid=9, mean=0.0, std=0.02)
    c = orc.synthetic((1 << 20,), seed=5, tid=10, mean=0.0, std=0.02)
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    f = orc.bf16_to_f32(a).astype(np.float64)
    assert abs(f.mean()) < 1e-4
    assert abs(f.std() - 0.02) < 2e-4
    # Irwin-Hall(4): kurtosis 3 - 1.2/4 = 2.7, support +-sqrt(12)*sigma
    assert 2.6 < ((f - f.mean()) ** 4).mean() / f.var() ** 2 < 2.8
    assert np.abs(f).max() <= 0.02 * np.sqrt(12) * 1.01
    n = orc.bf16_to_f32(orc.synthetic((1 << 16,), 5, 2, 1.0, 0.02))
    assert abs(n.mean() - 1.0) < 1e-3


# ---------------------------------------------------------------- embedding gather
def test_emblookup_is_a_row_gather():
    """orc.emblookup == table[ids] (emblookup.cu:19-24), first and last rows included, ids
    repeated and unsorted; a transposed or off-by-one gather fails."""
    table = orc.synthetic((orc.VOCAB, orc.HIDDEN), 9, 1, 0.0, 0.02)
    ids = np.array([0, orc.VOCAB - 1, 5, 5, 128000, 1, 77777, 0], np.int32)
    got = orc.emblookup(ids, table)
    assert got.shape == (ids.size, orc.HIDDEN)
    assert np.array_equal(got, table[ids])
    assert not np.array_equal(got[0], got[1])


# ---------------------------------------------------------------- rope tables
def test_rope_tables_match_hf_llama3():
    g = np.load(GOLD / "rope_llama3_hf.npz")
    cos, sin = orc.rope_tables()
    # Frequencies: angle at position 1 recovers freq_i; HF computes them in fp32.
    freqs = np.arctan2(sin[1].astype(np.float64), cos[1].astype(np.float64))
    np.testing.assert_allclose(freqs, g["inv_freq"].astype(np.float64), rtol=2e-6, atol=1e-12)
    # Tables at sampled positions within the reference test's 1e-3 (test_rope.cu:56-59)
    pos = g["positions"]
    assert np.abs(cos[pos] - g["cos"]).max() < 1e-3
    assert np.abs(sin[pos] - g["sin"]).max() < 1e-3
    assert np.all(cos[0] == 1.0) and np.all(sin[0] == 0.0)
    np.testing.assert_allclose(cos.astype(np.float64) ** 2 + sin.astype(np.float64) ** 2, 1.0, atol=1e-6)


def test_rope_tables_past_8192_positions():
    """Rows past the reference's 8192 (the paged paths run to 131072 positions).  Closed form:
    each row is cos / sin of the fp32 product position * freq_i (numpy's float32 multiply is the
    same IEEE product).  Against HF's own LlamaRotaryEmbedding forward (fixture): the only
    difference is the inverse frequencies' rounding (the reference rounds a double, HF computes
    them in fp32), so |ours - HF| <= pos * |freq_i - inv_freq_i| + ulp(pos * freq_i) per element,
    a bound a wrong position, frequency or pairing exceeds."""
    g = np.load(GOLD / "rope_llama3_hf_long.npz")
    h = np.load(GOLD / "rope_llama3_hf.npz")
    cos, sin = orc.rope_tables(orc.LONGCTX)
    freqs = orc.rope_freqs()
    np.testing.assert_allclose(freqs, h["inv_freq"], rtol=4e-7)
    short_cos, short_sin = orc.rope_tables()
    assert np.array_equal(cos[:8192], short_cos) and np.array_equal(sin[:8192], short_sin)
    pos = g["positions"]
    ang = (pos.astype(np.float32)[:, None] * freqs[None, :]).astype(np.float64)
    np.testing.assert_allclose(cos[pos], np.cos(ang), rtol=0, atol=2e-7)
    np.testing.assert_allclose(sin[pos], np.sin(ang), rtol=0, atol=2e-7)
    p64 = pos.astype(np.float64)[:, None]
    dfreq = np.abs(freqs.astype(np.float64) - h["inv_freq"].astype(np.float64))[None, :]
    prod = np.abs(ang)
    ulp = np.spacing(prod.astype(np.float32)).astype(np.float64)
    bound = p64 * dfreq + ulp + 1e-6
    assert (np.abs(cos[pos] - g["cos"]) <= bound).all()
    assert (np.abs(sin[pos] - g["sin"]) <= bound).all()
    np.testing.assert_allclose(cos[pos].astype(np.float64) ** 2 + sin[pos].astype(np.float64) ** 2,
                               1.0, atol=1e-6)


# ---------------------------------------------------------------- rmsnorm
def test_rmsnorm_matches_hf_fixture():
    g = np.load(GOLD / "rmsnorm_hf.npz")
    y = orc.rmsnorm(g["x"], g["w"])
    d = ulp_diff(y, g["y"])
    assert d.max() <= 1 and (d == 0).mean() > 0.99


def test_rmsnorm_closed_form_constant_row():
    # x = c everywhere -> mean square c^2 -> output ~ sign(c) * w
    x = orc.f32_to_bf16(np.full((1, 4096), 3.0, np.float32))
    w = orc.f32_to_bf16(np.linspace(0.5, 1.5, 4096).astype(np.float32))
    y = orc.bf16_to_f32(orc.rmsnorm(x, w))
    np.testing.assert_allclose(y[0], orc.bf16_to_f32(w), rtol=8e-3)


# ---------------------------------------------------------------- matmul
@pytest.mark.parametrize("m,k,n", [(1, 512, 96), (3, 4096, 64), (5, 1024, 33)])
def test_matmul_matches_float64_bruteforce(m, k, n):
    x = orc.synthetic((m, k), 1, 100 + m, 0.0, 1.0)
    w = orc.synthetic((n, k), 1, 200 + n, 0.0, 0.02)
    ref = orc.bf16_to_f32(x).astype(np.float64) @ orc.bf16_to_f32(w).astype(np.float64).T
    y32 = orc.matmul(x, w, out_f32=True)
    np.testing.assert_allclose(y32, ref, rtol=1e-5, atol=1e-5)
    y = orc.matmul(x, w)
    assert ulp_diff(y, orc.f32_to_bf16(ref.astype(np.float32))).max() <= 1
    # a transposed operand would not match: row j of W must pair with column j of Y
    assert not np.allclose(y32[:, 0], (orc.bf16_to_f32(x) @ orc.bf16_to_f32(w)[::-1].T)[:, 0])


def test_matmul_matches_torch_linear_bf16():
    x = orc.synthetic((4, 4096), 2, 1, 0.0, 1.0)
    w = orc.synthetic((256, 4096), 2, 2, 0.0, 0.02)
    ref = torch.nn.functional.linear(t_bf16(x).float(), t_bf16(w).float())
    d = ulp_diff(orc.matmul(x, w), bits(ref))
    assert d.max() <= 1


# ---------------------------------------------------------------- swiglu / residual
def test_swiglu_matches_torch_silu():
    g = orc.synthetic((4, 14336), 3, 1, 0.0, 2.0)
    u = orc.synthetic((4, 14336), 3, 2, 0.0, 2.0)
    ref = torch.nn.functional.silu(t_bf16(g).float()) * t_bf16(u).float()
    assert ulp_diff(orc.swiglu(g, u), bits(ref)).max() <= 1


def test_residual_add_exact():
    x = orc.synthetic((8, 4096), 4, 1, 0.0, 1.0)
    d = orc.synthetic((8, 4096), 4, 2, 0.0, 1.0)
    ref = bits(t_bf16(x).float() + t_bf16(d).float())
    assert np.array_equal(orc.residual_add(x, d), ref)


# ---------------------------------------------------------------- rope
def test_apply_rope_matches_hf_and_preserves_pair_norms():
    from transformers.models.llama.modeling_llama import apply_rotary_pos_emb
    cos, sin = orc.rope_tables()
    S, start = 16, 2040
    q = orc.synthetic((32, S, 128), 5, 1, 0.0, 1.0)
    k = orc.synthetic((8, S, 128), 5, 2, 0.0, 1.0)
    qo = orc.apply_rope(q, start, 32, S, S, cos, sin)
    ko = orc.apply_rope(k, start, 8, S, S, cos, sin)
    c = torch.from_numpy(cos[start:start + S])
    s = torch.from_numpy(sin[start:start + S])
    cf = torch.cat([c, c], -1)[None, None]
    sf = torch.cat([s, s], -1)[None, None]
    qr, kr = apply_rotary_pos_emb(t_bf16(q).float()[None], t_bf16(k).float()[None], cf, sf)
    assert ulp_diff(qo, bits(qr[0])).max() <= 1
    assert ulp_diff(ko, bits(kr[0])).max() <= 1
    qf, of = orc.bf16_to_f32(q), orc.bf16_to_f32(qo)
    n0 = qf[..., :64] ** 2 + qf[..., 64:] ** 2
    n1 = of[..., :64] ** 2 + of[..., 64:] ** 2
    np.testing.assert_allclose(n1, n0, rtol=2e-2, atol=1e-3)


def test_apply_rope_cache_stride():
    cos, sin = orc.rope_tables()
    plane = orc.synthetic((2, 8192, 128), 6, 1, 0.0, 1.0)
    out = orc.apply_rope(plane, 100, 2, 3, 8192, cos, sin)   # rows 0..2 of each head plane
    assert np.array_equal(out[:, 3:], plane[:, 3:])
    ref = orc.apply_rope(np.ascontiguousarray(plane[:, :3]), 100, 2, 3, 3, cos, sin)
    assert np.array_equal(out[:, :3], ref)


# ---------------------------------------------------------------- softmax
@pytest.mark.parametrize("causal", [True, False])
def test_softmax_matches_torch(causal):
    S = 64
    x = orc.synthetic((4, S, S) if causal else (32, S), 7, 1, 0.0, 3.0)
    y = orc.bf16_to_f32(orc.softmax_scaled(x, S, causal))
    xs = t_bf16(x).float() / np.sqrt(128.0)
    if causal:
        xs = xs + torch.triu(torch.full((S, S), float("-inf")), diagonal=1)
    ref = torch.softmax(xs, dim=-1).numpy()
    np.testing.assert_allclose(y, ref, atol=4e-3, rtol=1e-2)
    np.testing.assert_allclose(y.astype(np.float64).sum(-1), 1.0, atol=2e-2)


# ---------------------------------------------------------------- attention
def test_attention_matches_hf_repeat_kv():
    from transformers.models.llama.modeling_llama import repeat_kv
    ctx, q_start, n_q = 96, 80, 16
    q = orc.synthetic((n_q, 32, 128), 8, 1, 0.0, 1.0)
    kp = orc.synthetic((8, ctx, 128), 8, 2, 0.0, 1.0)
    vp = orc.synthetic((8, ctx, 128), 8, 3, 0.0, 1.0)
    out = orc.bf16_to_f32(orc.attention(q, kp, vp, q_start, ctx))
    qt = t_bf16(q).float().permute(1, 0, 2)[None]                  # [1, 32, n_q, 128]
    kt = repeat_kv(t_bf16(kp).float()[None], 4)                      # [1, 32, ctx, 128]
    vt = repeat_kv(t_bf16(vp).float()[None], 4)
    sc = qt @ kt.transpose(-1, -2) / np.sqrt(128.0)
    pos = torch.arange(n_q)[:, None] + q_start
    sc = sc.masked_fill(torch.arange(ctx)[None, :] > pos, float("-inf"))
    ref = (torch.softmax(sc, -1) @ vt)[0].permute(1, 0, 2).reshape(n_q, 4096).numpy()
    assert_close(out, ref, what="attention vs repeat_kv")


def _attn_scores(q, kp, q_start, ctx, n_q):
    """fp32 scores [32, n_q, ctx] (raw q.k, unscaled) with the causal mask as -inf."""
    from transformers.models.llama.modeling_llama import repeat_kv
    qt = t_bf16(q).float().permute(1, 0, 2)                          # [32, n_q, 128]
    kt = repeat_kv(t_bf16(kp).float()[None], 4)[0]                   # [32, ctx, 128]
    sc = qt @ kt.transpose(-1, -2)
    pos = torch.arange(n_q)[:, None] + q_start
    return sc.masked_fill(torch.arange(ctx)[None, :] > pos, float("-inf"))


def _vrep(vp):
    from transformers.models.llama.modeling_llama import repeat_kv
    return repeat_kv(t_bf16(vp).float()[None], 4)[0]                 # [32, ctx, 128]


def _heads_out(o, n_q):
    return o.permute(1, 0, 2).reshape(n_q, 4096).numpy()


def _assert_rounding_equal(got, ref, sc, vp, n_q, what):
    """Equal up to rare flips of one probability's bf16 rounding: > 99% of elements bit-identical,
    and every element within one ulp of the reference plus 2 x 2^-8 max_t p_t |v_t| (the shift one
    flipped probability causes; the fp32 scores of two implementations differ in the last bits)."""
    p = torch.softmax(sc.double() / np.sqrt(128.0), -1)                       # [32, n_q, ctx]
    flip = _heads_out((p[..., None] * _vrep(vp).double().abs()[:, None]).amax(2), n_q)
    g, w = orc.bf16_to_f32(got).astype(np.float64), orc.bf16_to_f32(ref).astype(np.float64)
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(w), 1e-30))) - 7)
    err = np.abs(g - w)
    assert (err <= ulp + 2.0 ** -7 * flip).all(), f"{what}: worst {err.max():.3e}"
    assert (got == ref).mean() > 0.99, f"{what}: {(got == ref).mean():.4f} exact"


def test_attention_reference_rounding_point_matches_torch():
    """PROB_REFERENCE: softmax in fp32, probabilities stored as bf16 (softmax.cu:105,158), then
    the fp32 A.V product (attn.cu:167-204) rounded to bf16 -- torch's softmax, .to(bfloat16),
    fp32 matmul.  The fp32 mode is measurably further from that reference than the rounded mode
    is, so a mode that skipped the rounding would fail."""
    ctx, q_start, n_q = 160, 130, 24
    q = orc.synthetic((n_q, 32, 128), 81, 1, 0.0, 1.0)
    kp = orc.synthetic((8, ctx, 128), 81, 2, 0.0, 1.0)
    vp = orc.synthetic((8, ctx, 128), 81, 3, 0.0, 1.0)
    sc = _attn_scores(q, kp, q_start, ctx, n_q)
    p = torch.softmax(sc / np.sqrt(128.0), -1).to(torch.bfloat16).float()
    ref = bits(torch.from_numpy(_heads_out(p @ _vrep(vp), n_q)))
    with orc.prob_rounding(orc.PROB_REFERENCE):
        got = orc.attention(q, kp, vp, q_start, ctx)
    exact = orc.attention(q, kp, vp, q_start, ctx)
    _assert_rounding_equal(got, ref, sc, vp, n_q, "reference rounding point")
    assert (exact != ref).sum() > 5 * max(1, (got != ref).sum())


def test_attention_flash_rounding_single_tile_closed_form():
    """PROB_FLASH with every row's keys in one 64-key tile: out = bf16(sum_t p_t v_t * (1 / sum_t
    p_t)), p_t = bf16(exp2((s_t - max s) log2(e) / sqrt(128))) (one max, no rescaling)."""
    ctx, q_start, n_q = 64, 40, 24
    q = orc.synthetic((n_q, 32, 128), 82, 1, 0.0, 1.0)
    kp = orc.synthetic((8, ctx, 128), 82, 2, 0.0, 1.0)
    vp = orc.synthetic((8, ctx, 128), 82, 3, 0.0, 1.0)
    c = np.float32(np.log2(np.e) / np.sqrt(128.0))
    sc = _attn_scores(q, kp, q_start, ctx, n_q)
    e = torch.exp2((sc - sc.amax(-1, keepdim=True)) * c).to(torch.bfloat16).float()
    ref = bits(torch.from_numpy(_heads_out((e @ _vrep(vp)) * (1.0 / e.sum(-1, keepdim=True)), n_q)))
    with orc.prob_rounding(orc.PROB_FLASH):
        got = orc.attention(q, kp, vp, q_start, ctx)
    _assert_rounding_equal(got, ref, sc, vp, n_q, "flash rounding, one tile")


def test_attention_flash_rounding_fixed_max_closed_form():
    """PROB_FLASH over many tiles where key 0 holds every row's maximum score (k_0 = 8 q-ish):
    the running max never moves after the first tile, so the tiled sums equal the one-max closed
    form over all keys -- pins the accumulation across tiles and the causal extent."""
    ctx, q_start, n_q = 300, 260, 16
    q = orc.synthetic((n_q, 32, 128), 83, 1, 0.0, 0.5)
    kp = orc.synthetic((8, ctx, 128), 83, 2, 0.0, 0.2)
    vp = orc.synthetic((8, ctx, 128), 83, 3, 0.0, 1.0)
    # dim 0 of every q row is 4 and key 0 is 3 e_0: its score 12 tops every row (others ~N(0, 1.4))
    q[..., 0] = orc.f32_to_bf16(np.float32([4.0]))[0]
    kp[:, 0] = 0
    kp[:, 0, 0] = orc.f32_to_bf16(np.float32([3.0]))[0]
    c = np.float32(np.log2(np.e) / np.sqrt(128.0))
    sc = _attn_scores(q, kp, q_start, ctx, n_q)
    assert torch.equal(sc.amax(-1), sc[..., 0]), "key 0 must hold every row's maximum"
    e = torch.exp2((sc - sc[..., :1]) * c).to(torch.bfloat16).float()
    ref = bits(torch.from_numpy(_heads_out((e @ _vrep(vp)) * (1.0 / e.sum(-1, keepdim=True)), n_q)))
    with orc.prob_rounding(orc.PROB_FLASH):
        got = orc.attention(q, kp, vp, q_start, ctx)
    _assert_rounding_equal(got, ref, sc, vp, n_q, "flash rounding, fixed max")


def test_attention_flash_rounding_within_its_error_bound():
    """PROB_FLASH with growing maxima (rescaling on most tiles) stays within the bound that bf16
    probabilities allow around the exact (fp32) attention: each p_t carries a relative error
    <= 2^-9 in numerator and denominator alike, so |out - exact| <= 2^-8 sum p|v| / sum p plus
    the two outputs' bf16 roundings; and it differs from the fp32 mode (the rounding is on)."""
    ctx, q_start, n_q = 400, 330, 16
    q = orc.synthetic((n_q, 32, 128), 84, 1, 0.0, 1.0)
    kp = orc.synthetic((8, ctx, 128), 84, 2, 0.0, 1.0)
    ramp = np.linspace(0.5, 3.0, ctx, dtype=np.float32)[None, :, None]   # scores grow with t
    kp = orc.f32_to_bf16(orc.bf16_to_f32(kp) * ramp)
    vp = orc.synthetic((8, ctx, 128), 84, 3, 0.0, 1.0)
    sc = _attn_scores(q, kp, q_start, ctx, n_q).double() / np.sqrt(128.0)
    p = torch.softmax(sc, -1)
    va = _vrep(vp).double()
    bound = _heads_out(2.0 ** -8 * (p @ va.abs()), n_q)
    exact64 = _heads_out(p @ va, n_q)
    with orc.prob_rounding(orc.PROB_FLASH):
        got = orc.bf16_to_f32(orc.attention(q, kp, vp, q_start, ctx)).astype(np.float64)
    fp32 = orc.attention(q, kp, vp, q_start, ctx)
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(exact64), 1e-30))) - 7)
    assert (np.abs(got - exact64) <= bound + ulp).all()
    assert (orc.f32_to_bf16(got.astype(np.float32)) != fp32).mean() > 0.05


# ---------------------------------------------------------------- decoder layer
def _hf_layer(w):
    from transformers import LlamaConfig
    from transformers.models.llama.modeling_llama import LlamaDecoderLayer
    cfg = LlamaConfig(hidden_size=4096, intermediate_size=14336, num_attention_heads=32,
                      num_key_value_heads=8, head_dim=128, rms_norm_eps=1e-5,
                      attention_bias=False, mlp_bias=False, attn_implementation="eager")
    layer = LlamaDecoderLayer(cfg, layer_idx=0).float().eval()
    f = lambda a: t_bf16(a).float()
    with torch.no_grad():
        layer.input_layernorm.weight.copy_(f(w["input_layernorm"]))
        layer.post_attention_layernorm.weight.copy_(f(w["post_attention_layernorm"]))
        layer.self_attn.q_proj.weight.copy_(f(w["w_q"]))
        layer.self_attn.k_proj.weight.copy_(f(w["w_k"]))
        layer.self_attn.v_proj.weight.copy_(f(w["w_v"]))
        layer.self_attn.o_proj.weight.copy_(f(w["w_o"]))
        layer.mlp.gate_proj.weight.copy_(f(w["w_gate"]))
        layer.mlp.up_proj.weight.copy_(f(w["w_up"]))
        layer.mlp.down_proj.weight.copy_(f(w["w_down"]))
    return layer


def test_decoder_layer_matches_hf_llama_layer():
    """Layer order, residuals, GQA and RoPE pairing against HF LlamaDecoderLayer (fp32)."""
    S = 6
    w = orc.layer_weights(seed=21, layer=0)
    x = orc.synthetic((S, 4096), 21, 999, 0.0, 1.0)
    cos, sin = orc.rope_tables()
    kp = np.zeros((8, 16, 128), np.uint16)
    vp = np.zeros((8, 16, 128), np.uint16)
    xo = x.copy()
    orc.decoder_layer(xo, w, 0, cos, sin, kp, vp, 16)
    layer = _hf_layer(w)
    c = torch.from_numpy(cos[:S])
    s = torch.from_numpy(sin[:S])
    pe = (torch.cat([c, c], -1)[None], torch.cat([s, s], -1)[None])
    mask = torch.triu(torch.full((S, S), float("-inf")), 1)[None, None]
    with torch.no_grad():
        ref = layer(t_bf16(x).float()[None], attention_mask=mask, position_embeddings=pe)
    ref = ref[0] if isinstance(ref, tuple) else ref
    got, want, xin = orc.bf16_to_f32(xo), ref[0].numpy(), orc.bf16_to_f32(x)
    err = np.abs(got - want)
    assert err.max() < 1e-2 * (1 + np.abs(want).max())
    # the layer's own contribution (want - x) is matched to bf16 rounding level
    # (~2^-7 per rounding); a wrong op order, sign or pairing is O(1) here
    assert err.mean() / np.abs(want - xin).mean() < 1.5e-2


def test_decoder_layer_prefill_equals_stepwise_decode():
    """Causality: rows of one S-row pass == the same rows fed one position at a time."""
    S = 5
    w = orc.layer_weights(seed=22, layer=3)
    x = orc.synthetic((S, 4096), 22, 1, 0.0, 1.0)
    cos, sin = orc.rope_tables()
    kp1 = np.zeros((8, 8, 128), np.uint16)
    vp1 = np.zeros_like(kp1)
    xa = x.copy()
    orc.decoder_layer(xa, w, 0, cos, sin, kp1, vp1, 8)
    kp2 = np.zeros_like(kp1)
    vp2 = np.zeros_like(kp1)
    xb = x.copy()
    for t in range(S):
        row = np.ascontiguousarray(xb[t:t + 1])
        orc.decoder_layer(row, w, t, cos, sin, kp2, vp2, 8)
        xb[t] = row[0]
    assert np.array_equal(kp1, kp2) and np.array_equal(vp1, vp2)
    assert np.array_equal(xa, xb)


def test_ffn_matches_hf_llama_mlp():
    from transformers import LlamaConfig
    from transformers.models.llama.modeling_llama import LlamaMLP
    w = orc.layer_weights(seed=23, layer=1)
    x = orc.synthetic((3, 4096), 23, 1, 0.0, 1.0)
    mlp = LlamaMLP(LlamaConfig(hidden_size=4096, intermediate_size=14336)).float()
    with torch.no_grad():
        mlp.gate_proj.weight.copy_(t_bf16(w["w_gate"]).float())
        mlp.up_proj.weight.copy_(t_bf16(w["w_up"]).float())
        mlp.down_proj.weight.copy_(t_bf16(w["w_down"]).float())
        ref = mlp(t_bf16(x).float()).numpy()
    got = orc.bf16_to_f32(orc.ffn(x, w["w_gate"], w["w_up"], w["w_down"]))
    assert_close(got, ref, what="ffn vs LlamaMLP")


# ---------------------------------------------------------------- sampling
def test_argmax_matches_torch_fixture():
    g = np.load(GOLD / "argmax_torch.npz")
    for row, want in zip(g["logits"], g["expect"]):
        assert orc.argmax(row) == int(want)


def test_top_p_kept_set_matches_hf_warper():
    g = np.load(GOLD / "top_p_hf.npz")
    T, p = float(g["temperature"]), float(g["top_p"])
    for r, logits in enumerate(g["logits"]):
        kept_hf = np.unpackbits(g["kept"][r])[: logits.size].astype(bool)
        tok, info = orc.top_p(logits, T, p, seed=3, row=r, step=0)
        # the oracle's kept set is {l >= cut}; recover it from the sampled cut point
        l = logits / np.float32(T)
        cut = l[kept_hf].min()
        assert kept_hf[tok], "sampled token must be inside HF's nucleus"
        assert np.array_equal(l >= cut, kept_hf)
        assert info["lo"] <= info["t"] < info["hi"] <= info["z_kept"]


def test_top_p_minimal_prefix_bruteforce():
    rng = np.random.default_rng(4)
    for trial in range(20):
        logits = (rng.standard_normal(257) * rng.uniform(0.2, 4)).astype(np.float32)
        T, p = 0.7, float(rng.uniform(0.05, 0.99))
        seen = set()
        for step in range(40):
            tok, info = orc.top_p(logits, T, p, seed=trial, row=0, step=step)
            seen.add(tok)
        # kept set = minimal prefix (descending prob) whose mass reaches p
        pr = np.exp((logits / np.float32(T)).astype(np.float64))
        order = np.argsort(-pr, kind="stable")
        cum = np.cumsum(pr[order]) / pr.sum()
        k = int(np.searchsorted(cum, p - 1e-9)) + 1
        kept = set(order[:k].tolist())
        assert seen <= kept
    # p -> tiny keeps only the argmax
    tok, _ = orc.top_p(logits, 0.7, 1e-6, seed=1, row=0, step=0)
    assert tok == int(np.argmax(logits))


def test_top_p_sample_frequencies_follow_probabilities():
    logits = np.array([2.0, 1.0, 0.5, 0.0, -1.0, -3.0], np.float32)
    T, p = 0.7, 0.9
    counts = np.zeros(6)
    for step in range(4000):
        tok, _ = orc.top_p(logits, T, p, seed=9, row=0, step=step)
        counts[tok] += 1
    pr = np.exp(logits / T)
    pr /= pr.sum()
    order = np.argsort(-pr)
    cum = np.cumsum(pr[order])
    k = int(np.searchsorted(cum, p)) + 1
    kept = order[:k]
    want = np.zeros(6)
    want[kept] = pr[kept] / pr[kept].sum()
    np.testing.assert_allclose(counts / counts.sum(), want, atol=0.03)
    assert counts[[i for i in range(6) if i not in kept]].sum() == 0
