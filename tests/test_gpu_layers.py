"""Per-layer parity of the prefill and batched-decode paths on the full random-init
Llama-3.1-8B, through the C-ABI (ie_decoder_layer_prefill, ie_decoder_layer_batched).

Two bars, as test_gpu_model holds the batch-1 decode to:
  * integration: ie_prefill / ie_decode_step_batched equal the embedding followed by the 32
    per-layer calls, bit for bit (residual rows, K/V cache, prefill logits; ie_prefill's last
    layer is ie_decoder_layer_prefill_last_row, which computes the last row's output only);
  * per layer: a layer fed the GPU's own input matches the oracle's layer to 1e-2
    (tests/tolerance.py), so errors cannot hide in the accumulation across 32 layers.
The prefill rows are checked at S = 2048 (the 8-wave flash-attention form and the M = 2048
MFMA GEMMs) with the oracle's attention over the GPU's K/V rows of earlier positions and its
probabilities rounded as the MFMA attention rounds them (oracle.PROB_FLASH).
"""
import ctypes as C

import numpy as np
import pytest
import torch

import oracle as orc
from conftest import MODEL_SEED
from gpu_util import (assert_bf16_close, assert_delta_close, check_token, e2e_tol, host,
                      report_close, say)
from tolerance import assert_close

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(900)]
SEED = MODEL_SEED
V = 128256


def _ptr(t: torch.Tensor) -> C.c_void_p:
    return C.c_void_p(t.data_ptr())


def _check_layer_row(l, x_in, x_out, kv_got, w, pos, planes, cos, sin, what):
    """The oracle's layer l on one row at position pos over planes [2][8][pos+1][128] (rows
    < pos set): its output row against x_out, its new K/V row against kv_got [2][8][128]."""
    x = x_in.reshape(1, 4096).copy()
    orc.decoder_layer(x, w, pos, cos, sin, planes[0], planes[1], pos + 1)
    report_close(orc.bf16_to_f32(x_out), orc.bf16_to_f32(x[0]), what=f"{what} output")
    assert_delta_close(x_in, x_out, x[0], what=f"{what} delta")
    assert_bf16_close(kv_got, planes[:, :, pos], what=f"{what} kv row", outlier_frac=2e-3)


# ---------------------------------------------------------------- prefill, S = 2048
PREFILL_LAYERS = (0, 1, 15, 31)
PREFILL_ROWS = (0, 63, 64, 1000, 2047)


def _last_layer_and_head(hip, c, model, b, S):
    """Layer 31 of a chained prefill (b holds layers 0..30's output) as ie_prefill runs it
    (ie_decoder_layer_prefill_last_row), then the final norm + lm_head of the last row; returns
    (rows, logits, the layer's input rows).  b.data is left holding layer 31's input."""
    x31 = b.data.clone()
    hip.check(hip.lib.ie_decoder_layer_prefill_last_row(c.handle, model.ref(), 31, S, _ptr(b.data),
                                                        _ptr(b.aux), _ptr(b.attn),
                                                        _ptr(b.workspace), _ptr(b.kv)))
    logits = torch.zeros(V, dtype=torch.float32, device="cuda")
    hip.check(hip.lib.ie_final_norm_lm_head(c.handle, 1, _ptr(b.data[S - 1]),
                                            _ptr(model.view(None, "final_norm")),
                                            _ptr(model.view(None, "lm_head")), _ptr(logits)))
    torch.cuda.synchronize()
    rows = host(b.data[:S].view(torch.int16)).copy()
    b.data.copy_(x31)
    return rows, host(logits).copy(), x31


def test_prefill_2048_layers(hip, model, oracle_model, noise_floor):
    """ie_prefill(2048) equals ie_emblookup + 31 x ie_decoder_layer_prefill +
    ie_decoder_layer_prefill_last_row + the last row's final norm / lm_head bit for bit; layers
    0, 1, 15 and 31 (the full layer) at rows 0, 63, 64, 1000 and 2047 against the oracle fed the
    same input rows and the GPU's K/V rows of earlier positions; the last-row-only layer 31
    against the full one (its K/V rows bit for bit, its last row and the logits within the
    tolerance of two summation orders)."""
    from infengine_amd.engine import Context, Request
    S = 2048
    ids = np.random.default_rng(2048).integers(0, V, S).astype(np.int32)
    c = Context(0, graph=False)
    say(f"ie_prefill S={S}")
    req = Request(c, model, max_seq_len=S + 8)
    req.tokens[:S] = torch.from_numpy(ids).cuda()
    tok = req.prefill(S)
    want_x = host(req.data[:S].view(torch.int16)).copy()
    want_logits = host(req.logits).copy()
    want_kv = req.kv.clone()
    del req

    say("emblookup + 32 ie_decoder_layer_prefill calls")
    b = Request(c, model, max_seq_len=S + 8)
    b.tokens[:S] = torch.from_numpy(ids).cuda()
    hip.check(hip.lib.ie_emblookup(S, _ptr(b.tokens), _ptr(model.view(None, "emb_lookup")),
                                   _ptr(b.data), c.stream_ptr))
    kv6 = b.kv.view(torch.int16).view(32, 2, 8, 8192, 128)
    saved = {}
    for l in range(32):
        x_in = host(b.data[list(PREFILL_ROWS)].view(torch.int16)).copy() if l in PREFILL_LAYERS else None
        if l == 31:
            say("layer 31 as ie_prefill runs it (last row only)")
            rows, logits, _ = _last_layer_and_head(hip, c, model, b, S)
            assert np.array_equal(rows, want_x)
            assert np.array_equal(logits, want_logits) and tok == int(np.argmax(want_logits))
            assert torch.equal(b.kv, want_kv)
            say("layer 31 over all rows")
        hip.check(hip.lib.ie_decoder_layer_prefill(c.handle, model.ref(), l, S, _ptr(b.data),
                                                   _ptr(b.aux), _ptr(b.attn), _ptr(b.workspace),
                                                   _ptr(b.kv)))
        if l in PREFILL_LAYERS:
            torch.cuda.synchronize()
            saved[l] = (x_in, host(b.data[list(PREFILL_ROWS)].view(torch.int16)).copy(),
                        host(kv6[l, :, :, :S].contiguous()))
    full_logits = torch.zeros(V, dtype=torch.float32, device="cuda")
    hip.check(hip.lib.ie_final_norm_lm_head(c.handle, 1, _ptr(b.data[S - 1]),
                                            _ptr(model.view(None, "final_norm")),
                                            _ptr(model.view(None, "lm_head")), _ptr(full_logits)))
    torch.cuda.synchronize()
    assert torch.equal(b.kv, want_kv)   # the full layer 31 writes the same K/V rows
    # the last row through the decode kernels against the full layer's GEMMs and flash attention
    report_close(orc.bf16_to_f32(want_x[S - 1]),
                 orc.bf16_to_f32(host(b.data[S - 1].view(torch.int16))),
                 what="layer 31 last row: last-row path vs full layer")
    assert_close(want_logits, host(full_logits), tol=e2e_tol(noise_floor),
                 what="logits: last-row layer 31 vs full layer 31")
    check_token(tok, host(full_logits), want_logits, noise_floor)
    del b, want_kv
    c.close()

    cos, sin = oracle_model.cos, oracle_model.sin
    for l in PREFILL_LAYERS:
        say(f"oracle: prefill layer {l} at rows {PREFILL_ROWS}")
        w = orc.layer_weights(SEED, l)
        x_in, x_out, gkv = saved[l]
        for i, p in enumerate(PREFILL_ROWS):
            planes = np.zeros((2, 8, p + 1, 128), np.uint16)
            planes[:, :, :p] = gkv[:, :, :p]
            with orc.prob_rounding(orc.PROB_FLASH):
                _check_layer_row(l, x_in[i], x_out[i], gkv[:, :, p], w, p, planes, cos, sin,
                                 f"prefill layer {l} row {p}")


@pytest.mark.parametrize("S", [100, 512])
def test_prefill_split_k_equals_chained_layers(hip, model, S):
    """At prompt lengths whose projections split K, ie_prefill runs the residual reductions
    together with the RMSNorm that follows (the down projection's with the next layer's input
    norm) and the QKV reduction with RoPE and the K/V scatter; the per-layer entry point runs the
    standalone RMSNorm for its input.  Residual rows, K/V cache and logits must agree bit for
    bit."""
    from infengine_amd.engine import Context, Request
    ids = np.random.default_rng(S).integers(0, V, S).astype(np.int32)
    c = Context(0, graph=False)
    say(f"ie_prefill S={S}")
    req = Request(c, model, max_seq_len=S + 8)
    req.tokens[:S] = torch.from_numpy(ids).cuda()
    tok = req.prefill(S)
    want_x = host(req.data[:S].view(torch.int16)).copy()
    want_logits = host(req.logits).copy()
    want_kv = req.kv.clone()
    del req
    say(f"emblookup + 32 ie_decoder_layer_prefill calls, S={S}")
    b = Request(c, model, max_seq_len=S + 8)
    b.tokens[:S] = torch.from_numpy(ids).cuda()
    hip.check(hip.lib.ie_emblookup(S, _ptr(b.tokens), _ptr(model.view(None, "emb_lookup")),
                                   _ptr(b.data), c.stream_ptr))
    for l in range(31):
        hip.check(hip.lib.ie_decoder_layer_prefill(c.handle, model.ref(), l, S, _ptr(b.data),
                                                   _ptr(b.aux), _ptr(b.attn), _ptr(b.workspace),
                                                   _ptr(b.kv)))
    rows, logits, _ = _last_layer_and_head(hip, c, model, b, S)
    assert np.array_equal(rows, want_x)
    assert np.array_equal(logits, want_logits) and tok == int(np.argmax(want_logits))
    assert torch.equal(b.kv, want_kv)
    del b, want_kv
    c.close()


# ---------------------------------------------------------------- batched decode, B = 16
def test_batched16_layers(hip, model, oracle_model):
    """ie_decode_step_batched with 16 sequences at staggered contexts equals ie_emblookup + 32 x
    ie_decoder_layer_batched bit for bit (residual rows and new K/V rows); every one of the 32
    layers, fed the GPU's rows, matches the oracle's layer for all 16 sequences."""
    from infengine_amd.engine import Context
    B = 16
    lens = [33 + 61 * b for b in range(B)]            # 33 .. 948
    c = Context(0, graph=False)
    say(f"decode_step_batched B={B} lens {lens[0]}..{lens[-1]}")
    kvs = torch.zeros(B * hip.lib.ie_kv_cache_size() // 2, dtype=torch.int16, device="cuda")
    kv7 = kvs.view(B, 32, 2, 8, 8192, 128)
    toks = torch.zeros(B, 8192, dtype=torch.int32, device="cuda")
    priors, tk = [], []
    for b in range(B):
        prior = orc.synthetic((32, 2, 8, lens[b] - 1, 128), SEED, 5000 + b, 0.0, 1.0)
        kv7[b, :, :, :, :lens[b] - 1] = torch.from_numpy(prior.view(np.int16)).cuda()
        tk.append(1231 * (b + 3) + 7)
        toks[b, lens[b] - 1] = tk[-1]
        priors.append(prior)
    data = torch.zeros(B, 4096, dtype=torch.bfloat16, device="cuda")
    attn = torch.zeros_like(data)
    logits = torch.zeros(B, V, dtype=torch.float32, device="cuda")
    out = torch.zeros(B, dtype=torch.int32, device="cuda")
    ws = torch.zeros(hip.lib.ie_batch_workspace_size(B), dtype=torch.uint8, device="cuda")
    seq = (C.c_int * B)(*lens)
    th = (C.c_int * B)()
    hip.check(hip.lib.ie_decode_step_batched(c.handle, model.ref(), B, seq, _ptr(toks), _ptr(data),
                                             _ptr(attn), _ptr(logits), _ptr(out), th, _ptr(ws),
                                             _ptr(kvs)))
    torch.cuda.synchronize()
    want_x = host(data.view(torch.int16)).copy()
    want_rows = np.stack([host(kv7[b, :, :, :, lens[b] - 1].contiguous()) for b in range(B)])
    for b in range(B):
        kv7[b, :, :, :, lens[b] - 1] = 0

    say("emblookup + 32 ie_decoder_layer_batched calls")
    ids = torch.tensor(tk, dtype=torch.int32, device="cuda")
    hip.check(hip.lib.ie_emblookup(B, _ptr(ids), _ptr(model.view(None, "emb_lookup")), _ptr(data),
                                   c.stream_ptr))
    xs = [host(data.view(torch.int16)).copy()]
    for l in range(32):
        hip.check(hip.lib.ie_decoder_layer_batched(c.handle, model.ref(), l, B, seq, _ptr(data),
                                                   _ptr(attn), _ptr(ws), _ptr(kvs)))
        xs.append(host(data.view(torch.int16)).copy())
    got_rows = np.stack([host(kv7[b, :, :, :, lens[b] - 1].contiguous()) for b in range(B)])
    del kvs, kv7
    c.close()
    assert np.array_equal(xs[-1], want_x)
    assert np.array_equal(got_rows, want_rows)

    cos, sin = oracle_model.cos, oracle_model.sin
    for l in range(32):
        say(f"oracle: batched layer {l}, 16 rows")
        w = orc.layer_weights(SEED, l)
        for b in range(B):
            p = lens[b] - 1
            planes = np.zeros((2, 8, p + 1, 128), np.uint16)
            planes[:, :, :p] = priors[b][l]
            _check_layer_row(l, xs[l][b], xs[l + 1][b], got_rows[b, l], w, p, planes, cos, sin,
                             f"batched layer {l} row {b}")
