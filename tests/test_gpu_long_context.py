"""Long context past the reference's static 8192 positions, on the paged KV paths (pages of 64
positions, block tables), through the C-ABI, against the CPU oracle and a PyTorch fp32
attention reference.  The reference's cache and RoPE tables stop at 8192 (config.h:7,
attn.cu:304-307, rope.cu:68-103); here the paged entry points run to IE_MAX_LONG_CONTEXT
(131072, Llama-3.1's max_position_embeddings) with the RoPE formula continued.

Bars: RoPE tables bit-identical to the oracle's; the attention core within tests/tolerance.py
of fp32 torch; full-model logits within the end-to-end tolerance of test_gpu_model (2x the
stack's summation-order noise floor), tokens equal to the oracle's argmax outside that noise,
K/V rows of layer 0 to bf16 rounding and of layer 1 (one layer deep, the oracle rounding the
attention probabilities as the MFMA attention does) to 1e-2.
"""
import ctypes as C
import math

import numpy as np
import pytest
import torch

import oracle as orc
from conftest import MODEL_SEED
from gpu_util import assert_bf16_close, check_token, dev, e2e_tol, host, report_close, say
from tolerance import TOL, assert_close

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(900)]
SEED = MODEL_SEED
V = 128256
PAGE_POS = 64


def _ptr(t: torch.Tensor) -> C.c_void_p:
    return C.c_void_p(t.data_ptr())


def _pool(hip, n_pages: int) -> torch.Tensor:
    """A zeroed page pool viewed [page][layer][K|V][kv head][64][128] (int16 = bf16 bits)."""
    assert hip.lib.ie_kv_page_size() == 32 * 2 * 8 * PAGE_POS * 128 * 2
    return torch.zeros(n_pages, 32, 2, 8, PAGE_POS, 128, dtype=torch.int16, device="cuda")


def _rotate_heads(k_rows: np.ndarray, start_pos: int, cos, sin) -> np.ndarray:
    S = k_rows.shape[0]
    heads = k_rows.shape[1] // 128
    kt = np.ascontiguousarray(k_rows.reshape(S, heads, 128).transpose(1, 0, 2))
    return orc.apply_rope(kt, start_pos, heads, S, S, cos, sin)


def test_rope_tables_on_device_equal_oracle(hip, model):
    """All 131072 rows of the model's RoPE tables, bit for bit."""
    from infengine_amd.engine import device_view
    say("RoPE tables [131072][64] vs the oracle's")
    c, s = orc.rope_tables(orc.LONGCTX)
    gc = host(device_view(model.s.rope.cos, (orc.LONGCTX, 64), torch.float32))
    gs = host(device_view(model.s.rope.sin, (orc.LONGCTX, 64), torch.float32))
    assert np.array_equal(gc.view(np.uint32), c.view(np.uint32))
    assert np.array_equal(gs.view(np.uint32), s.view(np.uint32))


def _attn_reference(q, k, v, start_pos):
    """q [S][32][128], k/v [8][n][128] -> [S][32][128] fp32 (causal, scale 1/sqrt(128))."""
    S = q.shape[0]
    n = start_pos + S
    out = torch.empty(S, 32, 128, dtype=torch.float32, device="cuda")
    pos = torch.arange(S, device="cuda")[:, None] + start_pos
    masked = torch.arange(n, device="cuda")[None, :] > pos
    for h in range(32):
        s = torch.matmul(q[:, h].float(), k[h // 4, :n].float().t().contiguous()) / math.sqrt(128.0)
        out[:, h] = torch.matmul(torch.softmax(s.masked_fill(masked, float("-inf")), dim=-1),
                                 v[h // 4, :n].float())
    return out


# start positions past 8192, a chunk that crosses it, the 16384 mark, and the last rows of the
# 131072-position limit (2048 pages of 64)
@pytest.mark.parametrize("S,start_pos", [(300, 9000), (1100, 7800), (64, 16371), (2048, 14336),
                                         (2600, 9000), (64, 131000)])
def test_attn_prefill_core_paged_long(hip, ctx, S, start_pos):
    say(f"attn_prefill_core_paged S={S} start_pos={start_pos}")
    n = start_pos + S
    g = torch.Generator(device="cuda").manual_seed(n)
    q = torch.randn(S, 32, 128, generator=g, device="cuda").to(torch.bfloat16)
    k = torch.randn(8, n, 128, generator=g, device="cuda").to(torch.bfloat16)
    v = torch.randn(8, n, 128, generator=g, device="cuda").to(torch.bfloat16)
    nblk = (n + PAGE_POS - 1) // PAGE_POS
    n_pages = nblk + 5
    order = torch.from_numpy(np.random.default_rng(n).permutation(n_pages)[:nblk].astype(np.int32))
    pool = _pool(hip, n_pages)
    layer = 5
    for i in range(nblk):
        rows = min(PAGE_POS, n - PAGE_POS * i)
        pg = int(order[i])
        pool[pg, layer, 0, :, :rows] = k[:, PAGE_POS * i:PAGE_POS * i + rows].view(torch.int16)
        pool[pg, layer, 1, :, :rows] = v[:, PAGE_POS * i:PAGE_POS * i + rows].view(torch.int16)
        # the rest of the last page holds large finite values: the kernel must not read them
        pool[pg, layer, :, :, rows:] = torch.tensor(3.0e4, dtype=torch.bfloat16).view(torch.int16)
    table = order.cuda()
    out = torch.empty(S, 32 * 128, dtype=torch.bfloat16, device="cuda")
    hip.check(hip.lib.ie_attn_prefill_core_paged(ctx.handle, S, start_pos, _ptr(q), _ptr(pool),
                                                 n_pages, _ptr(table), layer, _ptr(out)))
    torch.cuda.synchronize()
    want = _attn_reference(q, k, v, start_pos)
    assert_close(out.float().view(S, 32, 128).cpu().numpy(), want.cpu().numpy(),
                 what=f"paged attention core S={S} start={start_pos}")


def _prior_into_pages(pool, prior, table_row):
    """K/V rows 0..n-1 of every layer ([32, 2, 8, n, 128] uint16) into a sequence's pages."""
    n = prior.shape[3]
    t = dev(prior)
    for i in range((n + PAGE_POS - 1) // PAGE_POS):
        rows = min(PAGE_POS, n - PAGE_POS * i)
        pool[int(table_row[i]), :, :, :, :rows] = t[:, :, :, PAGE_POS * i:PAGE_POS * i + rows]


def test_long_decode_batched_paged_vs_oracle(hip, model, oracle_model, noise_floor):
    """ie_decode_step_batched_paged with two sequences at 9001 and 66001 positions of cached
    context (split + merge attention over 141 and 1032 pages, the second past 65536 positions):
    logits of each row against the oracle's decode of that sequence, tokens against its argmax,
    the new layer-0 K/V rows against the oracle's."""
    from infengine_amd.engine import Context
    lens = [9001, 66001]
    B = len(lens)
    say(f"decode_step_batched_paged lens={lens}")
    nblk = [(n + PAGE_POS - 1) // PAGE_POS for n in lens]
    stride = max(nblk) + 1
    n_pages = sum(nblk) + 4
    order = np.random.default_rng(99).permutation(n_pages).astype(np.int32)
    table = np.full((B, stride), -1, np.int32)
    k = 0
    for b in range(B):
        table[b, :nblk[b]] = order[k:k + nblk[b]]
        k += nblk[b]
    pool = _pool(hip, n_pages)
    priors = []
    for b in range(B):
        prior = orc.synthetic((32, 2, 8, lens[b] - 1, 128), SEED, 5000 + b, 0.0, 1.0)
        _prior_into_pages(pool, prior, table[b])
        priors.append(prior)
    toks_stride = max(lens) + 7
    toks = torch.zeros(B, toks_stride, dtype=torch.int32, device="cuda")
    tk = [31337, 777]
    for b in range(B):
        toks[b, lens[b] - 1] = tk[b]
    c = Context(0, graph=False)
    data = torch.zeros(B, 4096, dtype=torch.bfloat16, device="cuda")
    attn = torch.zeros_like(data)
    logits = torch.zeros(B, V, dtype=torch.float32, device="cuda")
    out = torch.zeros(B, dtype=torch.int32, device="cuda")
    ws = torch.zeros(hip.lib.ie_batch_workspace_size(B), dtype=torch.uint8, device="cuda")
    seq = (C.c_int * B)(*lens)
    th = (C.c_int * B)()
    d_table = torch.from_numpy(table).cuda()
    hip.check(hip.lib.ie_decode_step_batched_paged(
        c.handle, model.ref(), B, seq, _ptr(toks), toks_stride, _ptr(data), _ptr(attn),
        _ptr(logits), _ptr(out), th, _ptr(ws), _ptr(pool), n_pages, _ptr(d_table), stride))
    torch.cuda.synchronize()
    got = host(logits).copy()
    new_rows = []
    for b in range(B):
        p = lens[b] - 1
        new_rows.append(host(pool[int(table[b, p // PAGE_POS]), 0, :, :, p % PAGE_POS].contiguous()))
    del pool
    c.close()

    tol = e2e_tol(noise_floor)
    for b in range(B):
        say(f"oracle decode at position {lens[b] - 1}")
        kv = np.zeros((32, 2, 8, lens[b], 128), np.uint16)
        kv[:, :, :, :lens[b] - 1] = priors[b]
        want = oracle_model.decode(tk[b], lens[b] - 1, kv)
        assert_close(got[b], want, tol=tol, what=f"long decode row {b} (context {lens[b]})")
        check_token(th[b], want, got[b], noise_floor)
        assert_bf16_close(new_rows[b], kv[0, :, :, lens[b] - 1], what=f"row {b} layer-0 kv",
                          outlier_frac=2e-3)


def test_long_prefill_paged_vs_oracle(hip, model, oracle_model, noise_floor):
    """ie_prefill_paged of a 9000-token prompt (past the reference's 8192): every layer-0 K/V
    row against the oracle, layer 0's output at sampled rows (8191, 8192, 8999 among them)
    through the layer-1 K/V rows; the same prompt prefilled in two chunks (8192 + 808,
    ie_prefill_paged_chunk) against the one-shot logits; and a decode step at 9001 positions
    after it against prefill_paged(9001)."""
    from infengine_amd.engine import Context, workspace_size
    S = 9000
    rng = np.random.default_rng(9000)
    ids = rng.integers(0, V, S + 1).astype(np.int32)
    nblk = (S + 1 + PAGE_POS - 1) // PAGE_POS
    n_pages = nblk + 3
    table = torch.from_numpy(rng.permutation(n_pages)[:nblk].astype(np.int32)).cuda()
    toks = torch.from_numpy(ids).cuda()
    c = Context(0, graph=False)

    def buffers(rows):
        data = torch.zeros(rows, 4096, dtype=torch.bfloat16, device="cuda")
        return dict(data=data, aux=torch.zeros_like(data), attn=torch.zeros_like(data),
                    logits=torch.zeros(V, dtype=torch.float32, device="cuda"),
                    out=torch.zeros(1, dtype=torch.int32, device="cuda"),
                    ws=torch.zeros(workspace_size(rows), dtype=torch.uint8, device="cuda"))

    def chunk(pool, bf, start, n):
        t = hip.check(hip.lib.ie_prefill_paged_chunk(
            c.handle, model.ref(), start, n, _ptr(toks), _ptr(bf["data"]), _ptr(bf["aux"]),
            _ptr(bf["attn"]), _ptr(bf["logits"]), _ptr(bf["out"]), _ptr(bf["ws"]), _ptr(pool),
            n_pages, _ptr(table)))
        torch.cuda.synchronize()
        return t, host(bf["logits"]).copy()

    say(f"ie_prefill_paged S={S}")
    pool = _pool(hip, n_pages)
    bf = buffers(S + 1)
    tok = hip.check(hip.lib.ie_prefill_paged(
        c.handle, model.ref(), S, _ptr(toks), _ptr(bf["data"]), _ptr(bf["aux"]), _ptr(bf["attn"]),
        _ptr(bf["logits"]), _ptr(bf["out"]), _ptr(bf["ws"]), _ptr(pool), n_pages, _ptr(table)))
    torch.cuda.synchronize()
    logits = host(bf["logits"]).copy()
    assert tok == int(np.argmax(logits))
    tbl = host(table)
    # layers 0 and 1, positions 0..S-1, gathered from the pages: [2 layers][2][8][S][128]
    pv = pool[torch.from_numpy(tbl.astype(np.int64)).cuda(), :2]          # [nblk][2][2][8][64][128]
    gkv = host(pv.permute(1, 2, 3, 0, 4, 5).reshape(2, 2, 8, nblk * PAGE_POS, 128)[:, :, :, :S]
               .contiguous())
    del pv

    say("the same prompt in two chunks: 8192 + 808")
    pool2 = _pool(hip, n_pages)
    bf2 = buffers(8192)
    chunk(pool2, bf2, 0, 8192)
    tok_c, logits_c = chunk(pool2, bf2, 8192, S - 8192)
    tol = e2e_tol(noise_floor)
    assert_close(logits_c, logits, tol=tol, what="chunked vs one-shot prefill logits")
    check_token(tok_c, logits, logits_c, noise_floor)
    pv2 = pool2[torch.from_numpy(tbl.astype(np.int64)).cuda(), 0]
    gkv2 = host(pv2.permute(1, 2, 0, 3, 4).reshape(2, 8, nblk * PAGE_POS, 128)[:, :, :S].contiguous())
    del pv2, pool2, bf2
    assert_bf16_close(gkv2, gkv[0], what="chunked layer-0 kv", outlier_frac=1e-3)

    say(f"decode at {S + 1} positions after the prefill vs prefill_paged({S + 1})")
    seq = (C.c_int * 1)(S + 1)
    th = (C.c_int * 1)()
    dl = torch.zeros(1, V, dtype=torch.float32, device="cuda")
    dws = torch.zeros(hip.lib.ie_batch_workspace_size(1), dtype=torch.uint8, device="cuda")
    dd = torch.zeros(1, 4096, dtype=torch.bfloat16, device="cuda")
    da = torch.zeros_like(dd)
    hip.check(hip.lib.ie_decode_step_batched_paged(
        c.handle, model.ref(), 1, seq, _ptr(toks), toks.numel(), _ptr(dd), _ptr(da), _ptr(dl),
        _ptr(bf["out"]), th, _ptr(dws), _ptr(pool), n_pages, _ptr(table), nblk))
    torch.cuda.synchronize()
    dec = host(dl[0]).copy()
    t1, want1 = chunk(pool, bf, 0, S + 1)
    assert_close(dec, want1, tol=tol, what="decode(9001) vs prefill_paged(9001)")
    check_token(th[0], want1, dec, noise_floor)
    del pool, bf
    c.close()

    say("oracle: layer-0 K/V of all 9000 rows")
    cos, sin = oracle_model.cos, oracle_model.sin
    w0 = orc.layer_weights(SEED, 0)
    x0 = oracle_model.embed(ids[:S])
    xn = orc.rmsnorm(x0, w0["input_layernorm"])
    k0 = _rotate_heads(orc.matmul(xn, w0["w_k"]), 0, cos, sin)
    v0 = np.ascontiguousarray(orc.matmul(xn, w0["w_v"]).reshape(S, 8, 128).transpose(1, 0, 2))
    assert_bf16_close(gkv[0, 0], k0, what="layer-0 K, 9000 rows", outlier_frac=1e-3)
    assert_bf16_close(gkv[0, 1], v0, what="layer-0 V, 9000 rows")

    # one layer deep, as in the 2048-token prefill test (the oracle rounds the attention
    # probabilities as the MFMA attention does)
    say("oracle: layer 0 at sampled rows -> layer-1 K/V rows")
    w1 = orc.layer_weights(SEED, 1)
    for p in (0, 4096, 8191, 8192, 8999):
        planes = np.zeros((2, 8, p + 1, 128), np.uint16)
        planes[0, :, :p] = k0[:, :p]
        planes[1, :, :p] = v0[:, :p]
        x = x0[p:p + 1].copy()
        with orc.prob_rounding(orc.PROB_FLASH):
            orc.decoder_layer(x, w0, p, cos, sin, planes[0], planes[1], p + 1)
        xn1 = orc.rmsnorm(x, w1["input_layernorm"])
        k1 = _rotate_heads(orc.matmul(xn1, w1["w_k"]), p, cos, sin)[:, 0]
        v1 = orc.matmul(xn1, w1["w_v"]).reshape(8, 128)
        report_close(orc.bf16_to_f32(gkv[1, 0, :, p]), orc.bf16_to_f32(k1), what=f"layer-1 K row {p}")
        report_close(orc.bf16_to_f32(gkv[1, 1, :, p]), orc.bf16_to_f32(v1), what=f"layer-1 V row {p}")


def test_long_context_limits_rejected_on_the_host(hip, ctx, model):
    """Positions past what an entry point's cache holds are refused before any GPU work: the
    reference-layout prefill at 8193 tokens, a paged chunk ending past 131072, a paged step
    whose token rows are shorter than its context, a block table wider than 131072 / 64."""
    say("long-context limits")
    bogus = C.c_void_p(0x1000)        # never dereferenced: validation fails first
    assert hip.lib.ie_prefill(ctx.handle, model.ref(), 8193, *[bogus] * 8) == -1
    assert "8192" in hip.last_error()
    assert hip.lib.ie_prefill_paged_chunk(ctx.handle, model.ref(), 131000, 100, *[bogus] * 8,
                                          4, bogus) == -1
    seq = (C.c_int * 1)(9001)
    assert hip.lib.ie_decode_step_batched_paged(ctx.handle, model.ref(), 1, seq, bogus, 9000,
                                                *[bogus] * 4, None, bogus, bogus, 4, bogus,
                                                200) == -1
    assert "token rows" in hip.last_error()
    assert hip.lib.ie_decode_step_batched_paged(ctx.handle, model.ref(), 1, seq, bogus, 9001,
                                                *[bogus] * 4, None, bogus, bogus, 4, bogus,
                                                131072 // 64 + 1) == -1


def test_positions_past_the_rope_tables_rejected(hip, ctx, model):
    """Weights whose RoPE tables have the reference's 8192 rows (rope_rows 0, as a caller
    assembling its own ie_model_weights leaves it) are refused past position 8191 by the paged
    entry points, before any GPU work; the library's own weights carry 131072 rows."""
    from infengine_amd._lib import ModelWeightsStruct
    say("positions past the weights' RoPE table rows")
    assert model.s.rope_rows == orc.LONGCTX
    w = ModelWeightsStruct()
    C.memmove(C.byref(w), C.byref(model.s), C.sizeof(w))
    w.rope_rows = 0
    bogus = C.c_void_p(0x1000)        # never dereferenced: validation fails first
    assert hip.lib.ie_prefill_paged_chunk(ctx.handle, C.byref(w), 8000, 200, *[bogus] * 8, 4,
                                          bogus) == -1
    assert "rope_rows" in hip.last_error()
    seq = (C.c_int * 1)(8193)
    assert hip.lib.ie_decode_step_batched_paged(ctx.handle, C.byref(w), 1, seq, bogus, 9000,
                                                *[bogus] * 4, None, bogus, bogus, 4, bogus,
                                                200) == -1
    assert "rope_rows" in hip.last_error()
