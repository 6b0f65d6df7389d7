"""BASELINE configs 4 and 5 at their real sizes on the full 32-layer random-init
Llama-3.1-8B, through the C-ABI, against the CPU oracle regenerating the same weights.

  config 4  ie_prefill of a 2048-token prompt (prefill.cu:11-48): the MFMA projections,
            32-row flash-attention workgroups and the K/V write-out at M = 2048.
  config 5  512-token prompts then 256 greedy decode steps (manager.cpp:60-86), KV up to 768
            positions per sequence: bs=1 through ie_generate, bs=16 through
            ie_decode_step_batched.
  bs=16     one batched decode step at staggered contexts, every row against the oracle.

Bars as in test_gpu_model: logits within the end-to-end tolerance (1e-2, or 2x the stack's
own summation-order noise floor), tokens equal to the oracle's argmax outside that noise,
bit-exact equality between the library's own equivalent paths, K/V rows of the first layers
against the oracle to bf16 rounding.
"""
import ctypes as C

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


def _ptr(t: torch.Tensor) -> C.c_void_p:
    return C.c_void_p(t.data_ptr())


def _kv6(kv: torch.Tensor) -> torch.Tensor:
    return kv.view(torch.int16).view(32, 2, 8, 8192, 128)


def _oracle_decode_rows(om, toks, poss, kvs):
    """oracle decode_step of several independent sequences, layer by layer (each layer's weights
    generated once): row b embeds toks[b] at position poss[b] over its cache kvs[b]
    [32, 2, 8, ctx_b, 128] (rows 0..poss[b]-1 set; row poss[b] is written).  Returns the logits."""
    xs = [om.embed([t]) for t in toks]
    for l in range(32):
        w = orc.layer_weights(SEED, l)
        for x, p, kv in zip(xs, poss, kvs):
            orc.decoder_layer(x, w, p, om.cos, om.sin, kv[l, 0], kv[l, 1], kv.shape[3])
    return [om.logits(x[0]) for x in xs]


def _rotate_heads(k_rows: np.ndarray, start_pos: int, cos, sin) -> np.ndarray:
    """RoPE of [S][heads * 128] rows at positions start_pos.. -> [heads][S][128]."""
    S = k_rows.shape[0]
    heads = k_rows.shape[1] // 128
    kt = np.ascontiguousarray(k_rows.reshape(S, heads, 128).transpose(1, 0, 2))
    return orc.apply_rope(kt, start_pos, heads, S, S, cos, sin)


# ---------------------------------------------------------------- config 4
def test_prefill_2048_config4(hip, model, oracle_model, noise_floor):
    """ie_prefill at S = 2048: every layer-0 K/V row against the oracle; layer 0's full output
    (attention + O + FFN) at sampled rows, seen through the layer-1 K/V rows it produces; logits
    and token bit-identical to ie_prefill_paged; last-row logits against prefill(2047) +
    decode_step(2048) (a different code path for the last token)."""
    from infengine_amd.engine import Context, Request
    S = 2048
    rng = np.random.default_rng(2048)
    ids = rng.integers(0, V, S).astype(np.int32)
    c = Context(0, graph=False)
    say(f"ie_prefill S={S}")
    req = Request(c, model, max_seq_len=S + 8)
    req.tokens[:S] = torch.from_numpy(ids).cuda()
    tok = req.prefill(S)
    logits = host(req.logits).copy()
    gkv = host(_kv6(req.kv)[:2, :, :, :S + 1].contiguous())
    assert np.isfinite(logits).all()
    assert tok == int(np.argmax(logits))
    assert gkv[:, :, :, :S].any(axis=-1).all() and not gkv[:, :, :, S].any()

    say(f"ie_prefill_paged S={S} (pages in a shuffled order)")
    page_elems = hip.lib.ie_kv_page_size() // 2
    nblk = S // 64
    n_pages = nblk + 3
    order = rng.permutation(n_pages)[:nblk].astype(np.int32)
    pool = torch.zeros(n_pages * page_elems, dtype=torch.int16, device="cuda")
    d_table = torch.from_numpy(order).cuda()
    logits_p = torch.zeros(V, dtype=torch.float32, device="cuda")
    out_p = torch.zeros(1, dtype=torch.int32, device="cuda")
    tok_p = hip.check(hip.lib.ie_prefill_paged(
        c.handle, model.ref(), S, _ptr(req.tokens), _ptr(req.data), _ptr(req.aux), _ptr(req.attn),
        _ptr(logits_p), _ptr(out_p), _ptr(req.workspace), _ptr(pool), n_pages, _ptr(d_table)))
    torch.cuda.synchronize()
    assert tok_p == tok and np.array_equal(host(logits_p), logits)
    pool6 = pool.view(n_pages, 32, 2, 8, 64, 128)
    kv_full = _kv6(req.kv)
    for i in range(0, nblk, 7):
        assert torch.equal(pool6[int(order[i])], kv_full[:, :, :, 64 * i:64 * i + 64]), i
    del pool

    say("prefill(2047) + decode_step(2048)")
    req2 = Request(c, model, max_seq_len=S + 8)
    req2.tokens[:S] = torch.from_numpy(ids).cuda()
    req2.prefill(S - 1)
    tok2 = req2.decode_step(S)
    logits2 = host(req2.logits).copy()
    del req2
    c.close()
    tol = e2e_tol(noise_floor)
    assert_close(logits, logits2, tol=tol, what="prefill(2048) vs prefill(2047) + decode")
    check_token(tok, logits2, logits, noise_floor)
    assert tok2 == int(np.argmax(logits2))

    say("oracle: layer-0 K/V of all 2048 rows")
    cos, sin = oracle_model.cos, oracle_model.sin
    w0 = orc.layer_weights(SEED, 0)
    x0 = oracle_model.embed(ids)
    xn = orc.rmsnorm(x0, w0["input_layernorm"])
    k0 = _rotate_heads(orc.matmul(xn, w0["w_k"]), 0, cos, sin)              # [8][S][128]
    v0 = np.ascontiguousarray(orc.matmul(xn, w0["w_v"]).reshape(S, 8, 128).transpose(1, 0, 2))
    assert_bf16_close(gkv[0, 0, :, :S], k0, what="layer-0 K, 2048 rows", outlier_frac=1e-3)
    assert_bf16_close(gkv[0, 1, :, :S], v0, what="layer-0 V, 2048 rows")

    # Layer 0's output at row p, seen through the layer-1 K/V row it produces, one layer deep.
    # The oracle rounds the attention probabilities as the MFMA attention does (bf16 against the
    # running max of 64-key tiles): where it keeps them in fp32, or rounds the normalised ones as
    # the reference's softmax does, these rows move by 0.7-1.2% (max-abs / scale) and ~0.7%
    # (mean-rel) from the rounding point alone -- the same distance either way, measured on the
    # CPU at rows 63 / 64 / 1000 / 1537 / 2047.
    say("oracle: layer 0 at sampled rows -> layer-1 K/V rows")
    w1 = orc.layer_weights(SEED, 1)
    for p in (0, 1, 63, 64, 1000, 1537, 2047):
        planes = np.zeros((2, 8, p + 1, 128), np.uint16)
        planes[0, :, :p] = k0[:, :p]
        planes[1, :, :p] = v0[:, :p]
        x = x0[p:p + 1].copy()
        with orc.prob_rounding(orc.PROB_FLASH):
            orc.decoder_layer(x, w0, p, cos, sin, planes[0], planes[1], p + 1)   # layer 0, row p
        xn1 = orc.rmsnorm(x, w1["input_layernorm"])
        k1 = _rotate_heads(orc.matmul(xn1, w1["w_k"]), p, cos, sin)[:, 0]   # [8][128]
        v1 = orc.matmul(xn1, w1["w_v"]).reshape(8, 128)
        report_close(orc.bf16_to_f32(gkv[1, 0, :, p]), orc.bf16_to_f32(k1), what=f"layer-1 K row {p}")
        report_close(orc.bf16_to_f32(gkv[1, 1, :, p]), orc.bf16_to_f32(v1), what=f"layer-1 V row {p}")


@pytest.mark.parametrize("S", [2048, 2000, 512, 100])
def test_prefill_fused_qkv_rope_equals_scatter(hip, model, S):
    """The prefill QKV projection with RoPE and the K/V write fused (ie_tune_gemm_schedule 1: in
    the epilogue of the ping-pong 192 x 256 tiles at S = 2048 / 2000, in the K-split reduction at
    S = 512 / 100) against the bf16 product + scatter kernel (schedule 0), whose other products
    are the same kernels: residual rows, every K/V row and the logits bit for bit, on the
    reference-layout cache (S = 2000: a last row tile of 208 rows) and for a chunk at start
    position 1000 over shuffled pages.  (At S <= 128 the default schedule runs the 64-weight-row
    kernel with other K splits; the prefill-vs-oracle tests cover it.)"""
    from infengine_amd.engine import Context, Request
    rng = np.random.default_rng(S)
    ids = rng.integers(0, V, S + 1000).astype(np.int32)
    c = Context(0, graph=False)
    page_elems = hip.lib.ie_kv_page_size() // 2
    nblk = (S + 1000 + 63) // 64
    order = rng.permutation(nblk + 2)[:nblk].astype(np.int32)
    d_table = torch.from_numpy(order).cuda()
    outs = {}
    try:
        for sched in (0, 1):
            hip.check(hip.lib.ie_tune_gemm_schedule(sched))
            say(f"ie_prefill S={S}, gemm schedule {sched}")
            req = Request(c, model, max_seq_len=S + 1008)
            req.tokens[:S + 1000] = torch.from_numpy(ids).cuda()
            tok = req.prefill(S)
            torch.cuda.synchronize()
            res = [tok, host(req.logits).copy(), host(req.data[:S].view(torch.int16)).copy(),
                   req.kv.clone()]
            say(f"ie_prefill_paged_chunk start 1000, {S} tokens, gemm schedule {sched}")
            pool = torch.zeros((nblk + 2) * page_elems, dtype=torch.int16, device="cuda")
            lg = torch.zeros(V, dtype=torch.float32, device="cuda")
            out = torch.zeros(1, dtype=torch.int32, device="cuda")
            # positions 0..999 first (the chunk attends to them), then the chunk under test
            hip.check(hip.lib.ie_prefill_paged_chunk(
                c.handle, model.ref(), 0, 1000, _ptr(req.tokens), _ptr(req.data), _ptr(req.aux),
                _ptr(req.attn), _ptr(lg), _ptr(out), _ptr(req.workspace), _ptr(pool), nblk + 2,
                _ptr(d_table)))
            tok_c = hip.check(hip.lib.ie_prefill_paged_chunk(
                c.handle, model.ref(), 1000, S, _ptr(req.tokens), _ptr(req.data), _ptr(req.aux),
                _ptr(req.attn), _ptr(lg), _ptr(out), _ptr(req.workspace), _ptr(pool), nblk + 2,
                _ptr(d_table)))
            torch.cuda.synchronize()
            res += [tok_c, host(lg).copy(), pool.clone()]
            outs[sched] = res
            del req, pool
    finally:
        hip.check(hip.lib.ie_tune_gemm_schedule(2))
    a, b = outs[0], outs[1]
    assert a[0] == b[0] and np.array_equal(a[1], b[1]) and np.array_equal(a[2], b[2])
    assert torch.equal(a[3], b[3])
    assert a[4] == b[4] and np.array_equal(a[5], b[5]) and torch.equal(a[6], b[6])
    c.close()


# ---------------------------------------------------------------- config 5, bs = 1
def test_generate_512_then_256_config5(hip, model, oracle_model, noise_floor):
    """ie_generate with a 512-token prompt and 256 decode steps (KV to 768 positions) equals the
    host-driven reference loop (ie_prefill, ie_decode_step, device write-back) bit for bit; its
    last step's logits match one oracle decode fed the GPU's cache and token."""
    from infengine_amd.engine import Context, Request
    S, N = 512, 257                      # the prefill's token + 256 decode steps
    ids = np.random.default_rng(512).integers(0, V, S).astype(np.int32)
    c = Context(0, graph=True)
    say(f"ie_generate prompt={S} new={N}")
    a = Request(c, model, max_seq_len=S + 8)
    got, _ = a.generate(ids, N)
    assert len(got) == N
    say("host-driven prefill + 256 decode_step loop")
    b = Request(c, model, max_seq_len=S + 8)
    b.tokens[:S] = torch.from_numpy(ids).cuda()
    want = [b.prefill(S)]
    b.tokens[S] = b.token[0]
    for i in range(1, N):
        want.append(b.decode_step(S + i))
        b.tokens[S + i] = b.token[0]
    assert got == want
    assert torch.equal(a.tokens[:S + N], b.tokens[:S + N])
    assert torch.equal(_kv6(a.kv)[:, :, :, :S + N], _kv6(b.kv)[:, :, :, :S + N])
    assert torch.equal(a.logits, b.logits)
    last = S + N - 2                     # position of the last step's token
    gkv = host(_kv6(a.kv)[:, :, :, :last + 1].contiguous())
    got_logits = host(a.logits).copy()
    c.close()

    say(f"oracle decode at position {last} over the GPU's cache")
    kv = np.zeros((32, 2, 8, last + 1, 128), np.uint16)
    kv[:, :, :, :last] = gkv[:, :, :, :last]
    want_logits = oracle_model.decode(got[-2], last, kv)
    assert_close(got_logits, want_logits, tol=e2e_tol(noise_floor), what="step 256 logits")
    check_token(got[-1], want_logits, got_logits, noise_floor)
    assert_bf16_close(gkv[0, :, :, last], kv[0, :, :, last], what="layer-0 kv row 767",
                      outlier_frac=1e-3)


# ---------------------------------------------------------------- batched decode, bs = 16
def _batched_buffers(hip, B):
    data = torch.zeros(B, 4096, dtype=torch.bfloat16, device="cuda")
    return dict(data=data, attn=torch.zeros_like(data),
                logits=torch.zeros(B, V, dtype=torch.float32, device="cuda"),
                out=torch.zeros(B, dtype=torch.int32, device="cuda"),
                ws=torch.zeros(hip.lib.ie_batch_workspace_size(B), dtype=torch.uint8,
                               device="cuda"))


def _batched_step(hip, c, model, lens, toks, kvs, buf):
    B = len(lens)
    seq = (C.c_int * B)(*lens)
    th = (C.c_int * B)()
    hip.check(hip.lib.ie_decode_step_batched(c.handle, model.ref(), B, seq, _ptr(toks),
                                             _ptr(buf["data"]), _ptr(buf["attn"]),
                                             _ptr(buf["logits"]), _ptr(buf["out"]), th,
                                             _ptr(buf["ws"]), _ptr(kvs)))
    return list(th)


# all contexts <= 2048: one workgroup per (sequence, kv head) writes the output; with a context
# past 2048 every row takes split + merge
@pytest.mark.parametrize("lens", [[101 + 97 * b for b in range(16)],
                                  [513 + 3 * b for b in range(15)] + [2100]])
def test_batched16_rows_vs_oracle(hip, model, oracle_model, noise_floor, lens):
    """ie_decode_step_batched with 16 sequences at staggered contexts: each row's logits against
    the oracle's decode of that sequence, its token against the oracle's argmax, its new layer-0
    K/V row against the oracle's."""
    from infengine_amd.engine import Context
    B = len(lens)
    say(f"decode_step_batched B={B} lens {lens[0]}..{lens[-1]}")
    c = Context(0, graph=False)
    kvs = torch.zeros(B * hip.lib.ie_kv_cache_size() // 2, dtype=torch.int16, device="cuda")
    kv7 = kvs.view(B, 32, 2, 8, 8192, 128)
    toks = torch.zeros(B, 8192, dtype=torch.int32, device="cuda")
    priors, tk = [], []
    for b in range(B):
        prior = orc.synthetic((32, 2, 8, lens[b] - 1, 128), SEED, 3000 + b, 0.0, 1.0)
        kv7[b, :, :, :, :lens[b] - 1] = dev(prior)
        tk.append(977 * (b + 1) + 13)
        toks[b, lens[b] - 1] = tk[-1]
        priors.append(prior)
    buf = _batched_buffers(hip, B)
    th = _batched_step(hip, c, model, lens, toks, kvs, buf)
    torch.cuda.synchronize()
    got = host(buf["logits"]).copy()
    new_rows = [host(kv7[b, 0, :, :, lens[b] - 1].contiguous()) for b in range(B)]
    del kvs, kv7
    c.close()

    say("oracle: 16 decode rows")
    kvo = []
    for b in range(B):
        kv = np.zeros((32, 2, 8, lens[b], 128), np.uint16)
        kv[:, :, :, :lens[b] - 1] = priors[b]
        kvo.append(kv)
    want = _oracle_decode_rows(oracle_model, tk, [n - 1 for n in lens], kvo)
    tol = e2e_tol(noise_floor)
    for b in range(B):
        assert_close(got[b], want[b], tol=tol, what=f"batched row {b} (context {lens[b]})")
        check_token(th[b], want[b], got[b], noise_floor)
        # the batched projection sums in MFMA order; RoPE's a*c - b*s magnifies a rare 1-ulp
        # product difference past 2 ulp: up to 0.2% of the elements (each within 1e-2 of scale)
        assert_bf16_close(new_rows[b], kvo[b][0, :, :, lens[b] - 1], what=f"row {b} layer-0 kv",
                          outlier_frac=2e-3)


# ---------------------------------------------------------------- config 5, bs = 16
def test_batched_generate_512_then_256_config5(hip, model, oracle_model, noise_floor):
    """Config 5 at bs=16: 16 independent 512-token prompts, each prefilled into its own cache,
    then 256 batched greedy steps (tokens fed back on the device; contexts 513..768).  The last
    step's logits of every row against an oracle decode over that row's GPU cache and token."""
    from infengine_amd.engine import Context
    B, S, N = 16, 512, 256
    c = Context(0, graph=False)
    kvsz = hip.lib.ie_kv_cache_size()
    kvs = torch.zeros(B * kvsz // 2, dtype=torch.int16, device="cuda")
    kv7 = kvs.view(B, 32, 2, 8, 8192, 128)
    toks = torch.zeros(B, 8192, dtype=torch.int32, device="cuda")
    rng = np.random.default_rng(516)
    data = torch.zeros(S, 4096, dtype=torch.bfloat16, device="cuda")
    aux, attn = torch.zeros_like(data), torch.zeros_like(data)
    logits1 = torch.zeros(V, dtype=torch.float32, device="cuda")
    out1 = torch.zeros(1, dtype=torch.int32, device="cuda")
    ws = torch.zeros(max(hip.lib.ie_attn_workspace_size(S), hip.lib.ie_ffn_workspace_size(S)),
                     dtype=torch.uint8, device="cuda")
    say(f"16 prefills of {S} tokens")
    for b in range(B):
        toks[b, :S] = torch.from_numpy(rng.integers(0, V, S).astype(np.int32)).cuda()
        t = hip.check(hip.lib.ie_prefill(c.handle, model.ref(), S, _ptr(toks[b]), _ptr(data),
                                         _ptr(aux), _ptr(attn), _ptr(logits1), _ptr(out1),
                                         _ptr(ws), C.c_void_p(kvs.data_ptr() + b * kvsz)))
        toks[b, S] = t
    del data, aux, attn, ws
    buf = _batched_buffers(hip, B)
    say(f"{N} batched steps, contexts {S + 1}..{S + N}")
    for i in range(N):
        th = _batched_step(hip, c, model, [S + 1 + i] * B, toks, kvs, buf)
        toks[:, S + 1 + i] = buf["out"]
        if i % 64 == 63:
            say(f"  step {i + 1}")
    torch.cuda.synchronize()
    last = S + N - 1                     # position of the last step's token (767)
    got = host(buf["logits"]).copy()
    ht = host(toks[:, :last + 2])
    assert [int(ht[b, last + 1]) for b in range(B)] == th
    gkv = [host(kv7[b, :, :, :, :last + 1].contiguous()) for b in range(B)]
    del kvs, kv7
    c.close()

    say("oracle: 16 decode rows at position 767 over the GPU's caches")
    kvo = []
    for b in range(B):
        kv = np.zeros((32, 2, 8, last + 1, 128), np.uint16)
        kv[:, :, :, :last] = gkv[b][:, :, :, :last]
        kvo.append(kv)
    want = _oracle_decode_rows(oracle_model, [int(ht[b, last]) for b in range(B)], [last] * B, kvo)
    tol = e2e_tol(noise_floor)
    for b in range(B):
        assert_close(got[b], want[b], tol=tol, what=f"row {b} step {N} logits")
        check_token(th[b], want[b], got[b], noise_floor)
        assert_bf16_close(gkv[b][0, :, :, last], kvo[b][0, :, :, last],
                          what=f"row {b} layer-0 kv row {last}", outlier_frac=2e-3)
