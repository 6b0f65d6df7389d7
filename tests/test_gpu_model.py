"""The engine entry points on the full 32-layer random-init Llama-3.1-8B (bf16),
through the C-ABI (ie_decode_step / ie_prefill / ie_decode_step_batched),
against the CPU oracle regenerating the same weights.

Three bars:
  * per layer: every one of the 32 layers, fed the GPU's own input, matches the
    oracle layer to tests/tolerance.py (no error accumulation across layers);
  * integration: ie_decode_step is bitwise identical to chaining the per-layer
    entry point plus final norm / lm_head / argmax (eager and hipGraph replay);
  * end to end: logits of the 32-layer stack are within 2x the stack's own fp32
    noise floor, measured as the oracle vs the oracle with every dot product
    summed in the opposite order (bf16 storage amplifies rounding-order noise
    through 32 layers to a few percent on this random-init model).  Token ids
    equal the oracle's argmax unless its top-2 gap is inside that noise.
KV-cache placement is bit-exact: untouched rows stay exactly as they were.
"""
import ctypes as C

import numpy as np
import pytest
import torch

import oracle as orc
from conftest import MODEL_SEED, NOISE_POS
from gpu_util import (P, assert_bf16_close, assert_delta_close, check_token, dev, e2e_tol, host,
                      say)
from tolerance import assert_close

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(900)]
SEED = MODEL_SEED
POS = NOISE_POS


@pytest.fixture(scope="module")
def prior():
    return orc.synthetic((32, 2, 8, POS, 128), SEED, 900, 0.0, 1.0)


def test_weights_match_oracle_generator(model):
    W = model
    assert np.array_equal(host(W.view(7, "w_k").view(torch.int16)),
                          orc.layer_weights(SEED, 7)["w_k"])
    assert np.array_equal(host(W.view(None, "final_norm").view(torch.int16)),
                          orc.final_norm(SEED))


def _chained_layers(hip, ctx, model, prior, tok, oracle_check):
    """Embed tok at position POS and run the 32 layers one entry point call at a
    time; with oracle_check, compare each layer against the oracle fed the same
    input.  Returns (hidden, logits, kv)."""
    kv = torch.zeros(hip.lib.ie_kv_cache_size() // 2, dtype=torch.int16, device="cuda")
    kv.view(32, 2, 8, 8192, 128)[:, :, :, :POS] = dev(prior)
    emb = model.view(None, "emb_lookup").view(torch.int16)
    x = emb[tok:tok + 1].clone()
    attn = torch.empty(1, 4096, dtype=torch.int16, device="cuda")
    ws = torch.zeros(hip.lib.ie_attn_workspace_size(1), dtype=torch.uint8, device="cuda")
    cos, sin = orc.rope_tables()
    for l in range(32):
        x_in = host(x).copy()
        hip.check(hip.lib.ie_decoder_layer_decode(ctx.handle, model.ref(), l, POS + 1, P(x),
                                                  P(attn), P(ws), P(kv)))
        torch.cuda.synchronize()
        if oracle_check:
            w = orc.layer_weights(SEED, l)
            planes = np.zeros((2, 8, POS + 1, 128), np.uint16)
            planes[:, :, :POS] = prior[l]
            xo = x_in.copy()
            orc.decoder_layer(xo, w, POS, cos, sin, planes[0], planes[1], POS + 1)
            got = orc.bf16_to_f32(host(x))
            assert_close(got, orc.bf16_to_f32(xo), what=f"layer {l}")
            assert_delta_close(x_in, host(x), xo, what=f"layer {l} delta")
            gkv = host(kv.view(32, 2, 8, 8192, 128)[l, :, :, POS])
            assert_bf16_close(gkv, planes[:, :, POS], what=f"layer {l} kv row", outlier_frac=1e-3)
    logits = torch.empty(128256, dtype=torch.float32, device="cuda")
    hip.check(hip.lib.ie_final_norm_lm_head(ctx.handle, 1, P(x),
                                            P(model.view(None, "final_norm")),
                                            P(model.view(None, "lm_head")), P(logits)))
    torch.cuda.synchronize()
    return host(x), host(logits), kv


def test_every_layer_matches_oracle(hip, ctx, model, prior):
    say("32 layers one at a time vs the oracle (each fed the GPU's input)")
    _chained_layers(hip, ctx, model, prior, 4242, oracle_check=True)


@pytest.mark.parametrize("graph", [False, True])
def test_decode_step_equals_chained_layers(hip, ctx, model, prior, graph):
    from infengine_amd.engine import Context, Request
    say(f"decode_step (graph={graph}) vs chained per-layer calls, bitwise")
    _, want_logits, want_kv = _chained_layers(hip, ctx, model, prior, 4242, oracle_check=False)
    c = Context(0, graph=graph)
    req = Request(c, model, max_seq_len=POS + 8)
    req.kv_view()[:, :, :, :POS] = dev(prior).view(torch.bfloat16)
    req.tokens[POS] = 4242
    for rep in range(3 if graph else 1):          # graph replays: same input, same output
        req.kv_view()[:, :, :, POS:] = 0
        tok = req.decode_step(POS + 1)
        got = host(req.logits)
        assert np.array_equal(got, want_logits), f"replay {rep}"
        assert tok == int(np.argmax(want_logits))
        assert int(req.token.item()) == tok
    gkv = host(req.kv.view(torch.int16).view(32, 2, 8, 8192, 128)[:, :, :, :POS + 2])
    assert np.array_equal(gkv, host(want_kv.view(32, 2, 8, 8192, 128)[:, :, :, :POS + 2]))
    c.close()
    torch.cuda.set_stream(ctx.stream)


def test_decode_steps_vs_oracle(hip, model, oracle_model, prior, noise_floor):
    from infengine_amd.engine import Context, Request
    say(f"decode_step x2 from position {POS} vs oracle (tol {e2e_tol(noise_floor):.3e})")
    c = Context(0, graph=True)
    req = Request(c, model, max_seq_len=POS + 8)
    req.kv_view()[:, :, :, :POS] = dev(prior).view(torch.bfloat16)
    req.tokens[POS] = 4242
    t1 = req.decode_step(POS + 1)
    got1 = host(req.logits).copy()
    req.tokens[POS + 1] = t1
    t2 = req.decode_step(POS + 2)
    got2 = host(req.logits).copy()
    gkv = host(req.kv.view(torch.int16).view(32, 2, 8, 8192, 128)[:, :, :, :POS + 3])
    c.close()

    kv = np.zeros((32, 2, 8, POS + 2, 128), np.uint16)
    kv[:, :, :, :POS] = prior
    want1 = oracle_model.decode(4242, POS, kv)
    assert_close(got1, want1, tol=e2e_tol(noise_floor), what="decode step 1 logits")
    check_token(t1, want1, got1, noise_floor)
    want2 = oracle_model.decode(t1, POS + 1, kv)
    assert_close(got2, want2, tol=e2e_tol(noise_floor), what="decode step 2 logits")
    check_token(t2, want2, got2, noise_floor)
    assert np.array_equal(gkv[:, :, :, :POS], prior)              # old rows untouched
    assert gkv[:, :, :, POS:POS + 2].any(axis=-1).all()            # rows POS, POS+1 written
    assert not gkv[:, :, :, POS + 2].any()                         # next row still empty
    assert_bf16_close(gkv[0, :, :, POS:POS + 2], kv[0, :, :, POS:POS + 2], what="layer-0 kv", outlier_frac=1e-3)


# 1 / 2 / 16: the M <= 16 skinny projections (at 1 the last layer's last row is its only row);
# 24 / 40 / 100: the 64-weight-row streaming projections (64 and 128 X rows; K split into fp32
# planes in the workspace, O aliased over q/k/v, SwiGLU in the kernel); 256: split-K MFMA tiles,
# the SwiGLU split and 16-row flash-attention workgroups; 128 / 129: the last medium-row size and
# the first split-K one
@pytest.mark.parametrize("S", [1, 2, 16, 17, 24, 40, 64, 65, 100, 128, 129, 256])
def test_prefill_then_decode_vs_oracle(hip, model, oracle_model, noise_floor, S):
    from infengine_amd.engine import Context, Request
    say(f"prefill seq_len={S} then decode_step vs oracle")
    rng = np.random.default_rng(5)
    ids = rng.integers(0, 128256, S).astype(np.int32)
    c = Context(0)
    req = Request(c, model, max_seq_len=S + 8)
    req.tokens[:S] = torch.from_numpy(ids).cuda()
    t = req.prefill(S)
    got = host(req.logits).copy()
    gkv = host(req.kv.view(torch.int16).view(32, 2, 8, 8192, 128)[:, :, :, :S + 1])
    req.tokens[S] = t
    t2 = req.decode_step(S + 1)
    got2 = host(req.logits).copy()
    # invariant: decode at position S == last row of a causal prefill over S+1 tokens
    req2 = Request(c, model, max_seq_len=S + 8)
    req2.tokens[:S + 1] = torch.from_numpy(np.append(ids, t).astype(np.int32)).cuda()
    req2.prefill(S + 1)
    got3 = host(req2.logits).copy()
    c.close()

    say(f"oracle prefill seq_len={S}")
    kv = np.zeros((32, 2, 8, S + 2, 128), np.uint16)
    want = oracle_model.prefill(ids, kv)
    tol = e2e_tol(noise_floor)
    assert_close(got, want, tol=tol, what="prefill logits")
    check_token(t, want, got, noise_floor)
    assert_bf16_close(gkv[0, :, :, :S], kv[0, :, :, :S], what="layer-0 kv", outlier_frac=1e-3)
    # every layer's K/V rows: within the end-to-end tolerance (deeper layers carry the
    # differences of the layers below them)
    for l in range(32):
        assert_close(orc.bf16_to_f32(gkv[l, :, :, :S]), orc.bf16_to_f32(kv[l, :, :, :S]), tol=tol,
                     what=f"layer {l} kv rows")
    assert gkv[:, :, :, :S].any(axis=-1).all() and not gkv[:, :, :, S].any()
    want2 = oracle_model.decode(t, S, kv)
    assert_close(got2, want2, tol=tol, what="decode after prefill")
    check_token(t2, want2, got2, noise_floor)
    assert_close(got3, got2, tol=tol, what="prefill(S+1) vs prefill(S)+decode")


# contexts up to 2048 take the one-workgroup-per-(sequence, kv head) attention; a longer one
# takes split + merge
LENS16 = [101 + 97 * b for b in range(16)]
LENS16_LONG = [513 + 3 * b for b in range(15)] + [2100]


# B = 1; B = 7 with contexts at the first position and around the 64-position tile edges
@pytest.mark.parametrize("lens", [[300], [1, 2, 63, 64, 65, 129, 500], [101, 257, 64],
                                  [2100, 257, 64], LENS16, LENS16_LONG])
def test_batched_decode_matches_single(hip, model, noise_floor, lens):
    from infengine_amd.engine import Context, Request, ptr
    B = len(lens)
    say(f"decode_step_batched B={B} lens={lens}")
    c = Context(0, graph=False)
    kvsz = hip.lib.ie_kv_cache_size()
    kvs = torch.zeros(B * kvsz // 2, dtype=torch.int16, device="cuda")
    toks = torch.zeros(B, 8192, dtype=torch.int32, device="cuda")
    singles = []
    for b in range(B):
        prior = orc.synthetic((32, 2, 8, lens[b] - 1, 128), SEED, 1000 + b, 0.0, 1.0)
        kvs.view(B, 32, 2, 8, 8192, 128)[b, :, :, :, :lens[b] - 1] = dev(prior)
        toks[b, lens[b] - 1] = 1000 * (b + 1)
        req = Request(c, model, max_seq_len=lens[b] + 4)
        req.kv_view()[:, :, :, :lens[b] - 1] = dev(prior).view(torch.bfloat16)
        req.tokens[lens[b] - 1] = 1000 * (b + 1)
        t = req.decode_step(lens[b])
        # the new token's K (rotated) and V rows of every layer
        kv_row = host(req.kv_view()[:, :, :, lens[b] - 1].contiguous().view(torch.int16)).copy()
        singles.append((t, host(req.logits).copy(), kv_row))
        del req
    data = torch.zeros(B, 4096, dtype=torch.bfloat16, device="cuda")
    attn = torch.zeros_like(data)
    logits = torch.zeros(B, 128256, dtype=torch.float32, device="cuda")
    out = torch.zeros(B, dtype=torch.int32, device="cuda")
    ws = torch.zeros(hip.lib.ie_batch_workspace_size(B), dtype=torch.uint8, device="cuda")
    seq = (C.c_int * B)(*lens)
    th = (C.c_int * B)()
    hip.check(hip.lib.ie_decode_step_batched(c.handle, model.ref(), B, seq, ptr(toks), ptr(data),
                                             ptr(attn), ptr(logits), ptr(out), th, ptr(ws),
                                             ptr(kvs)))
    torch.cuda.synchronize()
    for b in range(B):
        assert_close(host(logits[b]), singles[b][1], tol=e2e_tol(noise_floor),
                     what=f"batched row {b}")
        assert list(th)[b] == int(out[b].item()) == int(np.argmax(host(logits[b])))
        # the projection + RoPE + cache write fused into the batched QKV GEMM (RMSNorm applied
        # to the rows inside it, with the reference's two roundings) writes the same rows as the
        # single-sequence path: bf16-close at layer 0 (the two sum in different orders; RoPE's
        # a*c - b*s magnifies a rare 1-ulp product difference), within the end-to-end tolerance
        # through all 32 layers
        got_row = host(kvs.view(B, 32, 2, 8, 8192, 128)[b, :, :, :, lens[b] - 1].contiguous())
        assert_bf16_close(got_row[0], singles[b][2][0], ulps=2, what=f"batched kv row {b} layer 0",
                          outlier_frac=2e-3)
        assert_close(orc.bf16_to_f32(got_row), orc.bf16_to_f32(singles[b][2]),
                     tol=e2e_tol(noise_floor), what=f"batched kv row {b}")
    c.close()


# 40 / 100: the 64-weight-row streaming projections (64 and 128 X rows); 600: split-K MFMA tiles
# and 16-row attention workgroups; 1024: the last split-K size; 1100: unsplit projections, 16-row
# workgroups; 1800: the 32-row attention workgroups
@pytest.mark.parametrize("S", [17, 40, 64, 65, 100, 129, 600, 1024, 1100, 1800])
def test_prefill_paged_equals_contiguous(hip, model, S):
    """ie_prefill_paged (K/V rows into pages scattered over a pool) against ie_prefill (reference-
    layout cache): bit-identical logits and token, and every K/V row in its page."""
    from infengine_amd.engine import Context, ptr
    say(f"prefill_paged S={S}")
    c = Context(0, graph=False)
    page_elems = hip.lib.ie_kv_page_size() // 2
    nblk = (S + 63) // 64
    n_pages = nblk + 2
    order = np.random.default_rng(S).permutation(n_pages)[:nblk].astype(np.int32)
    pool = torch.zeros(n_pages * page_elems, dtype=torch.int16, device="cuda")
    kv = torch.zeros(hip.lib.ie_kv_cache_size() // 2, dtype=torch.int16, device="cuda")
    toks = torch.from_numpy(((np.arange(8192) * 7919 + 31) % 128256).astype(np.int32)).cuda()
    ws = torch.zeros(max(hip.lib.ie_attn_workspace_size(S), hip.lib.ie_ffn_workspace_size(S)),
                     dtype=torch.uint8, device="cuda")
    d_table = torch.from_numpy(order).cuda()
    outs = []
    for paged in (False, True):
        data = torch.zeros(S, 4096, dtype=torch.bfloat16, device="cuda")
        aux, attn = torch.zeros_like(data), torch.zeros_like(data)
        logits = torch.zeros(128256, dtype=torch.float32, device="cuda")
        out = torch.zeros(1, dtype=torch.int32, device="cuda")
        if paged:
            t = hip.lib.ie_prefill_paged(c.handle, model.ref(), S, ptr(toks), ptr(data), ptr(aux),
                                         ptr(attn), ptr(logits), ptr(out), ptr(ws), ptr(pool),
                                         n_pages, ptr(d_table))
        else:
            t = hip.lib.ie_prefill(c.handle, model.ref(), S, ptr(toks), ptr(data), ptr(aux),
                                   ptr(attn), ptr(logits), ptr(out), ptr(ws), ptr(kv))
        hip.check(t)
        outs.append((t, host(logits).copy()))
    assert outs[0][0] == outs[1][0] and np.array_equal(outs[0][1], outs[1][1])
    kv6 = kv.view(32, 2, 8, 8192, 128)
    pool6 = pool.view(n_pages, 32, 2, 8, 64, 128)
    for i in range(nblk):
        n = min(64, S - 64 * i)
        assert torch.equal(pool6[int(order[i]), :, :, :, :n], kv6[:, :, :, 64 * i:64 * i + n]), i
    c.close()


def test_batched_graph_replays_equal_eager(hip, ctx, model):
    """Batched steps replayed from captured graphs against the same steps launched eagerly, on
    paged caches: batches of 16 and 3 alternate (a graph per composition, reused), and sequence 0
    crosses the 2048-position switch of the attention path (a new capture); the next tokens are
    written back by eager device work between replays.  Every step's logits and tokens and the
    final pools bit-identical."""
    from infengine_amd.engine import Context, ptr
    B = 16
    lens0 = [2046] + [300 + 37 * b for b in range(1, B)]
    schedule = [16, 16, 3, 16, 3, 3, 16, 16]
    say(f"batched graph replays vs eager, schedule {schedule}")
    page_elems = hip.lib.ie_kv_page_size() // 2
    stride = (max(lens0) + len(schedule) + 63) // 64
    nblk = [(n + len(schedule) + 63) // 64 for n in lens0]
    n_pages = sum(nblk)
    tab = np.full((B, stride), -1, dtype=np.int32)
    first = np.cumsum([0] + nblk[:-1])
    for b in range(B):
        tab[b, :nblk[b]] = first[b] + np.arange(nblk[b])
    table = torch.from_numpy(tab).cuda()
    g = torch.Generator(device="cuda").manual_seed(SEED)
    pool0 = (torch.randn(n_pages * page_elems, device="cuda", generator=g) * 0.5).to(torch.bfloat16)
    toks0 = torch.randint(0, 128256, (B, stride * 64), dtype=torch.int32, device="cuda",
                          generator=g)
    runs = []
    for graph in (False, True):
        c = Context(0, graph=graph)
        pool = pool0.clone().view(torch.int16)
        toks = toks0.clone()
        ws = torch.zeros(hip.lib.ie_batch_workspace_size(B), dtype=torch.uint8, device="cuda")
        data = torch.zeros(B, 4096, dtype=torch.bfloat16, device="cuda")
        attn = torch.zeros_like(data)
        logits = torch.zeros(B, 128256, dtype=torch.float32, device="cuda")
        out = torch.zeros(B, dtype=torch.int32, device="cuda")
        lens = list(lens0)
        steps = []
        for nb in schedule:
            seq = (C.c_int * nb)(*lens[:nb])
            th = (C.c_int * nb)()
            hip.check(hip.lib.ie_decode_step_batched_paged(
                c.handle, model.ref(), nb, seq, ptr(toks), toks.shape[1], ptr(data), ptr(attn),
                ptr(logits), ptr(out), th, ptr(ws), ptr(pool), n_pages, ptr(table), stride))
            torch.cuda.synchronize()
            assert list(th) == host(out[:nb]).tolist()
            steps.append((host(logits[:nb]).copy(), list(th)))
            # eager device work between replays: the new tokens into the token rows
            rows = torch.arange(nb, device="cuda")
            cols = torch.tensor(lens[:nb], device="cuda", dtype=torch.long)
            toks[rows, cols] = out[:nb]
            for b in range(nb):
                lens[b] += 1
        runs.append((steps, pool))
        c.close()
    assert lens0[0] < 2049 <= lens0[0] + schedule.count(16) + schedule.count(3)
    for i, ((le, te), (lg, tg)) in enumerate(zip(runs[0][0], runs[1][0])):
        assert te == tg, f"step {i}: tokens differ"
        assert np.array_equal(le, lg), f"step {i}: logits differ"
    assert torch.equal(runs[0][1], runs[1][1]), "pools differ"
    torch.cuda.set_stream(ctx.stream)


def test_closing_graphed_contexts_frees_their_batched_graphs(hip, ctx, model):
    """Contexts that captured batched-step graphs (two batch compositions each) are created and
    closed six times: the device memory in use returns to where it started (ie_context_destroy
    destroys the cached graph executables with the context)."""
    from infengine_amd.engine import Context, ptr
    B, L = 4, 200
    say("graphed batched contexts: create, step (2 captures), close x6")
    kvs = torch.zeros(B * hip.lib.ie_kv_cache_size() // 2, dtype=torch.int16, device="cuda")
    toks = torch.zeros(B, 8192, dtype=torch.int32, device="cuda")
    ws = torch.zeros(hip.lib.ie_batch_workspace_size(B), dtype=torch.uint8, device="cuda")
    data = torch.zeros(B, 4096, dtype=torch.bfloat16, device="cuda")
    attn = torch.zeros_like(data)
    logits = torch.zeros(B, 128256, dtype=torch.float32, device="cuda")
    out = torch.zeros(B, dtype=torch.int32, device="cuda")

    def cycle():
        c = Context(0, graph=True)
        for nb in (B, 2, B):
            seq = (C.c_int * nb)(*[L] * nb)
            hip.check(hip.lib.ie_decode_step_batched(c.handle, model.ref(), nb, seq, ptr(toks),
                                                     ptr(data), ptr(attn), ptr(logits), ptr(out),
                                                     None, ptr(ws), ptr(kvs)))
        torch.cuda.synchronize()
        c.close()
        torch.cuda.synchronize()

    cycle()                                  # first-use allocations (module loads, pools)
    free0 = torch.cuda.mem_get_info()[0]
    for _ in range(6):
        cycle()
    grown = free0 - torch.cuda.mem_get_info()[0]
    say(f"  device memory in use grew by {grown / 2**20:.2f} MiB over 6 cycles")
    assert grown <= 4 << 20
    torch.cuda.set_stream(ctx.stream)


@pytest.mark.parametrize("lens", [[101, 257, 64], [2100, 257, 64], LENS16, LENS16_LONG])
def test_batched_paged_equals_contiguous(hip, model, lens):
    """ie_decode_step_batched_paged on a page pool (the sequences' 64-position blocks scattered
    over the pool in a random order) against ie_decode_step_batched on per-sequence caches:
    bit-identical logits and tokens, and the new K/V rows written into the right page rows."""
    from infengine_amd.engine import Context, ptr
    B = len(lens)
    say(f"decode_step_batched_paged B={B} lens={lens}")
    c = Context(0, graph=False)
    kvsz = hip.lib.ie_kv_cache_size()
    page_elems = hip.lib.ie_kv_page_size() // 2
    assert page_elems == 32 * 2 * 8 * 64 * 128
    kvs = torch.zeros(B * kvsz // 2, dtype=torch.int16, device="cuda")
    kv6 = kvs.view(B, 32, 2, 8, 8192, 128)
    toks = torch.zeros(B, 8192, dtype=torch.int32, device="cuda")
    for b in range(B):
        kv6[b, :, :, :, :lens[b] - 1] = dev(orc.synthetic((32, 2, 8, lens[b] - 1, 128), SEED,
                                                          2000 + b, 0.0, 1.0))
        toks[b, lens[b] - 1] = 700 * (b + 3)
    nblk = [(n + 63) // 64 for n in lens]
    n_pages = sum(nblk) + 3  # a few pages no table points at
    order = np.random.default_rng(SEED).permutation(n_pages)
    stride = max(nblk) + 1
    table = np.full((B, stride), -1, dtype=np.int32)
    pool = torch.zeros(n_pages * page_elems, dtype=torch.int16, device="cuda")
    pool6 = pool.view(n_pages, 32, 2, 8, 64, 128)
    k = 0
    for b in range(B):
        for i in range(nblk[b]):
            table[b, i] = order[k]
            pool6[order[k]] = kv6[b, :, :, :, 64 * i:64 * i + 64]
            k += 1
    d_table = torch.from_numpy(table).cuda()
    seq = (C.c_int * B)(*lens)
    outs = []
    for paged in (False, True):
        data = torch.zeros(B, 4096, dtype=torch.bfloat16, device="cuda")
        attn = torch.zeros_like(data)
        logits = torch.zeros(B, 128256, dtype=torch.float32, device="cuda")
        out = torch.zeros(B, dtype=torch.int32, device="cuda")
        ws = torch.zeros(hip.lib.ie_batch_workspace_size(B), dtype=torch.uint8, device="cuda")
        th = (C.c_int * B)()
        if paged:
            hip.check(hip.lib.ie_decode_step_batched_paged(
                c.handle, model.ref(), B, seq, ptr(toks), 8192, ptr(data), ptr(attn), ptr(logits),
                ptr(out), th, ptr(ws), ptr(pool), n_pages, ptr(d_table), stride))
        else:
            hip.check(hip.lib.ie_decode_step_batched(
                c.handle, model.ref(), B, seq, ptr(toks), ptr(data), ptr(attn), ptr(logits),
                ptr(out), th, ptr(ws), ptr(kvs)))
        torch.cuda.synchronize()
        outs.append((host(logits).copy(), list(th)))
    assert np.array_equal(outs[0][0], outs[1][0]), "paged logits differ from contiguous"
    assert outs[0][1] == outs[1][1]
    for b in range(B):
        pos = lens[b] - 1
        got = host(pool6[table[b, pos // 64], :, :, :, pos % 64].contiguous())
        want = host(kv6[b, :, :, :, pos].contiguous())
        assert got.any() and np.array_equal(got, want), f"new K/V row of sequence {b}"
    # pages no table entry points at are untouched
    for pid in order[sum(nblk):]:
        assert not host(pool6[int(pid)].reshape(-1)[:4096].contiguous()).any()
    c.close()


@pytest.mark.parametrize("graph", [False, True])
def test_generate_equals_manual_loop(hip, model, graph):
    """ie_generate (the Manager loop in the library, token write-back fused into the argmax)
    is bitwise identical to the reference loop driven from the host: ie_prefill, then
    ie_decode_step with a device-to-device write-back after each token (manager.cpp:70-86).
    Also covers the skipped position upload (the argmax advances it) and a decode step whose
    position does not follow the previous one."""
    from infengine_amd.engine import Context, Request
    S, N = 24, 6
    say(f"generate prompt={S} new={N} graph={graph} vs manual decode loop")
    rng = np.random.default_rng(77)
    ids = rng.integers(0, 128256, S).astype(np.int32)
    c = Context(0, graph=graph)
    a = Request(c, model, max_seq_len=S + N + 8)
    a.tokens[:S] = torch.from_numpy(ids).cuda()
    want = [a.prefill(S)]
    a.tokens[S] = a.token[0]
    for i in range(1, N):
        t = a.decode_step(S + i)
        a.tokens[S + i] = a.token[0]
        want.append(t)
    kv_want = host(a.kv.view(torch.int16).view(32, 2, 8, 8192, 128)[:, :, :, :S + N]).copy()
    logits_want = host(a.logits).copy()
    b = Request(c, model, max_seq_len=S + N + 8)
    got, ms = b.generate(ids, N, timed_from=2)
    assert got == want
    assert ms is not None and ms > 0
    assert host(b.tokens[:S + N]).tolist() == ids.tolist() + want[:N]
    assert np.array_equal(host(b.kv.view(torch.int16).view(32, 2, 8, 8192, 128)[:, :, :, :S + N]),
                          kv_want)
    assert np.array_equal(host(b.logits), logits_want)
    # a step at a position the previous step did not advance to still reads it (re-upload)
    t_again = b.decode_step(S + N - 1)
    assert t_again == want[N - 1]
    c.close()


def test_generate_stops_at_eos(hip, model):
    """ie_generate with an EOS id stops right after the first occurrence of that token (kept in
    the output), with the same tokens as the full run up to there; an EOS equal to the
    prefill's token ends the loop after the prefill."""
    from infengine_amd.engine import Context, Request
    S, N = 24, 10
    say(f"generate prompt={S} new={N} with EOS ids")
    ids = np.random.default_rng(78).integers(0, 128256, S).astype(np.int32)
    c = Context(0, graph=True)
    r = Request(c, model, max_seq_len=S + N + 8)
    full, _ = r.generate(ids, N)
    assert len(full) == N
    eos = full[5]
    stop = full.index(eos) + 1
    got, ms = r.generate(ids, N, timed_from=1, eos_token=eos)
    assert got == full[:stop]
    assert ms is not None and (ms > 0) == (stop > 1)
    assert host(r.tokens[S:S + stop]).tolist() == full[:stop]
    first, _ = r.generate(ids, N, eos_token=full[0])
    assert first == full[:1]
    c.close()
