"""Decode benchmark: random-init Llama-3.1-8B (bf16), batch 1, on one MI355X.

One timed "step" is one decode step of ie_generate, the library's Manager loop
(manager.cpp:60-86): decode.cuh:6-9 semantics (embed the last token, 32 layers,
final norm, lm_head, argmax, token returned to the host) plus the reference's
device-side token write-back (manager.cpp:84).  The KV cache is first filled by
the loop's prefill over a random prompt, so the timed steps run at real positions
(prompt_len + warmup .. prompt_len + warmup + steps - 1).

Also reported, on the same run:
  roofline      the dominant decode kernel (fused RMSNorm -> gate/up GEMV -> SwiGLU,
                234,926,080 algorithmic bytes per launch), timed with HIP events
                on the stream it runs on, rotating over the 32 layers' weights so
                the 256 MB Infinity Cache cannot serve repeats.
  batched       config 5's bs=16 leg: 16 independent sequences (staggered contexts
                from prompt_len+1) per ie_decode_step_batched, tokens/s and GB/s.
  batched_paged the same leg over a paged KV pool (ie_decode_step_batched_paged, each
                sequence's 64-position blocks on shuffled pages).
  prefill_2048  config 4: a 2048-token prefill of the full model (mean of 3 after three
                untimed calls), and the four prefill GEMM shapes at M = 2048 (QKV, O with
                residual, gate/up with SwiGLU, down with residual) timed with HIP events
                on the engine stream after 150 ms of warm-up (median of 3 runs of 10
                launches), as TFLOP/s and fraction of the 2.5 PFLOP/s dense bf16 MFMA peak,
                with torch.matmul (hipBLASLt) on the same shapes and protocol beside them.
  prefill_64    a 64-token prefill (mean of 3 warm calls): every weight is read once, so it
                is reported against HBM as the weight bytes (32 layers + lm_head) per second.
  cpu_baseline  the CPU oracle (oracle/, OpenMP) decoding the same model on this
                host: whole decode steps (32 layers + lm_head + argmax) for about
                10 s after one untimed step.

    python bench.py [--gpus 1] [--steps 128] [--warmup 16] [--prompt 512]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HIDDEN, FFN, VOCAB, LAYERS = 4096, 14336, 128256, 32
WEIGHT_BYTES_PER_TOKEN = 15_009_849_344          # every weight byte read once per bs=1 step
KV_BYTES_PER_POS = 131_072                       # 32 layers x (K+V) x 8 heads x 128 x 2 B
GATE_UP_BYTES = 2 * FFN * HIDDEN * 2 + 2 * HIDDEN * 2 + FFN * 2
HBM_PEAK_GBPS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0                   # dense bf16 MFMA, MI355X
LAYER_GEMM_PARAMS = (6144 + 4096 + 2 * FFN) * HIDDEN + HIDDEN * FFN   # QKV, O, gate+up, down


def prefill_gemm_flops(P: int) -> float:
    """Flops of the layer products an ie_prefill of P tokens runs: 31 layers over P rows, then
    the last layer's QKV over P rows (its K/V cache rows) and its O, gate/up and down products
    over the last row only (the one row the final norm and lm_head read)."""
    qkv = 6144 * HIDDEN
    return 2.0 * (P * LAYER_GEMM_PARAMS * (LAYERS - 1) + P * qkv + (LAYER_GEMM_PARAMS - qkv))
# HBM bytes per gate/up launch from rocprofv3 FETCH_SIZE (x2.000) + WRITE_SIZE (x1.000), each
# factor calibrated on a 256 MiB copy; profiles/decode_gemv_hbm_traffic.md.
GATE_UP_TRAFFIC = 235_190_000


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def cpu_baseline(prompt: int, budget_s: float = 10.0) -> dict:
    """The oracle decoding the same model on this host: full decode steps
    (embedding, 32 decoder layers, final norm, lm_head, argmax) at positions
    prompt, prompt+1, ... against a synthetic KV prefix, for about budget_s
    seconds.  Weights are generated once beforehand and not timed."""
    import numpy as np

    import oracle as orc
    threads = int(os.environ.get("OMP_NUM_THREADS", len(os.sched_getaffinity(0))))
    threads = min(threads, len(os.sched_getaffinity(0)))
    seed = 0
    cos, sin = orc.rope_tables()
    layers = [orc.layer_weights(seed, l) for l in range(LAYERS)]
    emb = orc.embedding(seed)
    lm = orc.lm_head_weight(seed)
    fn = orc.final_norm(seed)
    cap = prompt + 1024
    kv = np.zeros((LAYERS, 2, 8, cap, 128), np.uint16)
    kv[:, :, :, :prompt] = orc.synthetic((LAYERS, 2, 8, prompt, 128), seed, 9000, 0.0, 1.0)

    def step(tok: int, pos: int) -> int:
        x = orc.emblookup(np.array([tok], np.int32), emb)
        for l in range(LAYERS):
            orc.decoder_layer(x, layers[l], pos, cos, sin, kv[l, 0], kv[l, 1], cap)
        return orc.argmax(orc.matmul(orc.rmsnorm(x, fn), lm, out_f32=True)[0])

    tok = step(1234, prompt)             # untimed: first touch of every weight page
    pos, n = prompt + 1, 0
    t0 = time.perf_counter()
    while n < 2 or (time.perf_counter() - t0 < budget_s and pos + 1 < cap):
        tok = step(tok, pos)
        pos += 1
        n += 1
    dt = time.perf_counter() - t0
    return {"value": round(n / dt, 4), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"{n} full oracle decode steps (32 layers + lm_head + argmax) at positions "
                      f"{prompt + 1}..{pos - 1} after one untimed step, {dt:.1f} s on "
                      f"{threads} threads"}


def cpu_config_legs(budget_s: float = 2.0) -> dict:
    """The oracle on configs 1-4 on this host (same thread count as cpu_baseline), each repeated
    for about budget_s seconds after one untimed call; inputs generated beforehand, not timed.
    Configs 1-3 in full; config 4 (2048-token prefill of 32 layers) from one layer at 256 rows,
    extrapolated by flop count (linear products, causal attention, the last row's lm_head).
    Threads: OpenMP's default (the host's cores available to this process)."""
    import numpy as np

    import oracle as orc
    seed = 0
    cos, sin = orc.rope_tables()
    w = orc.layer_weights(seed, 5)
    x = orc.synthetic((1, HIDDEN), seed, 77, 0.0, 1.0)

    def timed(fn, min_n: int = 2) -> float:
        fn()
        n, t0 = 0, time.perf_counter()
        while n < min_n or time.perf_counter() - t0 < budget_s:
            fn()
            n += 1
        return (time.perf_counter() - t0) / n

    def c1() -> None:
        xn = orc.rmsnorm(x, w["post_attention_layernorm"])
        orc.residual_add(x, orc.ffn(xn, w["w_gate"], w["w_up"], w["w_down"]))

    P = 2047
    planes = np.zeros((2, 8, P + 1, 128), np.uint16)
    planes[:, :, :P] = orc.synthetic((2, 8, P, 128), seed, 78, 0.0, 1.0)

    def c2() -> None:
        orc.decoder_layer(x.copy(), w, P, cos, sin, planes[0], planes[1], P + 1)

    lm, fn = orc.lm_head_weight(seed), orc.final_norm(seed)
    x16 = orc.synthetic((16, HIDDEN), seed, 79, 0.0, 1.0)

    def c3(rows) -> None:
        logits = orc.matmul(orc.rmsnorm(rows, fn), lm, out_f32=True)
        for r in range(rows.shape[0]):
            orc.argmax(logits[r])
            orc.top_p(logits[r], 0.7, 0.9, 1234, r, 0)

    S4 = 128
    x4 = orc.synthetic((S4, HIDDEN), seed, 80, 0.0, 1.0)
    p4 = np.zeros((2, 8, S4, 128), np.uint16)

    def c4() -> None:
        orc.decoder_layer(x4.copy(), w, 0, cos, sin, p4[0], p4[1], S4)

    def layer_flops(S: int) -> float:
        return 2.0 * S * (LAYER_GEMM_PARAMS) + 4.0 * 32 * 128 * S * (S + 1) / 2

    t1, t2, t3a, t3b = timed(c1), timed(c2), timed(lambda: c3(x)), timed(lambda: c3(x16))
    t4 = timed(c4, 1)
    t4_full = t4 * (LAYERS * layer_flops(2048) + 2.0 * VOCAB * HIDDEN) / layer_flops(S4)
    return {"config1_ffn_block_us": round(t1 * 1e6, 1), "config2_layer_us": round(t2 * 1e6, 1),
            "config3_b1_us": round(t3a * 1e6, 1), "config3_b16_us": round(t3b * 1e6, 1),
            "config4_prefill_2048_ms": round(t4_full * 1e3, 1),
            "config4_sample": f"one layer at {S4} rows ({t4 * 1e3:.1f} ms), extrapolated by flops",
            "cores": len(os.sched_getaffinity(0)), "kind": "port"}


def calibration_copy(nbytes: int = 256 << 20) -> None:
    """A plain device-to-device copy of known size, for scaling the HBM
    FETCH_SIZE / WRITE_SIZE counters of a --pmc run."""
    import torch
    src = torch.ones(nbytes // 4, dtype=torch.int32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(4):
        dst.copy_(src)
    torch.cuda.synchronize()


def timed_launches(stream, fn) -> float:
    """Microseconds per call of fn, timed with HIP events on `stream`. The clocks settle over the
    first ~0.1 s of sustained MFMA load (a cold launch runs 10-15 % slow), as they do inside a
    prefill's 32 back-to-back layers: warm up for 150 ms, then take the median of three timed
    runs of 10 launches."""
    import torch

    t_end = time.perf_counter() + 0.15
    while time.perf_counter() < t_end:
        for _ in range(8):
            fn()
        torch.cuda.synchronize()
    runs = []
    for _ in range(3):
        g0, g1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        g0.record(stream)
        for _ in range(10):
            fn()
        g1.record(stream)
        g1.synchronize()
        runs.append(g0.elapsed_time(g1) * 1e3 / 10)
    return sorted(runs)[1]


def prefill_attention(ctx, S: int) -> dict:
    """One layer's causal flash attention at S query rows (start 0) through
    ie_attn_prefill_core, timed like the GEMMs: 4 * 32 * 128 * S (S + 1) / 2 flop of causal
    work against the bf16 MFMA peak."""
    import torch

    from infengine_amd import check, lib
    from infengine_amd.engine import ptr

    q = torch.randn(S, 32, 128, device="cuda").to(torch.bfloat16)
    k = torch.randn(8, 8192, 128, device="cuda").to(torch.bfloat16)
    v = torch.randn(8, 8192, 128, device="cuda").to(torch.bfloat16)
    out = torch.empty(S, HIDDEN, dtype=torch.bfloat16, device="cuda")
    torch.cuda.synchronize()
    us = timed_launches(ctx.stream, lambda: check(lib.ie_attn_prefill_core(
        ctx.handle, S, 0, ptr(q), ptr(k), ptr(v), ptr(out))))
    flop = 4.0 * 32 * 128 * S * (S + 1) / 2
    tf = flop / (us * 1e-6) / 1e12
    del q, k, v, out
    return {"seq_len": S, "us": round(us, 1), "tflops": round(tf, 1),
            "frac": round(tf / MFMA_BF16_PEAK_TFLOPS, 4)}


def prefill_gemms(ctx, P: int) -> dict:
    """The four prefill GEMM shapes at M = P (QKV, O with residual, gate/up with SwiGLU, down with
    residual) through ie_gemm_ex, and the same products through torch.matmul (hipBLASLt), each
    timed with HIP events on the engine stream after 150 ms of warm-up (median of 3 runs of 10
    launches)."""
    import torch

    from infengine_amd import check, lib
    from infengine_amd.engine import ptr

    def timed(fn) -> float:
        return timed_launches(ctx.stream, fn)

    gemms = {}
    for name, epi, k, n in (("qkv", 0, HIDDEN, 6144), ("o", 1, HIDDEN, HIDDEN),
                            ("gate_up", 3, HIDDEN, FFN), ("down", 1, FFN, HIDDEN)):
        gx = (torch.randn(P, k, device="cuda") * 0.5).to(torch.bfloat16)
        gw0 = (torch.randn(n, k, device="cuda") * 0.02).to(torch.bfloat16)
        gw1 = (torch.randn(n, k, device="cuda") * 0.02).to(torch.bfloat16) if epi == 3 else gw0
        gy = torch.zeros(P, n, dtype=torch.bfloat16, device="cuda")
        torch.cuda.synchronize()

        def run() -> None:
            check(lib.ie_gemm_ex(ctx.handle, epi, P, k, n, ptr(gx), ptr(gw0), ptr(gw1), ptr(gy)))

        us = timed(run)
        flop = 2.0 * P * n * k * (2 if epi == 3 else 1)
        tf = flop / (us * 1e-6) / 1e12
        # the same product through torch.matmul (hipBLASLt), same protocol: gate and up as
        # one [2 * 14336, 4096] weight, no fused epilogue
        gw = torch.cat([gw0, gw1]) if epi == 3 else gw0
        ref_us = timed(lambda: torch.matmul(gx, gw.t()))
        gemms[name] = {"m": P, "n": n, "k": k, "us": round(us, 1), "tflops": round(tf, 1),
                       "frac": round(tf / MFMA_BF16_PEAK_TFLOPS, 4),
                       "torch_matmul_us": round(ref_us, 1),
                       "torch_matmul_tflops": round(flop / (ref_us * 1e-6) / 1e12, 1)}
        del gx, gw0, gw1, gy, gw
    return gemms


def config_legs(ctx, W, iters: int = 32) -> dict:
    """BASELINE configs 1-3 timed alone with HIP events on the engine stream: 8 untimed launches,
    then `iters` launches rotating through the 32 layers' weights (config 3: through two
    [128256][4096] tables, the lm_head and the embedding), so the 256 MB Infinity Cache cannot
    serve repeats.  Bytes are the algorithmic weight (+ K/V) bytes per launch.
      config1  the FFN block of one decode token (ie_ffn_block_decode): RMSNorm, gate/up GEMV +
               SwiGLU, down GEMV + residual
      config2  one decoder layer decode step at position 2047 over 2047 cached K/V rows
               (ie_decoder_layer_decode)
      config3  final RMSNorm + lm_head to fp32 logits, argmax, temperature 0.7 / top-p 0.9
               sampling: B = 1 (the decode step's GEMV) and B = 16 (the batched step's RMSNorm +
               skinny MFMA product)"""
    import ctypes as C

    import torch

    from infengine_amd import check, lib
    from infengine_amd.engine import ptr

    st = ctx.stream

    def timed(launch) -> float:
        for i in range(8):
            launch(i)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(st)
        for i in range(iters):
            launch(8 + i)
        e1.record(st)
        e1.synchronize()
        return e0.elapsed_time(e1) * 1e3 / iters

    def leg(us: float, nbytes: int) -> dict:
        gbps = nbytes / (us * 1e-6) / 1e9
        return {"us": round(us, 2), "bytes": nbytes, "GBps": round(gbps, 1),
                "hbm_frac": round(gbps / HBM_PEAK_GBPS, 4)}

    L = W.s.layers
    ws = torch.zeros(lib.ie_batch_workspace_size(16), dtype=torch.uint8, device="cuda")
    x = (torch.randn(1, HIDDEN, device="cuda")).to(torch.bfloat16)
    x0 = x.clone()

    def ffn(i: int) -> None:
        l = L[i % LAYERS]
        check(lib.ie_ffn_block_decode(ctx.handle, ptr(x), C.c_void_p(l.post_attention_layernorm),
                                      C.c_void_p(l.ffn_block.w_gate), C.c_void_p(l.ffn_block.w_up),
                                      C.c_void_p(l.ffn_block.w_down), ptr(ws)))
        if i % LAYERS == LAYERS - 1:
            x.copy_(x0)           # keep the residual stream at unit scale
    c1 = leg(timed(ffn), 3 * FFN * HIDDEN * 2 + 2 * HIDDEN * 2)

    pos = 2047
    kv = torch.zeros(lib.ie_kv_cache_size() // 2, dtype=torch.int16, device="cuda")
    kv6 = kv.view(LAYERS, 2, 8, 8192, 128)
    for l in range(LAYERS):
        kv6[l, :, :, :pos] = torch.randn(2, 8, pos, 128, device="cuda").to(torch.bfloat16).view(torch.int16)
    attn = torch.zeros(1, HIDDEN, dtype=torch.bfloat16, device="cuda")

    def layer(i: int) -> None:
        check(lib.ie_decoder_layer_decode(ctx.handle, W.ref(), i % LAYERS, pos + 1, ptr(x),
                                          ptr(attn), ptr(ws), ptr(kv)))
        if i % LAYERS == LAYERS - 1:
            x.copy_(x0)
    layer_w = (HIDDEN * HIDDEN * 2 + 2 * 1024 * HIDDEN + 3 * FFN * HIDDEN + 2 * HIDDEN) * 2
    c2 = leg(timed(layer), layer_w + KV_BYTES_PER_POS // LAYERS * (pos + 1))
    del kv, kv6

    tables = (W.s.lm_head, W.s.emb_lookup)
    c3 = {}
    for B in (1, 16):
        xb = torch.randn(B, HIDDEN, device="cuda").to(torch.bfloat16)
        xn = torch.empty_like(xb)
        logits = torch.empty(B, VOCAB, dtype=torch.float32, device="cuda")
        out = torch.zeros(B, dtype=torch.int32, device="cuda")
        out2 = torch.zeros(B, dtype=torch.int32, device="cuda")
        tws = torch.zeros(lib.ie_top_p_workspace_size(B, VOCAB), dtype=torch.uint8, device="cuda")

        def head(i: int, B=B, xb=xb, xn=xn, logits=logits, out=out, out2=out2, tws=tws) -> None:
            table = C.c_void_p(tables[i % 2])
            if B == 1:
                check(lib.ie_final_norm_lm_head(ctx.handle, 1, ptr(xb), C.c_void_p(W.s.final_norm),
                                                table, ptr(logits)))
                check(lib.ie_sample_token_amax(ctx.handle, ptr(logits), ptr(out)))
            else:
                check(lib.ie_rmsnorm(B, ptr(xb), C.c_void_p(W.s.final_norm), ptr(xn), ptr_stream))
                check(lib.ie_gemm_ex(ctx.handle, 2, B, HIDDEN, VOCAB, ptr(xn), table, table,
                                     ptr(logits)))
                check(lib.ie_sample_argmax_rows(ctx.handle, B, VOCAB, ptr(logits), ptr(out)))
            check(lib.ie_sample_top_p(ctx.handle, B, VOCAB, ptr(logits), 0.7, 0.9, 1234, i,
                                      ptr(out2), ptr(tws)))
        ptr_stream = C.c_void_p(st.cuda_stream)
        c3[f"b{B}"] = leg(timed(head), VOCAB * HIDDEN * 2 + HIDDEN * 2)
        del xb, xn, logits, out, out2, tws
    return {"config1_ffn_block": c1, "config2_layer_pos2047": c2, "config3_head_sampling": c3,
            "iters": iters}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--prompt", type=int, default=512)
    ap.add_argument("--kernel-iters", type=int, default=64)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--batch", type=int, default=16, help="batched-decode sequences (1: skip)")
    ap.add_argument("--batch-steps", type=int, default=32)
    ap.add_argument("--prefill-len", type=int, default=2048,
                    help="config 4 prefill leg and its GEMM roofline (0: skip)")
    ap.add_argument("--gemm-only", action="store_true",
                    help="only the prefill GEMM shapes at M = --prefill-len, ours and torch.matmul "
                         "(for profiling them); prints their JSON")
    ap.add_argument("--attn-only", action="store_true",
                    help="only the prefill attention at S = --prefill-len (for profiling it); "
                         "prints its JSON")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only the --prefill-len prefill of the full model, 3 untimed + 3 timed "
                         "(for a kernel trace of whole prefills); prints its JSON")
    ap.add_argument("--no-config-legs", action="store_true",
                    help="skip the configs 1-3 legs (GPU) and the per-config CPU figures")
    ap.add_argument("--calibration-copy", action="store_true",
                    help="also run a 256 MiB device copy (counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported in this build "
              "(the single-GPU path is the whole deliverable of this build)",
              file=sys.stderr)
        return 2

    import ctypes as C

    import numpy as np
    import torch

    from infengine_amd import check, lib
    from infengine_amd.engine import Context, ModelWeights, Request, ptr

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    torch.cuda.set_device(0)
    if args.calibration_copy:
        calibration_copy()
    ctx = Context(0, graph=not args.no_graph)
    if args.gemm_only:
        print(json.dumps({"prefill_gemm": prefill_gemms(ctx, args.prefill_len or 2048)}), flush=True)
        ctx.close()
        return 0
    if args.attn_only:
        print(json.dumps({"prefill_attention": prefill_attention(ctx, args.prefill_len or 2048)}),
              flush=True)
        ctx.close()
        return 0
    if args.prefill_only:
        P = args.prefill_len or 2048
        W = ModelWeights.random_init(seed=0, std=0.02)
        req = Request(ctx, W, max_seq_len=P + 8)
        req.tokens[:P] = torch.from_numpy(
            np.random.default_rng(0).integers(0, VOCAB, P).astype(np.int32)).cuda()
        for _ in range(3):
            req.prefill(P)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(3):
            tok = req.prefill(P)
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) / 3 * 1e3
        flops = prefill_gemm_flops(P)
        print(json.dumps({"prefill": {"seq_len": P, "ms": round(ms, 3), "token": tok,
                                      "layer_gemm_tflops_per_s": round(flops / ms / 1e9, 1)}}),
              flush=True)
        del req
        W.free()
        ctx.close()
        return 0
    log("random-init weights (16.06 GB)")
    W = ModelWeights.random_init(seed=0, std=0.02)
    total = args.prompt + args.warmup + args.steps + 1
    req = Request(ctx, W, max_seq_len=total + 8)
    rng = np.random.default_rng(0)
    ids = rng.integers(0, VOCAB, args.prompt).astype(np.int32)
    req.tokens[: args.prompt] = torch.from_numpy(ids).cuda()

    log(f"prefill {args.prompt} tokens")
    req.prefill(args.prompt)          # untimed first call (code loading, clocks)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    tok = req.prefill(args.prompt)
    prefill_s = time.perf_counter() - t0
    req.tokens[args.prompt] = tok

    # ---- decode: the Manager loop (manager.cpp:60-86) in the library: prefill, then decode
    # steps, each with its device-side token write-back (manager.cpp:84) and the token returned
    # to the host; steps 1..warmup are untimed
    n_new = 1 + args.warmup + args.steps
    toks, timed_ms = req.generate(ids, n_new, timed_from=1 + args.warmup)
    assert toks[0] == tok, "ie_generate's prefill token differs from ie_prefill's"
    assert len(toks) == n_new, "ie_generate stopped early"
    first_pos = args.prompt + args.warmup          # position of the first timed step's token
    last_pos = args.prompt + args.warmup + args.steps - 1
    dt = timed_ms / 1e3
    ms_per_step = dt * 1e3 / args.steps
    tok_s = args.steps / dt
    kv_bytes = KV_BYTES_PER_POS * sum(p + 1 for p in range(first_pos, last_pos + 1)) / args.steps
    step_gbps = (WEIGHT_BYTES_PER_TOKEN + kv_bytes) / (dt / args.steps) / 1e9

    # ---- batched decode (config 5): 16 independent sequences per step, one KV cache each
    batched = batched_paged = None
    if args.batch > 1:
        B = args.batch
        log(f"batched decode B={B}")
        kvs = torch.zeros(B * lib.ie_kv_cache_size() // 2, dtype=torch.int16, device="cuda")
        toks = torch.randint(0, VOCAB, (B, 8192), dtype=torch.int32, device="cuda")
        bdata = torch.zeros(B, HIDDEN, dtype=torch.bfloat16, device="cuda")
        battn = torch.zeros_like(bdata)
        blogits = torch.zeros(B, VOCAB, dtype=torch.float32, device="cuda")
        bout = torch.zeros(B, dtype=torch.int32, device="cuda")
        bws = torch.zeros(lib.ie_batch_workspace_size(B), dtype=torch.uint8, device="cuda")
        th = (C.c_int * B)()
        # the same leg on a paged KV pool: each sequence's 64-position blocks on pages in a
        # shuffled order (ie_decode_step_batched_paged)
        last = args.prompt + B + 4 + args.batch_steps
        nblk = (last + 63) // 64
        pool = torch.zeros(B * nblk * lib.ie_kv_page_size() // 2, dtype=torch.int16, device="cuda")
        table = torch.from_numpy(np.random.default_rng(7).permutation(B * nblk).astype(np.int32)
                                 .reshape(B, nblk)).cuda()

        def run_leg(paged: bool) -> dict:
            lens = [args.prompt + 1 + b for b in range(B)]     # staggered contexts

            def bstep() -> None:
                seq = (C.c_int * B)(*lens)
                if paged:
                    check(lib.ie_decode_step_batched_paged(
                        ctx.handle, W.ref(), B, seq, ptr(toks), toks.shape[1], ptr(bdata), ptr(battn),
                        ptr(blogits), ptr(bout), th, ptr(bws), ptr(pool), B * nblk, ptr(table),
                        nblk))
                else:
                    check(lib.ie_decode_step_batched(ctx.handle, W.ref(), B, seq, ptr(toks),
                                                     ptr(bdata), ptr(battn), ptr(blogits),
                                                     ptr(bout), th, ptr(bws), ptr(kvs)))
                for b in range(B):
                    lens[b] += 1

            for _ in range(4):
                bstep()
            torch.cuda.synchronize()
            kv_b = KV_BYTES_PER_POS * sum(lens)
            t0 = time.perf_counter()
            for _ in range(args.batch_steps):
                bstep()
            torch.cuda.synchronize()
            bdt = (time.perf_counter() - t0) / args.batch_steps
            kv_b = (kv_b + KV_BYTES_PER_POS * sum(lens)) / 2          # mean over the timed steps
            return {"batch": B, "steps": args.batch_steps, "tokens_per_s": round(B / bdt, 1),
                    "ms_per_step": round(bdt * 1e3, 4),
                    "step_GBps": round((WEIGHT_BYTES_PER_TOKEN + kv_b) / bdt / 1e9, 1),
                    "contexts": [args.prompt + 5, lens[-1]]}

        batched = run_leg(False)
        log(f"batched decode B={B}, paged KV")
        batched_paged = run_leg(True)
        del pool, table
        del kvs, toks, bdata, battn, blogits, bout, bws

    # ---- configs 1-3, each timed alone
    configs = None
    if not args.no_config_legs:
        log("configs 1-3 (FFN block, one layer at position 2047, head + sampling)")
        configs = config_legs(ctx, W)

    # ---- config 4: 2048-token prefill, and its four GEMM shapes against the MFMA peak
    prefill2048 = None
    if args.prefill_len > 0:
        P = args.prefill_len
        log(f"prefill {P} tokens")
        req2 = Request(ctx, W, max_seq_len=P + 8)
        req2.tokens[:P] = torch.from_numpy(rng.integers(0, VOCAB, P).astype(np.int32)).cuda()
        for _ in range(3):                                # untimed: allocation, clocks
            req2.prefill(P)
        torch.cuda.synchronize()
        reps = 3
        t0 = time.perf_counter()
        for _ in range(reps):
            req2.prefill(P)
        torch.cuda.synchronize()
        pdt = (time.perf_counter() - t0) / reps
        del req2
        gemms = prefill_gemms(ctx, P)
        attention = prefill_attention(ctx, P)
        flops = prefill_gemm_flops(P)
        prefill2048 = {"seq_len": P, "ms": round(pdt * 1e3, 2), "tokens_per_s": round(P / pdt, 1),
                       "layer_gemm_tflops_per_s": round(flops / pdt / 1e12, 1),
                       "gemm": gemms, "attention": attention,
                       "mfma_peak_tflops": MFMA_BF16_PEAK_TFLOPS}

    # ---- a short prompt (64 tokens): every weight read once, so the prefill is HBM-bound;
    # warm calls (two untimed, then the mean of three), bytes = the 32 layers' products + lm_head
    log("prefill 64 tokens")
    P64 = 64
    req3 = Request(ctx, W, max_seq_len=P64 + 8)
    req3.tokens[:P64] = torch.from_numpy(rng.integers(0, VOCAB, P64).astype(np.int32)).cuda()
    for _ in range(2):
        req3.prefill(P64)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(3):
        req3.prefill(P64)
    torch.cuda.synchronize()
    p64 = (time.perf_counter() - t0) / 3
    del req3
    w_bytes = 2 * (LAYERS * LAYER_GEMM_PARAMS + VOCAB * HIDDEN)
    prefill64 = {"seq_len": P64, "ms": round(p64 * 1e3, 3), "tokens_per_s": round(P64 / p64, 1),
                 "weight_GBps": round(w_bytes / p64 / 1e9, 1),
                 "weight_hbm_frac": round(w_bytes / p64 / 1e9 / HBM_PEAK_GBPS, 4)}

    # ---- dominant kernel, timed live on its own stream with HIP events
    log("gate/up GEMV kernel timing")
    h = torch.empty(FFN, dtype=torch.bfloat16, device="cuda")
    x = req.data[0]
    launches = []
    for i in range(args.kernel_iters + 8):
        L = W.s.layers[i % LAYERS]
        launches.append((L.post_attention_layernorm, L.ffn_block.w_gate, L.ffn_block.w_up))
    stream = ctx.stream
    for (nw, wg, wu) in launches[:8]:
        check(lib.ie_ffn_gate_up_decode(ctx.handle, ptr(x), C.c_void_p(nw), C.c_void_p(wg),
                                        C.c_void_p(wu), ptr(h)))
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for (nw, wg, wu) in launches[8:]:
        check(lib.ie_ffn_gate_up_decode(ctx.handle, ptr(x), C.c_void_p(nw), C.c_void_p(wg),
                                        C.c_void_p(wu), ptr(h)))
    e1.record(stream)
    e1.synchronize()
    k_us = e0.elapsed_time(e1) * 1e3 / args.kernel_iters
    k_gbps = GATE_UP_BYTES / (k_us * 1e-6) / 1e9

    out = {
        "metric": "decode tokens/s + weight-stream HBM GB/s (% of 8 TB/s), Llama-3.1-8B bs=1",
        "value": round(tok_s, 3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init weights ~N(0,0.02), random prompt ids)",
        "config": {"workload": "llama-3.1-8b decode step, batch 1, 32 layers, random-init bf16",
                   "batch": 1, "prompt_len": args.prompt,
                   "decode_positions": [first_pos, last_pos],
                   "graph": not args.no_graph},
        "step_GBps": round(step_gbps, 1),
        "step_hbm_frac": round(step_gbps / HBM_PEAK_GBPS, 4),
        "prefill": {"seq_len": args.prompt, "ms": round(prefill_s * 1e3, 2),
                    "tokens_per_s": round(args.prompt / prefill_s, 1), "call": "second (warm)"},
        "batched": batched,
        "batched_paged": batched_paged,
        "configs": configs,
        "prefill_2048": prefill2048,
        "prefill_64": prefill64,
        "roofline": {"bound": "hbm", "kernel": "gemv_kernel<4096, SwiGLU, RMSNorm> (gate/up)",
                     "achieved": round(k_gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(k_gbps / HBM_PEAK_GBPS, 4), "traffic": GATE_UP_TRAFFIC,
                     "traffic_source": "rocprofv3 --pmc FETCH_SIZE (x2.000) and WRITE_SIZE "
                                       "(x1.000) per dispatch, factors from a 256 MiB copy: "
                                       "profiles/decode_gemv_hbm_traffic.md",
                     "avg_launch_us": round(k_us, 2), "bytes_per_launch": GATE_UP_BYTES},
    }
    del req
    W.free()
    ctx.close()
    torch.cuda.synchronize()
    if not args.no_cpu_baseline:
        log("cpu baseline (oracle)")
        out["cpu_baseline"] = cpu_baseline(args.prompt)
        if not args.no_config_legs:
            log("cpu configs 1-4 (oracle)")
            cpu = cpu_config_legs()
            out["cpu_configs"] = cpu
            if configs is not None:
                configs["config1_ffn_block"]["cpu_us"] = cpu["config1_ffn_block_us"]
                configs["config2_layer_pos2047"]["cpu_us"] = cpu["config2_layer_us"]
                configs["config3_head_sampling"]["b1"]["cpu_us"] = cpu["config3_b1_us"]
                configs["config3_head_sampling"]["b16"]["cpu_us"] = cpu["config3_b16_us"]
            if prefill2048 is not None:
                prefill2048["cpu_ms_extrapolated"] = cpu["config4_prefill_2048_ms"]
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
