"""GPU parity of every hot-path op, called through the C-ABI, against the CPU
oracle on the same seeded inputs at the BASELINE shapes.

Bars: bit-exact for byte/index work (synthetic generator, embedding rows,
residual add, KV-cache row placement, argmax ids); tests/tolerance.py
(max-abs / rel <= 1e-2, fp32 accumulation) for floating point.
"""
import ctypes as C
import pathlib

import numpy as np
import pytest
import torch

import oracle as orc
from gpu_util import (P, assert_bf16_close, assert_delta_close, bf16_empty, bf16_zeros, dev, host,
                      say, ulp_diff)
from tolerance import assert_close

pytestmark = pytest.mark.gpu
GOLD = pathlib.Path(__file__).resolve().parent / "golden"
H, F, V = 4096, 14336, 128256


@pytest.fixture(scope="module")
def rope():
    cos, sin = orc.rope_tables()
    return cos, sin, dev(cos), dev(sin)


def sync():
    torch.cuda.synchronize()


# ---------------------------------------------------------------- generator / gathers
def test_synthetic_generator_bit_exact(hip, ctx):
    n = 3_000_007
    say(f"fill_synthetic n={n}")
    out = bf16_empty(n)
    hip.check(hip.lib.ie_fill_synthetic_bf16(P(out), n, 77, 5, 0.0, 0.02, ctx.stream_ptr))
    sync()
    assert np.array_equal(host(out), orc.synthetic((n,), 77, 5, 0.0, 0.02))


def test_emblookup_bit_exact(hip, ctx):
    say("emblookup 128 ids over the full [128256, 4096] table")
    table = orc.synthetic((V, H), 3, 1, 0.0, 0.02)
    rng = np.random.default_rng(0)
    ids = rng.integers(0, V, 128).astype(np.int32)
    ids[:3] = [0, V - 1, 12345]
    d_table, d_ids, out = dev(table), dev(ids), bf16_empty(128, H)
    hip.check(hip.lib.ie_emblookup(128, P(d_ids), P(d_table), P(out), ctx.stream_ptr))
    sync()
    assert np.array_equal(host(out), orc.emblookup(ids, table))
    # out-of-range ids give a zero row instead of reading outside the table
    bad = dev(np.array([-1, V], np.int32))
    out2 = bf16_empty(2, H).fill_(7)
    hip.check(hip.lib.ie_emblookup(2, P(bad), P(d_table), P(out2), ctx.stream_ptr))
    sync()
    assert not host(out2).any()


# ---------------------------------------------------------------- elementwise
def test_rmsnorm(hip, ctx):
    say("rmsnorm [128, 4096]")
    x = orc.synthetic((128, H), 4, 1, 0.0, 1.0)
    w = orc.synthetic((H,), 4, 2, 1.0, 0.02)
    out = bf16_empty(128, H)
    hip.check(hip.lib.ie_rmsnorm(128, P(dev(x)), P(dev(w)), P(out), ctx.stream_ptr))
    sync()
    got, want = host(out), orc.rmsnorm(x, w)
    assert_bf16_close(got, want, ulps=2, what="rmsnorm")
    assert (ulp_diff(got, want) == 0).mean() > 0.99
    # and against HF LlamaRMSNorm's own output (fixture)
    g = np.load(GOLD / "rmsnorm_hf.npz")
    out = bf16_empty(16, H)
    hip.check(hip.lib.ie_rmsnorm(16, P(dev(g["x"])), P(dev(g["w"])), P(out), ctx.stream_ptr))
    sync()
    assert_bf16_close(host(out), g["y"], ulps=2, what="rmsnorm vs HF")
    assert (ulp_diff(host(out), g["y"]) == 0).mean() > 0.99
    # fewer rows (1, 7, 126): each row as in the 128-row call, bit for bit, and nothing written
    # past the last row
    ref = bf16_empty(128, H)
    hip.check(hip.lib.ie_rmsnorm(128, P(dev(x)), P(dev(w)), P(ref), ctx.stream_ptr))
    for rows in (1, 7, 126):
        say(f"rmsnorm rows={rows}")
        o2 = torch.full((rows + 4, H), 0x40E0, dtype=torch.int16, device="cuda")  # bf16 7.0
        hip.check(hip.lib.ie_rmsnorm(rows, P(dev(x)), P(dev(w)), P(o2), ctx.stream_ptr))
        sync()
        assert torch.equal(o2[:rows], ref[:rows]), rows
        assert bool((o2[rows:] == 0x40E0).all()), rows


def test_residual_add_bit_exact(hip, ctx):
    say("residual_add [128, 4096]")
    x = orc.synthetic((128, H), 5, 1, 0.0, 1.0)
    d = orc.synthetic((128, H), 5, 2, 0.0, 1.0)
    dx = dev(x)
    hip.check(hip.lib.ie_residual_add(128, H, P(dx), P(dev(d)), ctx.stream_ptr))
    sync()
    assert np.array_equal(host(dx), orc.residual_add(x, d))


def test_swiglu(hip, ctx):
    say("swiglu [128, 14336]")
    g = orc.synthetic((128, F), 6, 1, 0.0, 2.0)
    u = orc.synthetic((128, F), 6, 2, 0.0, 2.0)
    out = bf16_empty(128, F)
    hip.check(hip.lib.ie_swiglu(128, P(dev(g)), P(dev(u)), P(out), ctx.stream_ptr))
    sync()
    assert_bf16_close(host(out), orc.swiglu(g, u), ulps=1, what="swiglu")


def test_apply_rope_activations_and_cache(hip, ctx, rope):
    cos, sin, dcos, dsin = rope
    say("apply_rope q [32,128,128] and k-cache rows 1000..1015")
    q = orc.synthetic((32, 128, 128), 7, 1, 0.0, 1.0)
    out = bf16_empty(32, 128, 128)
    hip.check(hip.lib.ie_apply_rope(0, 32, 128, P(dcos), P(dsin), P(dev(q)), P(out), 0, ctx.stream_ptr))
    sync()
    assert_bf16_close(host(out), orc.apply_rope(q, 0, 32, 128, 128, cos, sin), ulps=1, what="rope q")
    plane = orc.synthetic((8, 8192, 128), 7, 2, 0.0, 1.0)
    dp = dev(plane)
    hip.check(hip.lib.ie_apply_rope(1000, 8, 16, P(dcos), P(dsin), P(dp), P(dp), 1, ctx.stream_ptr))
    sync()
    got = host(dp)
    # only rows 0..15 of each head plane change (is_kv_cache stride), start_pos 1000
    want = orc.apply_rope(plane, 1000, 8, 16, 8192, cos, sin)
    assert np.array_equal(got[:, 16:], plane[:, 16:])
    assert_bf16_close(got[:, :16], want[:, :16], ulps=1, what="rope k cache")


@pytest.mark.parametrize("causal", [True, False])
def test_scale_softmax(hip, ctx, causal):
    S = 128 if causal else 2048
    say(f"scale_softmax causal={causal} S={S}")
    x = orc.synthetic((32, S, S) if causal else (32, S), 8, 1, 0.0, 4.0)
    out = bf16_empty(*x.shape)
    hip.check(hip.lib.ie_scale_causal_softmax(S, P(dev(x)), P(out), 0 if causal else 1, ctx.stream_ptr))
    sync()
    want = orc.softmax_scaled(x, S, causal)
    assert_close(orc.bf16_to_f32(host(out)), orc.bf16_to_f32(want), what="softmax")
    assert_bf16_close(host(out), want, ulps=2, what="softmax")


# ---------------------------------------------------------------- GEMV / GEMM
@pytest.mark.parametrize("k,n", [(4096, 14336), (14336, 4096), (4096, 6144), (4096, 1024)])
def test_multiply_by_weight_gemv(hip, ctx, k, n):
    say(f"multiply_by_weight m=1 k={k} n={n}")
    x = orc.synthetic((1, k), 9, k, 0.0, 1.0)
    w = orc.synthetic((n, k), 9, n, 0.0, 0.02)
    out = bf16_empty(1, n)
    hip.check(hip.lib.ie_multiply_by_weight(ctx.handle, 1, k, n, P(dev(x)), P(dev(w)), P(out)))
    sync()
    want = orc.matmul(x, w)
    assert_close(orc.bf16_to_f32(host(out)), orc.bf16_to_f32(want), what="gemv")
    assert_bf16_close(host(out), want, ulps=2, what="matmul")


@pytest.mark.parametrize("waves,ppw", [(4, 1), (16, 1), (8, 3), (8, 7), (4, 5)])
def test_gemv_tuning_knobs(hip, ctx, waves, ppw):
    """The decode GEMV under forced waves per workgroup / row pairs per wave (the multi-pair loop
    and the 4- and 16-wave instances; partial last waves at 3072 and 2048 pairs) computes the
    default's values: bit-identical without RMSNorm (a pair's dot product does not depend on
    where it runs), within tolerance of the oracle with it (the sum of squares is added over a
    different number of waves)."""
    say(f"gemv knobs waves={waves} pairs/wave={ppw}")
    cases = [(14336, 4096), (4096, 6144)]
    xs = {k: orc.synthetic((1, k), 21, k, 0.0, 1.0) for k, _ in cases}
    ws = {(k, n): orc.synthetic((n, k), 21, n, 0.0, 0.02) for k, n in cases}

    def run_plain():
        outs = []
        for k, n in cases:
            out = bf16_empty(1, n)
            hip.check(hip.lib.ie_multiply_by_weight(ctx.handle, 1, k, n, P(dev(xs[k])),
                                                    P(dev(ws[(k, n)])), P(out)))
            outs.append(out)
        sync()
        return [host(o) for o in outs]

    wg, wu, wd = _ffn_weights(22)
    x = orc.synthetic((1, H), 22, 10, 0.0, 1.0)
    nw = orc.synthetic((H,), 22, 11, 1.0, 0.02)
    wsp = torch.zeros(hip.lib.ie_ffn_workspace_size(1), dtype=torch.uint8, device="cuda")
    dwg, dwu, dwd, dnw = dev(wg), dev(wu), dev(wd), dev(nw)

    def run_ffn():
        dx = dev(x)
        hip.check(hip.lib.ie_ffn_block_decode(ctx.handle, P(dx), P(dnw), P(dwg), P(dwu), P(dwd),
                                              P(wsp)))
        sync()
        return host(dx)

    default = run_plain()
    try:
        hip.check(hip.lib.ie_tune_gemv_waves(waves))
        hip.check(hip.lib.ie_tune_gemv_pairs_per_wave(ppw))
        tuned = run_plain()
        ffn = run_ffn()
    finally:
        hip.check(hip.lib.ie_tune_gemv_waves(0))
        hip.check(hip.lib.ie_tune_gemv_pairs_per_wave(0))
    for (k, n), a, b in zip(cases, default, tuned):
        assert np.array_equal(a, b), f"gemv k={k} n={n} differs under waves={waves} ppw={ppw}"
        assert_close(orc.bf16_to_f32(b), orc.bf16_to_f32(orc.matmul(xs[k], ws[(k, n)])),
                     what=f"gemv k={k} n={n}")
    want = orc.residual_add(x, orc.ffn(orc.rmsnorm(x, nw), wg, wu, wd))
    assert_close(orc.bf16_to_f32(ffn), orc.bf16_to_f32(want), what="ffn block (tuned)")
    assert_delta_close(x, ffn, want, what="ffn block delta (tuned)")
    hip.check(hip.lib.ie_tune_gemv_waves(0))
    assert np.array_equal(run_plain()[0], default[0]), "knobs reset"


def test_rope_buffer_tables(hip, ctx):
    """ie_init_rope_buffer (rope.cu:68-103; the [8192][64] tables continued by the same formula to
    131072 rows) equals the oracle's tables bit for bit; ie_cleanup_rope_buffer frees them."""
    from infengine_amd._lib import MAX_LONG_CONTEXT
    from infengine_amd.engine import device_view
    n = MAX_LONG_CONTEXT
    say(f"init_rope_buffer [{n}][64] vs oracle")
    cos, sin = C.c_void_p(), C.c_void_p()
    hip.check(hip.lib.ie_init_rope_buffer(C.byref(cos), C.byref(sin)))
    try:
        want_cos, want_sin = orc.rope_tables(n)
        sync()
        assert torch.equal(device_view(cos.value, (n, 64), torch.float32).cpu(),
                           torch.from_numpy(want_cos))
        assert torch.equal(device_view(sin.value, (n, 64), torch.float32).cpu(),
                           torch.from_numpy(want_sin))
    finally:
        hip.check(hip.lib.ie_cleanup_rope_buffer(cos, sin))


def test_kv_cache_to_pages(hip, ctx):
    """ie_kv_cache_to_pages: positions [37, 287) of every layer of a reference-layout cache
    ([32][K|V][8][8192][128]) land in the pages the block table names ([page][32][K|V][8][64]
    [128]), bit for bit; blocks whose id is outside the pool (-1, 9) are skipped and every
    other page row keeps its contents."""
    say("kv_cache_to_pages, 250 positions over 5 blocks")
    Lr, KVH, MAXC, D, PP, n_pages = 32, 8, 8192, 128, 64, 6
    g = torch.Generator(device="cuda").manual_seed(5)
    cache = torch.randint(-32768, 32767, (Lr, 2, KVH, MAXC, D), dtype=torch.int16, device="cuda",
                          generator=g)
    pool = torch.randint(-32768, 32767, (n_pages, Lr, 2, KVH, PP, D), dtype=torch.int16,
                         device="cuda", generator=g)
    want = pool.clone()
    tab = [3, -1, 0, 5, 1, 9]
    table = torch.tensor(tab, dtype=torch.int32, device="cuda")
    first, npos = 37, 250
    hip.check(hip.lib.ie_kv_cache_to_pages(ctx.handle, P(cache), first, npos, P(pool), n_pages,
                                           P(table)))
    sync()
    for blk in range(first // PP, (first + npos - 1) // PP + 1):
        pg = tab[blk]
        if not 0 <= pg < n_pages:
            continue
        lo, hi = max(first, blk * PP), min(first + npos, (blk + 1) * PP)
        want[pg, :, :, :, lo - blk * PP:hi - blk * PP, :] = cache[:, :, :, lo:hi, :]
    assert torch.equal(pool, want)
    del cache


def test_lm_head_logits(hip, ctx):
    say("lm_head [1,4096] x [128256,4096] -> fp32")
    x = orc.synthetic((3, H), 10, 1, 0.0, 1.0)
    w = orc.synthetic((V, H), 10, 2, 0.0, 0.02)
    out = torch.empty(V, dtype=torch.float32, device="cuda")
    hip.check(hip.lib.ie_lm_head(ctx.handle, 3, P(dev(x)), P(dev(w)), P(out)))
    sync()
    want = orc.matmul(x[2:3], w, out_f32=True)[0]           # lm_head.cu:7: last row only
    got = host(out)
    assert_close(got, want, tol=1e-4, what="lm_head")        # fp32 out: only summation order differs


@pytest.mark.parametrize("m,k,n", [(1, 4096, 256), (16, 4096, 1024), (100, 4096, 512),
                                   (256, 4096, 1024), (64, 14336, 4096), (300, 4096, 132),
                                   (8, 14336, 512), (4, 1536, 200)])
def test_gemm_mfma(hip, ctx, m, k, n):
    say(f"gemm_bf16 m={m} k={k} n={n}")
    x = orc.synthetic((m, k), 11, m, 0.0, 1.0)
    w = orc.synthetic((n, k), 11, n + 7, 0.0, 0.02)
    out = bf16_empty(m, n)
    hip.check(hip.lib.ie_gemm_bf16(ctx.handle, m, k, n, P(dev(x)), P(dev(w)), P(out)))
    sync()
    want = orc.matmul(x, w)
    assert_close(orc.bf16_to_f32(host(out)), orc.bf16_to_f32(want), what="gemm")
    assert_bf16_close(host(out), want, ulps=2, what="matmul")


def test_gemm_mfma_prefill_shape_sampled_rows(hip, ctx):
    m, k, n = 2048, 4096, 6144
    say(f"gemm_bf16 m={m} k={k} n={n} (64 sampled rows checked)")
    x = orc.synthetic((m, k), 12, 1, 0.0, 1.0)
    w = orc.synthetic((n, k), 12, 2, 0.0, 0.02)
    out = bf16_empty(m, n)
    hip.check(hip.lib.ie_gemm_bf16(ctx.handle, m, k, n, P(dev(x)), P(dev(w)), P(out)))
    sync()
    rows = np.random.default_rng(1).choice(m, 64, replace=False)
    rows[:2] = [0, m - 1]
    want = orc.matmul(np.ascontiguousarray(x[rows]), w)
    got = host(out)[rows]
    assert_close(orc.bf16_to_f32(got), orc.bf16_to_f32(want), what="gemm 2048")


GEMM_EPI = {"bf16": 0, "resid": 1, "f32": 2, "swiglu": 3}


@pytest.mark.parametrize("epi", list(GEMM_EPI))
@pytest.mark.parametrize("m,n", [(7, 1000), (16, 4096), (17, 4096), (24, 1000), (32, 4096),
                                 (33, 6144), (40, 1000), (48, 4096), (64, 4096), (64, 14336),
                                 (100, 4096), (300, 1000), (512, 4096), (2048, 6144),
                                 (2048, 4096), (2048, 14336)])
def test_gemm_epilogues(hip, ctx, epi, m, n):
    """Every fused epilogue of the MFMA GEMM on each kernel the launcher picks: the skinny
    streaming kernel (m <= 16, ragged n), the 64-weight-row streaming kernel at m = 17-100
    (bf16 / resid / SwiGLU; 64 X rows up to m = 64, 128 at m = 100; K split with a reduction, or
    SwiGLU in the kernel at n = 14336), 128 x 128 tiles (m = 300: f32 / SwiGLU; f32 at
    m = 17..100), K split across workgroups with a reduction (bf16 / resid at m = 300, 512), and
    the prefill sizes:
    192 x 256 tiles (bf16 / resid at n = 6144), 256 x 256 tiles (SwiGLU at n = 4096), 256 x 128
    tiles (the others at n = 4096 and 6144), and at n = 14336 a launch split by output columns
    (full rounds of the big tile, then the remaining columns with another shape: SwiGLU 256 x 256
    then 256 x 128, bf16 / resid 256 x 256 then 192 x 256, fp32 256 x 128 then 128 x 128);
    sampled rows at m = 2048."""
    k = 4096
    say(f"gemm_ex {epi} m={m} k={k} n={n}")
    x = orc.synthetic((m, k), 21, m, 0.0, 1.0)
    w0 = orc.synthetic((n, k), 21, n + 1, 0.0, 0.02)
    w1 = orc.synthetic((n, k), 21, n + 2, 0.0, 0.02)
    y0 = orc.synthetic((m, n), 21, n + 3, 0.0, 1.0)
    if epi == "f32":
        out = torch.empty(m, n, dtype=torch.float32, device="cuda")
    else:
        out = dev(y0) if epi == "resid" else bf16_empty(m, n)
    hip.check(hip.lib.ie_gemm_ex(ctx.handle, GEMM_EPI[epi], m, k, n, P(dev(x)), P(dev(w0)),
                                 P(dev(w1)), P(out)))
    sync()
    rows = np.arange(m) if m <= 512 else np.random.default_rng(2).choice(m, 48, replace=False)
    rows[:2] = [0, m - 1]
    xs = np.ascontiguousarray(x[rows])
    got = host(out)[rows]
    if epi == "f32":
        assert_close(got, orc.matmul(xs, w0, out_f32=True), tol=1e-4, what="gemm f32")
        return
    if epi == "bf16":
        want = orc.matmul(xs, w0)
    elif epi == "resid":
        want = orc.residual_add(np.ascontiguousarray(y0[rows]), orc.matmul(xs, w0))
    else:
        want = orc.swiglu(orc.matmul(xs, w0), orc.matmul(xs, w1))
    assert_close(orc.bf16_to_f32(got), orc.bf16_to_f32(want), what=f"gemm {epi}")
    # SwiGLU compounds a 1-ulp difference in gate or up (summation order) through g*silu(g)*u;
    # the residual add cancels (y0 ~ -acc), so a 1-ulp product difference can be several ulps
    # of a small sum: admit 1e-3 of such elements (each still within 1e-2 of the scale)
    assert_bf16_close(got, want, ulps=4 if epi == "swiglu" else 2, what=f"gemm {epi}",
                      outlier_frac=1e-3 if epi == "resid" else 0.0)


# ragged rows and columns on every tile kind: 256 x 256 and 192 x 256 (QKV split points at
# 4096 / 5120), 256 x 128 (two k-groups), SwiGLU with a column-split launch
@pytest.mark.parametrize("epi,m,k,n", [("bf16", 300, 4096, 6144), ("resid", 1300, 4096, 4096),
                                       ("resid", 2048, 14336, 4096), ("swiglu", 700, 4096, 14336),
                                       ("swiglu", 2048, 4096, 14336), ("bf16", 2048, 4096, 6144),
                                       ("bf16", 555, 4096, 1000)])
def test_gemm_schedules_bit_identical(hip, ctx, epi, m, k, n):
    """The prefill GEMM's tile schedules (ie_tune_gemm_schedule: the DMA-ring kernels, the
    ping-pong kernel for 256-row tiles, for all bf16 tiles, and with 4 W ring slots) give
    identical bits: the MFMAs of every accumulator run in the same k order."""
    say(f"gemm schedules {epi} m={m} k={k} n={n}")
    x = dev(orc.synthetic((m, k), 31, m, 0.0, 1.0))
    w0 = dev(orc.synthetic((n, k), 31, n + 1, 0.0, 0.02))
    w1 = dev(orc.synthetic((n, k), 31, n + 2, 0.0, 0.02))
    y0 = dev(orc.synthetic((m, n), 31, n + 3, 0.0, 1.0))
    outs = []
    try:
        for sched in (0, 1, 2, 3):
            hip.check(hip.lib.ie_tune_gemm_schedule(sched))
            out = y0.clone()
            hip.check(hip.lib.ie_gemm_ex(ctx.handle, GEMM_EPI[epi], m, k, n, P(x), P(w0), P(w1),
                                         P(out)))
            sync()
            outs.append(host(out))
    finally:
        hip.check(hip.lib.ie_tune_gemm_schedule(2))
    for o in outs[1:]:
        assert np.array_equal(outs[0], o)
    assert np.isfinite(orc.bf16_to_f32(outs[2])).all() and outs[2][[0, m // 2, m - 1]].any()


# The skinny kernel at M <= 16: the fp32 epilogue's 32-row tiles (K = 4096 / 14336) with the
# last partial round in K halves (n = 8224: 257 tiles, one split; the lm_head's 128256 columns:
# 4008 tiles, 168 split) or none (n = 4100: 129 tiles, the last with 4 rows), and the bf16 /
# residual 16-row tiles at ragged widths.
@pytest.mark.parametrize("epi,m,k,n", [("bf16", 16, 4096, 4096), ("resid", 9, 4096, 4112),
                                       ("resid", 16, 14336, 4096), ("f32", 1, 14336, 4100),
                                       ("f32", 3, 4096, 8224), ("f32", 16, 4096, 128256),
                                       ("f32", 7, 14336, 8224)])
def test_gemm_skinny_wide_tiles(hip, ctx, epi, m, k, n):
    """M <= 16 products, the split tiles handing partials over through device-scope stores and
    an arrival counter: against the oracle, and bit-identical on a second call (the counters were
    reset by the first call's finishers)."""
    say(f"gemm_ex skinny 32-row tiles {epi} m={m} k={k} n={n}")
    x = orc.synthetic((m, k), 41, m, 0.0, 1.0)
    w0 = orc.synthetic((n, k), 41, n + 1, 0.0, 0.02)
    y0 = orc.synthetic((m, n), 41, n + 3, 0.0, 1.0)
    dx, dw = dev(x), dev(w0)
    outs = []
    for _ in range(2):
        if epi == "f32":
            out = torch.empty(m, n, dtype=torch.float32, device="cuda")
        else:
            out = dev(y0) if epi == "resid" else bf16_empty(m, n)
        hip.check(hip.lib.ie_gemm_ex(ctx.handle, GEMM_EPI[epi], m, k, n, P(dx), P(dw), P(dw),
                                     P(out)))
        sync()
        outs.append(host(out))
    assert np.array_equal(outs[0], outs[1])
    got = outs[0]
    if epi == "f32":
        assert_close(got, orc.matmul(x, w0, out_f32=True), tol=1e-4, what="skinny f32")
        return
    want = orc.matmul(x, w0) if epi == "bf16" else orc.residual_add(y0, orc.matmul(x, w0))
    assert_close(orc.bf16_to_f32(got), orc.bf16_to_f32(want), what=f"skinny {epi}")
    assert_bf16_close(got, want, ulps=2, what=f"skinny {epi}",
                      outlier_frac=1e-3 if epi == "resid" else 0.0)


@pytest.mark.parametrize("epi", ["bf16", "resid"])
@pytest.mark.parametrize("m", [17, 24, 40, 64, 2048])
def test_gemm_down_projection_shapes(hip, ctx, epi, m):
    """The down projection (k 14336, n 4096) as prefill runs it: the 64-weight-row streaming
    kernel at 17-64 rows (K split 4 ways, then the residual reduction) and the 2048-row MFMA tiles
    of config 4; every row up to 64, sampled rows at 2048, against the oracle."""
    k, n = 14336, 4096
    say(f"gemm_ex down {epi} m={m} k={k} n={n}")
    x = orc.synthetic((m, k), 25, m, 0.0, 1.0)
    w0 = orc.synthetic((n, k), 25, n + 1, 0.0, 0.02)
    y0 = orc.synthetic((m, n), 25, n + 3, 0.0, 1.0)
    out = dev(y0) if epi == "resid" else bf16_empty(m, n)
    hip.check(hip.lib.ie_gemm_ex(ctx.handle, GEMM_EPI[epi], m, k, n, P(dev(x)), P(dev(w0)),
                                 P(dev(w0)), P(out)))
    sync()
    rows = np.arange(m) if m <= 64 else np.random.default_rng(4).choice(m, 40, replace=False)
    rows[:2] = [0, m - 1]
    xs = np.ascontiguousarray(x[rows])
    got = host(out)[rows]
    want = orc.matmul(xs, w0)
    if epi == "resid":
        want = orc.residual_add(np.ascontiguousarray(y0[rows]), want)
    assert_close(orc.bf16_to_f32(got), orc.bf16_to_f32(want), what=f"gemm down {epi} m={m}")
    assert_bf16_close(got, want, ulps=2, what=f"gemm down {epi} m={m}",
                      outlier_frac=1e-3 if epi == "resid" else 0.0)


@pytest.mark.parametrize("epi,m,k,n", [("bf16", 17, 4096, 6144), ("resid", 33, 4096, 4096),
                                       ("swiglu", 64, 4096, 14336), ("resid", 65, 14336, 4096),
                                       ("bf16", 100, 4096, 1000), ("swiglu", 128, 256, 520),
                                       ("bf16", 128, 192, 16384), ("resid", 48, 4096, 4104),
                                       ("swiglu", 96, 4096, 4104), ("swiglu", 100, 4096, 14336),
                                       ("swiglu", 128, 256, 12288)])
def test_gemm_medium_rows(hip, ctx, epi, m, k, n):
    """17-128 rows (prompts of a few dozen tokens): the 64-weight-row streaming kernel with 64 X
    rows (m <= 64) or 128.  K split into fp32 planes then reduced: 2 ways (bf16 n = 6144, resid
    n = 4104), 4 (resid n = 4096 at k 4096 and 14336, SwiGLU n = 520 over its 1040-column gate|up
    planes), 16 (bf16 n = 1000), and one plane (SwiGLU n = 4104: 129 tiles, no split divides);
    unsplit with the epilogue in the kernel where the tiles alone fill the chip (SwiGLU n = 14336
    over 32-column tiles at m = 64; over 64-column tiles of 128 weight rows and 8 waves at m = 100
    and 128, n = 14336 and 12288; bf16 n = 16384 at k = 192, three stages).  Ragged n, every row
    against the oracle, and the same bits on a second call."""
    say(f"gemm_ex medium rows {epi} m={m} k={k} n={n}")
    x = orc.synthetic((m, k), 27, m, 0.0, 1.0)
    w0 = orc.synthetic((n, k), 27, n + 1, 0.0, 0.02)
    w1 = orc.synthetic((n, k), 27, n + 2, 0.0, 0.02)
    y0 = orc.synthetic((m, n), 27, n + 3, 0.0, 1.0)
    dx, dw0, dw1 = dev(x), dev(w0), dev(w1)
    outs = []
    for _ in range(2):
        out = dev(y0) if epi == "resid" else bf16_empty(m, n)
        hip.check(hip.lib.ie_gemm_ex(ctx.handle, GEMM_EPI[epi], m, k, n, P(dx), P(dw0), P(dw1),
                                     P(out)))
        sync()
        outs.append(host(out))
    assert np.array_equal(outs[0], outs[1])
    got = outs[0]
    if epi == "bf16":
        want = orc.matmul(x, w0)
    elif epi == "resid":
        want = orc.residual_add(y0, orc.matmul(x, w0))
    else:
        want = orc.swiglu(orc.matmul(x, w0), orc.matmul(x, w1))
    assert_close(orc.bf16_to_f32(got), orc.bf16_to_f32(want), what=f"gemm medium {epi}")
    assert_bf16_close(got, want, ulps=4 if epi == "swiglu" else 2, what=f"gemm medium {epi}",
                      outlier_frac=1e-3 if epi == "resid" else 0.0)


@pytest.mark.parametrize("epi", ["bf16", "resid"])
def test_gemm_split_k_long(hip, ctx, epi):
    """The down-projection shape of a 512-token prefill (m 512, k 14336, n 4096): 64 wide tiles
    would leave the chip mostly idle, so K is split 4 ways (fp32 partials, then the reduction
    applies the epilogue); sampled rows against the oracle."""
    m, k, n = 512, 14336, 4096
    say(f"gemm_ex split-K {epi} m={m} k={k} n={n}")
    x = orc.synthetic((m, k), 23, m, 0.0, 1.0)
    w0 = orc.synthetic((n, k), 23, n + 1, 0.0, 0.02)
    y0 = orc.synthetic((m, n), 23, n + 3, 0.0, 1.0)
    out = dev(y0) if epi == "resid" else bf16_empty(m, n)
    hip.check(hip.lib.ie_gemm_ex(ctx.handle, GEMM_EPI[epi], m, k, n, P(dev(x)), P(dev(w0)),
                                 P(dev(w0)), P(out)))
    sync()
    rows = np.random.default_rng(3).choice(m, 40, replace=False)
    rows[:2] = [0, m - 1]
    xs = np.ascontiguousarray(x[rows])
    got = host(out)[rows]
    want = orc.matmul(xs, w0)
    if epi == "resid":
        want = orc.residual_add(np.ascontiguousarray(y0[rows]), want)
    assert_close(orc.bf16_to_f32(got), orc.bf16_to_f32(want), what=f"gemm split-K {epi}")
    assert_bf16_close(got, want, ulps=2, what=f"gemm split-K {epi}",
                      outlier_frac=1e-3 if epi == "resid" else 0.0)


# ---------------------------------------------------------------- FFN (config 1)
def _ffn_weights(seed):
    return (orc.synthetic((F, H), seed, 1, 0.0, 0.02), orc.synthetic((F, H), seed, 2, 0.0, 0.02),
            orc.synthetic((H, F), seed, 3, 0.0, 0.02))


def test_ffn_block_decode_config1(hip, ctx):
    """x + W_down(silu(W_gate n) * (W_up n)), n = rmsnorm(x): the fused decode FFN."""
    say("ffn_block_decode (config 1)")
    wg, wu, wd = _ffn_weights(13)
    x = orc.synthetic((1, H), 13, 10, 0.0, 1.0)
    nw = orc.synthetic((H,), 13, 11, 1.0, 0.02)
    dx = dev(x)
    ws = torch.zeros(hip.lib.ie_ffn_workspace_size(1), dtype=torch.uint8, device="cuda")
    hip.check(hip.lib.ie_ffn_block_decode(ctx.handle, P(dx), P(dev(nw)), P(dev(wg)), P(dev(wu)),
                                          P(dev(wd)), P(ws)))
    sync()
    want = orc.residual_add(x, orc.ffn(orc.rmsnorm(x, nw), wg, wu, wd))
    got = orc.bf16_to_f32(host(dx))
    assert_close(got, orc.bf16_to_f32(want), what="ffn block")
    assert_delta_close(x, host(dx), want, what="ffn block delta")


@pytest.mark.parametrize("S", [1, 64])
def test_ffn_op(hip, ctx, S):
    say(f"ffn op seq_len={S}")
    wg, wu, wd = _ffn_weights(14)
    x = orc.synthetic((S, H), 14, 10, 0.0, 1.0)
    out = bf16_empty(S, H)
    ws = torch.zeros(hip.lib.ie_ffn_workspace_size(S), dtype=torch.uint8, device="cuda")
    hip.check(hip.lib.ie_ffn(ctx.handle, S, P(dev(x)), P(out), P(dev(wu)), P(dev(wd)), P(dev(wg)),
                             P(ws)))
    sync()
    assert_close(orc.bf16_to_f32(host(out)), orc.bf16_to_f32(orc.ffn(x, wg, wu, wd)), what="ffn")


# ---------------------------------------------------------------- attention
def _attn_weights(seed):
    w = orc.layer_weights(seed, 0)
    return w, {k: dev(v) for k, v in w.items()}


@pytest.mark.parametrize("pos", [0, 99, 2047, 3000])
def test_decode_attn_config2(hip, ctx, rope, pos):
    """decode_attn at position pos over pos cached rows (config 2: 2047); KV placement
    bit-exact.  Covers one row, a partial 64-row tile, one tile per split (2048) and
    several tiles per split (3001)."""
    cos, sin, dcos, dsin = rope
    say(f"decode_attn seq_len={pos + 1} layer 5")
    w, dw = _attn_weights(15)
    layer = 5
    kv = torch.zeros(hip.lib.ie_kv_cache_size() // 2, dtype=torch.int16, device="cuda")
    kv5 = kv.view(32, 2, 8, 8192, 128)[layer]
    prior = orc.synthetic((2, 8, pos, 128), 15, 500, 0.0, 1.0)
    if pos:
        kv5[:, :, :pos] = dev(prior)
    x = orc.synthetic((1, H), 15, 501, 0.0, 1.0)           # the already-normalised input
    out = bf16_empty(1, H)
    ws = torch.zeros(hip.lib.ie_attn_workspace_size(1), dtype=torch.uint8, device="cuda")
    hip.check(hip.lib.ie_decode_attn(ctx.handle, P(dcos), P(dsin), pos + 1, P(dev(x)),
                                     P(dw["w_q"]), P(dw["w_k"]), P(dw["w_v"]), P(dw["w_o"]),
                                     P(out), P(ws), P(kv), layer))
    sync()
    # oracle: projections, rope at pos, cache write, attention, O projection
    q = orc.apply_rope(orc.matmul(x, w["w_q"]), pos, 32, 1, 1, cos, sin)
    k = orc.apply_rope(orc.matmul(x, w["w_k"]), pos, 8, 1, 1, cos, sin)
    v = orc.matmul(x, w["w_v"])
    planes = np.zeros((2, 8, 8192, 128), np.uint16)
    planes[:, :, :pos] = prior
    planes[0, :, pos] = k.reshape(8, 128)
    planes[1, :, pos] = v.reshape(8, 128)
    a = orc.attention(q, planes[0], planes[1], pos, 8192)
    want = orc.matmul(a, w["w_o"])
    assert_close(orc.bf16_to_f32(host(out)), orc.bf16_to_f32(want), what="decode_attn")
    got_kv = host(kv.view(32, 2, 8, 8192, 128)[layer])
    assert np.array_equal(got_kv[:, :, :pos], prior)                # earlier rows untouched
    assert not got_kv[:, :, pos + 1:].any()                          # later rows untouched
    assert_bf16_close(got_kv[:, :, pos], planes[:, :, pos], what="kv row", outlier_frac=1e-3)  # row seq_len-1
    others = kv.view(32, 2, 8, 8192, 128)
    assert int(torch.count_nonzero(others[:layer])) == 0
    assert int(torch.count_nonzero(others[layer + 1:])) == 0


# S = 256: both projections split K (fp32 partials + reduction), the q/k/v one over three matrices
@pytest.mark.parametrize("S", [96, 256])
def test_attn_prefill_op(hip, ctx, rope, S):
    cos, sin, dcos, dsin = rope
    layer = 2
    say(f"attn (prefill) seq_len={S}")
    w, dw = _attn_weights(16)
    x = orc.synthetic((S, H), 16, 600, 0.0, 1.0)
    kv = torch.zeros(hip.lib.ie_kv_cache_size() // 2, dtype=torch.int16, device="cuda")
    out = bf16_empty(S, H)
    ws = torch.zeros(hip.lib.ie_attn_workspace_size(S), dtype=torch.uint8, device="cuda")
    hip.check(hip.lib.ie_attn(ctx.handle, P(dcos), P(dsin), S, P(dev(x)), P(dw["w_q"]),
                              P(dw["w_k"]), P(dw["w_v"]), P(dw["w_o"]), P(out), P(ws), P(kv),
                              layer))
    sync()
    q = orc.matmul(x, w["w_q"])
    k = orc.matmul(x, w["w_k"])
    v = orc.matmul(x, w["w_v"])
    qr = np.stack([orc.apply_rope(q[t], t, 32, 1, 1, cos, sin) for t in range(S)])
    kr = np.stack([orc.apply_rope(k[t], t, 8, 1, 1, cos, sin) for t in range(S)])
    planes = np.zeros((2, 8, 8192, 128), np.uint16)
    planes[0, :, :S] = kr.reshape(S, 8, 128).transpose(1, 0, 2)
    planes[1, :, :S] = v.reshape(S, 8, 128).transpose(1, 0, 2)
    a = orc.attention(qr.reshape(S, H), planes[0], planes[1], 0, 8192)
    want = orc.matmul(a, w["w_o"])
    assert_close(orc.bf16_to_f32(host(out)), orc.bf16_to_f32(want), what="attn prefill")
    got_kv = host(kv.view(32, 2, 8, 8192, 128)[layer])
    assert_bf16_close(got_kv[:, :, :S], planes[:, :, :S], what="kv rows", outlier_frac=1e-3)
    assert not got_kv[:, :, S:].any()


def test_attn_prefill_op_2048(hip, ctx, rope):
    """The attention op at S = 2048: the QKV projection runs as one GEMM over the three
    concatenated weights on 192 x 256 tiles, two of which straddle the Q|K and K|V split points.
    Every K and V cache row is checked, and the output at sampled query rows."""
    cos, sin, dcos, dsin = rope
    S, layer = 2048, 1
    say(f"attn (prefill) seq_len={S}")
    w, dw = _attn_weights(17)
    x = orc.synthetic((S, H), 17, 700, 0.0, 1.0)
    kv = torch.zeros(hip.lib.ie_kv_cache_size() // 2, dtype=torch.int16, device="cuda")
    out = bf16_empty(S, H)
    ws = torch.zeros(hip.lib.ie_attn_workspace_size(S), dtype=torch.uint8, device="cuda")
    hip.check(hip.lib.ie_attn(ctx.handle, P(dcos), P(dsin), S, P(dev(x)), P(dw["w_q"]),
                              P(dw["w_k"]), P(dw["w_v"]), P(dw["w_o"]), P(out), P(ws), P(kv),
                              layer))
    sync()
    k = orc.matmul(x, w["w_k"])
    v = orc.matmul(x, w["w_v"])
    kh = np.ascontiguousarray(k.reshape(S, 8, 128).transpose(1, 0, 2))    # [head][t][128]
    planes = np.zeros((2, 8, 8192, 128), np.uint16)
    planes[0, :, :S] = orc.apply_rope(kh, 0, 8, S, S, cos, sin).reshape(8, S, 128)
    planes[1, :, :S] = v.reshape(S, 8, 128).transpose(1, 0, 2)
    got_kv = host(kv.view(32, 2, 8, 8192, 128)[layer])
    assert_bf16_close(got_kv[:, :, :S], planes[:, :, :S], what="kv rows", outlier_frac=1e-3)
    assert not got_kv[:, :, S:].any()
    got = host(out)
    for t in (0, 1, 767, 1500, 2047):
        q = orc.apply_rope(orc.matmul(x[t:t + 1], w["w_q"]), t, 32, 1, 1, cos, sin)
        a = orc.attention(q, planes[0], planes[1], t, 8192)
        want = orc.matmul(a, w["w_o"])
        assert_close(orc.bf16_to_f32(got[t:t + 1]), orc.bf16_to_f32(want), what=f"attn row {t}")


@pytest.fixture(scope="module")
def model31():
    from infengine_amd.engine import ModelWeights
    W = ModelWeights.random_init(seed=31, std=0.02)
    yield W
    W.free()


@pytest.mark.parametrize("pos", [100, 1023, 1024, 2047, 3000, 4095, 4096, 5000, 8191])
def test_decoder_layer_decode_config2(hip, ctx, rope, model31, pos):
    """One full fused decoder layer, token at position pos (2047).  Up to
    4096 rows the O projection merges the attention partials itself (one tile per wave at
    100, several at 2047 and 3000; 4 splits up to 1024 rows, 8 from 1025); 4097 rows and more
    take the merge kernel (up to 32 splits; 8192: the cache's last row)."""
    cos, sin, dcos, dsin = rope
    say(f"decoder_layer_decode layer 0 pos {pos} (random-init weights)")
    seed, layer = 31, 0
    W = model31
    kv = torch.zeros(hip.lib.ie_kv_cache_size() // 2, dtype=torch.int16, device="cuda")
    prior = orc.synthetic((2, 8, pos, 128), seed, 700, 0.0, 1.0)
    kv.view(32, 2, 8, 8192, 128)[layer][:, :, :pos] = dev(prior)
    x = orc.synthetic((1, H), seed, 701, 0.0, 1.0)
    dx = dev(x)
    attn = bf16_empty(1, H)
    ws = torch.zeros(hip.lib.ie_attn_workspace_size(1), dtype=torch.uint8, device="cuda")
    hip.check(hip.lib.ie_decoder_layer_decode(ctx.handle, W.ref(), layer, pos + 1, P(dx), P(attn),
                                              P(ws), P(kv)))
    sync()
    w = orc.layer_weights(seed, layer)
    planes = np.zeros((2, 8, 8192, 128), np.uint16)
    planes[:, :, :pos] = prior
    xo = x.copy()
    orc.decoder_layer(xo, w, pos, cos, sin, planes[0], planes[1], 8192)
    got = orc.bf16_to_f32(host(dx))
    assert_close(got, orc.bf16_to_f32(xo), what="decoder layer")
    assert_delta_close(x, host(dx), xo, what="decoder layer delta")
    got_kv = host(kv.view(32, 2, 8, 8192, 128)[layer])
    assert np.array_equal(got_kv[:, :, :pos], prior)
    assert_bf16_close(got_kv[:, :, pos], planes[:, :, pos], what="kv row", outlier_frac=1e-3)


# ---------------------------------------------------------------- sampling (config 3)
def test_argmax_fixtures_bit_exact(hip, ctx):
    say("argmax rows (torch.argmax fixtures: ties, NaN, signed zeros)")
    g = np.load(GOLD / "argmax_torch.npz")
    logits = dev(g["logits"])
    out = torch.full((logits.shape[0],), -7, dtype=torch.int32, device="cuda")
    hip.check(hip.lib.ie_sample_argmax_rows(ctx.handle, logits.shape[0], V, P(logits), P(out)))
    sync()
    assert host(out).tolist() == g["expect"].tolist()
    one = torch.empty(1, dtype=torch.int32, device="cuda")
    for r in range(logits.shape[0]):                       # single-row entry point, repeated
        hip.check(hip.lib.ie_sample_token_amax(ctx.handle, P(logits[r]), P(one)))
        sync()
        assert int(one.item()) == int(g["expect"][r])


def test_top_p_fixture_and_oracle(hip, ctx):
    say("top-p T=0.7 p=0.9 on HF fixture logits")
    g = np.load(GOLD / "top_p_hf.npz")
    logits = dev(g["logits"])
    R = logits.shape[0]
    out = torch.empty(R, dtype=torch.int32, device="cuda")
    ws = torch.empty(hip.lib.ie_top_p_workspace_size(R, V), dtype=torch.uint8, device="cuda")
    for step in range(8):
        hip.check(hip.lib.ie_sample_top_p(ctx.handle, R, V, P(logits), 0.7, 0.9, 1234, step,
                                          P(out), P(ws)))
        sync()
        for r in range(R):
            kept = np.unpackbits(g["kept"][r])[:V].astype(bool)
            tok = int(out[r].item())
            want, info = orc.top_p(g["logits"][r], 0.7, 0.9, 1234, r, step)
            assert kept[tok]
            margin = min(info["t"] - info["lo"], info["hi"] - info["t"]) / info["z_kept"]
            if margin > 1e-6:
                assert tok == want, (r, step, tok, want)


def test_top_p_ties_and_flat_rows(hip, ctx):
    """Rows whose cut bin holds more tokens than the sampler's candidate list (all logits equal; a
    20000-way tie at the top; a near-flat row), where it selects over the row itself, and a
    sharp row: the kept set and the sample equal the oracle's (masses in exact fixed point)."""
    say("top-p on tied and flat rows")
    rng = np.random.default_rng(17)
    rows = [np.zeros(V, np.float32),
            np.where(np.arange(V) < 20000, 3.0, -1.0).astype(np.float32),
            (rng.standard_normal(V) * 0.01).astype(np.float32),
            (rng.standard_normal(V) * 8.0).astype(np.float32)]
    lg = np.stack(rows)
    R = lg.shape[0]
    logits = torch.from_numpy(lg).cuda()
    out = torch.empty(R, dtype=torch.int32, device="cuda")
    ws = torch.empty(hip.lib.ie_top_p_workspace_size(R, V), dtype=torch.uint8, device="cuda")
    for step in range(4):
        hip.check(hip.lib.ie_sample_top_p(ctx.handle, R, V, P(logits), 0.7, 0.9, 555, step,
                                          P(out), P(ws)))
        sync()
        for r in range(R):
            want, info = orc.top_p(lg[r], 0.7, 0.9, 555, r, step)
            assert int(out[r].item()) == want, (r, step, int(out[r].item()), want)


def test_final_norm_lm_head_sampling_config3(hip, ctx):
    """Config 3: final RMSNorm + lm_head GEMV -> fp32 logits, argmax and top-p, B=1 and B=16."""
    say("final_norm_lm_head rows=16 + argmax + top-p")
    R = 16
    x = orc.synthetic((R, H), 41, 1, 0.0, 1.0)
    nw = orc.synthetic((H,), 41, 2, 1.0, 0.02)
    wl = orc.synthetic((V, H), 41, 3, 0.0, 0.02)
    dwl = dev(wl)
    logits = torch.empty(R, V, dtype=torch.float32, device="cuda")
    hip.check(hip.lib.ie_final_norm_lm_head(ctx.handle, R, P(dev(x)), P(dev(nw)), P(dwl),
                                            P(logits)))
    one = torch.empty(V, dtype=torch.float32, device="cuda")
    hip.check(hip.lib.ie_final_norm_lm_head(ctx.handle, 1, P(dev(x[:1])), P(dev(nw)), P(dwl),
                                            P(one)))
    sync()
    want = orc.matmul(orc.rmsnorm(x, nw), wl, out_f32=True)
    got = host(logits)
    assert_close(got, want, what="lm_head logits")
    assert np.array_equal(host(one), got[0])                 # B=1 row == row 0 of B=16, bitwise
    toks = torch.empty(R, dtype=torch.int32, device="cuda")
    hip.check(hip.lib.ie_sample_argmax_rows(ctx.handle, R, V, P(logits), P(toks)))
    sync()
    for r in range(R):
        assert int(toks[r].item()) == orc.argmax(got[r])     # identical logits -> identical id
        top2 = np.sort(want[r])[-2:]
        if top2[1] - top2[0] > 1e-3 * np.abs(want[r]).max():
            assert int(toks[r].item()) == orc.argmax(want[r])
    ws = torch.empty(hip.lib.ie_top_p_workspace_size(R, V), dtype=torch.uint8, device="cuda")
    hip.check(hip.lib.ie_sample_top_p(ctx.handle, R, V, P(logits), 0.7, 0.9, 99, 3, P(toks),
                                      P(ws)))
    sync()
    for r in range(R):
        want_tok, info = orc.top_p(got[r], 0.7, 0.9, 99, r, 3)
        margin = min(info["t"] - info["lo"], info["hi"] - info["t"]) / info["z_kept"]
        if margin > 1e-6:
            assert int(toks[r].item()) == want_tok
