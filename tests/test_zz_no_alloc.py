"""ie_sample_top_p_noalloc (the top-p sampler with its scratch in the library's static
per-device array, no workspace argument, no allocation) against ie_sample_top_p (the same
kernel with a caller-allocated workspace): identical token ids, bit for bit, on two calls in
a row where the second is smaller than the first, and a clear rejection past the limit.
"""
import ctypes as C

import numpy as np
import pytest
import torch

from gpu_util import P, host, say

pytestmark = pytest.mark.gpu
V = 128256
IE_ERR_INVALID_ARG = -1
NOALLOC_MAX = 16 * 131072


def _logits(rows, vocab, seed):
    rng = np.random.default_rng(seed)
    # rows with a sharp head, a flat tail and everything between
    scale = np.linspace(0.5, 12.0, rows, dtype=np.float32)[:, None]
    return torch.from_numpy((rng.standard_normal((rows, vocab)).astype(np.float32) * scale)).cuda()


def _with_workspace(hip, ctx, logits, rows, vocab, seed, step):
    out = torch.full((rows,), -7, dtype=torch.int32, device="cuda")
    ws = torch.empty(hip.lib.ie_top_p_workspace_size(rows, vocab), dtype=torch.uint8,
                     device="cuda")
    hip.check(hip.lib.ie_sample_top_p(ctx.handle, rows, vocab, P(logits), 0.7, 0.9, seed, step,
                                      P(out), P(ws)))
    torch.cuda.synchronize()
    return host(out).tolist()


def _noalloc(hip, ctx, logits, rows, vocab, seed, step):
    out = torch.full((rows,), -7, dtype=torch.int32, device="cuda")
    hip.check(hip.lib.ie_sample_top_p_noalloc(ctx.handle, rows, vocab, P(logits), 0.7, 0.9, seed,
                                              step, P(out)))
    torch.cuda.synchronize()
    return host(out).tolist()


def test_top_p_noalloc_matches_workspace_entry(hip, ctx):
    # first call: 16 full-vocabulary rows (2,052,096 of the 2,097,152 scratch floats)
    rows, vocab = 16, V
    say(f"top-p noalloc call 1: rows={rows} vocab={vocab}")
    big = _logits(rows, vocab, 1)
    for step in (0, 5):
        got = _noalloc(hip, ctx, big, rows, vocab, 42, step)
        want = _with_workspace(hip, ctx, big, rows, vocab, 42, step)
        assert got == want, (step, got, want)
        assert all(0 <= t < vocab for t in got)
    # second call, smaller: the scratch still holds the first call's exponentials
    rows2, vocab2 = 3, 50_000
    say(f"top-p noalloc call 2: rows={rows2} vocab={vocab2}")
    small = _logits(rows2, vocab2, 2)
    got2 = _noalloc(hip, ctx, small, rows2, vocab2, 7, 1)
    want2 = _with_workspace(hip, ctx, small, rows2, vocab2, 7, 1)
    assert got2 == want2, (got2, want2)
    assert all(0 <= t < vocab2 for t in got2)


def test_top_p_noalloc_rejects_past_its_scratch(hip, ctx):
    say("top-p noalloc: over-limit shapes are rejected on the host")
    logits = torch.zeros(8, dtype=torch.float32, device="cuda")
    out = torch.zeros(17, dtype=torch.int32, device="cuda")
    for rows, vocab in ((17, 131072), (1, NOALLOC_MAX + 1), (17, 1000)):
        rc = hip.lib.ie_sample_top_p_noalloc(ctx.handle, rows, vocab, P(logits), 0.7, 0.9, 1, 0,
                                             P(out))
        assert rc == IE_ERR_INVALID_ARG
        assert "static scratch" in hip.last_error()
    # exactly at the limit (rows * vocab == the scratch size) the call runs
    rows, vocab = 16, 131072
    say(f"top-p noalloc at the limit: rows={rows} vocab={vocab}")
    lg = _logits(rows, vocab, 3)
    assert _noalloc(hip, ctx, lg, rows, vocab, 5, 2) == _with_workspace(hip, ctx, lg, rows, vocab,
                                                                          5, 2)
