"""GPU parity of the causal GQA prefill attention core (ie_attn_prefill_core) against a plain
PyTorch fp32 reference of the same op, at prompt lengths up to BASELINE config 4's 2048 rows
and with a cached prefix (start_pos > 0).  Tolerance: tests/tolerance.py (max-abs / scale and
mean relative error <= 1e-2); the kernel rounds the probabilities to bf16 before P.V, as the
reference's fp16 softmax output does (softmax.cu:55-107).
"""
import math

import pytest
import torch

from gpu_util import P, say
from tolerance import assert_close

pytestmark = pytest.mark.gpu
CTX = 8192


def reference(q, k, v, start_pos):
    """q [S][32][128], k/v [8][CTX][128] (bf16 tensors) -> [S][32][128] fp32."""
    S = q.shape[0]
    n = start_pos + S
    out = torch.empty(S, 32, 128, dtype=torch.float32, device="cuda")
    pos = torch.arange(S, device="cuda")[:, None] + start_pos
    keys = torch.arange(n, device="cuda")[None, :]
    masked = keys > pos
    for h in range(32):
        qh = q[:, h].float()
        kh = k[h // 4, :n].float()
        vh = v[h // 4, :n].float()
        s = torch.matmul(qh, kh.t().contiguous()) / math.sqrt(128.0)
        s = s.masked_fill(masked, float("-inf"))
        out[:, h] = torch.matmul(torch.softmax(s, dim=-1), vh)
    return out


# the kernel forms: 16 rows per 4-wave workgroup below 1280 rows, two 16-row blocks per 8-wave
# workgroup up to 2559 (1500 + 37: the two blocks of a workgroup end in different key tiles), 32
# rows per wave from 2560
@pytest.mark.parametrize("S,start_pos", [(1, 0), (17, 0), (96, 0), (300, 5), (1000, 0),
                                         (1500, 37), (2048, 0), (200, 2000), (2600, 0),
                                         (3000, 1000)])
def test_attn_prefill_core(hip, ctx, S, start_pos):
    say(f"attn_prefill_core S={S} start_pos={start_pos}")
    g = torch.Generator(device="cuda").manual_seed(1000 + S + start_pos)
    q = torch.randn(S, 32, 128, generator=g, device="cuda").to(torch.bfloat16)
    k = torch.zeros(8, CTX, 128, dtype=torch.bfloat16, device="cuda")
    v = torch.zeros_like(k)
    n = start_pos + S
    k[:, :n] = torch.randn(8, n, 128, generator=g, device="cuda").to(torch.bfloat16)
    v[:, :n] = torch.randn(8, n, 128, generator=g, device="cuda").to(torch.bfloat16)
    # rows past the context hold large finite values: the kernel must not read them
    k[:, n:n + 64] = 3.0e4
    v[:, n:n + 64] = 3.0e4
    out = torch.empty(S, 32 * 128, dtype=torch.bfloat16, device="cuda")
    hip.check(hip.lib.ie_attn_prefill_core(ctx.handle, S, start_pos, P(q), P(k), P(v), P(out)))
    torch.cuda.synchronize()
    want = reference(q, k, v, start_pos)
    assert_close(out.float().view(S, 32, 128).cpu().numpy(), want.cpu().numpy(),
                 what=f"attn prefill core S={S} start={start_pos}")
