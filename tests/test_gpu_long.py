"""Long sequences (32K keys): forward rows against an exact fp32 reference
computed for a subset of rows, and backward through size-independent
identities (sum_j dV_j = sum_i dO_i over rows that see a key; sum_j dK_j = 0
because every row of dS sums to zero)."""

import math

import pytest
import torch

from fa_rdna3 import flash_attention

pytestmark = pytest.mark.gpu
DEVICE = "cuda"


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_long_causal_forward_rows(dtype):
    torch.manual_seed(0)
    S, D = 32768, 128
    q = torch.randn(1, 4, S, D, device=DEVICE, dtype=dtype)
    k = torch.randn(1, 2, S, D, device=DEVICE, dtype=dtype)
    v = torch.randn_like(k)
    with torch.no_grad():
        out = flash_attention(q, k, v, causal=True)
    scale = 1.0 / math.sqrt(D)
    tol = 2e-3 if dtype == torch.float16 else 1e-2
    for r0 in (0, S // 2 - 32, S - 64):
        rows = torch.arange(r0, r0 + 64, device=DEVICE)
        for h in range(4):
            s = (q[0, h, rows].float() @ k[0, h // 2].float().T) * scale
            s = s.masked_fill(torch.arange(S, device=DEVICE)[None, :] > rows[:, None], float("-inf"))
            ref = torch.softmax(s, dim=-1) @ v[0, h // 2].float()
            torch.testing.assert_close(out[0, h, rows].float(), ref, atol=tol, rtol=0)


def test_long_causal_backward_identities():
    torch.manual_seed(1)
    S, D = 32768, 128
    q = torch.randn(1, 4, S, D, device=DEVICE, dtype=torch.float16, requires_grad=True)
    k = torch.randn(1, 4, S, D, device=DEVICE, dtype=torch.float16, requires_grad=True)
    v = torch.randn(1, 4, S, D, device=DEVICE, dtype=torch.float16, requires_grad=True)
    do = torch.randn(1, 4, S, D, device=DEVICE, dtype=torch.float16)
    out = flash_attention(q, k, v, causal=True)
    out.backward(do)
    for name, t in (("dq", q.grad), ("dk", k.grad), ("dv", v.grad)):
        assert torch.isfinite(t).all(), name
    # Every row sees at least its own key, so the rows of P sum to one.
    sum_dv = v.grad.float().sum(dim=2)
    sum_do = do.float().sum(dim=2)
    torch.testing.assert_close(sum_dv, sum_do, atol=2.0, rtol=2e-3)
    # Rows of dS sum to zero: sum_j dK_j = scale * sum_i (sum_j dS_ij) q_i = 0.
    sum_dk = k.grad.float().sum(dim=2)
    scale_dk = k.grad.float().abs().sum(dim=2)
    assert (sum_dk.abs() <= 2e-3 * scale_dk + 1.0).all()
