"""Paged decode of several query rows per sequence (speculative / chunked
decode over a block-table cache) against the CPU oracle, and against the
contiguous kv-cache path on the same keys (paged == contiguous within fp16
rounding)."""

import numpy as np
import pytest
import torch

from fa_rdna3 import flash_attention_decode_paged, flash_attention_decode_paged_multi, flash_attention_with_kvcache
from oracle import attention as oracle

pytestmark = pytest.mark.gpu
DEVICE = "cuda"
TOL = {torch.float16: 2e-3, torch.bfloat16: 1e-2}


def _paged_case(seed, B, Hq, Hkv, Sq, D, P, max_blocks, dtype):
    g = torch.Generator().manual_seed(seed)
    nb = B * max_blocks + 3
    q = torch.randn(B, Hq, Sq, D, generator=g).to(dtype)
    kc = torch.randn(nb, P, Hkv, D, generator=g).to(dtype)
    vc = torch.randn(nb, P, Hkv, D, generator=g).to(dtype)
    bt = torch.randperm(nb, generator=g)[:B * max_blocks].reshape(B, max_blocks).to(torch.int32)
    return q, kc, vc, bt


def _check(q, kc, vc, bt, ctx, causal, dtype, **kw):
    out = flash_attention_decode_paged_multi(q.to(DEVICE), kc.to(DEVICE), vc.to(DEVICE), bt.to(DEVICE),
                                             ctx.to(DEVICE), causal=causal, **kw)
    ref = oracle.paged_attention(q.float().numpy(), kc.float().numpy(), vc.float().numpy(), bt.numpy(),
                                 ctx.numpy(), causal=causal)
    np.testing.assert_allclose(out.float().cpu().numpy(), ref, atol=TOL[dtype], rtol=0)
    return out


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("P", [16, 64])
@pytest.mark.parametrize("Sq", [2, 4, 8])
def test_paged_multi_causal(dtype, P, Sq):
    q, kc, vc, bt = _paged_case(P + Sq, 3, 32, 8, Sq, 128, P, 2048 // P, dtype)
    ctx = torch.tensor([5, 1000, 2048], dtype=torch.int32)
    _check(q, kc, vc, bt, ctx, True, dtype)


@pytest.mark.parametrize("P", [1, 8])
def test_paged_multi_small_pages(P):
    # Pages under 16 keys take the generic kernel.
    q, kc, vc, bt = _paged_case(P, 2, 8, 2, 3, 64, P, 512 // P, torch.float16)
    ctx = torch.tensor([2, 500], dtype=torch.int32)
    _check(q, kc, vc, bt, ctx, True, torch.float16)


def test_paged_multi_non_causal_and_forced_splits():
    q, kc, vc, bt = _paged_case(3, 2, 16, 4, 5, 128, 16, 64, torch.float16)
    ctx = torch.tensor([300, 1024], dtype=torch.int32)
    for splits in (1, 7, 32):
        _check(q, kc, vc, bt, ctx, False, torch.float16, num_splits=splits)


def test_paged_multi_one_row_equals_paged_decode():
    q, kc, vc, bt = _paged_case(4, 4, 32, 8, 1, 128, 16, 256, torch.float16)
    ctx = torch.tensor([4096, 17, 3000, 1], dtype=torch.int32).to(DEVICE)
    a = flash_attention_decode_paged_multi(q.to(DEVICE), kc.to(DEVICE), vc.to(DEVICE), bt.to(DEVICE), ctx)
    b = flash_attention_decode_paged(q[:, :, 0].to(DEVICE), kc.to(DEVICE), vc.to(DEVICE), bt.to(DEVICE), ctx)
    torch.testing.assert_close(a[:, :, 0], b, atol=0, rtol=0)


def test_paged_multi_equals_contiguous_kvcache():
    q, kc, vc, bt = _paged_case(5, 2, 16, 4, 4, 128, 16, 128, torch.float16)
    ctx = torch.tensor([777, 2048], dtype=torch.int32)
    out = flash_attention_decode_paged_multi(q.to(DEVICE), kc.to(DEVICE), vc.to(DEVICE), bt.to(DEVICE),
                                             ctx.to(DEVICE), causal=True)
    # The same keys gathered into a contiguous cache.
    gk = torch.stack([kc[bt[b].long()].reshape(2048, 4, 128).transpose(0, 1) for b in range(2)])
    gv = torch.stack([vc[bt[b].long()].reshape(2048, 4, 128).transpose(0, 1) for b in range(2)])
    ref = flash_attention_with_kvcache(q.to(DEVICE), gk.contiguous().to(DEVICE), gv.contiguous().to(DEVICE),
                                       cache_seqlens=ctx.to(DEVICE), causal=True)
    torch.testing.assert_close(out, ref, atol=1e-3, rtol=0)
