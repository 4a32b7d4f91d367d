"""Split-K decode and paged-KV decode against fp32 math and the CPU oracle
(behaviour contract of the reference tests test_decode.py, test_paged.py and
test_gqa.py::test_gqa_decode)."""

import math

import numpy as np
import pytest
import torch

from attn_refs import attention
from fa_rdna3 import flash_attention_decode, flash_attention_decode_paged
from oracle import attention as oracle

pytestmark = pytest.mark.gpu
DEVICE = "cuda"
TOL = {torch.float16: 3e-3, torch.bfloat16: 2e-2}


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("seqlen_q", [1, 4])
@pytest.mark.parametrize("seqlen_k", [128, 1000, 4096, 16384])
def test_decode_matches_reference(dtype, head_dim, seqlen_q, seqlen_k):
    torch.manual_seed(seqlen_k + head_dim + seqlen_q)
    q = torch.randn(2, 8, seqlen_q, head_dim, device=DEVICE, dtype=dtype)
    k = torch.randn(2, 8, seqlen_k, head_dim, device=DEVICE, dtype=dtype)
    v = torch.randn_like(k)
    with torch.no_grad():
        out = flash_attention_decode(q, k, v)
    ref = attention(q.float(), k.float(), v.float())
    torch.testing.assert_close(out.float(), ref, atol=TOL[dtype], rtol=TOL[dtype])


@pytest.mark.parametrize("q_heads,kv_heads", [(32, 8), (16, 2), (8, 8)])
def test_gqa_decode(q_heads, kv_heads):
    torch.manual_seed(q_heads + kv_heads)
    q = torch.randn(1, q_heads, 1, 128, device=DEVICE, dtype=torch.float16)
    k = torch.randn(1, kv_heads, 8192, 128, device=DEVICE, dtype=torch.float16)
    v = torch.randn_like(k)
    out = flash_attention_decode(q, k, v)
    torch.testing.assert_close(out.float(), attention(q.float(), k.float(), v.float()), atol=3e-3, rtol=3e-3)


@pytest.mark.parametrize("head_dim", [16, 32, 256, 512])
def test_decode_head_dims(head_dim):
    torch.manual_seed(head_dim)
    q = torch.randn(2, 4, 2, head_dim, device=DEVICE, dtype=torch.float16)
    k = torch.randn(2, 2, 3000, head_dim, device=DEVICE, dtype=torch.float16)
    v = torch.randn_like(k)
    out = flash_attention_decode(q, k, v)
    torch.testing.assert_close(out.float(), attention(q.float(), k.float(), v.float()), atol=3e-3, rtol=3e-3)


def test_decode_many_query_rows():
    # group 4 x Sq 12 = 48 packed rows: more than one 32-row block per KV head
    torch.manual_seed(12)
    q = torch.randn(2, 8, 12, 64, device=DEVICE, dtype=torch.bfloat16)
    k = torch.randn(2, 2, 2048, 64, device=DEVICE, dtype=torch.bfloat16)
    v = torch.randn_like(k)
    out = flash_attention_decode(q, k, v)
    torch.testing.assert_close(out.float(), attention(q.float(), k.float(), v.float()), atol=2e-2, rtol=2e-2)


def test_decode_cache_seqlens_matches_oracle():
    torch.manual_seed(21)
    lens = torch.tensor([0, 1, 31, 1000, 2047], dtype=torch.int32)
    q = torch.randn(5, 8, 1, 64, dtype=torch.float16)
    k = torch.randn(5, 2, 2047, 64, dtype=torch.float16)
    v = torch.randn_like(k)
    out = flash_attention_decode(q.to(DEVICE), k.to(DEVICE), v.to(DEVICE), cache_seqlens=lens.to(DEVICE))
    ref = oracle.decode(q.float().numpy(), k.float().numpy(), v.float().numpy(), cache_seqlens=lens.numpy())
    np.testing.assert_allclose(out.float().cpu().numpy(), ref, atol=2e-3, rtol=0)
    assert torch.all(out[0] == 0)


def test_decode_is_inference_only():
    q = torch.randn(1, 2, 1, 64, device=DEVICE, dtype=torch.float16, requires_grad=True)
    k = torch.randn(1, 2, 128, 64, device=DEVICE, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="inference-only"):
        flash_attention_decode(q, k, k)


def _paged_reference(query, k_cache, v_cache, block_table, context_lens, scale):
    return torch.from_numpy(oracle.paged_decode(
        query.float().cpu().numpy(), k_cache.float().cpu().numpy(), v_cache.float().cpu().numpy(),
        block_table.cpu().numpy(), context_lens.cpu().numpy(), scale)).float()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("q_heads,kv_heads", [(8, 8), (8, 2)])
@pytest.mark.parametrize("head_dim", [64, 128])
def test_paged_decode(dtype, q_heads, kv_heads, head_dim):
    torch.manual_seed(q_heads + kv_heads + head_dim)
    bs = 16
    context = torch.tensor([100, 63, 16], device=DEVICE, dtype=torch.int32)
    nblk = math.ceil(100 / bs)
    q = torch.randn(3, q_heads, head_dim, device=DEVICE, dtype=dtype)
    kc = torch.randn(3 * nblk, bs, kv_heads, head_dim, device=DEVICE, dtype=dtype)
    vc = torch.randn_like(kc)
    bt = torch.arange(3 * nblk, device=DEVICE, dtype=torch.int32).reshape(3, nblk)
    out = flash_attention_decode_paged(q, kc, vc, bt, context)
    ref = _paged_reference(q, kc, vc, bt, context, 1 / math.sqrt(head_dim))
    torch.testing.assert_close(out.float().cpu(), ref, atol=TOL[dtype], rtol=TOL[dtype])


def test_paged_zero_context_returns_zeros():
    q = torch.randn(2, 4, 64, device=DEVICE, dtype=torch.float16)
    kc = torch.randn(4, 16, 4, 64, device=DEVICE, dtype=torch.float16)
    out = flash_attention_decode_paged(q, kc, torch.randn_like(kc), torch.zeros(2, 1, device=DEVICE, dtype=torch.int32),
                                       torch.zeros(2, device=DEVICE, dtype=torch.int32))
    assert torch.all(out == 0)


@pytest.mark.parametrize("num_splits", [1, 3, 7, 32])
def test_paged_forced_splits(num_splits):
    torch.manual_seed(31 + num_splits)
    ctx = torch.tensor([0, 1, 15, 16, 17, 49], device=DEVICE, dtype=torch.int32)
    nblk = math.ceil(49 / 16)
    q = torch.randn(6, 4, 64, device=DEVICE, dtype=torch.float16)
    kc = torch.randn(6 * nblk, 16, 2, 64, device=DEVICE, dtype=torch.float16)
    vc = torch.randn_like(kc)
    bt = torch.randperm(6 * nblk, device=DEVICE, dtype=torch.int32).reshape(6, nblk)
    out = flash_attention_decode_paged(q, kc, vc, bt, ctx, num_splits=num_splits)
    ref = _paged_reference(q, kc, vc, bt, ctx, 0.125)
    torch.testing.assert_close(out.float().cpu(), ref, atol=3e-3, rtol=3e-3)


@pytest.mark.parametrize("block_size", [1, 8, 32, 64, 256])
def test_paged_block_sizes(block_size):
    torch.manual_seed(block_size)
    ctx = torch.tensor([0, 1, block_size - 1, block_size, block_size + 5, 3 * block_size + 7],
                       device=DEVICE, dtype=torch.int32)
    nblk = math.ceil(int(ctx.max()) / block_size)
    q = torch.randn(6, 4, 64, device=DEVICE, dtype=torch.float16)
    kc = torch.randn(6 * nblk, block_size, 2, 64, device=DEVICE, dtype=torch.float16)
    vc = torch.randn_like(kc)
    bt = torch.arange(6 * nblk, device=DEVICE, dtype=torch.int32).reshape(6, nblk)
    out = flash_attention_decode_paged(q, kc, vc, bt, ctx, num_splits=3)
    torch.testing.assert_close(out.float().cpu(), _paged_reference(q, kc, vc, bt, ctx, 0.125), atol=3e-3, rtol=3e-3)


def test_paged_strided_metadata():
    torch.manual_seed(8)
    q = torch.randn(3, 4, 64, device=DEVICE, dtype=torch.float16)
    kc = torch.randn(6, 16, 4, 64, device=DEVICE, dtype=torch.float16)
    vc = torch.randn_like(kc)
    storage = torch.zeros(3, 4, device=DEVICE, dtype=torch.int32)
    bt = storage[:, ::2]
    bt.copy_(torch.arange(6, device=DEVICE, dtype=torch.int32).reshape(3, 2))
    ctx = torch.zeros(6, device=DEVICE, dtype=torch.int32)[::2]
    ctx.fill_(31)
    assert not bt.is_contiguous() and not ctx.is_contiguous()
    out = flash_attention_decode_paged(q, kc, vc, bt, ctx, num_splits=3)
    torch.testing.assert_close(out.float().cpu(), _paged_reference(q, kc, vc, bt, ctx, 0.125), atol=3e-3, rtol=3e-3)


def test_paged_invalid_blocks_are_ignored():
    q = torch.randn(2, 4, 64, device=DEVICE, dtype=torch.float16)
    kc = torch.randn(2, 16, 4, 64, device=DEVICE, dtype=torch.float16)
    bt = torch.tensor([[-1], [99]], device=DEVICE, dtype=torch.int32)
    out = flash_attention_decode_paged(q, kc, torch.randn_like(kc), bt,
                                       torch.full((2,), 16, device=DEVICE, dtype=torch.int32), num_splits=3)
    assert torch.all(out == 0)


def test_paged_context_clamped_to_table_capacity():
    q = torch.zeros(1, 2, 64, device=DEVICE, dtype=torch.float16)
    kc = torch.randn(1, 16, 2, 64, device=DEVICE, dtype=torch.float16)
    vc = torch.randn_like(kc)
    out = flash_attention_decode_paged(q, kc, vc, torch.zeros(1, 1, device=DEVICE, dtype=torch.int32),
                                       torch.tensor([32], device=DEVICE, dtype=torch.int32), num_splits=3)
    torch.testing.assert_close(out.float(), vc.float().mean(dim=1), atol=3e-3, rtol=3e-3)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("P", [16, 8, 4])
def test_paged_equals_contiguous_decode(dtype, P):
    """Scattering a contiguous cache into random pages must not change the
    answer beyond output rounding (pages of 16 keys and of 4 / 8 keys take
    two page-lookup variants of the streaming kernel)."""
    torch.manual_seed(77)
    B, Hq, Hkv, D, S = 3, 16, 4, 128, 3000
    q = torch.randn(B, Hq, 1, D, device=DEVICE, dtype=dtype)
    k = torch.randn(B, Hkv, S, D, device=DEVICE, dtype=dtype)
    v = torch.randn_like(k)
    lens = torch.tensor([3000, 1234, 17], device=DEVICE, dtype=torch.int32)
    contiguous = flash_attention_decode(q, k, v, cache_seqlens=lens)[:, :, 0]
    nblk = math.ceil(S / P)
    perm = torch.randperm(B * nblk, device=DEVICE)
    bt = perm.to(torch.int32).reshape(B, nblk)
    kc = torch.empty(B * nblk, P, Hkv, D, device=DEVICE, dtype=dtype)
    vc = torch.empty_like(kc)
    kpad = torch.nn.functional.pad(k, (0, 0, 0, nblk * P - S)).reshape(B, Hkv, nblk, P, D).permute(0, 2, 3, 1, 4)
    vpad = torch.nn.functional.pad(v, (0, 0, 0, nblk * P - S)).reshape(B, Hkv, nblk, P, D).permute(0, 2, 3, 1, 4)
    kc[bt.long().reshape(-1)] = kpad.reshape(B * nblk, P, Hkv, D)
    vc[bt.long().reshape(-1)] = vpad.reshape(B * nblk, P, Hkv, D)
    paged = flash_attention_decode_paged(q[:, :, 0], kc, vc, bt, lens)
    ulp = {torch.float16: 2 ** -10, torch.bfloat16: 2 ** -7}[dtype]
    bound = ulp * contiguous.float().abs().clamp_min(1.0)
    assert torch.all((paged.float() - contiguous.float()).abs() <= bound)
