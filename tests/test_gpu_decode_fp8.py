"""Split-K decode over an fp8 (OCP e4m3) KV cache against the CPU oracle on
the dequantised cache (the fp8 -> 16-bit conversion is exact, so the only
differences are the kernel's own rounding)."""

import numpy as np
import pytest
import torch

from fa_rdna3 import flash_attention_decode
from oracle import attention as oracle

pytestmark = pytest.mark.gpu
DEVICE = "cuda"
TOL = {torch.float16: 2e-3, torch.bfloat16: 1e-2}


def _fp8_case(seed, B, Hq, Hkv, Sq, Sk, D, k_scale, v_scale, qdtype):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Hq, Sq, D, generator=g).to(qdtype)
    k = (torch.randn(B, Hkv, Sk, D, generator=g) / k_scale).to(torch.float8_e4m3fn)
    v = (torch.randn(B, Hkv, Sk, D, generator=g) / v_scale).to(torch.float8_e4m3fn)
    return q, k, v


@pytest.mark.parametrize("qdtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("scales", [(1.0, 1.0), (0.25, 3.0)])
def test_fp8_decode_matches_oracle(qdtype, D, scales):
    ks, vs = scales
    q, k, v = _fp8_case(D + int(ks * 8), 4, 32, 8, 1, 4096, D, ks, vs, qdtype)
    lens = torch.tensor([4096, 1, 1000, 2500], dtype=torch.int32)
    out = flash_attention_decode(q.to(DEVICE), k.to(DEVICE), v.to(DEVICE), cache_seqlens=lens.to(DEVICE),
                                 k_scale=ks, v_scale=vs)
    kd = k.float().numpy() * ks
    vd = v.float().numpy() * vs
    ref = oracle.decode(q.float().numpy(), kd, vd, cache_seqlens=lens.numpy())
    np.testing.assert_allclose(out.float().cpu().numpy(), ref, atol=TOL[qdtype] * max(1.0, vs), rtol=0)


@pytest.mark.parametrize("qdtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("D", [256, 512])
def test_fp8_decode_wide_heads_match_oracle(qdtype, D):
    # head_dim > 128 runs the tiled split kernel with fp8 tiles.
    q, k, v = _fp8_case(D + 3, 2, 8, 2, 3, 1100, D, 0.5, 2.0, qdtype)
    lens = torch.tensor([1100, 37], dtype=torch.int32)
    out = flash_attention_decode(q.to(DEVICE), k.to(DEVICE), v.to(DEVICE), cache_seqlens=lens.to(DEVICE),
                                 k_scale=0.5, v_scale=2.0)
    ref = oracle.decode(q.float().numpy(), k.float().numpy() * 0.5, v.float().numpy() * 2.0,
                        cache_seqlens=lens.numpy())
    np.testing.assert_allclose(out.float().cpu().numpy(), ref, atol=2 * TOL[qdtype], rtol=0)


def test_fp8_decode_query_rows_and_head_dim_32():
    q, k, v = _fp8_case(7, 2, 8, 2, 5, 777, 32, 1.0, 1.0, torch.float16)
    out = flash_attention_decode(q.to(DEVICE), k.to(DEVICE), v.to(DEVICE))
    ref = oracle.decode(q.float().numpy(), k.float().numpy(), v.float().numpy())
    np.testing.assert_allclose(out.float().cpu().numpy(), ref, atol=2e-3, rtol=0)


def test_fp8_equals_16bit_decode_on_the_same_values():
    # Power-of-two scales keep the dequantised cache exact in fp16, so the fp8
    # read must agree with the 16-bit read of the same values.
    q, k, v = _fp8_case(8, 2, 16, 4, 1, 3000, 128, 0.5, 2.0, torch.float16)
    out8 = flash_attention_decode(q.to(DEVICE), k.to(DEVICE), v.to(DEVICE), k_scale=0.5, v_scale=2.0)
    k16 = (k.to(torch.float32) * 0.5).half().to(DEVICE)
    v16 = (v.to(torch.float32) * 2.0).half().to(DEVICE)
    out16 = flash_attention_decode(q.to(DEVICE), k16, v16)
    torch.testing.assert_close(out8, out16, atol=2e-3, rtol=0)


def test_fp8_strided_cache_is_copied_to_rows():
    q, k, v = _fp8_case(9, 1, 4, 4, 1, 512, 64, 1.0, 1.0, torch.float16)
    kt = k.to(DEVICE).transpose(2, 3).contiguous().transpose(2, 3)  # non-unit last stride
    out = flash_attention_decode(q.to(DEVICE), kt, v.to(DEVICE))
    ref = oracle.decode(q.float().numpy(), k.float().numpy(), v.float().numpy())
    np.testing.assert_allclose(out.float().cpu().numpy(), ref, atol=2e-3, rtol=0)


@pytest.mark.parametrize("P,D", [(16, 128), (64, 128), (8, 128), (4, 64), (16, 256)])
@pytest.mark.parametrize("Sq", [1, 4])
def test_fp8_paged_decode_matches_oracle(P, D, Sq):
    # Pages of >= 16 keys with head_dim <= 128 take the streaming kernel;
    # smaller pages and wider heads the tiled one.
    from fa_rdna3 import flash_attention_decode_paged, flash_attention_decode_paged_multi
    g = torch.Generator().manual_seed(P + Sq + D)
    B, Hq, Hkv, mb = 3, 32, 8, 2048 // P
    nb = B * mb + 5
    q = torch.randn(B, Hq, Sq, D, generator=g).half()
    kc = (torch.randn(nb, P, Hkv, D, generator=g) / 0.5).to(torch.float8_e4m3fn)
    vc = (torch.randn(nb, P, Hkv, D, generator=g) / 2.0).to(torch.float8_e4m3fn)
    bt = torch.randperm(nb, generator=g)[:B * mb].reshape(B, mb).to(torch.int32)
    ctx = torch.tensor([9, 1500, 2048], dtype=torch.int32)
    args = (kc.to(DEVICE), vc.to(DEVICE), bt.to(DEVICE), ctx.to(DEVICE))
    if Sq == 1:
        out = flash_attention_decode_paged(q[:, :, 0].to(DEVICE), *args, k_scale=0.5, v_scale=2.0)[:, :, None]
    else:
        out = flash_attention_decode_paged_multi(q.to(DEVICE), *args, causal=True, k_scale=0.5, v_scale=2.0)
    ref = oracle.paged_attention(q.float().numpy(), kc.float().numpy() * 0.5, vc.float().numpy() * 2.0,
                                 bt.numpy(), ctx.numpy(), causal=Sq > 1)
    np.testing.assert_allclose(out.float().cpu().numpy(), ref, atol=4e-3, rtol=0)
