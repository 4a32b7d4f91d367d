"""KV-cache entry point (cache append + causal decode over per-sequence
lengths) against the CPU oracle: the cache rows are compared bit for bit,
outputs within the fp16 / bf16 tolerances."""

import numpy as np
import pytest
import torch

from fa_rdna3 import flash_attention_decode, flash_attention_with_kvcache
from oracle import attention as oracle

pytestmark = pytest.mark.gpu
DEVICE = "cuda"
TOL = {torch.float16: 2e-3, torch.bfloat16: 1e-2}


def _case(seed, B, Hq, Hkv, Sq, Sc, Snew, D, dtype):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Hq, Sq, D, generator=g).to(dtype)
    kc = torch.randn(B, Hkv, Sc, D, generator=g).to(dtype)
    vc = torch.randn(B, Hkv, Sc, D, generator=g).to(dtype)
    kn = torch.randn(B, Hkv, Snew, D, generator=g).to(dtype) if Snew else None
    vn = torch.randn(B, Hkv, Snew, D, generator=g).to(dtype) if Snew else None
    return q, kc, vc, kn, vn


def _run(q, kc, vc, kn, vn, lens, causal):
    dq, dkc, dvc = q.to(DEVICE), kc.to(DEVICE), vc.to(DEVICE)
    dkn = None if kn is None else kn.to(DEVICE)
    dvn = None if vn is None else vn.to(DEVICE)
    dl = None if lens is None else lens.to(DEVICE)
    out = flash_attention_with_kvcache(dq, dkc, dvc, dkn, dvn, cache_seqlens=dl, causal=causal)
    torch.cuda.synchronize()
    ref, rk, rv = oracle.kvcache_attention(
        q.float().numpy(), kc.float().numpy(), vc.float().numpy(),
        None if kn is None else kn.float().numpy(), None if vn is None else vn.float().numpy(),
        None if lens is None else lens.numpy(), causal=causal)
    return out, dkc, dvc, ref, rk, rv


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("D", [64, 128])
def test_append_then_causal_decode(dtype, D):
    q, kc, vc, kn, vn = _case(1, 4, 8, 2, 4, 700, 4, D, dtype)
    lens = torch.tensor([0, 3, 345, 696], dtype=torch.int32)  # 696 + 4 fills the cache exactly
    out, dkc, dvc, ref, rk, rv = _run(q, kc, vc, kn, vn, lens, causal=True)
    # The appended rows are copies: exact.
    np.testing.assert_array_equal(dkc.float().cpu().numpy(), rk)
    np.testing.assert_array_equal(dvc.float().cpu().numpy(), rv)
    np.testing.assert_allclose(out.float().cpu().numpy(), ref, atol=TOL[dtype], rtol=0)


def test_rows_past_the_cache_are_dropped():
    q, kc, vc, kn, vn = _case(2, 2, 4, 4, 6, 128, 6, 64, torch.float16)
    lens = torch.tensor([125, 128], dtype=torch.int32)
    out, dkc, dvc, ref, rk, rv = _run(q, kc, vc, kn, vn, lens, causal=True)
    np.testing.assert_array_equal(dkc.float().cpu().numpy(), rk)
    np.testing.assert_array_equal(dvc.float().cpu().numpy(), rv)
    np.testing.assert_allclose(out.float().cpu().numpy(), ref, atol=2e-3, rtol=0)


@pytest.mark.parametrize("Sq", [1, 7, 33])
def test_causal_without_append(Sq):
    # Chunked prefill against a ready cache: bottom-right causal per sequence,
    # including rows that see no key (Sq > len) and a zero-length sequence.
    q, kc, vc, _, _ = _case(3 + Sq, 3, 8, 8, Sq, 1000, 0, 128, torch.float16)
    lens = torch.tensor([0, 20, 1000], dtype=torch.int32)
    out, _, _, ref, _, _ = _run(q, kc, vc, None, None, lens, causal=True)
    np.testing.assert_allclose(out.float().cpu().numpy(), ref, atol=2e-3, rtol=0)
    assert torch.all(out[0] == 0)
    if Sq > 20:
        assert torch.all(out[1, :, :Sq - 20] == 0)


def test_full_cache_causal_matches_forward_oracle():
    q, kc, vc, _, _ = _case(4, 2, 16, 4, 64, 512, 0, 128, torch.bfloat16)
    out, _, _, ref, _, _ = _run(q, kc, vc, None, None, None, causal=True)
    fwd = oracle.attention_forward(q.float().numpy(), kc.float().numpy(), vc.float().numpy(), causal=True)[0]
    np.testing.assert_allclose(ref, fwd, atol=1e-12)
    np.testing.assert_allclose(out.float().cpu().numpy(), ref, atol=1e-2, rtol=0)


def test_single_row_causal_equals_split_k_decode():
    q, kc, vc, _, _ = _case(5, 4, 32, 8, 1, 4096, 0, 128, torch.float16)
    lens = torch.tensor([4096, 1, 2000, 3333], dtype=torch.int32).to(DEVICE)
    dq, dkc, dvc = q.to(DEVICE), kc.to(DEVICE), vc.to(DEVICE)
    a = flash_attention_with_kvcache(dq, dkc, dvc, cache_seqlens=lens, causal=True)
    b = flash_attention_decode(dq, dkc, dvc, cache_seqlens=lens)
    torch.testing.assert_close(a, b, atol=0, rtol=0)


@pytest.mark.parametrize("D", [16, 256])
def test_other_head_dims(D):
    q, kc, vc, kn, vn = _case(6 + D, 2, 4, 2, 3, 300, 3, D, torch.float16)
    lens = torch.tensor([10, 290], dtype=torch.int32)
    out, dkc, dvc, ref, rk, rv = _run(q, kc, vc, kn, vn, lens, causal=True)
    np.testing.assert_array_equal(dkc.float().cpu().numpy(), rk)
    np.testing.assert_allclose(out.float().cpu().numpy(), ref, atol=2e-3, rtol=0)


def test_strided_cache_view_is_updated_in_place():
    # A cache that is a view into a larger buffer (e.g. one layer of a stack).
    q, kc, vc, kn, vn = _case(7, 2, 4, 2, 2, 256, 2, 64, torch.float16)
    big_k = torch.zeros(3, 2, 2, 256, 64, dtype=torch.float16, device=DEVICE)
    big_v = torch.zeros_like(big_k)
    big_k[1].copy_(kc.to(DEVICE))
    big_v[1].copy_(vc.to(DEVICE))
    lens = torch.tensor([100, 7], dtype=torch.int32)
    out = flash_attention_with_kvcache(q.to(DEVICE), big_k[1], big_v[1], kn.to(DEVICE), vn.to(DEVICE),
                                       cache_seqlens=lens.to(DEVICE), causal=True)
    ref, rk, _ = oracle.kvcache_attention(q.float().numpy(), kc.float().numpy(), vc.float().numpy(),
                                          kn.float().numpy(), vn.float().numpy(), lens.numpy(), causal=True)
    np.testing.assert_array_equal(big_k[1].float().cpu().numpy(), rk)
    assert torch.all(big_k[0] == 0) and torch.all(big_k[2] == 0)
    np.testing.assert_allclose(out.float().cpu().numpy(), ref, atol=2e-3, rtol=0)
