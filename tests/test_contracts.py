"""Host-side contracts that run on CPU: argument validation with the
reference's messages, the platform gate, split heuristics, ALiBi slopes and
the SDPA override's install/restore semantics (behaviour contract of the
reference tests test_validation.py, test_decode.py::test_decode_actually_splits,
test_paged.py::test_paged_split_heuristic, test_alibi.py and
test_sdpa_dispatch.py)."""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import fa_rdna3._validation as validation
from fa_rdna3 import (alibi_slopes, flash_attention, flash_attention_decode, flash_attention_decode_paged,
                      flash_attention_decode_paged_multi, flash_attention_varlen, flash_attention_with_kvcache,
                      sdpa)
from fa_rdna3.interface import _decode_num_splits, _paged_num_splits
from fa_rdna3.sdpa import disable_rdna3_flash_attention, enable_rdna3_flash_attention, use_rdna3_flash_attention
from oracle import attention as oracle


def _dense():
    q = torch.randn(1, 4, 8, 64, dtype=torch.float16)
    return q, torch.randn_like(q), torch.randn_like(q)


def test_platform_detection(monkeypatch):
    monkeypatch.setattr(torch.version, "hip", "7.0")
    monkeypatch.setattr(torch.cuda, "is_available", lambda: True)
    monkeypatch.setattr(torch.cuda, "current_device", lambda: 0)
    monkeypatch.setattr(validation, "_device_arch", lambda i: "gfx950")
    assert validation.unsupported_reason(torch.device("cuda:0")) is None
    assert validation.unsupported_reason("cuda:0") is None
    monkeypatch.setattr(validation, "_device_arch", lambda i: "gfx942")
    assert "gfx950" in validation.unsupported_reason(torch.device("cuda:0"))
    monkeypatch.setattr(torch.version, "hip", None)
    assert "ROCm" in validation.unsupported_reason(torch.device("cuda:0"))


def test_platform_rejects_old_torch(monkeypatch):
    monkeypatch.setattr(validation, "_TORCH_VERSION", (2, 7))
    assert validation.unsupported_reason() == "fa-rdna3 requires PyTorch 2.8 or newer"


def test_cpu_tensors_are_rejected_by_the_platform_gate():
    with pytest.raises(RuntimeError):
        flash_attention(*_dense())


@pytest.mark.parametrize("mutate,match", [
    (lambda q, k, v: (q[0], k, v), "query must have shape"),
    (lambda q, k, v: (q, k.expand(2, -1, -1, -1), v), "same batch size"),
    (lambda q, k, v: (q, k, v.double()), "same dtype"),
    (lambda q, k, v: (q, k[:, :3], v[:, :3]), "multiple"),
    (lambda q, k, v: (q, k[:, :, :-1], v), "same sequence length"),
])
def test_dense_shape_contracts(monkeypatch, mutate, match):
    monkeypatch.setattr(validation, "_require_platform", lambda d: None)
    with pytest.raises(ValueError, match=match):
        flash_attention(*mutate(*_dense()))


@pytest.mark.parametrize("kwargs,match", [
    ({"window_size": (1,)}, "window_size"),
    ({"window_size": (-2, 0)}, "window_size"),
    ({"softcap": -1.0}, "softcap"),
    ({"dropout_p": 1.0}, "dropout_p"),
    ({"softmax_scale": float("nan")}, "softmax_scale"),
    ({"bias": torch.zeros(3, 7)}, "broadcastable"),
    ({"alibi_slopes": torch.ones(3)}, "shape"),
])
def test_dense_modifier_contracts(monkeypatch, kwargs, match):
    monkeypatch.setattr(validation, "_require_platform", lambda d: None)
    with pytest.raises((TypeError, ValueError), match=match):
        flash_attention(*_dense(), **kwargs)


def test_decode_rejects_autograd(monkeypatch):
    monkeypatch.setattr(validation, "_require_platform", lambda d: None)
    q, k, v = _dense()
    q.requires_grad_(True)
    with pytest.raises(RuntimeError, match="inference-only"):
        flash_attention_decode(q, k, v)


def test_decode_cache_seqlens_contract(monkeypatch):
    monkeypatch.setattr(validation, "_require_platform", lambda d: None)
    with pytest.raises(ValueError, match="cache_seqlens"):
        flash_attention_decode(*_dense(), cache_seqlens=torch.zeros(2, dtype=torch.int32))


def test_kvcache_contracts(monkeypatch):
    monkeypatch.setattr(validation, "_require_platform", lambda d: None)
    q = torch.randn(2, 4, 3, 64, dtype=torch.float16)
    kc = torch.randn(2, 2, 32, 64, dtype=torch.float16)
    vc = torch.randn_like(kc)
    kn = torch.randn(2, 2, 3, 64, dtype=torch.float16)
    lens = torch.zeros(2, dtype=torch.int32)
    with pytest.raises(ValueError, match="together"):
        flash_attention_with_kvcache(q, kc, vc, kn, None, cache_seqlens=lens)
    with pytest.raises(ValueError, match="cache_seqlens is required"):
        flash_attention_with_kvcache(q, kc, vc, kn, kn.clone())
    with pytest.raises(ValueError, match="must have shape"):
        flash_attention_with_kvcache(q, kc, vc, kn[:, :1], kn[:, :1], cache_seqlens=lens)
    with pytest.raises(ValueError, match="dtype and device"):
        flash_attention_with_kvcache(q, kc, vc, kn.float(), kn.float(), cache_seqlens=lens)
    with pytest.raises(ValueError, match="in place"):
        kc_t = torch.randn(2, 2, 64, 32, dtype=torch.float16).transpose(2, 3)  # non-unit last stride
        flash_attention_with_kvcache(q, kc_t, vc, kn, kn.clone(), cache_seqlens=lens)
    with pytest.raises(ValueError, match="cache_seqlens"):
        flash_attention_with_kvcache(q, kc, vc, cache_seqlens=lens.long())


def test_kvcache_oracle_reduces_to_decode_and_forward():
    # The cache-update oracle is pinned by its two reductions: no new rows and
    # no mask is `decode`; a full cache with the causal mask is the forward.
    rng = np.random.default_rng(5)
    q = rng.standard_normal((2, 4, 3, 16))
    kc = rng.standard_normal((2, 2, 20, 16))
    vc = rng.standard_normal((2, 2, 20, 16))
    lens = np.array([7, 20])
    out, k2, v2 = oracle.kvcache_attention(q, kc, vc, cache_seqlens=lens)
    np.testing.assert_allclose(out, oracle.decode(q, kc, vc, cache_seqlens=lens), atol=1e-12)
    np.testing.assert_array_equal(k2, kc)
    out, _, _ = oracle.kvcache_attention(q, kc, vc, causal=True)
    np.testing.assert_allclose(out, oracle.attention_forward(q, kc, vc, causal=True)[0], atol=1e-12)
    kn = rng.standard_normal((2, 2, 3, 16))
    vn = rng.standard_normal((2, 2, 3, 16))
    out, k2, v2 = oracle.kvcache_attention(q, kc, vc, kn, vn, cache_seqlens=np.array([5, 18]), causal=True)
    np.testing.assert_array_equal(k2[0, :, 5:8], kn[0])
    np.testing.assert_array_equal(k2[1, :, 18:20], kn[1, :, :2])  # the row past the cache is dropped
    np.testing.assert_array_equal(v2[0, :, :5], vc[0, :, :5])
    ref0 = oracle.attention_forward(q[:1], k2[:1, :, :8], v2[:1, :, :8], causal=True)[0]
    np.testing.assert_allclose(out[:1], ref0, atol=1e-12)


def test_paged_attention_oracle_reductions():
    # Multi-row paged oracle: one row reduces to paged_decode; with all pages
    # valid it equals the kv-cache oracle over the gathered contiguous cache.
    rng = np.random.default_rng(9)
    kc = rng.standard_normal((12, 4, 2, 16))
    vc = rng.standard_normal((12, 4, 2, 16))
    bt = rng.permutation(12).reshape(2, 6)
    ctx = np.array([13, 24])
    q1 = rng.standard_normal((2, 4, 16))
    np.testing.assert_allclose(oracle.paged_attention(q1[:, :, None], kc, vc, bt, ctx)[:, :, 0],
                               oracle.paged_decode(q1, kc, vc, bt, ctx), atol=1e-12)
    q = rng.standard_normal((2, 4, 5, 16))
    gk = np.stack([kc[bt[b]].reshape(24, 2, 16).transpose(1, 0, 2) for b in range(2)])
    gv = np.stack([vc[bt[b]].reshape(24, 2, 16).transpose(1, 0, 2) for b in range(2)])
    ref, _, _ = oracle.kvcache_attention(q, gk, gv, cache_seqlens=ctx, causal=True)
    np.testing.assert_allclose(oracle.paged_attention(q, kc, vc, bt, ctx, causal=True), ref, atol=1e-12)


def test_paged_multi_contract(monkeypatch):
    monkeypatch.setattr(validation, "_require_platform", lambda d: None)
    q = torch.randn(2, 4, 64, dtype=torch.float16)
    kc = torch.randn(8, 16, 2, 64, dtype=torch.float16)
    bt = torch.zeros(2, 4, dtype=torch.int32)
    ctx = torch.ones(2, dtype=torch.int32)
    with pytest.raises(ValueError, match="seqlen_q"):
        flash_attention_decode_paged_multi(q, kc, kc.clone(), bt, ctx)
    with pytest.raises(ValueError, match="seqlen_q"):
        flash_attention_decode_paged_multi(q[:, :, None, :][:, :, :0], kc, kc.clone(), bt, ctx)


def test_fp8_decode_contracts(monkeypatch):
    monkeypatch.setattr(validation, "_require_platform", lambda d: None)
    q = torch.randn(2, 4, 1, 64, dtype=torch.float16)
    k8 = torch.randn(2, 2, 32, 64).to(torch.float8_e4m3fn)
    with pytest.raises(ValueError, match="both be float8"):
        flash_attention_decode(q, k8, torch.randn(2, 2, 32, 64, dtype=torch.float16))
    with pytest.raises(ValueError, match="k_scale"):
        flash_attention_decode(q, k8, k8.clone(), k_scale=0.0)
    with pytest.raises(ValueError, match="fp8 KV caches need head_dim"):
        flash_attention_decode(torch.randn(2, 4, 1, 80, dtype=torch.float16),
                               torch.randn(2, 2, 32, 80).to(torch.float8_e4m3fn),
                               torch.randn(2, 2, 32, 80).to(torch.float8_e4m3fn))
    with pytest.raises(ValueError, match="float8_e4m3fn key / value caches only"):
        flash_attention_decode(q, torch.randn(2, 2, 32, 64, dtype=torch.float16),
                               torch.randn(2, 2, 32, 64, dtype=torch.float16), v_scale=2.0)
    with pytest.raises(ValueError, match="same batch size"):
        flash_attention_decode(q, k8[:1], k8[:1].clone())


def test_varlen_metadata_contracts(monkeypatch):
    monkeypatch.setattr(validation, "_require_platform", lambda d: None)
    q = torch.randn(8, 4, 64, dtype=torch.float16)
    k = torch.randn(8, 2, 64, dtype=torch.float16)
    v = torch.randn_like(k)
    cu64 = torch.tensor([0, 8], dtype=torch.int64)
    cu32 = cu64.to(torch.int32)
    with pytest.raises(ValueError, match="contiguous int32"):
        flash_attention_varlen(q, k, v, cu64, cu64, 8, 8)
    with pytest.raises(ValueError, match="same batch size"):
        flash_attention_varlen(q, k, v, cu32, torch.tensor([0, 4, 8], dtype=torch.int32), 8, 8)
    with pytest.raises(ValueError, match="max_seqlen_q"):
        flash_attention_varlen(q, k, v, cu32, cu32, 9, 8)


def test_paged_metadata_contracts(monkeypatch):
    monkeypatch.setattr(validation, "_require_platform", lambda d: None)
    q = torch.randn(2, 4, 64, dtype=torch.float16)
    k = torch.randn(4, 24, 2, 64, dtype=torch.float16)
    bt = torch.zeros(2, 1, dtype=torch.int32)
    ctx = torch.ones(2, dtype=torch.int32)
    with pytest.raises(ValueError, match="power of two"):
        flash_attention_decode_paged(q, k, torch.randn_like(k), bt, ctx)
    k = torch.randn(4, 16, 2, 64, dtype=torch.float16)
    with pytest.raises(ValueError, match="int32"):
        flash_attention_decode_paged(q, k, torch.randn_like(k), bt.long(), ctx)
    with pytest.raises(ValueError, match="num_splits"):
        flash_attention_decode_paged(q, k, torch.randn_like(k), bt, ctx, num_splits=33)


def test_split_heuristics_match_reference_values():
    assert _decode_num_splits(batch=1, heads=4, seqlen_q=1, seqlen_k=16384) > 1
    assert _decode_num_splits(batch=8, heads=32, seqlen_q=512, seqlen_k=256) == 1
    assert _paged_num_splits(1, 8, 16, 256, 96, requested_splits=7) == 7
    assert _paged_num_splits(1, 8, 16, 4, 96) == 1
    assert _paged_num_splits(1, 8, 16, 256, 96) == 16
    assert _paged_num_splits(4, 32, 16, 256, 96, max_context_len=256) == 4
    assert _paged_num_splits(8, 32, 16, 256, 96, max_context_len=256) == 2
    assert _paged_num_splits(16, 32, 16, 256, 96, max_context_len=256) == 1
    assert _paged_num_splits(16, 32, 16, 256, 96, max_context_len=4096) == 16


@pytest.mark.parametrize("args", [(b, h, sq, sk, t) for b in (1, 4) for h in (4, 32) for sq in (1, 20)
                                  for sk in (100, 8192) for t in (192, 1024)])
def test_split_heuristics_agree_with_oracle(args):
    assert _decode_num_splits(*args) == oracle.decode_num_splits(*args)


@pytest.mark.parametrize("n", [1, 2, 3, 5, 6, 8, 12, 16, 24, 32, 48, 64])
def test_alibi_slopes(n):
    np.testing.assert_allclose(alibi_slopes(n, device="cpu").numpy(), oracle.alibi_slopes(n), rtol=1e-6)


@pytest.mark.parametrize("n_heads", [0, -1, 1.5, True])
def test_alibi_slopes_rejects_invalid(n_heads):
    with pytest.raises(ValueError, match="positive integer"):
        alibi_slopes(n_heads, device="cpu")


def test_dispatch_defers_cpu_tensors_to_original():
    q = torch.randn(1, 2, 4, 8)
    ref = F.scaled_dot_product_attention(q, q, q)
    with use_rdna3_flash_attention():
        torch.testing.assert_close(F.scaled_dot_product_attention(q, q, q), ref)


def test_disable_preserves_later_third_party_override():
    original = F.scaled_dot_product_attention
    q = torch.randn(1, 1, 4, 8)
    ref = original(q, q, q)
    enable_rdna3_flash_attention()
    installed = F.scaled_dot_product_attention

    def third_party(*a, **kw):
        return installed(*a, **kw)

    F.scaled_dot_product_attention = third_party
    disable_rdna3_flash_attention()
    try:
        assert F.scaled_dot_product_attention is third_party
        torch.testing.assert_close(F.scaled_dot_product_attention(q, q, q), ref)
        enable_rdna3_flash_attention()
        assert F.scaled_dot_product_attention is third_party
    finally:
        F.scaled_dot_product_attention = original


def test_context_manager_is_nestable():
    original = F.scaled_dot_product_attention
    with use_rdna3_flash_attention():
        installed = F.scaled_dot_product_attention
        assert installed is sdpa._dispatch_sdpa
        with use_rdna3_flash_attention():
            assert F.scaled_dot_product_attention is installed
        assert F.scaled_dot_product_attention is installed
    assert F.scaled_dot_product_attention is original


def test_context_manager_overlaps_are_refcounted():
    original = F.scaled_dot_product_attention
    first, second = use_rdna3_flash_attention(), use_rdna3_flash_attention()
    first.__enter__()
    installed = F.scaled_dot_product_attention
    second.__enter__()
    first.__exit__(None, None, None)
    assert F.scaled_dot_product_attention is installed
    second.__exit__(None, None, None)
    assert F.scaled_dot_product_attention is original


def test_bypass_routes_to_original():
    q = torch.randn(1, 1, 4, 8)
    with use_rdna3_flash_attention(), sdpa._bypass_rdna3_flash_attention():
        torch.testing.assert_close(F.scaled_dot_product_attention(q, q, q), sdpa._original_sdpa(q, q, q))
