"""Forward parity of the HIP kernels against fp32 math attention
(behaviour contract of the reference tests test_forward.py, test_gqa.py,
test_causal_align.py, test_window.py, test_softcap.py, test_alibi.py,
test_bias.py, test_fp32_headdim.py)."""

import math

import pytest
import torch

from attn_refs import assert_ratio, attention, max_err
from fa_rdna3 import alibi_slopes, flash_attention
from fa_rdna3.interface import _bias_args, _forward

pytestmark = pytest.mark.gpu
DEVICE = "cuda"
TOL = {torch.float16: 3e-3, torch.bfloat16: 2e-2}


def _rand(shape, dtype, seed=None):
    return torch.randn(shape, device=DEVICE, dtype=dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("seqlen", [128, 200, 512, 1000, 2048])
def test_matches_fp32_reference(dtype, causal, head_dim, seqlen):
    torch.manual_seed(seqlen + head_dim)
    shape = (2, 4, seqlen, head_dim)
    q, k, v = (_rand(shape, dtype) for _ in range(3))
    scale = 1.0 / math.sqrt(head_dim)
    out = flash_attention(q, k, v, causal=causal, softmax_scale=scale)
    ref = attention(q.float(), k.float(), v.float(), causal=causal, scale=scale)
    torch.testing.assert_close(out.float(), ref, atol=TOL[dtype], rtol=TOL[dtype])


@pytest.mark.parametrize("head_dim", [16, 32, 64, 128, 256, 512])
def test_head_dims(head_dim):
    torch.manual_seed(head_dim)
    q, k, v = (_rand((1, 2, 512, head_dim), torch.float16) for _ in range(3))
    out = flash_attention(q, k, v)
    ref = attention(q.float(), k.float(), v.float())
    torch.testing.assert_close(out.float(), ref, atol=3e-3, rtol=3e-3)


def test_cross_attention_shapes():
    torch.manual_seed(1)
    q = _rand((2, 8, 333, 64), torch.float16)
    k = _rand((2, 8, 777, 64), torch.float16)
    v = _rand((2, 8, 777, 64), torch.float16)
    out = flash_attention(q, k, v)
    torch.testing.assert_close(out.float(), attention(q.float(), k.float(), v.float()), atol=3e-3, rtol=3e-3)


def test_lse_matches_logsumexp():
    torch.manual_seed(0)
    q, k, v = (_rand((2, 4, 512, 64), torch.float16) for _ in range(3))
    scale = 0.125
    _, lse = _forward(q, k, v, False, scale, (-1, -1), 0.0, None, None, 0.0, 0)
    expected = torch.logsumexp((q.float() @ k.float().transpose(-1, -2)) * scale, dim=-1)
    assert max_err(lse, expected) < 1e-3


def test_empty_rows_give_zero_output_and_neg_inf_lse():
    # causal with Sq > Sk: the first Sq - Sk query rows see no key.
    torch.manual_seed(5)
    q = _rand((1, 2, 96, 64), torch.float16)
    k = _rand((1, 2, 40, 64), torch.float16)
    v = _rand((1, 2, 40, 64), torch.float16)
    out, lse = _forward(q, k, v, True, 0.125, (-1, -1), 0.0, None, None, 0.0, 0)
    assert torch.all(out[:, :, :56] == 0)
    assert torch.all(torch.isneginf(lse[:, :, :56]))
    assert torch.isfinite(lse[:, :, 56:]).all()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("q_heads,kv_heads", [(32, 8), (16, 4), (8, 1)])
def test_gqa_forward(dtype, causal, q_heads, kv_heads):
    torch.manual_seed(q_heads + kv_heads)
    q = _rand((2, q_heads, 512, 128), dtype)
    k = _rand((2, kv_heads, 512, 128), dtype)
    v = _rand((2, kv_heads, 512, 128), dtype)
    out = flash_attention(q, k, v, causal=causal)
    ref = attention(q.float(), k.float(), v.float(), causal=causal)
    torch.testing.assert_close(out.float(), ref, atol=TOL[dtype], rtol=TOL[dtype])


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("sq,sk", [(128, 384), (64, 256), (1, 256), (200, 200), (333, 512), (384, 128), (256, 64)])
def test_bottom_right_causal(dtype, sq, sk):
    torch.manual_seed(sq + sk)
    q = _rand((2, 4, sq, 64), dtype)
    k = _rand((2, 4, sk, 64), dtype)
    v = _rand((2, 4, sk, 64), dtype)
    out = flash_attention(q, k, v, causal=True)
    exact = attention(q.float(), k.float(), v.float(), causal=True)
    naive = attention(q, k, v, causal=True)
    assert_ratio(out, naive, exact)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("causal,window", [(True, (63, 0)), (True, (255, 0)), (False, (48, 48)), (False, (100, 0))])
@pytest.mark.parametrize("seqlen", [200, 512])
def test_window(dtype, causal, window, seqlen):
    torch.manual_seed(seqlen + window[0] + int(causal))
    q, k, v = (_rand((2, 4, seqlen, 64), dtype) for _ in range(3))
    out = flash_attention(q, k, v, causal=causal, window_size=window)
    exact = attention(q.float(), k.float(), v.float(), causal=causal, window=window)
    naive = attention(q, k, v, causal=causal, window=window)
    assert_ratio(out, naive, exact)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("softcap", [30.0, 50.0])
def test_softcap(dtype, causal, softcap):
    torch.manual_seed(int(softcap) + int(causal))
    q, k, v = (_rand((2, 4, 300, 64), dtype) for _ in range(3))
    out = flash_attention(q, k, v, causal=causal, softcap=softcap)
    exact = attention(q.float(), k.float(), v.float(), causal=causal, softcap=softcap)
    naive = attention(q, k, v, causal=causal, softcap=softcap)
    assert_ratio(out, naive, exact)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("heads", [8, 12])
def test_alibi(dtype, causal, heads):
    torch.manual_seed(heads + int(causal))
    slopes = alibi_slopes(heads, device=DEVICE)
    q, k, v = (_rand((2, heads, 300, 64), dtype) for _ in range(3))
    out = flash_attention(q, k, v, causal=causal, alibi_slopes=slopes)
    exact = attention(q.float(), k.float(), v.float(), causal=causal, alibi=slopes)
    naive = attention(q, k, v, causal=causal, alibi=slopes)
    assert_ratio(out, naive, exact)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("bias_shape", ["full", "broadcast_batch", "broadcast_head", "row"])
def test_bias(dtype, bias_shape):
    torch.manual_seed(len(bias_shape))
    b, h, s = 2, 4, 200
    q, k, v = (_rand((b, h, s, 64), dtype) for _ in range(3))
    shape = {"full": (b, h, s, s), "broadcast_batch": (1, h, s, s),
             "broadcast_head": (b, 1, s, s), "row": (1, 1, 1, s)}[bias_shape]
    bias = torch.randn(shape, device=DEVICE, dtype=torch.float32)
    out = flash_attention(q, k, v, bias=bias)
    full = bias.expand(b, h, s, s)
    assert_ratio(out, attention(q, k, v, bias=full), attention(q.float(), k.float(), v.float(), bias=full))


def test_bias_in_query_dtype():
    torch.manual_seed(9)
    q, k, v = (_rand((2, 4, 256, 64), torch.bfloat16) for _ in range(3))
    bias = torch.randn(2, 4, 256, 256, device=DEVICE, dtype=torch.bfloat16)
    out = flash_attention(q, k, v, bias=bias)
    assert_ratio(out, attention(q, k, v, bias=bias), attention(q.float(), k.float(), v.float(), bias=bias))


def test_bias_hard_mask():
    torch.manual_seed(3)
    q, k, v = (_rand((2, 4, 256, 64), torch.float16) for _ in range(3))
    keep = torch.rand(2, 4, 256, 256, device=DEVICE) < 0.5
    keep |= torch.eye(256, device=DEVICE, dtype=torch.bool)
    bias = torch.where(keep, 0.0, float("-inf")).float()
    out = flash_attention(q, k, v, bias=bias)
    torch.testing.assert_close(out.float(), attention(q.float(), k.float(), v.float(), bias=bias),
                               atol=3e-3, rtol=3e-3)


def test_bias_fully_masked_rows():
    torch.manual_seed(17)
    q, k, v = (_rand((1, 2, 256, 64), torch.float16).requires_grad_(True) for _ in range(3))
    bias = torch.zeros(1, 2, 256, 256, device=DEVICE)
    bias[:, :, :64] = float("-inf")
    out = flash_attention(q, k, v, bias=bias)
    assert torch.isfinite(out).all()
    torch.testing.assert_close(out.float(), attention(q.float(), k.float(), v.float(), bias=bias),
                               atol=3e-3, rtol=3e-3)
    out.backward(torch.randn_like(out))
    for t in (q, k, v):
        assert torch.isfinite(t.grad).all()
    assert torch.all(q.grad[:, :, :64] == 0)


def test_bias_masked_prefix_gives_mean_of_values():
    q = torch.zeros(1, 2, 256, 64, device=DEVICE, dtype=torch.float16)
    k = torch.zeros_like(q)
    v = torch.randn_like(q)
    bias = torch.full((1, 1, 1, 256), -1000.0, device=DEVICE)
    bias[..., :128] = float("-inf")
    out = flash_attention(q, k, v, bias=bias)
    expected = v[..., 128:, :].float().mean(dim=-2, keepdim=True).expand_as(out)
    torch.testing.assert_close(out.float(), expected, atol=3e-3, rtol=3e-3)


def test_low_precision_bias_is_not_materialized():
    q = torch.empty(2, 4, 64, 64, device=DEVICE, dtype=torch.float16)
    bias = torch.randn(1, 1, 64, 64, device=DEVICE, dtype=torch.float16)
    expanded, *_ = _bias_args(bias, q, 2, 4, 64, 64)
    assert expanded.dtype == bias.dtype and expanded.data_ptr() == bias.data_ptr()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("head_dim", [48, 80, 96, 192])
@pytest.mark.parametrize("causal", [False, True])
def test_nonpow2_head_dim(dtype, head_dim, causal):
    torch.manual_seed(head_dim + int(causal))
    q, k, v = (_rand((2, 4, 256, head_dim), dtype) for _ in range(3))
    out = flash_attention(q, k, v, causal=causal)
    assert out.shape == q.shape
    assert_ratio(out, attention(q, k, v, causal=causal), attention(q.float(), k.float(), v.float(), causal=causal),
                 slack=2e-3)


@pytest.mark.parametrize("causal", [False, True])
def test_fp32_forward(causal):
    torch.manual_seed(int(causal))
    q, k, v = (_rand((2, 4, 512, 64), torch.float32) for _ in range(3))
    out = flash_attention(q, k, v, causal=causal)
    torch.testing.assert_close(out, attention(q, k, v, causal=causal), atol=2e-3, rtol=2e-3)


def test_strided_views_are_accepted():
    # packed qkv (B, S, 3, H, D) viewed as (B, H, S, D): non-contiguous strides.
    torch.manual_seed(4)
    packed = torch.randn(2, 300, 3, 4, 64, device=DEVICE, dtype=torch.float16)
    q, k, v = (t.transpose(1, 2) for t in packed.unbind(2))
    out = flash_attention(q, k, v, causal=True)
    torch.testing.assert_close(out.float(), attention(q.float(), k.float(), v.float(), causal=True),
                               atol=3e-3, rtol=3e-3)


def test_rejects_unsupported_dtype():
    q = torch.randn(1, 1, 64, 64, device=DEVICE, dtype=torch.float64)
    with pytest.raises(ValueError, match="unsupported dtype"):
        flash_attention(q, q, q)


def test_gqa_rejects_indivisible_heads():
    q = torch.randn(1, 6, 128, 64, device=DEVICE, dtype=torch.float16)
    k = torch.randn(1, 4, 128, 64, device=DEVICE, dtype=torch.float16)
    with pytest.raises(ValueError, match="multiple"):
        flash_attention(q, k, k)
