"""Gradient parity of the HIP backward against fp32 autograd, judged relative
to the error a same-precision naive attention already makes (behaviour
contract of the reference tests test_backward.py, test_gqa.py,
test_causal_align.py, test_window.py, test_softcap.py, test_alibi.py,
test_bias.py, test_fp32_headdim.py)."""

import math

import pytest
import torch

from attn_refs import attention, check_grads, grads
from fa_rdna3 import alibi_slopes, flash_attention

pytestmark = pytest.mark.gpu
DEVICE = "cuda"


def _rand(shape, dtype):
    return torch.randn(shape, device=DEVICE, dtype=dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("seqlen", [128, 200, 512, 1000])
def test_backward_matches_reference(dtype, causal, head_dim, seqlen):
    torch.manual_seed(seqlen + head_dim)
    shape = (2, 4, seqlen, head_dim)
    q, k, v, do = (_rand(shape, dtype) for _ in range(4))
    check_grads(lambda a, b, c: flash_attention(a, b, c, causal),
                lambda a, b, c: attention(a, b, c, causal=causal), q, k, v, do)


def test_backward_cross_shapes():
    torch.manual_seed(1)
    q = _rand((2, 8, 333, 64), torch.float16)
    k = _rand((2, 8, 777, 64), torch.float16)
    v = _rand((2, 8, 777, 64), torch.float16)
    do = _rand((2, 8, 333, 64), torch.float16)
    check_grads(lambda a, b, c: flash_attention(a, b, c), lambda a, b, c: attention(a, b, c), q, k, v, do)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("q_heads,kv_heads", [(16, 4), (8, 1), (32, 8)])
def test_gqa_backward(causal, q_heads, kv_heads):
    torch.manual_seed(q_heads * 10 + kv_heads)
    q = _rand((2, q_heads, 512, 64), torch.float16)
    k = _rand((2, kv_heads, 512, 64), torch.float16)
    v = _rand((2, kv_heads, 512, 64), torch.float16)
    do = _rand((2, q_heads, 512, 64), torch.float16)
    check_grads(lambda a, b, c: flash_attention(a, b, c, causal),
                lambda a, b, c: attention(a, b, c, causal=causal), q, k, v, do)


@pytest.mark.parametrize("sq,sk", [(128, 384), (200, 200), (384, 128)])
def test_bottom_right_causal_backward(sq, sk):
    torch.manual_seed(sq + sk)
    q = _rand((2, 4, sq, 64), torch.float16)
    k = _rand((2, 4, sk, 64), torch.float16)
    v = _rand((2, 4, sk, 64), torch.float16)
    do = _rand((2, 4, sq, 64), torch.float16)
    check_grads(lambda a, b, c: flash_attention(a, b, c, causal=True),
                lambda a, b, c: attention(a, b, c, causal=True), q, k, v, do)


@pytest.mark.parametrize("causal,window", [(True, (63, 0)), (False, (48, 48)), (False, (100, 0))])
def test_window_backward(causal, window):
    torch.manual_seed(window[0] + int(causal))
    q, k, v, do = (_rand((2, 4, 512, 64), torch.float16) for _ in range(4))
    check_grads(lambda a, b, c: flash_attention(a, b, c, causal, window_size=window),
                lambda a, b, c: attention(a, b, c, causal=causal, window=window), q, k, v, do)


@pytest.mark.parametrize("causal,window", [(True, (31, 0)), (False, (16, 24))])
@pytest.mark.parametrize("sq,sk", [(96, 257), (257, 96)])
def test_window_cross_attention_backward(causal, window, sq, sk):
    torch.manual_seed(11 + int(causal) + sq)
    q = _rand((1, 2, sq, 64), torch.float16)
    k = _rand((1, 2, sk, 64), torch.float16)
    v = _rand((1, 2, sk, 64), torch.float16)
    do = _rand((1, 2, sq, 64), torch.float16)
    check_grads(lambda a, b, c: flash_attention(a, b, c, causal, window_size=window),
                lambda a, b, c: attention(a, b, c, causal=causal, window=window), q, k, v, do)


@pytest.mark.parametrize("causal", [False, True])
def test_softcap_backward(causal):
    torch.manual_seed(int(causal))
    q, k, v, do = (_rand((2, 4, 512, 64), torch.float16) for _ in range(4))
    check_grads(lambda a, b, c: flash_attention(a, b, c, causal, softcap=50.0),
                lambda a, b, c: attention(a, b, c, causal=causal, softcap=50.0), q, k, v, do)


@pytest.mark.parametrize("causal", [False, True])
def test_alibi_backward(causal):
    torch.manual_seed(int(causal))
    slopes = alibi_slopes(8, device=DEVICE)
    q, k, v, do = (_rand((2, 8, 512, 64), torch.float16) for _ in range(4))
    check_grads(lambda a, b, c: flash_attention(a, b, c, causal, alibi_slopes=slopes),
                lambda a, b, c: attention(a, b, c, causal=causal, alibi=slopes), q, k, v, do)


def test_bias_backward():
    torch.manual_seed(1)
    q, k, v, do = (_rand((2, 4, 512, 64), torch.float16) for _ in range(4))
    bias = torch.randn(2, 4, 512, 512, device=DEVICE, dtype=torch.float16)
    check_grads(lambda a, b, c: flash_attention(a, b, c, bias=bias),
                lambda a, b, c: attention(a, b, c, bias=bias), q, k, v, do)


@pytest.mark.parametrize("causal", [False, True])
def test_fp32_backward(causal):
    torch.manual_seed(int(causal))
    q, k, v, do = (_rand((2, 4, 512, 64), torch.float32) for _ in range(4))
    kernel = grads(lambda a, b, c: flash_attention(a, b, c, causal), q, k, v, do)
    exact = grads(lambda a, b, c: attention(a, b, c, causal=causal), q, k, v, do)
    for kg, eg in zip(kernel, exact):
        torch.testing.assert_close(kg, eg, atol=3e-3, rtol=3e-3)


@pytest.mark.parametrize("head_dim", [256, 512])
@pytest.mark.parametrize("causal", [False, True])
def test_large_head_dim(head_dim, causal):
    torch.manual_seed(head_dim + int(causal))
    q, k, v, do = (_rand((1, 2, 192, head_dim), torch.bfloat16) for _ in range(4))
    check_grads(lambda a, b, c: flash_attention(a, b, c, causal),
                lambda a, b, c: attention(a, b, c, causal=causal), q, k, v, do, slack=2e-3)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("head_dim", [16, 48, 80, 96, 192])
def test_nonpow2_head_dim_backward(dtype, head_dim):
    torch.manual_seed(head_dim)
    q, k, v, do = (_rand((2, 4, 256, head_dim), dtype) for _ in range(4))
    check_grads(lambda a, b, c: flash_attention(a, b, c, True),
                lambda a, b, c: attention(a, b, c, causal=True), q, k, v, do, slack=2e-3)


def test_backward_is_deterministic():
    torch.manual_seed(2)
    q, k, v, do = (_rand((2, 8, 384, 128), torch.bfloat16) for _ in range(4))
    k, v = k[:, :2].contiguous(), v[:, :2].contiguous()
    first = grads(lambda a, b, c: flash_attention(a, b, c, True), q, k, v, do)
    second = grads(lambda a, b, c: flash_attention(a, b, c, True), q, k, v, do)
    for a, b in zip(first, second):
        assert torch.equal(a, b)
