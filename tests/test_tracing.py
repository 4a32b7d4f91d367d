"""Tracers over the native dense operators: the differentiable
``fa_mi355x::attention`` reaches ``fa_mi355x::forward`` / ``backward`` through
the dispatcher, whose Meta kernels give FakeTensorMode and make_fx the output
shapes without a launch (the reference's ``register_fake`` contract,
interface.py:283-297, 420-422)."""

import math

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode
from torch.fx.experimental.proxy_tensor import make_fx

from fa_rdna3 import _native

ARGS = (True, 0.125, -1, -1, 0.0, None, None, 0.0, 0)


def _qkv(device, dtype=torch.float16, grad=False, d=40):
    q = torch.empty(2, 4, 64, d, device=device, dtype=dtype, requires_grad=grad)
    k = torch.empty(2, 2, 80, d, device=device, dtype=dtype, requires_grad=grad)
    v = torch.empty(2, 2, 80, d, device=device, dtype=dtype, requires_grad=grad)
    return q, k, v


def test_meta_forward_backward_shapes():
    ops = _native.ops()
    q, k, v = _qkv("meta", torch.bfloat16, grad=True)
    out = ops.attention(q, k, v, *ARGS)
    assert out.shape == q.shape and out.dtype == q.dtype and out.device.type == "meta"
    out.backward(torch.empty_like(out))
    assert q.grad.shape == q.shape and k.grad.shape == k.shape and v.grad.shape == v.shape
    o, lse = ops.forward(q.detach(), k.detach(), v.detach(), *ARGS)
    assert lse.shape == (2, 4, 64) and lse.dtype == torch.float32


def test_fake_tensor_mode_cpu():
    ops = _native.ops()
    with FakeTensorMode():
        q, k, v = _qkv("cpu", grad=True)
        out = ops.attention(q, k, v, *ARGS)
        assert out.shape == q.shape and out.dtype == torch.float16
        out.sum().backward()
        assert k.grad.shape == k.shape


def test_make_fx_records_native_operators():
    ops = _native.ops()

    def f(q, k, v):
        return ops.attention(q, k, v, *ARGS)

    gm = make_fx(f, tracing_mode="fake")(*_qkv("cpu"))
    targets = {str(n.target) for n in gm.graph.nodes if n.op == "call_function"}
    assert "fa_mi355x.forward.default" in targets, targets


@pytest.mark.gpu
def test_flash_attention_under_fake_mode_and_make_fx():
    """The public entry point on fake CUDA tensors and under make_fx (fake and
    real tracing): output shapes and dtypes, forward and backward recorded."""
    from fa_rdna3 import flash_attention

    for dtype in (torch.float16, torch.bfloat16):
        with FakeTensorMode():
            q, k, v = _qkv("cuda", dtype, grad=True, d=128)
            out = flash_attention(q, k, v, causal=True)
            assert out.shape == q.shape and out.dtype == dtype and out.device.type == "cuda"
            out.sum().backward()
            assert q.grad.shape == q.shape and v.grad.shape == v.shape

    def fwd_bwd(q, k, v, do):
        q, k, v = (t.detach().requires_grad_(True) for t in (q, k, v))
        out = flash_attention(q, k, v, causal=True, softmax_scale=1 / math.sqrt(64))
        return torch.autograd.grad(out, (q, k, v), do)

    g = torch.Generator().manual_seed(0)
    real = [torch.randn(1, 2, 96, 64, generator=g).half().cuda() for _ in range(4)]
    for mode in ("fake", "real"):
        gm = make_fx(fwd_bwd, tracing_mode=mode)(*real)
        targets = {str(n.target) for n in gm.graph.nodes if n.op == "call_function"}
        assert {"fa_mi355x.forward.default", "fa_mi355x.backward.default"} <= targets, targets
    # The real-mode graph replays on the GPU to the eager gradients.
    gm = make_fx(fwd_bwd, tracing_mode="real")(*real)
    for a, b in zip(gm(*real), fwd_bwd(*real)):
        torch.testing.assert_close(a, b, atol=0, rtol=0)
