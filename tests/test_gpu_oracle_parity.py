"""HIP kernels against the numpy CPU oracle on small seeded problems covering
every modifier combination the reference supports."""

import itertools
import math

import numpy as np
import pytest
import torch

from fa_rdna3 import alibi_slopes, flash_attention_varlen
from fa_rdna3.interface import _backward, _forward
from oracle import attention as oracle

pytestmark = pytest.mark.gpu
DEVICE = "cuda"
TOL = {torch.float16: (2e-3, 1e-3), torch.bfloat16: (1e-2, 1e-3), torch.float32: (1e-4, 1e-4)}

MODS = [
    dict(causal=False, window=(-1, -1), softcap=0.0, bias=False, alibi=False),
    dict(causal=True, window=(-1, -1), softcap=0.0, bias=False, alibi=False),
    dict(causal=True, window=(40, 0), softcap=0.0, bias=False, alibi=False),
    dict(causal=False, window=(17, 23), softcap=0.0, bias=False, alibi=False),
    dict(causal=False, window=(-1, -1), softcap=20.0, bias=False, alibi=False),
    dict(causal=False, window=(-1, -1), softcap=0.0, bias=True, alibi=False),
    dict(causal=True, window=(-1, -1), softcap=0.0, bias=False, alibi=True),
    dict(causal=True, window=(64, -1), softcap=30.0, bias=True, alibi=True),
]


def _case(dtype, sq, sk, hq, hk, d, m, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(2, hq, sq, d, generator=g).to(dtype)
    k = torch.randn(2, hk, sk, d, generator=g).to(dtype)
    v = torch.randn(2, hk, sk, d, generator=g).to(dtype)
    do = torch.randn(2, hq, sq, d, generator=g).to(dtype)
    bias = torch.randn(1, hq, sq, sk, generator=g) if m["bias"] else None
    slopes = alibi_slopes(hq, device="cpu") if m["alibi"] else None
    return q, k, v, do, bias, slopes


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("mi", range(len(MODS)))
@pytest.mark.parametrize("shape", [(77, 77, 4, 2, 64), (130, 45, 2, 2, 128), (33, 300, 4, 1, 32)])
def test_forward_backward_vs_oracle(dtype, mi, shape):
    m = MODS[mi]
    sq, sk, hq, hk, d = shape
    q, k, v, do, bias, slopes = _case(dtype, sq, sk, hq, hk, d, m, seed=mi * 7 + sq)
    scale = 1.0 / math.sqrt(d)
    dev = lambda t: None if t is None else t.to(DEVICE)
    args = (m["causal"], scale, m["window"], m["softcap"], dev(bias), dev(slopes), 0.0, 0)
    out, lse = _forward(dev(q), dev(k), dev(v), *args)
    dq, dk, dv = _backward(dev(do), dev(q), dev(k), dev(v), out, lse, *args)
    np_ = lambda t: None if t is None else t.float().numpy()
    ref_o, ref_l = oracle.attention_forward(np_(q), np_(k), np_(v), m["causal"], scale, m["window"], m["softcap"],
                                            np_(bias), np_(slopes))
    otol, ltol = TOL[dtype]
    assert np.abs(out.float().cpu().numpy() - ref_o).max() <= otol
    fin = np.isfinite(ref_l)
    l = lse.cpu().numpy()
    assert np.array_equal(np.isfinite(l), fin)
    assert np.abs(l[fin] - ref_l[fin]).max() <= ltol
    rg = oracle.attention_backward(np_(q), np_(k), np_(v), np_(do), m["causal"], scale, m["window"], m["softcap"],
                                   np_(bias), np_(slopes))
    for got, want, name in zip((dq, dk, dv), rg, "qkv"):
        err = np.abs(got.float().cpu().numpy() - want).max()
        # gradient error scales with the gradient magnitude and input rounding
        tol = 3e-3 if dtype == torch.float32 else (2e-2 if dtype == torch.float16 else 1.5e-1)
        assert err <= tol * max(1.0, np.abs(want).max()), (name, err)


def test_varlen_vs_oracle():
    g = torch.Generator().manual_seed(3)
    lengths = [1, 40, 129, 7, 200]
    cu = torch.tensor([0] + list(np.cumsum(lengths)), dtype=torch.int32)
    total = sum(lengths)
    q = torch.randn(total, 8, 64, generator=g).half()
    k = torch.randn(total, 2, 64, generator=g).half()
    v = torch.randn(total, 2, 64, generator=g).half()
    out = flash_attention_varlen(q.to(DEVICE), k.to(DEVICE), v.to(DEVICE), cu.to(DEVICE), cu.to(DEVICE), 200, 200,
                                 causal=True, window_size=(30, -1), softcap=15.0)
    ref, _ = oracle.varlen_forward(q.float().numpy(), k.float().numpy(), v.float().numpy(), cu.numpy(), cu.numpy(),
                                   causal=True, window=(30, -1), softcap=15.0)
    assert np.abs(out.float().cpu().numpy() - ref).max() <= 2e-3


VARLEN_MODS = [
    dict(causal=False, window=(-1, -1), softcap=0.0, alibi=False),
    dict(causal=True, window=(-1, -1), softcap=0.0, alibi=False),
    dict(causal=True, window=(31, 0), softcap=0.0, alibi=False),
    dict(causal=False, window=(-1, -1), softcap=30.0, alibi=False),
    dict(causal=True, window=(-1, -1), softcap=0.0, alibi=True),
    dict(causal=True, window=(100, -1), softcap=50.0, alibi=False),
]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("mi", range(len(VARLEN_MODS)))
@pytest.mark.parametrize("cross", [False, True])
def test_varlen_backward_vs_oracle(dtype, mi, cross):
    """Packed dQ/dK/dV (reference kernels/varlen.py:186-421, cases of
    tests/test_varlen_mods.py:17-43) against oracle.varlen_backward."""
    m = VARLEN_MODS[mi]
    g = torch.Generator().manual_seed(100 + mi * 2 + int(cross))
    lq = [1, 77, 200, 33, 130]
    lk = [5, 60, 200, 129, 1] if cross else lq
    cu_q = torch.tensor([0] + list(np.cumsum(lq)), dtype=torch.int32)
    cu_k = torch.tensor([0] + list(np.cumsum(lk)), dtype=torch.int32)
    hq, hk, d = 4, 2, 64
    q = torch.randn(sum(lq), hq, d, generator=g).to(dtype)
    k = torch.randn(sum(lk), hk, d, generator=g).to(dtype)
    v = torch.randn(sum(lk), hk, d, generator=g).to(dtype)
    do = torch.randn(sum(lq), hq, d, generator=g).to(dtype)
    slopes = alibi_slopes(hq, device="cpu") if m["alibi"] else None
    tq, tk, tv = (t.to(DEVICE).requires_grad_(True) for t in (q, k, v))
    out = flash_attention_varlen(tq, tk, tv, cu_q.to(DEVICE), cu_k.to(DEVICE), max(lq), max(lk),
                                 causal=m["causal"], window_size=m["window"], softcap=m["softcap"],
                                 alibi_slopes=None if slopes is None else slopes.to(DEVICE))
    out.backward(do.to(DEVICE))
    np_ = lambda t: None if t is None else t.float().numpy()
    args = (cu_q.numpy(), cu_k.numpy(), m["causal"], None, m["window"], m["softcap"], np_(slopes))
    ref_o, _ = oracle.varlen_forward(np_(q), np_(k), np_(v), *args)
    otol = TOL[dtype][0]
    assert np.abs(out.detach().float().cpu().numpy() - ref_o).max() <= otol
    rg = oracle.varlen_backward(np_(q), np_(k), np_(v), np_(do), *args)
    tol = 2e-2 if dtype == torch.float16 else 1.5e-1
    for got, want, name in zip((tq.grad, tk.grad, tv.grad), rg, "qkv"):
        err = np.abs(got.float().cpu().numpy() - want).max()
        assert err <= tol * max(1.0, np.abs(want).max()), (name, err)
