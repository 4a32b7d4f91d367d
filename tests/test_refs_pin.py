"""Pins of the two remaining checkers (CPU only).

* ``tests/attn_refs.py`` is the torch reference that the full-size GPU checks
  use (it runs on the GPU there, in fp32).  Here it runs in float64 on the CPU
  and must reproduce the oracle and the committed golden vectors, with every
  modifier it supports (GQA, bottom-right causal, windows, softcap, bias,
  ALiBi, empty rows) and for the packed varlen form.
* ``oracle.varlen_backward`` restates kernels/varlen.py:186-421 (dK/dV and
  dQ of packed sequences).  It is pinned by its reduction to the dense
  backward (equal lengths, packed = batched), by torch float64 autograd of a
  ragged packed case (an independent formulation: per-sequence attention
  concatenated, gradients from autograd), and by central finite differences
  of ``varlen_forward``.
* ``oracle.attention_flops`` is pinned to the reference benchmark's figures
  (bench/benchmark.py:32-36: two GEMMs of 2*Sq*Sk*D flops per (batch, head),
  halved when causal) through hand-computed known answers.
"""

import os

import numpy as np
import pytest
import torch

import attn_refs
from oracle import attention as A

RNG = np.random.default_rng(2024)
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "attention_small.npz")


def _t(x):
    return None if x is None else torch.tensor(x, dtype=torch.float64)


def _refs_forward_backward(q, k, v, do, **kw):
    fn = lambda a, b, c: attn_refs.attention(a, b, c, **kw)
    out = fn(_t(q), _t(k), _t(v))
    dq, dk, dv = attn_refs.grads(fn, _t(q), _t(k), _t(v), _t(do))
    return out.numpy(), dq.numpy(), dk.numpy(), dv.numpy()


def test_attn_refs_reproduce_golden_vectors():
    g = np.load(GOLDEN)
    kw = dict(causal=True, scale=float(g["scale"]), window=(5, -1), softcap=float(g["softcap"]),
              bias=_t(g["bias"]), alibi=_t(g["alibi"]))
    out, dq, dk, dv = _refs_forward_backward(g["q"], g["k"], g["v"], g["dout"], **kw)
    np.testing.assert_allclose(out, g["out"], atol=1e-12)
    np.testing.assert_allclose(dq, g["dq"], atol=1e-10)
    np.testing.assert_allclose(dk, g["dk"], atol=1e-10)
    np.testing.assert_allclose(dv, g["dv"], atol=1e-10)


CASES = [
    dict(causal=False, window=(-1, -1), softcap=0.0, bias=False, alibi=False),
    dict(causal=True, window=(-1, -1), softcap=0.0, bias=False, alibi=False),
    dict(causal=True, window=(4, -1), softcap=0.0, bias=False, alibi=False),
    dict(causal=False, window=(3, 2), softcap=5.0, bias=False, alibi=False),
    dict(causal=True, window=(6, -1), softcap=9.0, bias=True, alibi=True),
    dict(causal=False, window=(-1, -1), softcap=0.0, bias=True, alibi=True),
]


@pytest.mark.parametrize("case", CASES, ids=str)
@pytest.mark.parametrize("sq,sk", [(7, 7), (5, 11), (12, 4)])
def test_attn_refs_match_oracle(case, sq, sk):
    q = RNG.standard_normal((2, 4, sq, 16))
    k = RNG.standard_normal((2, 2, sk, 16))
    v = RNG.standard_normal((2, 2, sk, 16))
    do = RNG.standard_normal((2, 4, sq, 16))
    bias = RNG.standard_normal((2, 4, sq, sk)) if case["bias"] else None
    alibi = A.alibi_slopes(4) if case["alibi"] else None
    opts = dict(causal=case["causal"], scale=0.3, window=case["window"], softcap=case["softcap"])
    out, dq, dk, dv = _refs_forward_backward(q, k, v, do, bias=_t(bias), alibi=_t(alibi), **opts)
    ref_o, _ = A.attention_forward(q, k, v, bias=bias, alibi=alibi, **opts)
    rq, rk, rv = A.attention_backward(q, k, v, do, bias=bias, alibi=alibi, **opts)
    np.testing.assert_allclose(out, ref_o, atol=1e-12)
    np.testing.assert_allclose(dq, rq, atol=1e-10)
    np.testing.assert_allclose(dk, rk, atol=1e-10)
    np.testing.assert_allclose(dv, rv, atol=1e-10)


def test_attn_refs_varlen_matches_oracle():
    lq, lk = [3, 9, 1, 6], [5, 9, 4, 2]
    hq, hk, d = 4, 2, 8
    q = RNG.standard_normal((sum(lq), hq, d))
    k = RNG.standard_normal((sum(lk), hk, d))
    v = RNG.standard_normal((sum(lk), hk, d))
    do = RNG.standard_normal((sum(lq), hq, d))
    cu = lambda ls: np.concatenate([[0], np.cumsum(ls)])
    kw = dict(causal=True, window=(3, -1), softcap=4.0, alibi=A.alibi_slopes(hq))
    fn = lambda a, b, c: attn_refs.varlen_attention(a, b, c, lq, lk, causal=True, window=(3, -1), softcap=4.0,
                                                    alibi=_t(kw["alibi"]))
    out = fn(_t(q), _t(k), _t(v)).numpy()
    ref, _ = A.varlen_forward(q, k, v, cu(lq), cu(lk), **kw)
    np.testing.assert_allclose(out, ref, atol=1e-12)
    g = [x.numpy() for x in attn_refs.grads(fn, _t(q), _t(k), _t(v), _t(do))]
    rg = A.varlen_backward(q, k, v, do, cu(lq), cu(lk), **kw)
    for a, b in zip(g, rg):
        np.testing.assert_allclose(a, b, atol=1e-10)


def _autograd_varlen(q, k, v, do, lq, lk, causal, window, softcap, alibi):
    """Independent float64 formulation: each sequence's dense attention written
    out with torch ops, outputs concatenated, gradients from autograd."""
    tq, tk, tv = (torch.tensor(x, requires_grad=True) for x in (q, k, v))
    g = q.shape[1] // k.shape[1]
    outs, qs, ks = [], 0, 0
    for a, b in zip(lq, lk):
        qq = tq[qs:qs + a].transpose(0, 1)
        kk = tk[ks:ks + b].transpose(0, 1).repeat_interleave(g, 0)
        vv = tv[ks:ks + b].transpose(0, 1).repeat_interleave(g, 0)
        s = qq @ kk.transpose(1, 2) * (1.0 / np.sqrt(q.shape[-1]))
        if softcap > 0:
            s = softcap * torch.tanh(s / softcap)
        i = torch.arange(a)[:, None] + (b - a)
        j = torch.arange(b)[None, :]
        if alibi is not None:
            s = s - torch.tensor(alibi)[:, None, None] * (j - i).abs()
        keep = torch.ones(a, b, dtype=torch.bool)
        if causal:
            keep &= j <= i
        if window[0] >= 0:
            keep &= j >= i - window[0]
        if window[1] >= 0:
            keep &= j <= i + window[1]
        s = s.masked_fill(~keep, float("-inf"))
        has = keep.any(-1)[None, :, None]
        p = torch.where(has, torch.softmax(torch.where(has, s, torch.zeros_like(s)), -1), torch.zeros_like(s))
        outs.append((p @ vv).transpose(0, 1))
        qs += a
        ks += b
    torch.cat(outs, 0).mul(torch.tensor(do)).sum().backward()
    return tq.grad.numpy(), tk.grad.numpy(), tv.grad.numpy()


VARLEN_CASES = [
    dict(causal=False, window=(-1, -1), softcap=0.0, alibi=False),
    dict(causal=True, window=(-1, -1), softcap=0.0, alibi=False),
    dict(causal=True, window=(2, -1), softcap=3.0, alibi=False),
    dict(causal=False, window=(1, 3), softcap=0.0, alibi=True),
]


@pytest.mark.parametrize("case", VARLEN_CASES, ids=str)
def test_varlen_backward_matches_autograd(case):
    lq, lk = [4, 1, 7, 3], [6, 3, 7, 1]
    q = RNG.standard_normal((sum(lq), 4, 8))
    k = RNG.standard_normal((sum(lk), 2, 8))
    v = RNG.standard_normal((sum(lk), 2, 8))
    do = RNG.standard_normal((sum(lq), 4, 8))
    alibi = A.alibi_slopes(4) if case["alibi"] else None
    cu = lambda ls: np.concatenate([[0], np.cumsum(ls)])
    got = A.varlen_backward(q, k, v, do, cu(lq), cu(lk), case["causal"], None, case["window"], case["softcap"],
                            alibi)
    want = _autograd_varlen(q, k, v, do, lq, lk, case["causal"], case["window"], case["softcap"], alibi)
    for a, b in zip(got, want):
        np.testing.assert_allclose(a, b, atol=1e-10)


def test_varlen_backward_equal_lengths_is_dense_backward():
    q = RNG.standard_normal((3, 4, 6, 8))
    k = RNG.standard_normal((3, 2, 6, 8))
    v = RNG.standard_normal((3, 2, 6, 8))
    do = RNG.standard_normal((3, 4, 6, 8))
    pack = lambda t: t.transpose(0, 2, 1, 3).reshape(-1, t.shape[1], t.shape[3])
    cu = [0, 6, 12, 18]
    got = A.varlen_backward(pack(q), pack(k), pack(v), pack(do), cu, cu, causal=True, softcap=5.0)
    want = A.attention_backward(q, k, v, do, causal=True, softcap=5.0)
    for a, b in zip(got, want):
        np.testing.assert_allclose(a, pack(b), atol=1e-13)


def test_varlen_backward_finite_differences_with_bounded_intervals():
    # cu values outside the storage are clamped (varlen.py:21-27); rows outside
    # every interval get no gradient.
    q = RNG.standard_normal((9, 2, 4))
    k = RNG.standard_normal((8, 1, 4))
    v = RNG.standard_normal((8, 1, 4))
    do = RNG.standard_normal((9, 2, 4))
    cu_q, cu_k = [-2, 3, 7], [0, 5, 30]
    opts = dict(causal=True, window=(2, -1), softcap=2.5)
    grads = A.varlen_backward(q, k, v, do, cu_q, cu_k, **opts)
    loss = lambda q_, k_, v_: np.sum(A.varlen_forward(q_, k_, v_, cu_q, cu_k, **opts)[0] * do)
    eps = 1e-6
    for idx, (x, g) in enumerate(zip((q, k, v), grads)):
        fd = np.zeros_like(x)
        for i in np.ndindex(x.shape):
            xp, xm = x.copy(), x.copy()
            xp[i] += eps
            xm[i] -= eps
            a, b = [q, k, v], [q, k, v]
            a[idx], b[idx] = xp, xm
            fd[i] = (loss(*a) - loss(*b)) / (2 * eps)
        np.testing.assert_allclose(g, fd, atol=1e-6)
    assert np.all(grads[0][7:] == 0)


def test_attention_flops_known_answers():
    # bench/benchmark.py:32-36 of the reference: 2 * 2 * B * H * S * S * D,
    # halved (integer) when causal.  Values worked out by hand.
    assert A.attention_flops(2, 16, 2048, 2048, 128, True) == 34_359_738_368
    assert A.attention_flops(2, 16, 2048, 2048, 128, False) == 68_719_476_736
    assert A.attention_flops(1, 16, 1024, 1024, 64, False) == 4_294_967_296
    assert A.attention_flops(1, 1, 3, 5, 7, False) == 420
    # Non-causal: the two GEMMs QK^T and PV at 2*M*N*K flops each.
    b, h, sq, sk, d = 3, 5, 11, 13, 8
    assert A.attention_flops(b, h, sq, sk, d, False) == b * h * (2 * sq * sk * d) * 2
