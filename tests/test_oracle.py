"""Pins of the CPU oracle (oracle/attention.py) against things that do not
restate its formulas: torch float64 autograd (an independent implementation),
central finite differences, closed forms and the reference's own known-answer
values.  A dropped term, a wrong sign or index, or a transposed operand in the
oracle fails at least one of these."""

import math

import numpy as np
import pytest
import torch

from oracle import attention as A

RNG = np.random.default_rng(1234)


def _torch_reference(q, k, v, causal, scale, window, softcap, bias, alibi):
    """Independent float64 torch formulation with autograd."""
    q, k, v = (torch.tensor(x, dtype=torch.float64, requires_grad=True) for x in (q, k, v))
    g = q.shape[1] // k.shape[1]
    kk, vv = k.repeat_interleave(g, 1), v.repeat_interleave(g, 1)
    s = torch.einsum("bhid,bhjd->bhij", q, kk) * scale
    if softcap > 0:
        s = softcap * torch.tanh(s / softcap)
    if bias is not None:
        s = s + torch.tensor(bias, dtype=torch.float64)
    sq, sk = s.shape[-2:]
    qi = torch.arange(sq)[:, None] + (sk - sq)
    kj = torch.arange(sk)[None, :]
    if alibi is not None:
        s = s - torch.tensor(alibi, dtype=torch.float64)[None, :, None, None] * (kj - qi).abs()
    keep = torch.ones(sq, sk, dtype=torch.bool)
    if causal:
        keep &= kj <= qi
    if window[0] >= 0:
        keep &= kj >= qi - window[0]
    if window[1] >= 0:
        keep &= kj <= qi + window[1]
    s = s.masked_fill(~keep, float("-inf"))
    valid = keep.any(-1)[None, None, :, None]
    p = torch.where(valid, torch.softmax(torch.where(valid, s, torch.zeros_like(s)), -1), torch.zeros_like(s))
    out = p @ vv
    lse = torch.where(valid[..., 0], torch.logsumexp(torch.where(valid, s, torch.zeros_like(s)), -1),
                      torch.full_like(s[..., 0], float("-inf")))
    return q, k, v, out, lse


CASES = [
    dict(causal=False, window=(-1, -1), softcap=0.0, bias=False, alibi=False),
    dict(causal=True, window=(-1, -1), softcap=0.0, bias=False, alibi=False),
    dict(causal=True, window=(3, 0), softcap=0.0, bias=False, alibi=False),
    dict(causal=False, window=(2, 4), softcap=7.0, bias=True, alibi=True),
    dict(causal=True, window=(-1, -1), softcap=0.0, bias=True, alibi=True),
]


@pytest.mark.parametrize("case", CASES, ids=str)
@pytest.mark.parametrize("sq,sk", [(6, 6), (5, 9), (9, 4)])
def test_oracle_matches_torch_autograd(case, sq, sk):
    q = RNG.standard_normal((2, 4, sq, 8))
    k = RNG.standard_normal((2, 2, sk, 8))
    v = RNG.standard_normal((2, 2, sk, 8))
    do = RNG.standard_normal((2, 4, sq, 8))
    bias = RNG.standard_normal((1, 4, sq, sk)) if case["bias"] else None
    alibi = A.alibi_slopes(4) if case["alibi"] else None
    opts = (case["causal"], 0.4, case["window"], case["softcap"], bias, alibi)
    out, lse = A.attention_forward(q, k, v, *opts)
    tq, tk, tv, tout, tlse = _torch_reference(q, k, v, *opts)
    np.testing.assert_allclose(out, tout.detach().numpy(), atol=1e-12)
    np.testing.assert_array_equal(np.isneginf(lse), np.isneginf(tlse.detach().numpy()))
    fin = np.isfinite(lse)
    np.testing.assert_allclose(lse[fin], tlse.detach().numpy()[fin], atol=1e-12)
    (tout * torch.tensor(do)).sum().backward()
    dq, dk, dv = A.attention_backward(q, k, v, do, *opts)
    np.testing.assert_allclose(dq, tq.grad.numpy(), atol=1e-10)
    np.testing.assert_allclose(dk, tk.grad.numpy(), atol=1e-10)
    np.testing.assert_allclose(dv, tv.grad.numpy(), atol=1e-10)


@pytest.mark.parametrize("case", CASES, ids=str)
def test_backward_matches_finite_differences(case):
    q = RNG.standard_normal((1, 2, 5, 4))
    k = RNG.standard_normal((1, 1, 7, 4))
    v = RNG.standard_normal((1, 1, 7, 4))
    do = RNG.standard_normal((1, 2, 5, 4))
    bias = RNG.standard_normal((1, 2, 5, 7)) if case["bias"] else None
    alibi = A.alibi_slopes(2) if case["alibi"] else None
    opts = (case["causal"], 0.7, case["window"], case["softcap"], bias, alibi)
    grads = A.attention_backward(q, k, v, do, *opts)
    loss = lambda q_, k_, v_: np.sum(A.attention_forward(q_, k_, v_, *opts)[0] * do)
    eps = 1e-6
    for idx, (x, g) in enumerate(zip((q, k, v), grads)):
        fd = np.zeros_like(x)
        it = np.nditer(x, flags=["multi_index"])
        for _ in it:
            i = it.multi_index
            xp, xm = x.copy(), x.copy()
            xp[i] += eps
            xm[i] -= eps
            args_p = [q, k, v]
            args_m = [q, k, v]
            args_p[idx], args_m[idx] = xp, xm
            fd[i] = (loss(*args_p) - loss(*args_m)) / (2 * eps)
        np.testing.assert_allclose(g, fd, atol=1e-6)


def test_zero_query_gives_mean_of_values():
    v = RNG.standard_normal((1, 1, 10, 4))
    out, lse = A.attention_forward(np.zeros((1, 1, 3, 4)), RNG.standard_normal((1, 1, 10, 4)), v)
    np.testing.assert_allclose(out[0, 0], np.broadcast_to(v[0, 0].mean(0), (3, 4)), atol=1e-14)
    np.testing.assert_allclose(lse, math.log(10), atol=1e-14)


def test_single_visible_key_returns_its_value():
    k = RNG.standard_normal((1, 1, 4, 8))
    v = RNG.standard_normal((1, 1, 4, 8))
    q = RNG.standard_normal((1, 1, 4, 8))
    out, _ = A.attention_forward(q, k, v, causal=True, window=(0, 0))  # each query sees only key i
    np.testing.assert_allclose(out[0, 0], v[0, 0], atol=1e-14)


def test_empty_rows_are_zero_with_neg_inf_lse():
    q = RNG.standard_normal((1, 1, 6, 4))
    k = RNG.standard_normal((1, 1, 2, 4))
    out, lse = A.attention_forward(q, k, k, causal=True)
    assert np.all(out[0, 0, :4] == 0) and np.all(np.isneginf(lse[0, 0, :4]))
    assert np.all(np.isfinite(lse[0, 0, 4:]))


def test_bottom_right_alignment_last_row_sees_all_keys():
    q = RNG.standard_normal((1, 1, 2, 4))
    k = RNG.standard_normal((1, 1, 5, 4))
    v = RNG.standard_normal((1, 1, 5, 4))
    causal, _ = A.attention_forward(q, k, v, causal=True)
    full, _ = A.attention_forward(q, k, v)
    np.testing.assert_allclose(causal[0, 0, 1], full[0, 0, 1], atol=1e-14)


def test_softcap_large_cap_is_identity_and_small_cap_saturates():
    q, k, v = (RNG.standard_normal((1, 1, 4, 4)) for _ in range(3))
    np.testing.assert_allclose(A.attention_forward(q, k, v, softcap=1e9)[0], A.attention_forward(q, k, v)[0],
                               atol=1e-9)
    # cap -> 0: all logits -> 0, uniform weights
    np.testing.assert_allclose(A.attention_forward(q, k, v, softcap=1e-9)[0][0, 0],
                               np.broadcast_to(v[0, 0].mean(0), (4, 4)), atol=1e-6)


def test_alibi_zero_slope_equals_plain_and_bias_equivalence():
    q, k, v = (RNG.standard_normal((1, 2, 5, 4)) for _ in range(3))
    np.testing.assert_allclose(A.attention_forward(q, k, v, alibi=np.zeros(2))[0], A.attention_forward(q, k, v)[0],
                               atol=1e-14)
    slopes = np.array([0.5, 0.25])
    i = np.arange(5)[:, None]
    j = np.arange(5)[None, :]
    bias = -slopes[None, :, None, None] * np.abs(j - i)[None, None]
    np.testing.assert_allclose(A.attention_forward(q, k, v, alibi=slopes)[0],
                               A.attention_forward(q, k, v, bias=bias)[0], atol=1e-14)


def test_alibi_slopes_closed_form():
    np.testing.assert_allclose(A.alibi_slopes(8), [2.0 ** -(i + 1) for i in range(8)])
    np.testing.assert_allclose(A.alibi_slopes(4), [2.0 ** -(2 * (i + 1)) for i in range(4)])
    s12 = A.alibi_slopes(12)
    np.testing.assert_allclose(s12[:8], [2.0 ** -(i + 1) for i in range(8)])
    np.testing.assert_allclose(s12[8:], [2.0 ** -(0.5 + i) for i in range(4)])


def test_split_heuristic_known_answers():
    # interface.py:53-58 / tests/test_decode.py:38-42 of the reference
    assert A.decode_num_splits(1, 4, 1, 16384) > 1
    assert A.decode_num_splits(8, 32, 512, 256) == 1
    # tests/test_paged.py:172-179 of the reference
    assert A.paged_num_splits(1, 8, 16, 256, 96, requested_splits=7) == 7
    assert A.paged_num_splits(1, 8, 16, 4, 96) == 1
    assert A.paged_num_splits(1, 8, 16, 256, 96) == 16
    assert A.paged_num_splits(4, 32, 16, 256, 96, max_context_len=256) == 4
    assert A.paged_num_splits(8, 32, 16, 256, 96, max_context_len=256) == 2
    assert A.paged_num_splits(16, 32, 16, 256, 96, max_context_len=256) == 1
    assert A.paged_num_splits(16, 32, 16, 256, 96, max_context_len=4096) == 16


def test_split_combine_equals_unsplit():
    q = RNG.standard_normal((1, 2, 3, 4))
    k = RNG.standard_normal((1, 2, 20, 4))
    v = RNG.standard_normal((1, 2, 20, 4))
    full, _ = A.attention_forward(q, k, v)
    parts = [A.attention_forward(q, k[:, :, a:b], v[:, :, a:b]) for a, b in ((0, 7), (7, 8), (8, 20))]
    o = np.stack([p[0] for p in parts])
    l = np.stack([p[1] for p in parts])
    empty_o, empty_l = np.zeros_like(full)[None], np.full(l.shape[1:], -np.inf)[None]
    np.testing.assert_allclose(A.split_combine(np.concatenate([o, empty_o]), np.concatenate([l, empty_l])),
                               full, atol=1e-13)


def test_paged_decode_equals_contiguous_gather_and_special_cases():
    B, Hq, Hkv, D, P = 3, 4, 2, 8, 4
    kc = RNG.standard_normal((10, P, Hkv, D))
    vc = RNG.standard_normal((10, P, Hkv, D))
    bt = np.array([[3, 1, 7], [0, 9, 2], [5, 4, 6]])
    q = RNG.standard_normal((B, Hq, D))
    ctx = np.array([9, 12, 1])
    out = A.paged_decode(q, kc, vc, bt, ctx, 0.5)
    for b in range(B):
        keys = np.concatenate([kc[p] for p in bt[b]])[: ctx[b]]   # (n, Hkv, D)
        vals = np.concatenate([vc[p] for p in bt[b]])[: ctx[b]]
        dec = A.decode(q[b][None, :, None], keys.transpose(1, 0, 2)[None], vals.transpose(1, 0, 2)[None], 0.5)
        np.testing.assert_allclose(out[b], dec[0, :, 0], atol=1e-13)
    # zero context, invalid ids -> zeros; context beyond capacity is clamped
    assert np.all(A.paged_decode(q, kc, vc, bt, np.zeros(3), 0.5) == 0)
    assert np.all(A.paged_decode(q[:1], kc, vc, np.array([[-1, 99, 10]]), np.array([12]), 0.5) == 0)
    clamped = A.paged_decode(np.zeros((1, 2, D)), kc, vc, np.array([[0]]), np.array([50]), 0.5)
    np.testing.assert_allclose(clamped[0], vc[0].mean(0).repeat(1, 0), atol=1e-14)


def test_varlen_bounded_intervals_and_equal_lengths():
    assert A.bounded_intervals([-5, 3, 100], 10) == [(0, 3), (3, 7)]
    q = RNG.standard_normal((2, 3, 6, 4))
    packed = lambda t: t.transpose(0, 2, 1, 3).reshape(12, 3, 4)
    out, lse = A.varlen_forward(packed(q), packed(q), packed(q), [0, 6, 12], [0, 6, 12], causal=True)
    dense, dlse = A.attention_forward(q, q, q, causal=True)
    np.testing.assert_allclose(out, packed(dense), atol=1e-14)
    np.testing.assert_allclose(lse, dlse.transpose(1, 0, 2).reshape(3, 12), atol=1e-14)


def test_golden_fixtures():
    """Values written once by tests/golden/make_golden.py with torch float64
    (an implementation independent of the oracle)."""
    import os
    path = os.path.join(os.path.dirname(__file__), "golden", "attention_small.npz")
    data = np.load(path)
    out, lse = A.attention_forward(data["q"], data["k"], data["v"], True, float(data["scale"]), (5, -1),
                                   float(data["softcap"]), data["bias"], data["alibi"])
    np.testing.assert_allclose(out, data["out"], atol=1e-12)
    np.testing.assert_allclose(lse, data["lse"], atol=1e-12)
    dq, dk, dv = A.attention_backward(data["q"], data["k"], data["v"], data["dout"], True, float(data["scale"]),
                                      (5, -1), float(data["softcap"]), data["bias"], data["alibi"])
    np.testing.assert_allclose(dq, data["dq"], atol=1e-10)
    np.testing.assert_allclose(dk, data["dk"], atol=1e-10)
    np.testing.assert_allclose(dv, data["dv"], atol=1e-10)
