"""The C++ host path of the dense attention (libfa_torch.so, the
torch.ops.fa_mi355x operators): its autograd function must give exactly the
results of the separately called forward and backward operators (same
kernels, same parameters), across the argument handling it does itself:
head-dim padding, GQA, broadcast bias, ALiBi slopes, dropout seeds, strided
inputs and fp32.  Its backward honours the dS scratch limit."""

import pytest
import torch

from fa_rdna3 import _native, alibi_slopes, flash_attention
from fa_rdna3.interface import _backward, _forward

pytestmark = pytest.mark.gpu
DEVICE = "cuda"


def _rand(shape, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g).to(dtype).to(DEVICE)


CASES = [
    dict(dtype=torch.float16, hq=4, hk=4, sq=200, sk=200, d=64, causal=True),
    dict(dtype=torch.bfloat16, hq=8, hk=2, sq=130, sk=257, d=128, causal=True, window=(64, 0)),
    dict(dtype=torch.float16, hq=4, hk=2, sq=96, sk=96, d=16, causal=False),  # padded to 32
    dict(dtype=torch.float16, hq=4, hk=4, sq=64, sk=80, d=64, causal=False, bias=True),
    dict(dtype=torch.bfloat16, hq=4, hk=4, sq=128, sk=128, d=128, causal=True, softcap=20.0, alibi=True),
    dict(dtype=torch.float16, hq=2, hk=2, sq=128, sk=128, d=64, causal=False, dropout=0.2),
    dict(dtype=torch.float32, hq=2, hk=1, sq=70, sk=90, d=64, causal=True),
    dict(dtype=torch.float16, hq=4, hk=4, sq=100, sk=100, d=64, causal=True, strided=True),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "-".join(f"{k}={v}" for k, v in c.items()))
def test_autograd_operator_equals_forward_and_backward(case):
    dt, hq, hk, sq, sk, d = case["dtype"], case["hq"], case["hk"], case["sq"], case["sk"], case["d"]
    q = _rand((2, hq, sq, d), dt, 1)
    if case.get("strided"):
        # (B, S, H, D) storage viewed as (B, H, S, D): non-unit row stride
        q = _rand((2, sq, hq, d), dt, 1).transpose(1, 2)
    k, v, do = _rand((2, hk, sk, d), dt, 2), _rand((2, hk, sk, d), dt, 3), _rand((2, hq, sq, d), dt, 4)
    bias = _rand((1, hq, sq, sk), torch.float32, 5) if case.get("bias") else None
    alibi = alibi_slopes(hq) if case.get("alibi") else None
    window = case.get("window", (-1, -1))
    softcap = case.get("softcap", 0.0)
    p = case.get("dropout", 0.0)
    scale = d ** -0.5
    seed = 1234

    leaves = [t.detach().clone().requires_grad_(True) for t in (q, k, v)]
    out = _native.ops().attention(*leaves, case["causal"], scale, window[0], window[1], softcap, bias, alibi, p,
                                  seed)
    out.backward(do)

    ref_o, ref_lse = _forward(q, k, v, case["causal"], scale, window, softcap, bias, alibi, p, seed)
    ref_g = _backward(do, q, k, v, ref_o, ref_lse, case["causal"], scale, window, softcap, bias, alibi, p, seed)
    assert out.shape == q.shape and out.dtype == q.dtype
    assert torch.equal(out, ref_o)
    for got, want in zip((t.grad for t in leaves), ref_g):
        assert got.shape == want.shape
        assert torch.equal(got, want)


def test_flash_attention_eager_runs_the_native_operator():
    """flash_attention's eager path is the C++ autograd function: its output's
    grad_fn is the native node, not a Python autograd.Function."""
    q, k, v = (_rand((1, 2, 64, 64), torch.float16, s).requires_grad_(True) for s in (1, 2, 3))
    out = flash_attention(q, k, v, causal=True)
    assert "AttentionFn" in type(out.grad_fn).__name__ or "CppFunction" in type(out.grad_fn).__name__, \
        type(out.grad_fn).__name__


def test_backward_follows_the_ds_scratch_limit():
    """With the dS scratch disabled the native backward recomputes dQ: dV is
    the same kernel's and equal, dQ agrees to the output rounding."""
    q, k, v, do = (_rand((1, 4, 256, 128), torch.float16, s) for s in (1, 2, 3, 4))

    def grads():
        leaves = [t.detach().clone().requires_grad_(True) for t in (q, k, v)]
        flash_attention(*leaves, causal=True).backward(do)
        return [t.grad for t in leaves]

    a = grads()
    saved = _native.set_ds_scratch_limit(0)
    try:
        b = grads()
    finally:
        _native.set_ds_scratch_limit(saved)
    assert torch.equal(a[2], b[2])
    for x, y in zip(a[:2], b[:2]):
        scale = y.float().abs().max().item()
        assert (x.float() - y.float()).abs().max().item() <= 4 * 2 ** -10 * max(scale, 1e-3)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_forward_configurations_agree(dtype):
    """A dense grid of many workgroups runs the one-key-half forward (two
    workgroups per CU), a small one the key-split forward: the same rows
    through both agree to the output rounding, and the LSE to 1e-5."""
    # 4 row blocks x 640 (batch, head): 2560 workgroups, above 8 per CU of
    # the 256-CU MI355X, so the one-half form runs
    big = tuple(_rand((40, 16, 512, 128), dtype, s) for s in (1, 2, 3))
    out_b, lse_b = _forward(*big, True, 128 ** -0.5, (-1, -1), 0.0, None, None, 0.0, 0)
    one = tuple(t[:1].contiguous() for t in big)  # 64 blocks: key-split form
    out_1, lse_1 = _forward(*one, True, 128 ** -0.5, (-1, -1), 0.0, None, None, 0.0, 0)
    ulp = 2.0 ** -10 if dtype == torch.float16 else 2.0 ** -7
    bound = 2 * ulp * out_1.float().abs().clamp_min(1.0)
    assert torch.all((out_b[:1].float() - out_1.float()).abs() <= bound)
    assert not torch.equal(out_b[:1], out_1)  # the two forms did run
    assert (lse_b[:1] - lse_1).abs().max().item() <= 1e-5


@pytest.mark.parametrize("mods", [dict(window=(200, 0)), dict(softcap=30.0), dict(alibi=True), dict(bias=True)],
                         ids=["window", "softcap", "alibi", "bias"])
def test_forward_configurations_agree_with_modifiers(mods):
    """The one-key-half forward (large grid) against the key-split forward
    (small grid) on the same rows, with each score modifier."""
    dt = torch.bfloat16
    big = tuple(_rand((40, 16, 512, 128), dt, s) for s in (5, 6, 7))
    h = 16
    bias = _rand((1, h, 512, 512), torch.float32, 8) if mods.get("bias") else None
    alibi = alibi_slopes(h) if mods.get("alibi") else None
    args = (True, 128 ** -0.5, mods.get("window", (-1, -1)), mods.get("softcap", 0.0), bias, alibi, 0.0, 0)
    out_b, lse_b = _forward(*big, *args)
    out_1, lse_1 = _forward(*(t[:1].contiguous() for t in big), *args)
    bound = 2 * 2.0 ** -7 * out_1.float().abs().clamp_min(1.0)
    assert torch.all((out_b[:1].float() - out_1.float()).abs() <= bound)
    fin = torch.isfinite(lse_1)
    assert torch.equal(fin, torch.isfinite(lse_b[:1]))
    assert (lse_b[:1][fin] - lse_1[fin]).abs().max().item() <= 1e-5


def test_two_per_cu_dq_form_on_a_dense_grid():
    """A dense causal grid above three rounds of workgroups per CU runs dQ
    from stored dS in its two-per-CU form (16-key steps); its dQ equals,
    bit for bit, the one-per-CU form's on the same sequence (same products
    in the same order), and agrees with the recomputing dQ."""
    dt = torch.float16
    q, k, v, do = (_rand((8, 16, 1024, 128), dt, s) for s in (11, 12, 13, 14))  # 8 x 128 = 1024 workgroups

    def dq(*t):
        leaves = [x.detach().clone().requires_grad_(True) for x in t[:3]]
        flash_attention(*leaves, causal=True).backward(t[3])
        return [x.grad for x in leaves]

    big = dq(q, k, v, do)
    one = dq(*(t[:1].contiguous() for t in (q, k, v, do)))  # 128 workgroups: one-per-CU form
    for a, b in zip(big, one):
        assert torch.equal(a[:1], b)
    saved = _native.set_ds_scratch_limit(0)
    try:
        rec = dq(q, k, v, do)
    finally:
        _native.set_ds_scratch_limit(saved)
    scale = rec[0].float().abs().max().item()
    assert (big[0].float() - rec[0].float()).abs().max().item() <= 4 * 2 ** -10 * max(scale, 1e-3)
