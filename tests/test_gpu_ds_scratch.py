"""The dS-scratch backward (dK/dV stores dS, dQ = dS K) against the
recompute backward (dQ recomputes S and dP), on the same inputs: dV comes
from the same kernel and must match bit for bit; delta = rowsum(O dO) is
summed in another order (its own kernel instead of inside dQ), which moves
dK by rounding, and dQ differs in the accumulation order of its products, so
both must agree to a few units of the output dtype's rounding.  Covers dense, GQA, windows, softcap (its dS is
stored quartered), ALiBi, bias, dropout, cross shapes, head_dim 64 and varlen
packing."""

import ctypes

import pytest
import torch

from fa_rdna3 import _native, alibi_slopes, flash_attention, flash_attention_varlen

pytestmark = pytest.mark.gpu
DEVICE = "cuda"


def _both(fn, *tensors):
    def run():
        leaves = [t.detach().clone().requires_grad_(True) for t in tensors[:3]]
        out = fn(*leaves)
        out.backward(tensors[3])
        return out.detach(), [t.grad for t in leaves]

    out_a, g_a = run()
    saved = _native.set_ds_scratch_limit(0)
    try:
        out_b, g_b = run()
    finally:
        _native.set_ds_scratch_limit(saved)
    return out_a, g_a, out_b, g_b


def _check(g_a, g_b, dtype):
    dq_a, dk_a, dv_a = g_a
    dq_b, dk_b, dv_b = g_b
    assert torch.equal(dv_a, dv_b)
    ulp = 2.0 ** -10 if dtype == torch.float16 else 2.0 ** -7
    for x, y in ((dq_a, dq_b), (dk_a, dk_b)):
        scale = y.float().abs().max().item()
        err = (x.float() - y.float()).abs().max().item()
        assert torch.isfinite(x).all()
        assert err <= 4 * ulp * max(scale, 1e-3), (err, scale)


def _rand(shape, dtype):
    return torch.randn(shape, device=DEVICE, dtype=dtype)


CASES = [
    dict(),
    dict(causal=True),
    dict(causal=True, window_size=(100, 0)),
    dict(window_size=(64, 32)),
    dict(causal=True, softcap=30.0),
    dict(causal=True, softcap=30.0, window_size=(200, -1)),
    dict(alibi=True),
    dict(bias=True),
    dict(dropout_p=0.2),
]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("case", range(len(CASES)))
def test_dense_ds_path_matches_recompute(dtype, head_dim, case):
    opts = dict(CASES[case])
    torch.manual_seed(case * 7 + head_dim)
    hq, hk, sq, sk = 8, 2, 300, 421
    q, do = _rand((2, hq, sq, head_dim), dtype), _rand((2, hq, sq, head_dim), dtype)
    k, v = _rand((2, hk, sk, head_dim), dtype), _rand((2, hk, sk, head_dim), dtype)
    if opts.pop("alibi", False):
        opts["alibi_slopes"] = alibi_slopes(hq, device=DEVICE)
    if opts.pop("bias", False):
        opts["bias"] = _rand((1, hq, sq, sk), dtype)
    if "dropout_p" in opts:
        # the same dropout seed for both runs: re-seed torch before each
        gen_state = torch.get_rng_state()

        def fn(a, b, c):
            torch.set_rng_state(gen_state)
            return flash_attention(a, b, c, **opts)
    else:
        def fn(a, b, c):
            return flash_attention(a, b, c, **opts)
    out_a, g_a, out_b, g_b = _both(fn, q, k, v, do)
    assert torch.equal(out_a, out_b)
    _check(g_a, g_b, dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("opts", [dict(causal=True), dict(causal=True, window_size=(256, -1), softcap=50.0),
                                  dict(causal=False)])
def test_varlen_ds_path_matches_recompute(dtype, opts):
    torch.manual_seed(5)
    lengths = [1, 130, 7, 513, 64, 300]
    total = sum(lengths)
    cu = torch.tensor([0] + list(torch.tensor(lengths).cumsum(0)), dtype=torch.int32, device=DEVICE)
    q, do = _rand((total, 8, 128), dtype), _rand((total, 8, 128), dtype)
    k, v = _rand((total, 2, 128), dtype), _rand((total, 2, 128), dtype)
    mx = max(lengths)

    def fn(a, b, c):
        return flash_attention_varlen(a, b, c, cu, cu, mx, mx, **opts)

    out_a, g_a, out_b, g_b = _both(fn, q, k, v, do)
    assert torch.equal(out_a, out_b)
    _check(g_a, g_b, dtype)


@pytest.mark.parametrize("lengths", [[60, 40, 700, 20], [700, 60, 40, 20]])
def test_varlen_understated_max_seqlen_gets_recomputed_dq(lengths):
    """max_seqlen below a sequence's real length: the scratch bound (from
    max_seqlen and total) leaves that sequence's dS no room.  Its heads must
    get the recomputed dQ (as with no scratch at all), not a skipped one; the
    rows both paths define (the first max_seqlen of each sequence) agree."""
    dtype = torch.float16
    torch.manual_seed(11)
    total, mx = sum(lengths), 128
    cu = torch.tensor([0] + list(torch.tensor(lengths).cumsum(0)), dtype=torch.int32, device=DEVICE)
    q, do = _rand((total, 4, 128), dtype), _rand((total, 4, 128), dtype)
    k, v = _rand((total, 2, 128), dtype), _rand((total, 2, 128), dtype)
    # (Rows past max_seqlen are left unwritten by the forward; only dQ rows
    # that both paths define are compared.)
    def fn(a, b, c):
        return flash_attention_varlen(a, b, c, cu, cu, mx, mx, causal=True)

    def grads():
        leaves = [t.detach().clone().requires_grad_(True) for t in (q, k, v)]
        out = fn(*leaves)
        out.backward(do)
        return leaves[0].grad

    dq_a = grads()
    saved = _native.set_ds_scratch_limit(0)
    try:
        dq_b = grads()
    finally:
        _native.set_ds_scratch_limit(saved)
    start = 0
    for n in lengths:
        rows = slice(start, start + min(n, mx))
        a, b = dq_a[rows].float(), dq_b[rows].float()
        scale = b.abs().max().item()
        assert torch.isfinite(a).all() and scale > 0
        assert (a - b).abs().max().item() <= 4 * 2.0 ** -10 * max(scale, 1e-3), n
        start += n


def test_phase_api_dq_needs_its_dkdv_phase_first():
    """The per-kernel entry point (fa_bwd_phase): dQ from dS alone is refused
    until phase 1 of the same problem has filled the scratch, then matches
    the full backward's dQ bit for bit."""
    from fa_rdna3.interface import _backward, _backward_launcher, _forward

    torch.manual_seed(3)
    q, k, v, do = (_rand((1, 4, 300, 128), torch.float16) for _ in range(4))
    scale = 128 ** -0.5
    out, lse = _forward(q, k, v, True, scale, (-1, -1), 0.0, None, None, 0.0, 0)
    launch = _backward_launcher(do, q, k, v, out, lse, True, scale, (-1, -1), 0.0, None, None, 0.0, 0)
    launch(0)
    with pytest.raises(RuntimeError, match="phase 1"):
        launch(2)
    launch(1)
    dq, dk, dv, _ = launch(2)
    ref = _backward(do, q, k, v, out, lse, True, scale, (-1, -1), 0.0, None, None, 0.0, 0)
    torch.cuda.synchronize()
    assert torch.equal(dq, ref[0]) and torch.equal(dk, ref[1]) and torch.equal(dv, ref[2])


@pytest.mark.parametrize("understate", [False, True])
def test_varlen_large_batch_ds_path(understate):
    """A batch of 150 short sequences: the dS regions of sequences past the
    first 64 are found by more than one pass of the wave sum.  Against the
    recompute path; with `understate`, sequence 140 is longer than
    max_seqlen promised, so its heads (and every later sequence's, whose
    regions start after it) fall back to the recomputed dQ."""
    dtype = torch.float16
    g = torch.Generator().manual_seed(21)
    lengths = torch.randint(1, 97, (150,), generator=g).tolist()
    mx = max(lengths)
    if understate:
        lengths[140] = 3 * mx
    total = sum(lengths)
    cu = torch.tensor([0] + list(torch.tensor(lengths).cumsum(0)), dtype=torch.int32, device=DEVICE)
    q, do = _rand((total, 4, 128), dtype), _rand((total, 4, 128), dtype)
    k, v = _rand((total, 2, 128), dtype), _rand((total, 2, 128), dtype)

    def fn(a, b, c):
        return flash_attention_varlen(a, b, c, cu, cu, mx, mx, causal=True)

    out_a, g_a, out_b, g_b = _both(fn, q, k, v, do)
    if not understate:
        assert torch.equal(out_a, out_b)
        _check(g_a, g_b, dtype)
        return
    # Rows past max_seqlen of the long sequence are undefined in both paths.
    keep = torch.ones(total, dtype=torch.bool, device=DEVICE)
    s140 = sum(lengths[:140])
    keep[s140 + mx: s140 + lengths[140]] = False
    ulp = 2.0 ** -10
    for x, y in zip(g_a[:1], g_b[:1]):
        x, y = x[keep].float(), y[keep].float()
        scale = y.abs().max().item()
        assert torch.isfinite(x).all()
        assert (x - y).abs().max().item() <= 4 * ulp * max(scale, 1e-3)


def _grads_at_limit(fn, tensors, limit):
    saved = _native.set_ds_scratch_limit(limit)
    try:
        leaves = [t.detach().clone().requires_grad_(True) for t in tensors[:3]]
        out = fn(*leaves)
        out.backward(tensors[3])
        torch.cuda.synchronize()
        return [t.grad for t in leaves]
    finally:
        _native.set_ds_scratch_limit(saved)


def _min_and_full(q, k, varlen):
    """(one KV head's scratch, whole scratch) for these shapes, from the ABI."""
    p = _native.BwdParams()
    p.fwd.abi_version, p.fwd.dtype = _native.ABI_VERSION, _native.DTYPE_CODE[q.dtype]
    p.fwd.head_dim = q.shape[-1]
    if varlen:
        lengths, mx = varlen
        p.fwd.batch, p.fwd.heads_q, p.fwd.heads_kv = len(lengths), q.shape[1], k.shape[1]
        p.fwd.seqlen_q = p.fwd.seqlen_k = mx
        p.fwd.total_q = p.fwd.total_k = q.shape[0]
        cu = torch.zeros(len(lengths) + 1, dtype=torch.int32)
        p.fwd.cu_seqlens_q = p.fwd.cu_seqlens_k = cu.data_ptr()
    else:
        p.fwd.batch, p.fwd.heads_q, p.fwd.seqlen_q, _ = q.shape
        p.fwd.heads_kv, p.fwd.seqlen_k = k.shape[1], k.shape[2]
    lib = _native.lib()
    return int(lib.fa_bwd_workspace_min_bytes(ctypes.byref(p))), int(lib.fa_bwd_workspace_bytes(ctypes.byref(p)))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("opts", [dict(causal=True), dict(causal=True, window_size=(1500, -1), softcap=30.0)])
@pytest.mark.parametrize("varlen", [False, True])
def test_chunked_ds_path_equals_whole_scratch(dtype, opts, varlen):
    """A scratch of fa_bwd_workspace_min_bytes (half the KV heads' dS, at
    least 1 GiB): dK/dV and dQ run in two chunks of KV heads, the same
    kernels on the same heads, so every gradient is bit-identical to the
    whole-scratch run; both agree with the recompute path."""
    torch.manual_seed(7)
    if varlen:
        lengths = [8192, 5000, 3000, 7000]
        total, mx = sum(lengths), max(lengths)
        cu = torch.tensor([0] + list(torch.tensor(lengths).cumsum(0)), dtype=torch.int32, device=DEVICE)
        q, do = _rand((total, 8, 128), dtype), _rand((total, 8, 128), dtype)
        k, v = _rand((total, 4, 128), dtype), _rand((total, 4, 128), dtype)

        def fn(a, b, c):
            return flash_attention_varlen(a, b, c, cu, cu, mx, mx, **opts)
        half, full = _min_and_full(q, k, (lengths, mx))
    else:
        q, do = _rand((2, 8, 8192, 128), dtype), _rand((2, 8, 8192, 128), dtype)
        k, v = _rand((2, 4, 8192, 128), dtype), _rand((2, 4, 8192, 128), dtype)

        def fn(a, b, c):
            return flash_attention(a, b, c, **opts)
        half, full = _min_and_full(q, k, None)
    assert (1 << 30) < half < full
    whole = _grads_at_limit(fn, (q, k, v, do), full)
    chunked = _grads_at_limit(fn, (q, k, v, do), half)
    recompute = _grads_at_limit(fn, (q, k, v, do), 0)
    print(f"chunked dS: {half} of {full} bytes", flush=True)
    for a, b in zip(whole, chunked):
        assert torch.equal(a, b)
    _check(whole, recompute, dtype)


def test_chunked_ds_path_odd_kv_heads():
    """Three KV heads (GQA group 2) split into chunks of 2 and 1 KV heads:
    bit-identical to the whole scratch."""
    torch.manual_seed(8)
    dtype = torch.float16
    q, do = _rand((2, 6, 8192, 128), dtype), _rand((2, 6, 8192, 128), dtype)
    k, v = _rand((2, 3, 8192, 128), dtype), _rand((2, 3, 8192, 128), dtype)

    def fn(a, b, c):
        return flash_attention(a, b, c, causal=True)

    half, full = _min_and_full(q, k, None)
    assert (half - 1024) * 3 == (full - 1024) * 2
    whole = _grads_at_limit(fn, (q, k, v, do), full)
    chunked = _grads_at_limit(fn, (q, k, v, do), half)
    for a, b in zip(whole, chunked):
        assert torch.equal(a, b)
