"""User-facing FlashAttention entry points, backed by MI355X (gfx950) HIP kernels.

Drop-in for the reference's ``fa_rdna3/interface.py``: same public functions,
op names, op schemas, argument meaning and error behaviour.  Where the
reference launched Triton kernels (``kernel[grid](...)``), this module fills
the C-ABI parameter structs of ``include/fa_mi355x.h`` and calls
``libfa_mi355x.so`` through :mod:`fa_rdna3._native` on the current HIP stream.

``flash_attention`` takes ``(batch, heads, seqlen, head_dim)`` tensors matching
``torch.nn.functional.scaled_dot_product_attention`` and is a differentiable
``torch.library`` custom op (grouped-query attention supported).
``flash_attention_decode`` is the split-K path for small-query / long-KV
decode, ``flash_attention_decode_paged`` walks a vLLM-style block table, and
``flash_attention_varlen`` handles packed variable-length sequences via
``cu_seqlens`` through an ``autograd.Function``.
"""

import math
from numbers import Integral

import torch

from . import _native
from ._native import DTYPE_CODE, ABI_VERSION
from ._validation import (
    LOW_PRECISION_DTYPES,
    SUPPORTED_DTYPES,
    SUPPORTED_HEAD_DIMS,
    validate_attention_options,
    validate_dense_inputs,
    validate_inference_only,
    validate_paged_inputs,
    validate_softmax_scale,
    validate_varlen_inputs,
)

_SUPPORTED_HEAD_DIMS = SUPPORTED_HEAD_DIMS
_SUPPORTED_DTYPES = SUPPORTED_DTYPES

# Smallest head dim the kernels take; 16 is zero-padded to it (zeros add
# nothing to q.k^T or p.v, reference interface.py:406-417 does the same for
# non-power-of-two dims).
_KERNEL_MIN_HEAD_DIM = 32

# Reference default (interface.py:49).  The MI355X callers pass 4 * CU count.
_DECODE_TARGET_PROGRAMS = 192
_DECODE_BLOCK_M = 16


def _cdiv(a, b):
    return -(-a // b)


def _next_power_of_2(n):
    return 1 if n <= 1 else 1 << (int(n) - 1).bit_length()


def _decode_num_splits(batch, heads, seqlen_q, seqlen_k, target_programs=_DECODE_TARGET_PROGRAMS):
    """Split count of the split-K decode (reference interface.py:53-58)."""
    m_blocks = _cdiv(seqlen_q, _DECODE_BLOCK_M)
    base = batch * heads * m_blocks
    wanted = (target_programs + base - 1) // base
    key_blocks = _cdiv(seqlen_k, 64)
    return max(1, min(32, wanted, key_blocks))


def _paged_num_splits(batch, heads, block_size, max_blocks, target_programs,
                      max_context_len=None, requested_splits=None):
    """Split count of the paged decode (reference interface.py:61-77)."""
    if requested_splits is not None:
        return requested_splits
    if max_context_len is None:
        active_blocks = max_blocks
        active_tokens = active_blocks * block_size
    else:
        active_blocks = min(max_blocks, _cdiv(max_context_len, block_size))
        active_tokens = min(max_blocks * block_size, max_context_len)
    if active_tokens <= 64:
        return 1
    split_cap = min(16, active_blocks, target_programs)
    occupancy_splits = _cdiv(5 * target_programs, batch * heads)
    work_splits = min(16, _cdiv(active_tokens, 256))
    return min(split_cap, max(occupancy_splits, work_splits))


def _streaming_decode_splits(batch, kv_heads, packed_rows, max_keys, cus):
    """Split count for the streaming decode kernel (head_dim <= 128).

    That kernel packs the query heads of one KV head into a 16-column block,
    runs one 4-wave workgroup per CU and keeps each wave's chunk loads in
    flight, so the best grid is about one workgroup per CU; each split keeps
    at least 8 chunks of 32 keys (2 per wave) so the partials and their
    merge stay small next to the K/V stream.
    """
    workgroups = batch * kv_heads * _cdiv(packed_rows, 16)
    chunks = _cdiv(max(max_keys, 1), 32)
    return max(1, min(32, _cdiv(cus, workgroups), _cdiv(chunks, 8)))


def _cu_count(device):
    return torch.cuda.get_device_properties(device).multi_processor_count


def _bias_args(bias, query, batch, heads, seqlen_q, seqlen_k):
    """Return (bias_or_dummy_tensor, sbb, sbh, sbm, sbn, has_bias).

    A None bias uses ``query`` as an unused dummy with zero strides.  A present
    bias is broadcast to (batch, heads, seqlen_q, seqlen_k) as a view: the
    broadcast dims carry stride 0 so the kernel re-reads the shared value and
    nothing is materialised (reference interface.py:115-126).
    """
    if bias is None:
        return query, 0, 0, 0, 0, False
    bias = bias.expand(batch, heads, seqlen_q, seqlen_k)
    sbb, sbh, sbm, sbn = bias.stride()
    return bias, sbb, sbh, sbm, sbn, True


def _alibi_args(alibi_slopes, query):
    """Return (per-head fp32 slopes or dummy, has_alibi) (reference :129-133)."""
    if alibi_slopes is None:
        return query, False
    return alibi_slopes.to(torch.float32).contiguous(), True


def alibi_slopes(n_heads, device="cuda"):
    """Standard ALiBi per-head slopes (Press et al., 2021) as a (n_heads,) tensor.

    For n a power of two the slopes are the geometric sequence
    r, r^2, ..., r^n with r = 2^(-8/n); otherwise the closest power of two's
    sequence is extended with every other slope of the doubled sequence.
    """
    if isinstance(n_heads, bool) or not isinstance(n_heads, Integral) or n_heads <= 0:
        raise ValueError("n_heads must be a positive integer")

    def geometric(n):
        ratio = 2.0 ** (-8.0 / n)
        return [ratio ** (i + 1) for i in range(n)]

    n = int(n_heads)
    if n & (n - 1) == 0:
        slopes = geometric(n)
    else:
        lower = 1 << (n.bit_length() - 1)
        slopes = geometric(lower) + geometric(2 * lower)[0::2][: n - lower]
    return torch.tensor(slopes, dtype=torch.float32, device=device)


# ---------------------------------------------------------------------------
# Parameter-struct builders
# ---------------------------------------------------------------------------

def _set(arr, values):
    for i, v in enumerate(values):
        arr[i] = int(v)


def _pad_head_dim(t, dim):
    pad = dim - t.shape[-1]
    return torch.nn.functional.pad(t, (0, pad)) if pad > 0 else t


def _kernel_head_dim(head_dim):
    return max(_KERNEL_MIN_HEAD_DIM, head_dim)


def _fwd_params(q, k, v, out, lse, *, dense, causal, softmax_scale, window, softcap,
                bias, alibi, dropout_p, dropout_seed, varlen=None):
    """Fill fa_fwd_params.  ``dense``: (B,H,S,D) tensors; otherwise packed
    (T,H,D) with ``varlen = (cu_q, cu_k, max_q, max_k)``."""
    p = _native.FwdParams()
    p.abi_version = ABI_VERSION
    p.dtype = DTYPE_CODE[q.dtype]
    p.q, p.k, p.v, p.out, p.lse = q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse.data_ptr()
    if dense:
        for name, t in (("q_stride", q), ("k_stride", k), ("v_stride", v), ("out_stride", out)):
            _set(getattr(p, name), _native.strides(t))
        _set(p.lse_stride, [s if n > 1 else 0 for s, n in zip(lse.stride(), lse.shape)])
        p.batch, p.heads_q, p.seqlen_q, p.head_dim = q.shape
        p.heads_kv, p.seqlen_k = k.shape[1], k.shape[2]
    else:
        for name, t in (("q_stride", q), ("k_stride", k), ("v_stride", v), ("out_stride", out)):
            st = _native.strides(t)
            _set(getattr(p, name), (0, st[1], t.stride(0), 1))
        _set(p.lse_stride, (0, lse.stride(0), lse.stride(1)))
        cu_q, cu_k, max_q, max_k = varlen
        p.batch = cu_q.numel() - 1
        p.heads_q, p.head_dim = q.shape[1], q.shape[2]
        p.heads_kv = k.shape[1]
        p.seqlen_q, p.seqlen_k = int(max_q), int(max_k)
        p.cu_seqlens_q, p.cu_seqlens_k = cu_q.data_ptr(), cu_k.data_ptr()
        p.total_q, p.total_k = q.shape[0], k.shape[0]
    p.softmax_scale = float(softmax_scale)
    p.causal = int(bool(causal))
    p.window_left, p.window_right = int(window[0]), int(window[1])
    p.softcap = float(softcap)
    if bias is not None:
        p.bias = bias.data_ptr()
        p.bias_dtype = DTYPE_CODE[bias.dtype]
        _set(p.bias_stride, bias.stride())
    if alibi is not None:
        p.alibi_slopes = alibi.data_ptr()
    p.dropout_p = float(dropout_p)
    p.dropout_seed = int(dropout_seed) & 0xFFFFFFFFFFFFFFFF
    return p


def _prep(*tensors):
    return tuple(None if t is None else _native.kernel_ready(t) for t in tensors)


# ---------------------------------------------------------------------------
# Dense forward / backward (reference interface.py:154-277)
# ---------------------------------------------------------------------------

def _forward(query, key, value, causal, softmax_scale, window, softcap, bias, alibi, dropout_p, dropout_seed):
    """Dense forward -> (out, lse) through the native host path
    (``fa_mi355x::forward``: parameter packing and launch in C++)."""
    return _native.ops().forward(query, key, value, bool(causal), float(softmax_scale), int(window[0]),
                                 int(window[1]), float(softcap), bias, alibi, float(dropout_p),
                                 int(dropout_seed))


def _bwd_setup(dout, query, key, value, out, lse, causal, softmax_scale, window, softcap, bias, alibi,
               dropout_p, dropout_seed):
    """Allocate dq/dk/dv/delta and fill fa_bwd_params for one dense backward
    phase at a time (``_backward_launcher``; the backward itself packs its
    parameters in C++).  Returns (params, dq, dk, dv, tensors kept alive for
    the launch)."""
    batch, heads, seqlen_q, head_dim = query.shape
    seqlen_k = key.shape[2]
    kdim = _kernel_head_dim(head_dim)
    q, k, v, o, do = _prep(*(_pad_head_dim(t, kdim) for t in (query, key, value, out, dout)))
    lse = lse.contiguous()
    bias_t, *_, has_bias = _bias_args(bias, query, batch, heads, seqlen_q, seqlen_k)
    alibi_t, has_alibi = _alibi_args(alibi, query)
    delta = torch.empty_like(lse)
    dq = torch.empty(q.shape, dtype=query.dtype, device=query.device)
    dk = torch.empty(k.shape, dtype=key.dtype, device=key.device)
    dv = torch.empty(v.shape, dtype=value.dtype, device=value.device)
    params = _native.BwdParams()
    params.fwd = _fwd_params(q, k, v, o, lse, dense=True, causal=causal, softmax_scale=softmax_scale,
                             window=window, softcap=softcap, bias=bias_t if has_bias else None,
                             alibi=alibi_t if has_alibi else None, dropout_p=dropout_p,
                             dropout_seed=dropout_seed)
    params.dout, params.dq, params.dk, params.dv = do.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr()
    params.delta = delta.data_ptr()
    for name, t in (("dout_stride", do), ("dq_stride", dq), ("dk_stride", dk), ("dv_stride", dv)):
        _set(getattr(params, name), _native.strides(t))
    _set(params.delta_stride, [s if n > 1 else 0 for s, n in zip(delta.stride(), delta.shape)])
    ds = _native.attach_ds_scratch(params, query)
    keep = (q, k, v, o, do, lse, delta, bias_t, alibi_t, ds)
    return params, dq, dk, dv, keep


def _backward(dout, query, key, value, out, lse, causal, softmax_scale, window, softcap, bias, alibi,
              dropout_p, dropout_seed):
    """Dense backward -> (dq, dk, dv) through ``fa_mi355x::backward``
    (delta, dK/dV and dQ in one C-ABI call, dS scratch when it fits)."""
    return _native.ops().backward(dout, query, key, value, out, lse, bool(causal), float(softmax_scale),
                                  int(window[0]), int(window[1]), float(softcap), bias, alibi,
                                  float(dropout_p), int(dropout_seed))


def _backward_launcher(dout, query, key, value, out, lse, causal, softmax_scale, window, softcap, bias,
                       alibi, dropout_p, dropout_seed):
    """Profiling aid: returns launch(phase) running one backward kernel
    (0 delta, 1 dK/dV, 2 dQ) on the current stream with fixed buffers."""
    params, dq, dk, dv, keep = _bwd_setup(dout, query, key, value, out, lse, causal, softmax_scale,
                                          window, softcap, bias, alibi, dropout_p, dropout_seed)

    def launch(phase):
        _native.call_bwd_phase(params, phase, query)
        return dq, dk, dv, keep

    return launch


@torch.library.custom_op("fa_rdna3::flash_fwd", mutates_args=())
def _flash_fwd(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
               causal: bool, softmax_scale: float, window_left: int, window_right: int,
               softcap: float, bias: "torch.Tensor | None", alibi: "torch.Tensor | None",
               dropout_p: float, dropout_seed: int) -> "tuple[torch.Tensor, torch.Tensor]":
    return _forward(query, key, value, causal, softmax_scale, (window_left, window_right),
                    softcap, bias, alibi, dropout_p, dropout_seed)


@_flash_fwd.register_fake
def _(query, key, value, causal, softmax_scale, window_left, window_right,
      softcap, bias, alibi, dropout_p, dropout_seed):
    out = torch.empty_like(query)
    lse = query.new_empty((query.shape[0], query.shape[1], query.shape[2]), dtype=torch.float32)
    return out, lse


@torch.library.custom_op("fa_rdna3::flash_bwd", mutates_args=())
def _flash_bwd(dout: torch.Tensor, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
               out: torch.Tensor, lse: torch.Tensor, causal: bool, softmax_scale: float,
               window_left: int, window_right: int, softcap: float,
               bias: "torch.Tensor | None", alibi: "torch.Tensor | None",
               dropout_p: float, dropout_seed: int) -> "tuple[torch.Tensor, torch.Tensor, torch.Tensor]":
    dq, dk, dv = _backward(dout, query, key, value, out, lse, causal, softmax_scale,
                           (window_left, window_right), softcap, bias, alibi, dropout_p, dropout_seed)
    # Custom ops may not return views of internal padding buffers.
    return dq.contiguous(), dk.contiguous(), dv.contiguous()


@_flash_bwd.register_fake
def _(dout, query, key, value, out, lse, causal, softmax_scale, window_left, window_right,
      softcap, bias, alibi, dropout_p, dropout_seed):
    return torch.empty_like(query), torch.empty_like(key), torch.empty_like(value)


def _flash_fwd_setup_context(ctx, inputs, output):
    (query, key, value, causal, softmax_scale, window_left, window_right,
     softcap, bias, alibi, dropout_p, dropout_seed) = inputs
    out, lse = output
    ctx.save_for_backward(query, key, value, out, lse, bias, alibi)
    ctx.args = (causal, softmax_scale, window_left, window_right, softcap, dropout_p, dropout_seed)


def _flash_fwd_backward(ctx, grad_out, grad_lse):
    query, key, value, out, lse, bias, alibi = ctx.saved_tensors
    causal, softmax_scale, window_left, window_right, softcap, dropout_p, dropout_seed = ctx.args
    dquery, dkey, dvalue = _flash_bwd(
        grad_out.contiguous(), query, key, value, out, lse, causal, softmax_scale,
        window_left, window_right, softcap, bias, alibi, dropout_p, dropout_seed)
    return dquery, dkey, dvalue, None, None, None, None, None, None, None, None, None


_flash_fwd.register_autograd(_flash_fwd_backward, setup_context=_flash_fwd_setup_context)


# ---------------------------------------------------------------------------
# Tiny fp32 inference op (reference interface.py:84-104, :336-352)
# ---------------------------------------------------------------------------

@torch.library.custom_op("fa_rdna3::flash_tiny_fwd", mutates_args=())
def _flash_tiny_fwd(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                    softmax_scale: float, bias: "torch.Tensor | None",
                    block_n: int) -> torch.Tensor:
    batch, heads, seqlen, _ = query.shape
    out = torch.empty_like(query)
    bias_t, sbb, sbh, sbm, sbn, has_bias = _bias_args(bias, query, batch, heads, seqlen, seqlen)
    if has_bias and bias_t.dtype != torch.float32:
        bias_t = bias_t.float()
        sbb, sbh, sbm, sbn = bias_t.stride()
    p = _native.TinyParams()
    p.abi_version = ABI_VERSION
    p.seqlen = seqlen
    p.q, p.k, p.v, p.out = query.data_ptr(), key.data_ptr(), value.data_ptr(), out.data_ptr()
    for name, t in (("q_stride", query), ("k_stride", key), ("v_stride", value), ("out_stride", out)):
        _set(getattr(p, name), t.stride())
    if has_bias:
        p.bias = bias_t.data_ptr()
        _set(p.bias_stride, (sbb, sbh, sbm, sbn))
    p.batch, p.heads = batch, heads
    p.softmax_scale = float(softmax_scale)
    _native.call("fa_tiny_fwd_f32", p, query)
    return out


@_flash_tiny_fwd.register_fake
def _(query, key, value, softmax_scale, bias, block_n):
    return torch.empty_like(query)


def _can_use_tiny_forward(query, key, value, causal, window_size, softcap,
                          alibi_slopes, dropout_p, head_dim):
    requires_backward = torch.is_grad_enabled() and (
        query.requires_grad or key.requires_grad or value.requires_grad)
    return (
        not requires_backward
        and query.dtype == torch.float32
        and head_dim == 128
        and query.shape[1] == key.shape[1] == value.shape[1]
        and query.shape[2] == key.shape[2] == value.shape[2]
        and query.shape[2] <= 32
        and not causal
        and tuple(window_size) == (-1, -1)
        and softcap == 0.0
        and alibi_slopes is None
        and dropout_p == 0.0
    )


def flash_attention(query, key, value, causal=False, softmax_scale=None, window_size=(-1, -1),
                    softcap=0.0, bias=None, alibi_slopes=None, dropout_p=0.0):
    """Scaled dot-product attention on the MI355X FlashAttention kernels.

    Args:
        query, key, value: ``(batch, heads, seqlen, head_dim)`` in float16,
            bfloat16 or float32; key/value may have fewer heads (GQA).
        causal: causal mask, bottom-right aligned when seqlen_q != seqlen_k.
        softmax_scale: logit scale; defaults to ``1/sqrt(head_dim)``.
        window_size: ``(left, right)``; query i attends keys j with
            ``i - left <= j <= i + right`` (positions bottom-right aligned);
            ``-1`` means unbounded on that side.
        softcap: if > 0, logits become ``softcap * tanh(logit / softcap)``.
        bias: additive logit bias broadcastable to ``(B, H, Sq, Sk)`` (``-inf``
            entries mask); not differentiable.
        alibi_slopes: ``(heads,)`` slopes; adds ``-slope * |i - j|`` in-kernel.
        dropout_p: dropout on the softmax weights (kept entries scaled by
            ``1/(1-p)``); a fresh seed per forward is reused by the backward.

    Returns:
        The attention output shaped like ``query``; differentiable in q, k, v.
    """
    validate_dense_inputs(query, key, value)
    validate_attention_options(
        query, key, softmax_scale=softmax_scale, window_size=window_size, softcap=softcap,
        bias=bias, alibi_slopes=alibi_slopes, dropout_p=dropout_p)
    head_dim = query.shape[-1]
    softmax_scale = 1.0 / math.sqrt(head_dim) if softmax_scale is None else float(softmax_scale)
    window_size = tuple(window_size)
    softcap = float(softcap)
    dropout_p = float(dropout_p)

    if _can_use_tiny_forward(query, key, value, causal, window_size, softcap,
                             alibi_slopes, dropout_p, head_dim):
        seqlen = query.shape[2]
        block_n = 8 if seqlen <= 8 else 16 if seqlen <= 16 else 32
        return _flash_tiny_fwd(query, key, value, softmax_scale, bias, block_n)

    pad = 0
    if head_dim not in _SUPPORTED_HEAD_DIMS:
        padded = max(16, _next_power_of_2(head_dim))
        if padded not in _SUPPORTED_HEAD_DIMS:
            raise ValueError(f"head_dim {head_dim} not supported (would pad to {padded})")
        pad = padded - head_dim
        query = torch.nn.functional.pad(query, (0, pad))
        key = torch.nn.functional.pad(key, (0, pad))
        value = torch.nn.functional.pad(value, (0, pad))

    dropout_seed = int(torch.randint(0, 2 ** 31 - 1, (1,)).item()) if dropout_p > 0.0 else 0
    if torch.compiler.is_compiling():
        out, _ = _flash_fwd(query, key, value, causal, softmax_scale, window_size[0], window_size[1],
                            softcap, bias, alibi_slopes, dropout_p, dropout_seed)
    else:
        # Eager mode: the differentiable native operator (forward launch, and
        # a backward the autograd engine runs in C++ without Python).
        out = _native.ops().attention(query, key, value, bool(causal), softmax_scale, int(window_size[0]),
                                      int(window_size[1]), softcap, bias, alibi_slopes, dropout_p, dropout_seed)
    if pad:
        out = out[..., :head_dim]
    return out


# ---------------------------------------------------------------------------
# Split-K decode (reference interface.py:427-479)
# ---------------------------------------------------------------------------

def flash_attention_decode(query, key, value, softmax_scale=None, *, cache_seqlens=None, k_scale=None,
                           v_scale=None):
    """Split-K attention for autoregressive decode (small query, long KV).

    The key range is split across workgroups so a tiny query fills the GPU;
    partial outputs are merged with an LSE-weighted reduction.  Non-causal and
    inference-only.  ``cache_seqlens`` (optional int32 ``(batch,)``) limits
    sequence b to its first ``cache_seqlens[b]`` keys (an MI355X-build
    extension; absent, every key is visible as in the reference).

    ``key`` / ``value`` may also be ``torch.float8_e4m3fn`` caches holding
    K / k_scale and V / v_scale (per-tensor scales, default 1; head_dim 32, 64,
    128, 256 or 512; another MI355X-build extension): they are read as fp8, half the bytes of
    a 16-bit cache, and converted exactly to the query's type in registers.
    """
    kv_fp8 = isinstance(key, torch.Tensor) and key.dtype == torch.float8_e4m3fn
    if kv_fp8:
        _validate_fp8_kv(query, key, value, k_scale, v_scale)
    else:
        if k_scale is not None or v_scale is not None:
            raise ValueError("k_scale and v_scale apply to float8_e4m3fn key / value caches only")
        validate_dense_inputs(query, key, value, dtypes=LOW_PRECISION_DTYPES)
    validate_inference_only(query, key, value)
    validate_softmax_scale(softmax_scale)
    batch, heads, seqlen_q, head_dim = query.shape
    seqlen_k = key.shape[2]
    if head_dim not in _SUPPORTED_HEAD_DIMS:
        raise ValueError(f"head_dim {head_dim} not supported; expected one of {_SUPPORTED_HEAD_DIMS}")
    if cache_seqlens is not None:
        if (not isinstance(cache_seqlens, torch.Tensor) or cache_seqlens.dtype != torch.int32
                or cache_seqlens.device != query.device or cache_seqlens.shape != (batch,)):
            raise ValueError(f"cache_seqlens must be an int32 tensor of shape ({batch},) on {query.device}")
    softmax_scale = 1.0 / math.sqrt(head_dim) if softmax_scale is None else float(softmax_scale)
    if kv_fp8:
        return _decode_launch(query, key, value, softmax_scale, cache_seqlens, causal=False,
                              fp8_scales=(1.0 if k_scale is None else float(k_scale),
                                          1.0 if v_scale is None else float(v_scale)))
    return _decode_launch(query, key, value, softmax_scale, cache_seqlens, causal=False)


# fp8 caches are read at the kernel's own head dims (no padding of fp8 rows).
_FP8_HEAD_DIMS = (32, 64, 128, 256, 512)


def _validate_fp8_kv(query, key, value, k_scale, v_scale):
    """Contracts of an fp8 (e4m3) KV cache: the dense shape rules, checked on
    16-bit stand-ins of the same shapes, plus the fp8-specific ones."""
    _check_fp8_pair(value, k_scale, v_scale)
    if not isinstance(query, torch.Tensor) or query.dtype not in LOW_PRECISION_DTYPES:
        raise ValueError("query must be float16 or bfloat16 with an fp8 KV cache")
    stand_in = lambda t: torch.empty_strided(t.shape, [0] * t.dim(), dtype=query.dtype, device=t.device)
    validate_dense_inputs(query, stand_in(key), stand_in(value), dtypes=LOW_PRECISION_DTYPES)
    if query.shape[3] not in _FP8_HEAD_DIMS:
        raise ValueError(f"fp8 KV caches need head_dim 32, 64, 128, 256 or 512, got {query.shape[3]}")


def _decode_launch(query, key, value, softmax_scale, lens, causal, lens_add=0, fp8_scales=None):
    """Split-K decode launch shared by flash_attention_decode and
    flash_attention_with_kvcache (arguments already validated)."""
    batch, heads, seqlen_q, head_dim = query.shape
    seqlen_k = key.shape[2]
    kdim = _kernel_head_dim(head_dim)
    if fp8_scales is not None:
        # fp8 rows: unit last stride and 16-byte aligned rows (contiguous copy
        # otherwise); head_dim is one of the kernel's dims, so no padding.
        q = _prep(query)[0]
        k, v = _native.kernel_ready(key), _native.kernel_ready(value)
    else:
        q, k, v = _prep(_pad_head_dim(query, kdim), _pad_head_dim(key, kdim), _pad_head_dim(value, kdim))
    if kdim <= 128:
        group = heads // key.shape[1]
        num_splits = _streaming_decode_splits(batch, key.shape[1], group * seqlen_q, seqlen_k,
                                              _cu_count(query.device))
    else:
        num_splits = _decode_num_splits(batch, heads, seqlen_q, seqlen_k, 4 * _cu_count(query.device))
    out = torch.empty((batch, heads, seqlen_q, kdim), dtype=query.dtype, device=query.device)
    workspace = torch.empty(
        _native.decode_workspace_bytes(batch, heads, seqlen_q, kdim, num_splits),
        dtype=torch.uint8, device=query.device)
    p = _native.DecodeParams()
    p.abi_version = ABI_VERSION
    p.dtype = DTYPE_CODE[query.dtype]
    p.q, p.k, p.v, p.out = q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr()
    for name, t in (("q_stride", q), ("k_stride", k), ("v_stride", v), ("out_stride", out)):
        _set(getattr(p, name), _native.strides(t))
    p.batch, p.heads_q, p.seqlen_q, p.head_dim = batch, heads, seqlen_q, kdim
    p.heads_kv, p.seqlen_k = key.shape[1], seqlen_k
    if lens is not None:
        p.cache_seqlens = lens.data_ptr()
        p.cache_seqlens_stride = lens.stride(0)
    p.softmax_scale = softmax_scale
    p.num_splits = num_splits
    p.workspace = workspace.data_ptr()
    p.tickets = _native.decode_tickets(query, batch, heads, seqlen_q)
    p.causal = 1 if causal else 0
    p.cache_seqlens_add = int(lens_add)
    if fp8_scales is not None:
        p.kv_fp8 = 1
        p.k_scale, p.v_scale = fp8_scales
    _native.call("fa_decode_splitk", p, query)
    return out[..., :head_dim] if kdim != head_dim else out


def _rows_vector_ready(t):
    """True when ``t``'s rows can be written in place with 16-byte stores."""
    esize = t.element_size()
    return (t.stride(-1) == 1 and t.data_ptr() % 16 == 0
            and all((st * esize) % 16 == 0 for st, n in zip(t.stride()[:-1], t.shape[:-1]) if n > 1))


def flash_attention_with_kvcache(query, k_cache, v_cache, key=None, value=None, *, cache_seqlens=None,
                                 softmax_scale=None, causal=False):
    """Attention of new query rows against a contiguous KV cache, with an
    optional in-place append of new keys / values (the
    ``flash_attn_with_kvcache`` pattern; the reference's decode has no cache
    update, interface.py:427-479).

    ``query`` ``(B, Hq, Sq, D)``; ``k_cache``, ``v_cache`` ``(B, Hkv, Sc, D)``.
    When ``key`` and ``value`` ``(B, Hkv, Snew, D)`` are given they are written
    into the caches at rows ``[cache_seqlens[b], cache_seqlens[b] + Snew)``
    first (rows at or past ``Sc`` are dropped); ``cache_seqlens`` (int32
    ``(B,)``, required with ``key``) is not modified.  Sequence ``b`` then
    attends its first ``cache_seqlens[b] + Snew`` cache rows (all ``Sc`` rows
    when ``cache_seqlens`` is None).  ``causal`` aligns the mask bottom-right
    per sequence: query row ``i`` sees keys ``j <= len_b - Sq + i``; a row that
    sees no key returns zeros.  Inference-only.
    """
    validate_dense_inputs(query, k_cache, v_cache, dtypes=LOW_PRECISION_DTYPES)
    validate_inference_only(query, k_cache, v_cache)
    validate_softmax_scale(softmax_scale)
    batch, heads, seqlen_q, head_dim = query.shape
    heads_kv, seqlen_cache = k_cache.shape[1], k_cache.shape[2]
    if head_dim not in _SUPPORTED_HEAD_DIMS:
        raise ValueError(f"head_dim {head_dim} not supported; expected one of {_SUPPORTED_HEAD_DIMS}")
    if cache_seqlens is not None:
        if (not isinstance(cache_seqlens, torch.Tensor) or cache_seqlens.dtype != torch.int32
                or cache_seqlens.device != query.device or cache_seqlens.shape != (batch,)):
            raise ValueError(f"cache_seqlens must be an int32 tensor of shape ({batch},) on {query.device}")
    if (key is None) != (value is None):
        raise ValueError("key and value must be given together")
    lens = cache_seqlens
    if key is not None:
        if cache_seqlens is None:
            raise ValueError("cache_seqlens is required to append key / value to the cache")
        for name, t in (("key", key), ("value", value)):
            if not isinstance(t, torch.Tensor) or t.dim() != 4:
                raise ValueError(f"{name} must be a 4-D tensor (batch, heads_kv, seqlen_new, head_dim)")
            if t.dtype != query.dtype or t.device != query.device:
                raise ValueError(f"{name} must match query's dtype and device")
        if key.shape != value.shape or key.shape[0] != batch or key.shape[1] != heads_kv or key.shape[3] != head_dim:
            raise ValueError(f"key and value must have shape ({batch}, {heads_kv}, seqlen_new, {head_dim}); "
                             f"got {tuple(key.shape)} and {tuple(value.shape)}")
        for name, t in (("k_cache", k_cache), ("v_cache", v_cache)):
            if not _rows_vector_ready(t):
                raise ValueError(f"{name} must have a unit last stride and 16-byte aligned rows "
                                 "to be updated in place")
        seqlen_new = key.shape[2]
        if seqlen_new > 0:
            kn, vn = _native.kernel_ready(key), _native.kernel_ready(value)
            p = _native.AppendParams()
            p.abi_version = ABI_VERSION
            p.dtype = DTYPE_CODE[query.dtype]
            p.k_new, p.v_new = kn.data_ptr(), vn.data_ptr()
            p.k_cache, p.v_cache = k_cache.data_ptr(), v_cache.data_ptr()
            p.cache_seqlens, p.cache_seqlens_stride = cache_seqlens.data_ptr(), cache_seqlens.stride(0)
            for name, t in (("k_new_stride", kn), ("v_new_stride", vn), ("k_cache_stride", k_cache),
                            ("v_cache_stride", v_cache)):
                _set(getattr(p, name), _native.strides(t))
            p.batch, p.heads_kv, p.seqlen_new = batch, heads_kv, seqlen_new
            p.seqlen_cache, p.head_dim = seqlen_cache, head_dim
            _native.call("fa_kvcache_append", p, query)
    softmax_scale = 1.0 / math.sqrt(head_dim) if softmax_scale is None else float(softmax_scale)
    return _decode_launch(query, k_cache, v_cache, softmax_scale, lens, causal=bool(causal),
                          lens_add=0 if key is None else key.shape[2])


# ---------------------------------------------------------------------------
# Varlen (reference interface.py:482-640)
# ---------------------------------------------------------------------------

def _forward_varlen(query, key, value, cu_seqlens_q, cu_seqlens_k,
                    max_seqlen_q, max_seqlen_k, causal, softmax_scale, window, softcap, alibi):
    total_q, q_heads, head_dim = query.shape
    kdim = _kernel_head_dim(head_dim)
    q, k, v = _prep(_pad_head_dim(query, kdim), _pad_head_dim(key, kdim), _pad_head_dim(value, kdim))
    out = torch.empty((total_q, q_heads, kdim), dtype=query.dtype, device=query.device)
    lse = torch.empty((q_heads, total_q), dtype=torch.float32, device=query.device)
    alibi_t, has_alibi = _alibi_args(alibi, query)
    params = _fwd_params(q, k, v, out, lse, dense=False, causal=causal, softmax_scale=softmax_scale,
                         window=window, softcap=softcap, bias=None,
                         alibi=alibi_t if has_alibi else None, dropout_p=0.0, dropout_seed=0,
                         varlen=(cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k))
    _native.call("fa_fwd", params, query)
    return (out[..., :head_dim] if kdim != head_dim else out), lse


def _backward_varlen(dout, query, key, value, out, lse, cu_seqlens_q, cu_seqlens_k,
                     max_seqlen_q, max_seqlen_k, causal, softmax_scale, window, softcap, alibi):
    head_dim = query.shape[2]
    kdim = _kernel_head_dim(head_dim)
    q, k, v, o, do = _prep(*(_pad_head_dim(t, kdim) for t in (query, key, value, out, dout)))
    alibi_t, has_alibi = _alibi_args(alibi, query)
    delta = torch.empty_like(lse)
    dq = torch.empty(q.shape, dtype=query.dtype, device=query.device)
    dk = torch.empty(k.shape, dtype=key.dtype, device=key.device)
    dv = torch.empty(v.shape, dtype=value.dtype, device=value.device)
    params = _native.BwdParams()
    params.fwd = _fwd_params(q, k, v, o, lse, dense=False, causal=causal, softmax_scale=softmax_scale,
                             window=window, softcap=softcap, bias=None,
                             alibi=alibi_t if has_alibi else None, dropout_p=0.0, dropout_seed=0,
                             varlen=(cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k))
    params.dout, params.dq, params.dk, params.dv = do.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr()
    params.delta = delta.data_ptr()
    for name, t in (("dout_stride", do), ("dq_stride", dq), ("dk_stride", dk), ("dv_stride", dv)):
        st = _native.strides(t)
        _set(getattr(params, name), (0, st[1], t.stride(0), 1))
    _set(params.delta_stride, (0, delta.stride(0), delta.stride(1)))
    _ds = _native.attach_ds_scratch(params, query)
    _native.call("fa_bwd", params, query)
    if kdim != head_dim:
        dq, dk, dv = dq[..., :head_dim], dk[..., :head_dim], dv[..., :head_dim]
    return dq, dk, dv


class _FlashAttentionVarlen(torch.autograd.Function):
    @staticmethod
    def forward(ctx, query, key, value, cu_seqlens_q, cu_seqlens_k,
                max_seqlen_q, max_seqlen_k, causal, softmax_scale, window, softcap, alibi):
        out, lse = _forward_varlen(query, key, value, cu_seqlens_q, cu_seqlens_k,
                                   max_seqlen_q, max_seqlen_k, causal, softmax_scale, window, softcap, alibi)
        ctx.save_for_backward(query, key, value, out, lse, cu_seqlens_q, cu_seqlens_k, alibi)
        ctx.max_seqlen_q = max_seqlen_q
        ctx.max_seqlen_k = max_seqlen_k
        ctx.causal = causal
        ctx.softmax_scale = softmax_scale
        ctx.window = window
        ctx.softcap = softcap
        return out

    @staticmethod
    def backward(ctx, dout):
        query, key, value, out, lse, cu_seqlens_q, cu_seqlens_k, alibi = ctx.saved_tensors
        dquery, dkey, dvalue = _backward_varlen(
            dout, query, key, value, out, lse, cu_seqlens_q, cu_seqlens_k,
            ctx.max_seqlen_q, ctx.max_seqlen_k, ctx.causal, ctx.softmax_scale, ctx.window,
            ctx.softcap, alibi)
        return dquery, dkey, dvalue, None, None, None, None, None, None, None, None, None


def flash_attention_varlen(query, key, value, cu_seqlens_q, cu_seqlens_k,
                           max_seqlen_q, max_seqlen_k, causal=False, softmax_scale=None,
                           window_size=(-1, -1), softcap=0.0, alibi_slopes=None):
    """Attention over variable-length sequences packed without padding.

    Args:
        query: ``(total_q, q_heads, head_dim)``, sequences concatenated.
        key, value: ``(total_k, kv_heads, head_dim)`` (GQA allowed).
        cu_seqlens_q, cu_seqlens_k: int32 ``(batch + 1,)`` cumulative lengths;
            sequence i is rows ``cu_seqlens[i]:cu_seqlens[i+1]`` (clamped to
            the tensor).
        max_seqlen_q, max_seqlen_k: longest query / key sequence.
        causal, softmax_scale, window_size, softcap, alibi_slopes: as in
            :func:`flash_attention`, per sequence.  (No bias or dropout here.)

    Returns:
        ``(total_q, q_heads, head_dim)``; differentiable in q, k, v.
    """
    validate_varlen_inputs(query, key, value, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k)
    validate_attention_options(
        query, key, softmax_scale=softmax_scale, window_size=window_size, softcap=softcap,
        bias=None, alibi_slopes=alibi_slopes, dropout_p=0.0)
    head_dim = query.shape[-1]
    softmax_scale = 1.0 / math.sqrt(head_dim) if softmax_scale is None else float(softmax_scale)
    return _FlashAttentionVarlen.apply(query, key, value, cu_seqlens_q, cu_seqlens_k,
                                       int(max_seqlen_q), int(max_seqlen_k), causal, softmax_scale,
                                       tuple(window_size), float(softcap), alibi_slopes)


# ---------------------------------------------------------------------------
# Paged-KV decode (reference interface.py:643-728)
# ---------------------------------------------------------------------------

def flash_attention_decode_paged(query, k_cache, v_cache, block_table, context_lens,
                                 softmax_scale=None, *, max_context_len=None, num_splits=None, k_scale=None,
                                 v_scale=None):
    """Decode attention over a paged (block-table) KV cache, vLLM style.

    Args:
        query: ``(batch, q_heads, head_dim)``, one query row per sequence.
        k_cache, v_cache: ``(num_blocks, block_size, kv_heads, head_dim)``.
        block_table: int32 ``(batch, max_blocks_per_seq)`` physical block ids.
        context_lens: int32 ``(batch,)`` valid keys per sequence.
        softmax_scale: defaults to ``1/sqrt(head_dim)``.
        max_context_len: optional host-known bound used for split selection.
        num_splits: optional explicit split count from 1 to 32.

    Returns:
        ``(batch, q_heads, head_dim)``.  Non-causal, inference-only.

    ``k_cache`` / ``v_cache`` may be ``torch.float8_e4m3fn`` caches holding
    K / k_scale and V / v_scale (head_dim 32, 64, 128, 256 or 512; an
    MI355X-build extension, see :func:`flash_attention_decode`).
    """
    fp8 = _validate_paged(query, k_cache, v_cache, block_table, context_lens, k_scale, v_scale)
    validate_inference_only(query, k_cache, v_cache)
    validate_softmax_scale(softmax_scale)
    _paged_options(max_context_len, num_splits)
    out = _paged_launch(query.unsqueeze(2), k_cache, v_cache, block_table, context_lens, softmax_scale,
                        max_context_len, num_splits, causal=False, fp8_scales=fp8)
    return out.squeeze(2)


def _validate_paged(query, k_cache, v_cache, block_table, context_lens, k_scale, v_scale):
    """Paged contracts; returns (k_scale, v_scale) for fp8 caches, else None."""
    if not (isinstance(k_cache, torch.Tensor) and k_cache.dtype == torch.float8_e4m3fn):
        if k_scale is not None or v_scale is not None:
            raise ValueError("k_scale and v_scale apply to float8_e4m3fn key / value caches only")
        validate_paged_inputs(query, k_cache, v_cache, block_table, context_lens)
        return None
    _check_fp8_pair(v_cache, k_scale, v_scale)
    if not isinstance(query, torch.Tensor) or query.dtype not in LOW_PRECISION_DTYPES:
        raise ValueError("query must be float16 or bfloat16 with an fp8 KV cache")
    stand_in = lambda t: torch.empty_strided(t.shape, [0] * t.dim(), dtype=query.dtype, device=t.device)
    validate_paged_inputs(query, stand_in(k_cache), stand_in(v_cache), block_table, context_lens)
    if query.shape[-1] not in _FP8_HEAD_DIMS:
        raise ValueError("fp8 paged caches need head_dim 32, 64, 128, 256 or 512")
    return (1.0 if k_scale is None else float(k_scale), 1.0 if v_scale is None else float(v_scale))


def _check_fp8_pair(value, k_scale, v_scale):
    if not isinstance(value, torch.Tensor) or value.dtype != torch.float8_e4m3fn:
        raise ValueError("key and value must both be float8_e4m3fn caches")
    for name, sc in (("k_scale", k_scale), ("v_scale", v_scale)):
        if sc is not None and (isinstance(sc, bool) or not isinstance(sc, (int, float))
                               or not math.isfinite(float(sc)) or float(sc) <= 0.0):
            raise ValueError(f"{name} must be a positive finite number or None")


def _paged_options(max_context_len, num_splits):
    if (max_context_len is not None
            and (isinstance(max_context_len, bool) or not isinstance(max_context_len, Integral)
                 or max_context_len < 0)):
        raise ValueError("max_context_len must be a nonnegative integer or None")
    if (num_splits is not None
            and (isinstance(num_splits, bool) or not isinstance(num_splits, Integral)
                 or not 1 <= num_splits <= 32)):
        raise ValueError("num_splits must be an integer between 1 and 32 or None")


def _paged_launch(query, k_cache, v_cache, block_table, context_lens, softmax_scale, max_context_len,
                  num_splits, causal, fp8_scales=None):
    """Paged decode launch for a (batch, q_heads, Sq, head_dim) query (arguments
    already validated)."""
    max_context_len = None if max_context_len is None else int(max_context_len)
    num_splits = None if num_splits is None else int(num_splits)
    batch, q_heads, seqlen_q, head_dim = query.shape
    num_blocks, block_size, kv_heads = k_cache.shape[0], k_cache.shape[1], k_cache.shape[2]
    softmax_scale = 1.0 / math.sqrt(head_dim) if softmax_scale is None else float(softmax_scale)

    kdim = _kernel_head_dim(head_dim)
    if num_splits is None and kdim <= 128 and block_size >= 4:
        max_keys = block_table.shape[1] * block_size
        if max_context_len is not None:
            max_keys = min(max_keys, max_context_len)
        splits = _streaming_decode_splits(batch, kv_heads, (q_heads // kv_heads) * seqlen_q, max_keys,
                                          _cu_count(query.device))
    else:
        splits = int(_paged_num_splits(batch, q_heads, block_size, block_table.shape[1],
                                       2 * _cu_count(query.device), max_context_len=max_context_len,
                                       requested_splits=num_splits))
    if fp8_scales is not None:
        q, kc, vc = _prep(query, k_cache, v_cache)  # head_dim is a kernel dim: no padding
    else:
        q, kc, vc = _prep(_pad_head_dim(query, kdim), _pad_head_dim(k_cache, kdim),
                          _pad_head_dim(v_cache, kdim))
    out = torch.empty((batch, q_heads, seqlen_q, kdim), dtype=query.dtype, device=query.device)
    workspace = torch.empty(_native.decode_workspace_bytes(batch, q_heads, seqlen_q, kdim, splits),
                            dtype=torch.uint8, device=query.device)
    p = _native.PagedParams()
    p.abi_version = ABI_VERSION
    p.dtype = DTYPE_CODE[query.dtype]
    p.q, p.k_cache, p.v_cache, p.out = q.data_ptr(), kc.data_ptr(), vc.data_ptr(), out.data_ptr()
    p.block_table, p.context_lens = block_table.data_ptr(), context_lens.data_ptr()
    _set(p.q_stride, _native.strides(q))
    _set(p.k_stride, _native.strides(kc))
    _set(p.v_stride, _native.strides(vc))
    _set(p.out_stride, _native.strides(out))
    _set(p.block_table_stride, block_table.stride())
    p.context_lens_stride = context_lens.stride(0)
    p.batch, p.heads_q, p.heads_kv, p.head_dim = batch, q_heads, kv_heads, kdim
    p.num_blocks, p.block_size, p.max_blocks = num_blocks, block_size, block_table.shape[1]
    p.num_splits = splits
    p.softmax_scale = softmax_scale
    p.seqlen_q = seqlen_q
    p.causal = 1 if causal else 0
    if fp8_scales is not None:
        p.kv_fp8 = 1
        p.k_scale, p.v_scale = fp8_scales
    p.workspace = workspace.data_ptr()
    p.tickets = _native.decode_tickets(query, batch, q_heads, seqlen_q)
    _native.call("fa_decode_paged", p, query)
    return out[..., :head_dim] if kdim != head_dim else out


def flash_attention_decode_paged_multi(query, k_cache, v_cache, block_table, context_lens, softmax_scale=None,
                                       *, causal=True, max_context_len=None, num_splits=None, k_scale=None,
                                       v_scale=None):
    """Paged decode of several query rows per sequence (speculative or chunked
    decode over a vLLM-style cache; no counterpart in the reference, whose
    paged decode takes one row, interface.py:643-728).

    ``query`` ``(batch, q_heads, Sq, head_dim)``; the other arguments as in
    :func:`flash_attention_decode_paged`, with ``context_lens`` counting the
    query rows' own keys (already written to their pages).  ``causal`` aligns
    bottom-right per sequence: row ``i`` sees keys ``j <= context_len - Sq + i``.
    Returns ``(batch, q_heads, Sq, head_dim)``.  Inference-only.
    """
    _require_4d_query(query)
    fp8 = _validate_paged(query.select(2, 0), k_cache, v_cache, block_table, context_lens, k_scale, v_scale)
    validate_inference_only(query, k_cache, v_cache)
    validate_softmax_scale(softmax_scale)
    _paged_options(max_context_len, num_splits)
    return _paged_launch(query, k_cache, v_cache, block_table, context_lens, softmax_scale, max_context_len,
                         num_splits, causal=bool(causal), fp8_scales=fp8)


def _require_4d_query(query):
    if not isinstance(query, torch.Tensor) or query.dim() != 4 or query.shape[2] < 1:
        raise ValueError("query must be (batch, heads, seqlen_q, dim) with seqlen_q >= 1")
