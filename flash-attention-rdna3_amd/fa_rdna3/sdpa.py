"""Drop-in ``scaled_dot_product_attention`` override routed to the MI355X kernels.

:func:`enable_rdna3_flash_attention` swaps ``torch.nn.functional
.scaled_dot_product_attention`` for a dispatcher that sends supported calls to
:func:`fa_rdna3.flash_attention` / :func:`fa_rdna3.flash_attention_decode` and
everything else to the original implementation.  Routing rules, names and
refcounted context-manager semantics follow the reference
(fa_rdna3/sdpa.py:26-199).
"""

from contextlib import contextmanager
import math
from numbers import Real
import threading

import torch
import torch.nn.functional as F

from ._validation import is_available
from .interface import flash_attention, flash_attention_decode, _SUPPORTED_HEAD_DIMS

_original_sdpa = None
_patch_lock = threading.RLock()
_context_depth = 0
_context_installed = False
_dispatch_bypass_state = threading.local()

# A query this short against a cache at least this long goes to split-K decode.
_DECODE_MAX_QUERY = 8
_DECODE_MIN_KEY = 1024

# Training calls this short defer to torch: three backward launches cost more
# than torch's fused math backward on a handful of tokens.
_MIN_TRAIN_SEQLEN = 16


def _is_tiny_fp32_inference(query, key, value, attn_mask, is_causal, requires_backward):
    return (
        not requires_backward
        and not is_causal
        and query.dtype == torch.float32
        and query.shape[-1] == 128
        and query.shape == key.shape == value.shape
        and query.shape[-2] <= 32
        and (attn_mask is None or attn_mask.dtype == torch.float32)
    )


def _is_supported_mask(attn_mask, query, key):
    if attn_mask is None:
        return True
    if not isinstance(attn_mask, torch.Tensor):
        return False
    if (attn_mask.device != query.device or attn_mask.requires_grad
            or attn_mask.dtype not in (torch.bool, query.dtype, torch.float32)):
        return False
    target = (query.shape[0], query.shape[1], query.shape[2], key.shape[2])
    try:
        return torch.broadcast_shapes(tuple(attn_mask.shape), target) == target
    except RuntimeError:
        return False


def _is_supported_scale(scale):
    return scale is None or (
        not isinstance(scale, bool) and isinstance(scale, Real) and math.isfinite(float(scale)))


def _is_supported(query, key, value, attn_mask, dropout_p, enable_gqa, scale):
    tensors = (query, key, value)
    if not all(isinstance(t, torch.Tensor) for t in tensors):
        return False
    if not (query.is_cuda and is_available(query.device)):
        return False
    if key.device != query.device or value.device != query.device:
        return False
    if query.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        return False
    if key.dtype != query.dtype or value.dtype != query.dtype:
        return False
    if query.dim() != 4 or key.dim() != 4 or value.dim() != 4:
        return False
    if not (query.shape[0] == key.shape[0] == value.shape[0]):
        return False
    if min(query.shape[-2], key.shape[-2], query.shape[-1], query.shape[-3], key.shape[-3]) <= 0:
        return False
    if query.shape[-1] > 512:  # other dims are zero-padded internally
        return False
    if key.shape[-1] != query.shape[-1] or value.shape[-1] != query.shape[-1]:
        return False
    if key.shape[-2] != value.shape[-2] or key.shape[-3] != value.shape[-3]:
        return False
    if not (query.shape[-3] == key.shape[-3]
            or (enable_gqa and query.shape[-3] % key.shape[-3] == 0)):
        return False
    if not (_is_supported_mask(attn_mask, query, key) and _is_supported_scale(scale)):
        return False
    return not isinstance(dropout_p, bool) and isinstance(dropout_p, Real) and dropout_p == 0.0


def _mask_to_bias(attn_mask):
    """SDPA mask -> additive bias: a boolean mask becomes 0 / -inf fp32."""
    if attn_mask is None:
        return None
    if attn_mask.dtype == torch.bool:
        return torch.zeros_like(attn_mask, dtype=torch.float32).masked_fill(~attn_mask, float("-inf"))
    return attn_mask


def _dispatch_sdpa(query, key, value, attn_mask=None, dropout_p=0.0,
                   is_causal=False, scale=None, enable_gqa=False):
    if getattr(_dispatch_bypass_state, "depth", 0):
        if _original_sdpa is None:
            raise RuntimeError("RDNA3 SDPA bypass requires an installed dispatcher")
        return _original_sdpa(query, key, value, attn_mask=attn_mask, dropout_p=dropout_p,
                              is_causal=is_causal, scale=scale, enable_gqa=enable_gqa)
    # PyTorch's is_causal is top-left aligned; ours is bottom-right, so only
    # square causal calls without a mask are taken.
    supported = _is_supported(query, key, value, attn_mask, dropout_p, enable_gqa, scale) and (
        not is_causal or (attn_mask is None and query.shape[-2] == key.shape[-2]))
    if supported:
        requires_backward = torch.is_grad_enabled() and (
            query.requires_grad or key.requires_grad or value.requires_grad)
        if (_is_tiny_fp32_inference(query, key, value, attn_mask, is_causal, requires_backward)
                and torch.compiler.is_compiling()):
            torch._dynamo.mark_static(query, 2)
            torch._dynamo.mark_static(key, 2)
            torch._dynamo.mark_static(value, 2)
            return flash_attention(query, key, value, softmax_scale=scale, bias=_mask_to_bias(attn_mask))
        if (requires_backward
                and query.shape[-2] <= _MIN_TRAIN_SEQLEN and key.shape[-2] <= _MIN_TRAIN_SEQLEN):
            return _original_sdpa(query, key, value, attn_mask=attn_mask, dropout_p=dropout_p,
                                  is_causal=is_causal, scale=scale, enable_gqa=enable_gqa)
        bias = _mask_to_bias(attn_mask)
        if (bias is None and not is_causal and not requires_backward
                and query.dtype in (torch.float16, torch.bfloat16)
                and query.shape[-1] in _SUPPORTED_HEAD_DIMS
                and query.shape[-2] <= _DECODE_MAX_QUERY
                and key.shape[-2] >= _DECODE_MIN_KEY):
            return flash_attention_decode(query, key, value, softmax_scale=scale)
        return flash_attention(query, key, value, causal=is_causal, softmax_scale=scale, bias=bias)
    return _original_sdpa(query, key, value, attn_mask=attn_mask, dropout_p=dropout_p,
                          is_causal=is_causal, scale=scale, enable_gqa=enable_gqa)


def enable_rdna3_flash_attention():
    """Route supported ``scaled_dot_product_attention`` calls to the MI355X kernels."""
    global _original_sdpa
    with _patch_lock:
        if _original_sdpa is None:
            _original_sdpa = F.scaled_dot_product_attention
        if F.scaled_dot_product_attention is _original_sdpa:
            F.scaled_dot_product_attention = _dispatch_sdpa


def disable_rdna3_flash_attention():
    """Restore the original ``scaled_dot_product_attention`` (unless a later
    third-party override has replaced ours, which is then left in place)."""
    with _patch_lock:
        if _original_sdpa is not None and F.scaled_dot_product_attention is _dispatch_sdpa:
            F.scaled_dot_product_attention = _original_sdpa


@contextmanager
def _bypass_rdna3_flash_attention():
    depth = getattr(_dispatch_bypass_state, "depth", 0)
    _dispatch_bypass_state.depth = depth + 1
    try:
        yield
    finally:
        _dispatch_bypass_state.depth = depth


@contextmanager
def use_rdna3_flash_attention():
    """Temporarily route supported SDPA calls to the MI355X kernels (nestable,
    refcounted across overlapping contexts)."""
    global _context_depth, _context_installed
    with _patch_lock:
        if _context_depth == 0:
            already = F.scaled_dot_product_attention is _dispatch_sdpa
            enable_rdna3_flash_attention()
            _context_installed = not already and F.scaled_dot_product_attention is _dispatch_sdpa
        _context_depth += 1
    try:
        yield
    finally:
        with _patch_lock:
            _context_depth -= 1
            if _context_depth == 0:
                if _context_installed:
                    disable_rdna3_flash_attention()
                _context_installed = False
