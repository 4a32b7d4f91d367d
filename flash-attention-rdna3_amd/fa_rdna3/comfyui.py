"""ComfyUI adapter: an ``optimized_attention_override`` that sends ComfyUI's
attention calls to the MI355X kernels, and the model-patch node that installs it.

Same behaviour as the reference adapter (fa_rdna3/comfyui.py:27-302):

* ComfyUI hands attention ``(batch, tokens, heads * head_dim)`` tensors plus
  ``heads`` (or ``(batch, heads, tokens, head_dim)`` with ``skip_reshape``);
  the override splits the heads, runs :func:`flash_attention` and restores
  the caller's layout (``skip_output_reshape`` keeps the head layout);
* anything the kernels do not cover -- shapes that do not split into heads,
  an fp32 accumulation request for a 16-bit call, ``low_precision_attention
  =False``, or inputs the SDPA dispatcher's support test rejects -- goes to
  ComfyUI's own attention function, with the process-wide SDPA dispatch
  bypassed so the fallback really is ComfyUI's path;
* an override already installed on the model keeps precedence: it is called
  with an attention function that runs this adapter, so it can still
  delegate to the kernels.

Nothing here imports ComfyUI at module load; the node asks ComfyUI for its
attention-precision policy only when it patches a model.
"""

from collections.abc import Callable
from functools import wraps
import logging

import torch

from ._validation import unsupported_reason
from .interface import flash_attention
from .sdpa import (
    _bypass_rdna3_flash_attention,
    _is_supported,
    _mask_to_bias,
    enable_rdna3_flash_attention,
)

logger = logging.getLogger(__name__)


def _heads_layout(query, key, value, heads, skip_reshape, enable_gqa):
    """(q, k, v) as ``(batch, heads, tokens, head_dim)`` views, or None when
    the tensors do not describe a head split the kernels can take."""
    if isinstance(heads, bool) or not isinstance(heads, int) or heads <= 0:
        return None
    tensors = (query, key, value)
    if any(t.dim() != (4 if skip_reshape else 3) for t in tensors):
        return None
    if key.shape[0] != query.shape[0] or value.shape[0] != query.shape[0]:
        return None
    if skip_reshape:
        return tensors if query.shape[1] == heads else None
    width = query.shape[2]
    if width % heads:
        return None
    dim = width // heads
    if dim == 0 or key.shape[2] % dim or value.shape[2] % dim:
        return None
    kv_heads = key.shape[2] // dim
    if value.shape[2] // dim != kv_heads:
        return None
    if kv_heads != heads and not (enable_gqa and kv_heads > 0 and heads % kv_heads == 0):
        return None

    def split(t, h):
        return t.reshape(t.shape[0], t.shape[1], h, dim).transpose(1, 2)

    return split(query, heads), split(key, kv_heads), split(value, kv_heads)


def _mask_for_heads(mask):
    """ComfyUI masks are ``(q, k)``, ``(batch, q, k)`` or already 4-D; give the
    first two a broadcastable batch and head axis."""
    if isinstance(mask, torch.Tensor) and mask.dim() in (2, 3):
        return mask.unsqueeze(0) if mask.dim() == 2 else mask.unsqueeze(1)
    return mask


class ComfyUIAttentionOverride:
    """Callable installed as ComfyUI's ``optimized_attention_override``.

    ``previous_override``: an override that was on the model before (kept in
    front of this one).  ``precision_resolver(attn_precision, dtype)`` returns
    the accumulation dtype ComfyUI wants for a call (its global upcast
    policy); by default the call's own ``attn_precision``.
    """

    def __init__(self, previous_override=None, precision_resolver=None):
        self.previous_override = previous_override
        self.precision_resolver = precision_resolver or (lambda precision, dtype: precision)

    def _fallback(self, attention, query, key, value, heads, mask, attn_precision, skip_reshape,
                  skip_output_reshape, kwargs):
        with _bypass_rdna3_flash_attention():
            return attention(query, key, value, heads, mask=mask, attn_precision=attn_precision,
                             skip_reshape=skip_reshape, skip_output_reshape=skip_output_reshape, **kwargs)

    def _attend(self, attention, query, key, value, heads, mask=None, attn_precision=None,
                skip_reshape=False, skip_output_reshape=False, **kwargs):
        gqa = kwargs.get("enable_gqa") is True
        fallback_args = (attention, query, key, value, heads, mask, attn_precision, skip_reshape,
                         skip_output_reshape, kwargs)
        wants_fp32 = self.precision_resolver(attn_precision, query.dtype) == torch.float32
        if (wants_fp32 and query.dtype != torch.float32) or kwargs.get("low_precision_attention", True) is False:
            return self._fallback(*fallback_args)
        split = _heads_layout(query, key, value, heads, skip_reshape, gqa)
        if split is None:
            return self._fallback(*fallback_args)
        q, k, v = split
        mask4 = _mask_for_heads(mask)
        scale = kwargs.get("scale")
        if not _is_supported(q, k, v, mask4, 0.0, gqa, scale):
            return self._fallback(*fallback_args)
        out = flash_attention(q, k, v, softmax_scale=scale, bias=_mask_to_bias(mask4))
        if skip_output_reshape:
            return out
        batch, _, tokens, dim = out.shape
        return out.transpose(1, 2).reshape(batch, tokens, heads * dim)

    def __call__(self, original_attention, query, key, value, heads, mask=None, attn_precision=None,
                 skip_reshape=False, skip_output_reshape=False, **kwargs):
        if self.previous_override is None:
            return self._attend(original_attention, query, key, value, heads, mask, attn_precision,
                                skip_reshape, skip_output_reshape, **kwargs)

        @wraps(original_attention)
        def attention_via_kernels(q, k, v, h, mask=None, attn_precision=None, skip_reshape=False,
                                  skip_output_reshape=False, **kw):
            return self._attend(original_attention, q, k, v, h, mask, attn_precision, skip_reshape,
                                skip_output_reshape, **kw)

        with _bypass_rdna3_flash_attention():
            return self.previous_override(attention_via_kernels, query, key, value, heads, mask=mask,
                                          attn_precision=attn_precision, skip_reshape=skip_reshape,
                                          skip_output_reshape=skip_output_reshape, **kwargs)


def _get_comfyui_precision_resolver():
    from comfy.ldm.modules.attention import get_attn_precision

    return get_attn_precision


class ApplyRDNA3FlashAttention:
    """Model-patch node: installs :class:`ComfyUIAttentionOverride` on a clone
    of the model and turns on the process-wide SDPA dispatch."""

    @classmethod
    def INPUT_TYPES(cls):
        return {"required": {"model": ("MODEL",)}}

    RETURN_TYPES = ("MODEL",)
    RETURN_NAMES = ("model",)
    FUNCTION = "patch"
    CATEGORY = "model_patches/attention"
    DESCRIPTION = ("Routes this model's supported attention calls through the MI355X FlashAttention "
                   "kernels; other calls keep ComfyUI's own attention.")

    def patch(self, model):
        reason = unsupported_reason()
        if reason is not None:
            raise RuntimeError(f"Cannot enable RDNA3 Flash Attention: {reason}")
        patched = model.clone()
        options = patched.model_options["transformer_options"]
        previous = options.get("optimized_attention_override")
        if previous is not None and not callable(previous):
            raise TypeError("optimized_attention_override must be callable")
        if isinstance(previous, ComfyUIAttentionOverride):
            override = previous
        else:
            if previous is not None:
                logger.info("Composing MI355X Flash Attention under an existing attention override")
            override = ComfyUIAttentionOverride(previous, _get_comfyui_precision_resolver())
        options["optimized_attention_override"] = override
        enable_rdna3_flash_attention()
        logger.info("Enabled MI355X Flash Attention for the patched ComfyUI model")
        return (patched,)


# Node registry read by ComfyUI (names kept so saved workflows still resolve).
NODE_CLASS_MAPPINGS = {"ApplyRDNA3FlashAttention": ApplyRDNA3FlashAttention}
NODE_DISPLAY_NAME_MAPPINGS = {"ApplyRDNA3FlashAttention": "RDNA3 Flash Attention"}
