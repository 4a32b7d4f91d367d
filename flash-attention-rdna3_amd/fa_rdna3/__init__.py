"""FlashAttention-2 for AMD Instinct MI355X (gfx950), drop-in for ``fa_rdna3``.

Hand-written HIP kernels (``libfa_mi355x.so``, C ABI in include/fa_mi355x.h)
behind the reference package's Python surface.
"""

from ._validation import is_available, unsupported_reason
from .interface import (
    flash_attention,
    flash_attention_decode,
    flash_attention_varlen,
    flash_attention_decode_paged,
    flash_attention_decode_paged_multi,
    flash_attention_with_kvcache,
    alibi_slopes,
)
from .sdpa import (
    disable_rdna3_flash_attention,
    enable_rdna3_flash_attention,
    use_rdna3_flash_attention,
)

__all__ = [
    "flash_attention",
    "flash_attention_decode",
    "flash_attention_varlen",
    "flash_attention_decode_paged",
    "flash_attention_decode_paged_multi",
    "flash_attention_with_kvcache",
    "alibi_slopes",
    "is_available",
    "unsupported_reason",
    "enable_rdna3_flash_attention",
    "disable_rdna3_flash_attention",
    "use_rdna3_flash_attention",
]
