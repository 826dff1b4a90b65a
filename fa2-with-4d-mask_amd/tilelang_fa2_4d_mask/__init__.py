"""MI355X-native FlashAttention-2 with optional 4D mask/score.

Drop-in for the reference package of the same name
(tilelang_fa2_4d_mask/__init__.py:3-10): exports the raw autograd entry point
and the two model-facing wrappers.  The compute runs in the hand-written
gfx950 HIP kernels of libfa2_4d_mask.so (see ``_ext``).
"""

from .fa2 import flash_attention_with_4d_mask
from .modeling_attention import tilelang_attention_forward, tilelang_flash_attention

__all__ = [
    "flash_attention_with_4d_mask",
    "tilelang_attention_forward",
    "tilelang_flash_attention",
]
