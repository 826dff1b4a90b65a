"""Model-facing wrappers: the drop-in surface of the reference package.

Mirrors python/modeling_attention.py of the reference (names, keyword
defaults, argument meaning, ValueError messages):

* ``tilelang_flash_attention(query, key, value, *, attention_mask=None,
  mask=None, score=None, scale=None, is_causal=False, layout="bhsd",
  attention_mask_is_scaled=True, use_atomic_backward=True)``
  (modeling_attention.py:70-147);
* ``tilelang_attention_forward(module, query, key, value, attention_mask,
  scaling, dropout=0.0, **kwargs) -> (out, None)`` (modeling_attention.py:150-192).

One deliberate difference: a mask or score with a broadcast batch/head axis is
passed to the kernels as a stride-0 view instead of being materialised
(the reference's ``_expand_4d`` calls ``.contiguous()``,
modeling_attention.py:57-59), so a [B, 1, T, T] mask costs T*T bytes, not
Hq*T*T.  Values are identical.
"""

from __future__ import annotations

from typing import Literal, Optional

import torch

from .fa2 import flash_attention_with_4d_mask

Layout = Literal["bhsd", "bshd"]


def _dims(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, layout: str):
    """(batch, heads_q, seqlen_q, seqlen_k, head_dim) with the reference's checks
    (modeling_attention.py:21-45)."""
    if query.dim() != 4 or key.dim() != 4 or value.dim() != 4:
        raise ValueError("query, key, and value must be rank-4 tensors")
    if layout == "bhsd":
        h_ax, t_ax = 1, 2
    elif layout == "bshd":
        h_ax, t_ax = 2, 1
    else:
        raise ValueError(f"unsupported layout: {layout}")
    B, Hq, Tq, D = query.shape[0], query.shape[h_ax], query.shape[t_ax], query.shape[3]
    Bk, Hk, Tk, Dk = key.shape[0], key.shape[h_ax], key.shape[t_ax], key.shape[3]
    Bv, Hv, Tv, Dv = value.shape[0], value.shape[h_ax], value.shape[t_ax], value.shape[3]
    if Bk != B or Bv != B:
        raise ValueError("query, key, and value must have the same batch size")
    if Tk != Tv:
        raise ValueError("key and value must have the same sequence length")
    if Hk != Hv:
        raise ValueError("key and value must have the same number of heads")
    if Dk != D or Dv != D:
        raise ValueError("query, key, and value must have the same head dimension")
    if Hq % Hk != 0:
        raise ValueError(f"query heads ({Hq}) must be divisible by key/value heads ({Hk})")
    return B, Hq, Tq, Tk, D


def _broadcast_4d(x: torch.Tensor, *, batch: int, heads: int, seqlen_q: int, seqlen_k: int, name: str) -> torch.Tensor:
    """Validates a [B or 1, H or 1, Tq, Tk] tensor (modeling_attention.py:48-59)
    and returns it broadcast to [B, H, Tq, Tk] as a view (no copy)."""
    if x.dim() != 4:
        raise ValueError(f"{name} must have shape [B, H or 1, Tq, Tk]")
    if tuple(x.shape[-2:]) != (seqlen_q, seqlen_k):
        raise ValueError(f"{name} has trailing shape {tuple(x.shape[-2:])}, expected {(seqlen_q, seqlen_k)}")
    if x.shape[0] not in (1, batch):
        raise ValueError(f"{name} batch dimension must be 1 or {batch}")
    if x.shape[1] not in (1, heads):
        raise ValueError(f"{name} head dimension must be 1 or {heads}")
    return x.expand(batch, heads, seqlen_q, seqlen_k)


def tilelang_flash_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    *,
    attention_mask: Optional[torch.Tensor] = None,
    mask: Optional[torch.Tensor] = None,
    score: Optional[torch.Tensor] = None,
    scale: Optional[float] = None,
    is_causal: bool = False,
    layout: Layout = "bhsd",
    attention_mask_is_scaled: bool = True,
    use_atomic_backward: bool = True,
) -> torch.Tensor:
    """FlashAttention-2 on MI355X with optional 4D keep-mask / score.

    query/key/value: rank-4 fp16/bf16, ``layout="bhsd"`` ([B, H, T, D], default)
    or ``"bshd"`` ([B, T, H, D]); GQA/MQA with Hq % Hk == 0.
    mask: bool [B|1, Hq|1, Tq, Tk], True keeps.  score: float [B|1, Hq|1, Tq, Tk]
    added to Q K^T *before* scaling.  attention_mask: bool (AND-ed into mask) or
    float (added to score; divided by ``scale`` first when
    ``attention_mask_is_scaled``, the PyTorch/HF scaled-logit convention).
    is_causal: keep key j for query i iff j <= i, without a materialised mask.
    Returns the output in the input layout.
    """
    B, Hq, Tq, Tk, D = _dims(query, key, value, layout)
    if query.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError(f"TileLang attention expects fp16 or bf16 inputs, got {query.dtype}")
    if key.dtype != query.dtype or value.dtype != query.dtype:
        raise ValueError("query, key, and value must have the same dtype")
    scale = float(D ** -0.5 if scale is None else scale)
    shape = dict(batch=B, heads=Hq, seqlen_q=Tq, seqlen_k=Tk)

    if mask is not None:
        if mask.dtype != torch.bool:
            raise ValueError("mask must be a bool tensor with True for valid entries")
        mask = _broadcast_4d(mask, name="mask", **shape)

    if score is not None:
        if not torch.is_floating_point(score):
            raise ValueError("score must be a floating-point tensor")
        score = _broadcast_4d(score.to(device=query.device, dtype=torch.float32), name="score", **shape)

    if attention_mask is not None:
        attention_mask = _broadcast_4d(attention_mask.to(device=query.device), name="attention_mask", **shape)
        if attention_mask.dtype == torch.bool:
            mask = attention_mask if mask is None else (mask & attention_mask)
        elif torch.is_floating_point(attention_mask):
            additive = attention_mask.to(dtype=torch.float32)
            if attention_mask_is_scaled:
                additive = additive / scale
            score = additive if score is None else (score + additive)
        else:
            raise ValueError("attention_mask must be bool or floating point")

    return flash_attention_with_4d_mask(
        query, key, value, mask, score, scale, bool(is_causal), bool(use_atomic_backward), layout == "bhsd"
    )


def tilelang_attention_forward(
    module,
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    attention_mask: Optional[torch.Tensor],
    scaling: float,
    dropout: float = 0.0,
    **kwargs,
) -> tuple[torch.Tensor, None]:
    """HuggingFace-style ``attention_interface`` adapter returning
    ``(attn_output, None)``; the output stays in the input layout (BHSD by
    default).  Extra kwargs ``layout``, ``mask``, ``score``,
    ``use_atomic_backward``, ``attention_mask_is_scaled``, ``is_causal`` are
    honoured; ``is_causal`` defaults to ``attention_mask is None and
    module.is_causal`` (modeling_attention.py:167-177)."""
    if dropout not in (0, 0.0, None):
        raise ValueError("TileLang FA2 wrapper does not implement attention dropout")
    layout = kwargs.pop("layout", "bhsd")
    mask = kwargs.pop("mask", None)
    score = kwargs.pop("score", None)
    use_atomic_backward = kwargs.pop("use_atomic_backward", True)
    attention_mask_is_scaled = kwargs.pop("attention_mask_is_scaled", True)
    is_causal = kwargs.pop("is_causal", None)
    if is_causal is None:
        is_causal = attention_mask is None and bool(getattr(module, "is_causal", True))
    out = tilelang_flash_attention(
        query,
        key,
        value,
        attention_mask=attention_mask,
        mask=mask,
        score=score,
        scale=scaling,
        is_causal=bool(is_causal),
        layout=layout,
        attention_mask_is_scaled=attention_mask_is_scaled,
        use_atomic_backward=use_atomic_backward,
    )
    return out, None


__all__ = ["tilelang_flash_attention", "tilelang_attention_forward"]
