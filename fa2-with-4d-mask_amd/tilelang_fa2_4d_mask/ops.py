"""The attention as registered PyTorch custom ops.

``tilelang_fa2_4d_mask::fwd`` and ``tilelang_fa2_4d_mask::bwd`` wrap the host
code of the forward and backward (fa2.py ``_forward_impl`` / ``_backward_impl``)
with ``torch.library.custom_op``: fake (meta) implementations give the output
shapes without running anything, and ``register_autograd`` ties the backward op
to the forward one.  torch.compile traces a model through them without a graph
break, and the launches are stream-ordered and allocation-free inside the
kernels, so CUDA/HIP graph capture records them (the reference offers a
cudagraph mode in its benchmark, benchmark/throughput_check.py:249-250).

Operands are logical [B, T, H, D] tensors (any strides with a contiguous head
dimension); the mask / score arguments are the user's bool / float tensors of
shape [B|1, Hq|1, Tq, Tk].
"""

from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _ext
from . import fa2 as _fa2

_NS = "tilelang_fa2_4d_mask"


def _mask_ws_bytes(mask: Optional[torch.Tensor], B: int, Hq: int, Tq: int, Tk: int, is_causal: bool) -> int:
    """Prepared-mask workspace size for ``mask`` (host arithmetic only)."""
    if mask is None or B * Tq * Hq == 0 or Tk == 0:
        return 0
    m, mst = _fa2._kernel_side(mask, None, B, Hq, Tq, Tk, "mask", mask.device)
    lib = _ext.load_library()
    mp = _ext.FaMaskParams()
    mp.mask = 256   # never dereferenced by fa_mask_plan
    mp.mask_stride_b, mp.mask_stride_h, mp.mask_stride_q = mst
    mp.batch, mp.seqlen_q, mp.seqlen_k, mp.heads_q = B, Tq, Tk, Hq
    mp.is_causal = 1 if is_causal else 0
    n = ctypes.c_int64(0)
    _ext.check(lib.fa_mask_plan(ctypes.byref(mp), ctypes.byref(n)), "fa_mask_plan", lib)
    return n.value


@torch.library.custom_op(f"{_NS}::fwd", mutates_args=(), device_types="cuda")
def fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, mask: Optional[torch.Tensor],
        score: Optional[torch.Tensor], scale: float, is_causal: bool, use_atomic_backward: bool,
        residual: bool) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """O [B, Tq, Hq, D], LSE [B, Hq, Tq] fp32, the prepared mask (uint8, empty
    without a mask) and O's rounding residual (like O with ``residual`` and a
    mask or a score, else empty), which the backward adds to O for Delta.
    ``use_atomic_backward`` only selects the backward."""
    O, LSE, mask_ws, O_lo, _ = _fa2._forward_impl(q, k, v, mask, score, scale, is_causal, residual)
    if mask_ws is None:
        mask_ws = torch.empty((0,), dtype=torch.uint8, device=q.device)
    if O_lo is None:
        O_lo = q.new_empty((0,))
    return O, LSE, mask_ws, O_lo


def _residual_shape(q, mask, score, residual: bool) -> tuple:
    return tuple(q.shape) if residual and (mask is not None or score is not None) else (0,)


@fwd.register_fake
def _fwd_fake(q, k, v, mask, score, scale, is_causal, use_atomic_backward, residual):
    B, Tq, Hq, D = q.shape
    Tk = k.shape[1]
    O = q.new_empty((B, Tq, Hq, D))
    LSE = q.new_empty((B, Hq, Tq), dtype=torch.float32)
    ws = q.new_empty((_mask_ws_bytes(mask, B, Hq, Tq, Tk, is_causal),), dtype=torch.uint8)
    return O, LSE, ws, q.new_empty(_residual_shape(q, mask, score, residual))


@torch.library.custom_op(f"{_NS}::bwd", mutates_args=(), device_types="cuda")
def bwd(do: torch.Tensor, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, o: torch.Tensor, lse: torch.Tensor,
        mask: Optional[torch.Tensor], score: Optional[torch.Tensor], mask_ws: torch.Tensor, o_lo: torch.Tensor,
        scale: float, is_causal: bool, use_atomic_backward: bool) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """dQ, dK, dV ([B, T, H, D] contiguous, input dtype) of ``fwd``'s outputs."""
    B, Tq, Hq, D = q.shape
    Tk = k.shape[1]
    # the operands exactly as the forward's kernels saw them
    qk = _fa2._kernel_operand(q) if B * Tq * Hq > 0 and Tk > 0 else q
    kk = _fa2._kernel_operand(k) if B * Tq * Hq > 0 and Tk > 0 else k
    vk = _fa2._kernel_operand(v) if B * Tq * Hq > 0 and Tk > 0 else v
    m, mst = _fa2._kernel_side(mask, torch.bool, B, Hq, Tq, Tk, "mask", q.device)
    s, sst = _fa2._kernel_side(score, torch.float32, B, Hq, Tq, Tk, "score", q.device)
    ws = mask_ws if mask_ws.numel() else None
    lo = o_lo if o_lo.numel() else None
    dq, dk, dv = _fa2._backward_impl(do, qk, kk, vk, o, lse, m, s, ws, mst, sst, scale, is_causal,
                                     use_atomic_backward, lo)
    return dq, dk, dv


@bwd.register_fake
def _bwd_fake(do, q, k, v, o, lse, mask, score, mask_ws, o_lo, scale, is_causal, use_atomic_backward):
    return (q.new_empty(q.shape), k.new_empty(k.shape), v.new_empty(v.shape))


def _setup_context(ctx, inputs, output):
    q, k, v, mask, score, scale, is_causal, use_atomic_backward, residual = inputs
    O, LSE, mask_ws, O_lo = output
    ctx.save_for_backward(q, k, v, O, LSE, mask, score, mask_ws, O_lo)
    ctx.scale, ctx.is_causal, ctx.use_atomic_backward = scale, is_causal, use_atomic_backward
    # LSE and the mask workspace never receive a gradient: without this,
    # autograd launches a zero fill for each of them before every backward
    ctx.set_materialize_grads(False)


def _backward(ctx, dO, dLSE, dws, dlo):
    if dO is None:  # O itself does not reach the loss
        return None, None, None, None, None, None, None, None, None
    q, k, v, O, LSE, mask, score, mask_ws, O_lo = ctx.saved_tensors
    dq, dk, dv = torch.ops.tilelang_fa2_4d_mask.bwd(dO, q, k, v, O, LSE, mask, score, mask_ws, O_lo, ctx.scale,
                                                    ctx.is_causal, ctx.use_atomic_backward)
    return dq, dk, dv, None, None, None, None, None, None


fwd.register_autograd(_backward, setup_context=_setup_context)


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, mask: Optional[torch.Tensor],
              score: Optional[torch.Tensor], scale: float, is_causal: bool, use_atomic_backward: bool) -> torch.Tensor:
    """O [B, Tq, Hq, D] of logical [B, T, H, D] operands through the custom ops
    (differentiable in q, k, v).  O's rounding residual is kept for the
    backward only when a gradient can be asked for."""
    residual = torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad)
    return torch.ops.tilelang_fa2_4d_mask.fwd(q, k, v, mask, score, scale, is_causal, use_atomic_backward,
                                              residual)[0]


__all__ = ["fwd", "bwd", "attention"]
