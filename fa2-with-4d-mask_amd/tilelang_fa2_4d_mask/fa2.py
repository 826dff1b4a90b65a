"""Autograd Function over the gfx950 FlashAttention-2 kernels.

Host-side mirror of the reference's ``_flash_attention_with_4d_mask``
(python/fa2.py:437-558): same positional signature
``(Q, K, V, Mask, Score, scale, is_causal, use_atomic_backward, bhsd_input)``,
same defaults (``scale = D**-0.5``, python/fa2.py:456), same rank assert
(python/fa2.py:448), output in the input layout (python/fa2.py:488) and
gradients for Q, K, V only (python/fa2.py:556).

What differs on purpose:
* no layout copies: the kernels take (batch, time, head) strides, so both a
  BHSD view over BTHD storage and a BHSD-contiguous tensor are used in place
  (the reference copies the latter, python/fa2.py:433-435, 449-452);
* Mask/Score may be broadcast views ([B|1, Hq|1, Tq, Tk] with stride 0);
* dQ/dK/dV come back in the input dtype directly (the reference returns fp32
  dQ and lets autograd cast it, python/fa2.py:527,556);
* dQ goes through dS tiles the dK/dV kernel stores: ``False`` writes dQ in
  one deterministic pass; ``use_atomic_backward`` (default) does the same
  when the 256-row query blocks give every CU a workgroup, and on smaller
  grids adds fp32 partials over a few key ranges atomically (the reference
  adds a partial per 64-key block atomically in both modes,
  python/fa2.py:295-297, 420-421);
* a mask is prepared once per call (``fa_mask_prepare``: bits, block states,
  live-tile lists) and the workspace is kept for the backward, so the kernels
  skip tiles without a kept entry (the reference streams every tile's mask
  bytes, python/fa2.py:107-114, 261-280);
* the kernels exist for head dims 64, 128 and 256 (the reference compiles
  any D, python/fa2.py:33); other D up to 256 run zero-padded to the next of
  those, which is exact (see ``kernel_head_dim``), at the price of padded
  copies of the operands.  Head dim 256 has kernels of its own (128-row
  forward blocks, dK and dV in two launches, dQ recomputed in both backward
  modes: no dS workspace, no atomics).
"""

from __future__ import annotations

import contextlib
import ctypes
from typing import Optional

import torch
from torch.autograd.function import once_differentiable

from . import _ext

# Largest dS workspace (bytes) the backward may allocate to hand dS from the
# dK/dV kernel to the dQ kernel.  0 = the default, DS_LIMIT_DEFAULT (the
# library's own default; a constant, so that the backward's route, slices and
# head-group split depend on the problem alone: calls are bitwise repeatable
# whatever the allocator holds); negative = never (dQ is then recomputed from
# Q, K, V, dO: O(T) extra memory, as the reference's backward).  Below the
# whole need the backward runs in slices of (batch, kv-head) units, ranges of
# query rows (causal, or a unit above the limit; no mask) or parts of head
# groups (a unit above the limit, with a mask).
DS_LIMIT_BYTES = 0
DS_LIMIT_DEFAULT = 4 << 30


# Head dims the kernels are built for.
KERNEL_HEAD_DIMS = (64, 128, 256)


def kernel_head_dim(D: int) -> int:
    """Head dim the kernels run a problem of head dim ``D`` at: the smallest of
    KERNEL_HEAD_DIMS that is >= D (D itself when above them: the library then
    rejects it).  Zero columns appended to Q, K, V (and O, dO) leave Q K^T, the
    softmax and Delta = rowsum(O * dO) unchanged and give zero columns in O, dQ,
    dK, dV, which are dropped: the padded problem is exact."""
    for w in KERNEL_HEAD_DIMS:
        if D <= w:
            return w
    return D


def _pad_head_dim(x: torch.Tensor, Dp: int) -> torch.Tensor:
    """[B, T, H, D] -> [B, T, H, Dp], zeros appended (x itself when D == Dp)."""
    D = x.shape[3]
    return x if D == Dp else torch.nn.functional.pad(x, (0, Dp - D))


def ds_limit_bytes(device: Optional[torch.device] = None) -> int:
    """The dS workspace limit a backward uses (see DS_LIMIT_BYTES); the same
    on every device and in every memory state."""
    return int(DS_LIMIT_BYTES) if DS_LIMIT_BYTES != 0 else DS_LIMIT_DEFAULT


def _norm_strides(x: torch.Tensor) -> tuple:
    """Strides with size-1 dimensions reported as 0 (never stepped over)."""
    return tuple(0 if n == 1 else s for n, s in zip(x.shape, x.stride()))


def _kernel_operand(x: torch.Tensor) -> torch.Tensor:
    """A logical [B, T, H, D] operand the kernels can address: head dim
    contiguous, rows 16-byte aligned.  Copies only when that does not hold."""
    st = _norm_strides(x)
    if x.stride(3) != 1 and x.shape[3] > 1:
        return x.contiguous()
    if any(s % 8 for s in st[:3]) or x.data_ptr() % 16:
        return x.contiguous()
    return x


# The backward kernels reach a Q / dO row with a 32-bit byte offset from its
# head's first row (fa_api.cpp check_bwd: (Tq + 32) rows must span < 4 GiB).
ROW_SPAN_LIMIT = 1 << 32


def _rows_reachable(x: torch.Tensor, Tq: int) -> torch.Tensor:
    """x itself when (Tq + 32) of its rows span less than ROW_SPAN_LIMIT bytes,
    else a head-major copy (the rows of a head contiguous, D elements apart).
    A token-major layout with many heads reaches the limit at ~2^32 / (2 H D)
    tokens (524k at 32 heads of 128); head-major it moves to 2^31 / D rows."""
    if (Tq + 32) * 2 * abs(x.stride(1)) < ROW_SPAN_LIMIT:
        return x
    return x.transpose(1, 2).contiguous().transpose(1, 2)


def _bthd_strides(x: torch.Tensor) -> tuple:
    st = _norm_strides(x)
    return st[0], st[1], st[2]


def _kernel_side(x: Optional[torch.Tensor], dtype: Optional[torch.dtype], B: int, Hq: int, Tq: int, Tk: int,
                 name: str, device: torch.device):
    """Mask/Score as a broadcastable [B|1, Hq|1, Tq, Tk] view with a contiguous key axis."""
    if x is None:
        return None, (0, 0, 0)
    if x.dim() != 4:
        raise ValueError(f"{name} must have shape [B, H or 1, Tq, Tk]")
    if x.device != device:
        raise ValueError(f"{name} must be on {device}, got {x.device}")
    if dtype is not None and x.dtype != dtype:
        # convert the stored entries only: broadcast (stride-0) dimensions stay
        # broadcast, so the kernels and the workspaces see one plane for them
        base = x[tuple(slice(0, 1) if (x.stride(d) == 0 and x.shape[d] > 1) else slice(None) for d in range(4))]
        x = base.to(dtype).expand(x.shape)
    if tuple(x.shape[-2:]) != (Tq, Tk) or x.shape[0] not in (1, B) or x.shape[1] not in (1, Hq):
        raise ValueError(f"{name} has shape {tuple(x.shape)}, expected [{B} or 1, {Hq} or 1, {Tq}, {Tk}]")
    if x.stride(3) != 1 and Tk > 1:
        x = x.contiguous()
    st = _norm_strides(x)
    return x, (st[0], st[1], st[2])


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _prepare_mask(mask: torch.Tensor, mst: tuple, B: int, Hq: int, Tq: int, Tk: int, is_causal: bool,
                  device: torch.device) -> torch.Tensor:
    """Prepared-mask workspace of ``mask`` (a broadcastable [B|1, Hq|1, Tq, Tk]
    bool view), written on the current stream."""
    lib = _ext.load_library()
    mp = _ext.FaMaskParams()
    mp.mask = mask.data_ptr()
    mp.mask_stride_b, mp.mask_stride_h, mp.mask_stride_q = mst
    mp.batch, mp.seqlen_q, mp.seqlen_k, mp.heads_q = B, Tq, Tk, Hq
    mp.is_causal = 1 if is_causal else 0
    nbytes = ctypes.c_int64(0)
    _ext.check(lib.fa_mask_plan(ctypes.byref(mp), ctypes.byref(nbytes)), "fa_mask_plan", lib)
    ws = torch.empty((nbytes.value,), dtype=torch.uint8, device=device)
    mp.workspace = ws.data_ptr()
    mp.stream = _stream(device)
    _call(lib, "fa_mask_prepare", mp)
    return ws


class KernelEventLog:
    """HIP events recorded around every library call, on the stream the
    kernels are launched on (torch's current stream)."""

    def __init__(self):
        self.records = []  # (entry point, start event, end event)

    def elapsed_ms(self) -> dict:
        torch.cuda.synchronize()
        out: dict = {}
        for name, s, e in self.records:
            out.setdefault(name, []).append(s.elapsed_time(e))
        return out


_event_log: Optional[KernelEventLog] = None


@contextlib.contextmanager
def record_kernel_events():
    """Context manager yielding a :class:`KernelEventLog` of the library calls
    made inside it (forward and backward)."""
    global _event_log
    prev, log = _event_log, KernelEventLog()
    _event_log = log
    try:
        yield log
    finally:
        _event_log = prev


def _call(lib, entry: str, params) -> None:
    fn = getattr(lib, entry)
    log = _event_log
    if log is None:
        _ext.check(fn(ctypes.byref(params)), entry, lib)
        return
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    status = fn(ctypes.byref(params))
    end.record()
    log.records.append((entry, start, end))
    _ext.check(status, entry, lib)


def _check_qkv(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> None:
    if not q.is_cuda:
        raise ValueError("flash_attention_with_4d_mask runs on the GPU: inputs must be HIP/CUDA tensors")
    if k.device != q.device or v.device != q.device:
        raise ValueError("query, key and value must be on the same device")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("query, key, and value must have the same dtype")
    _ext.dtype_code(q.dtype)


def _forward_impl(q, k, v, Mask, Score, scale: float, is_causal: bool, residual: bool = False):
    """Host side of the forward (python/fa2.py:438-488) on logical [B, T, H, D]
    operands: O [B, Tq, Hq, D], LSE [B, Hq, Tq], the prepared mask (or None)
    and, with ``residual`` and a mask or a score, O's rounding residual (else
    None: the backward then takes Delta from O as stored), plus the operands
    as the kernels saw them (zero-padded to the kernel head dim, see
    ``kernel_head_dim``)."""
    B, Tq, Hq, D_in = q.shape
    _, Tk, Hk, _ = k.shape
    D = kernel_head_dim(D_in)
    q, k, v = (_pad_head_dim(x, D) for x in (q, k, v))
    mask, mst = _kernel_side(Mask, torch.bool, B, Hq, Tq, Tk, "mask", q.device)
    score, sst = _kernel_side(Score, torch.float32, B, Hq, Tq, Tk, "score", q.device)
    O = torch.empty((B, Tq, Hq, D), dtype=q.dtype, device=q.device)
    LSE = torch.empty((B, Hq, Tq), dtype=torch.float32, device=q.device)
    O_lo = torch.empty_like(O) if residual and (mask is not None or score is not None) else None
    mask_ws = None
    if B * Tq * Hq > 0:
        if Tk == 0:
            O.zero_()
            LSE.fill_(float("-inf"))
            if O_lo is not None:
                O_lo.zero_()
        else:
            q = _kernel_operand(q)
            k = _kernel_operand(k)
            v = _kernel_operand(v)
            # the parameter block is filled before the mask preparation is
            # launched, so that the forward's launch follows it closely
            p = _ext.FaFwdParams()
            p.q, p.k, p.v, p.o, p.lse = q.data_ptr(), k.data_ptr(), v.data_ptr(), O.data_ptr(), LSE.data_ptr()
            p.mask, p.score = _ext.ptr(mask), _ext.ptr(score)
            p.q_stride_b, p.q_stride_t, p.q_stride_h = _bthd_strides(q)
            p.k_stride_b, p.k_stride_t, p.k_stride_h = _bthd_strides(k)
            p.v_stride_b, p.v_stride_t, p.v_stride_h = _bthd_strides(v)
            p.o_stride_b, p.o_stride_t, p.o_stride_h = _bthd_strides(O)
            if O_lo is not None:
                p.o_lo = O_lo.data_ptr()
                p.o_lo_stride_b, p.o_lo_stride_t, p.o_lo_stride_h = _bthd_strides(O_lo)
            p.mask_stride_b, p.mask_stride_h, p.mask_stride_q = mst
            p.score_stride_b, p.score_stride_h, p.score_stride_q = sst
            p.batch, p.seqlen_q, p.seqlen_k, p.heads_q, p.heads_k, p.head_dim = B, Tq, Tk, Hq, Hk, D
            p.scale = scale
            p.is_causal = 1 if is_causal else 0
            p.dtype = _ext.dtype_code(q.dtype)
            p.stream = _stream(q.device)
            lib = _ext.load_library()
            if mask is not None:
                mask_ws = _prepare_mask(mask, mst, B, Hq, Tq, Tk, bool(is_causal), q.device)
                p.mask_ws = mask_ws.data_ptr()
            _call(lib, "fa_fwd", p)
    if D != D_in:
        O = O[..., :D_in].contiguous()
        O_lo = None if O_lo is None else O_lo[..., :D_in].contiguous()
    return O, LSE, mask_ws, O_lo, (q, k, v, mask, score, mst, sst)


def _backward_impl(do, q, k, v, O, LSE, mask, score, mask_ws, mst, sst, scale: float, is_causal: bool,
                   use_atomic_backward: bool, O_lo: Optional[torch.Tensor] = None):
    """Host side of the backward (python/fa2.py:490-556) on logical [B, T, H, D]
    operands (Q, K, V as given or as the forward's kernels saw them); returns
    dQ, dK, dV in the input dtype, [B, T, H, D] contiguous with D that of dO.
    ``O_lo``: the forward's rounding residual of O (with a mask or a score),
    added to O for Delta.  Head dims other than the kernels' run zero-padded
    (``kernel_head_dim``)."""
    B, Tq, Hq, D_in = do.shape
    _, Tk, Hk, _ = k.shape
    D = kernel_head_dim(D_in)
    q, k, v, O, do = (_pad_head_dim(x, D) for x in (q, k, v, O, do))
    if O_lo is not None:
        O_lo = _pad_head_dim(O_lo, D)
    dev = q.device
    dQ = torch.empty((B, Tq, Hq, D), dtype=q.dtype, device=dev)
    dK = torch.empty((B, Tk, Hk, D), dtype=q.dtype, device=dev)
    dV = torch.empty((B, Tk, Hk, D), dtype=q.dtype, device=dev)
    if B * Tq * Hq == 0 or Tk == 0:
        dQ.zero_()
        dK.zero_()
        dV.zero_()
        return tuple(x[..., :D_in].contiguous() for x in (dQ, dK, dV))
    do = _rows_reachable(_kernel_operand(do.to(q.dtype)), Tq)
    q = _rows_reachable(q, Tq)
    p = _ext.FaBwdParams()
    p.batch, p.seqlen_q, p.seqlen_k, p.heads_q, p.heads_k, p.head_dim = B, Tq, Tk, Hq, Hk, D
    p.scale = scale
    p.is_causal = 1 if is_causal else 0
    p.atomic_dq = 1 if use_atomic_backward else 0
    p.kv_split = 0
    p.dtype = _ext.dtype_code(q.dtype)
    p.ds_limit_bytes = ds_limit_bytes(dev)
    # the plan depends on whether a mask / score is given (dS tile pairs)
    p.mask, p.score = _ext.ptr(mask), _ext.ptr(score)
    lib = _ext.load_library()
    plan = _ext.FaBwdPlan()
    _ext.check(lib.fa_bwd_plan(ctypes.byref(p), ctypes.byref(plan)), "fa_bwd_plan", lib)
    p.kv_split = plan.kv_split

    delta = torch.empty((2, B, Hq, Tq), dtype=torch.float32, device=dev)   # Delta, backward LSE
    dead = torch.zeros((B * Hk,), dtype=torch.int32, device=dev)
    dq_acc = torch.empty((B, Tq, Hq, D), dtype=torch.float32, device=dev) if plan.needs_dq_accum else None
    dk_acc = dv_acc = None
    if plan.dkv_accum_elems > 0:
        # one fully overwritten fp32 slab per head-group part, or the running
        # sums of a backward over row ranges (zeroed only if the plan asks)
        alloc = torch.zeros if plan.dkv_accum_zeroed else torch.empty
        dk_acc = alloc((plan.dkv_accum_elems,), dtype=torch.float32, device=dev)
        dv_acc = alloc((plan.dkv_accum_elems,), dtype=torch.float32, device=dev)

    p.q, p.k, p.v, p.o, p.dout = q.data_ptr(), k.data_ptr(), v.data_ptr(), O.data_ptr(), do.data_ptr()
    p.lse, p.delta, p.dead_flags = LSE.data_ptr(), delta.data_ptr(), dead.data_ptr()
    p.mask_ws = _ext.ptr(mask_ws)
    # dS tiles handed from the dK/dV kernel to the dQ kernel
    ds = torch.empty((plan.ds_elems,), dtype=q.dtype, device=dev) if plan.ds_elems else None
    p.dq_accum, p.dk_accum, p.dv_accum = _ext.ptr(dq_acc), _ext.ptr(dk_acc), _ext.ptr(dv_acc)
    p.ds_tiles = _ext.ptr(ds)
    p.ds_tiles_elems = plan.ds_elems
    p.dq, p.dk, p.dv = dQ.data_ptr(), dK.data_ptr(), dV.data_ptr()
    p.q_stride_b, p.q_stride_t, p.q_stride_h = _bthd_strides(q)
    p.k_stride_b, p.k_stride_t, p.k_stride_h = _bthd_strides(k)
    p.v_stride_b, p.v_stride_t, p.v_stride_h = _bthd_strides(v)
    p.o_stride_b, p.o_stride_t, p.o_stride_h = _bthd_strides(O)
    if O_lo is not None:
        p.o_lo = O_lo.data_ptr()
        p.o_lo_stride_b, p.o_lo_stride_t, p.o_lo_stride_h = _bthd_strides(O_lo)
    p.do_stride_b, p.do_stride_t, p.do_stride_h = _bthd_strides(do)
    p.dq_stride_b, p.dq_stride_t, p.dq_stride_h = _bthd_strides(dQ)
    p.dk_stride_b, p.dk_stride_t, p.dk_stride_h = _bthd_strides(dK)
    p.dv_stride_b, p.dv_stride_t, p.dv_stride_h = _bthd_strides(dV)
    p.mask_stride_b, p.mask_stride_h, p.mask_stride_q = mst
    p.score_stride_b, p.score_stride_h, p.score_stride_q = sst
    p.stream = _stream(dev)
    _call(lib, "fa_bwd_preprocess", p)
    _call(lib, "fa_bwd", p)
    _call(lib, "fa_bwd_finalize", p)
    if D != D_in:
        dQ, dK, dV = (x[..., :D_in].contiguous() for x in (dQ, dK, dV))
    return dQ, dK, dV


class _flash_attention_with_4d_mask(torch.autograd.Function):
    """The reference's autograd Function (python/fa2.py:437-558), kept with its
    positional signature; ``flash_attention_with_4d_mask`` below reaches the
    same host code through the registered custom ops instead."""

    @staticmethod
    def forward(
        ctx,
        Q: torch.Tensor,
        K: torch.Tensor,
        V: torch.Tensor,
        Mask: Optional[torch.Tensor] = None,
        Score: Optional[torch.Tensor] = None,
        scale: Optional[float] = None,
        is_causal: Optional[bool] = False,
        use_atomic_backward: Optional[bool] = True,
        bhsd_input: Optional[bool] = True,
    ):
        assert Q.dim() == 4 and K.dim() == 4 and V.dim() == 4
        q = Q.transpose(1, 2) if bhsd_input else Q
        k = K.transpose(1, 2) if bhsd_input else K
        v = V.transpose(1, 2) if bhsd_input else V
        if scale is None:
            scale = q.shape[3] ** -0.5
        scale = float(scale)
        _check_qkv(q, k, v)
        O, LSE, mask_ws, O_lo, (q, k, v, mask, score, mst, sst) = _forward_impl(
            q, k, v, Mask, Score, scale, bool(is_causal), residual=any(ctx.needs_input_grad[:3]))
        ctx.save_for_backward(q, k, v, O, LSE, mask, score, mask_ws, O_lo)
        ctx.scale = scale
        ctx.is_causal = bool(is_causal)
        ctx.use_atomic_backward = bool(use_atomic_backward)
        ctx.mst, ctx.sst = mst, sst
        ctx.bhsd_input = bool(bhsd_input)
        return O.transpose(1, 2) if bhsd_input else O

    @staticmethod
    @once_differentiable
    def backward(ctx, dO: torch.Tensor):
        q, k, v, O, LSE, mask, score, mask_ws, O_lo = ctx.saved_tensors
        do = dO.transpose(1, 2) if ctx.bhsd_input else dO
        dQ, dK, dV = _backward_impl(do, q, k, v, O, LSE, mask, score, mask_ws, ctx.mst, ctx.sst, ctx.scale,
                                    ctx.is_causal, ctx.use_atomic_backward, O_lo)
        if ctx.bhsd_input:
            dQ, dK, dV = dQ.transpose(1, 2), dK.transpose(1, 2), dV.transpose(1, 2)
        return dQ, dK, dV, None, None, None, None, None, None


def flash_attention_with_4d_mask(Q, K, V, Mask=None, Score=None, scale=None, is_causal=False,
                                 use_atomic_backward=True, bhsd_input=True):
    """``flash_attention_with_4d_mask(Q, K, V, Mask, Score, scale, is_causal,
    use_atomic_backward, bhsd_input)`` (python/fa2.py:558): same positional
    signature, defaults, checks and autograd behaviour as the reference's
    ``Function.apply``; the work runs in the registered custom ops
    ``tilelang_fa2_4d_mask::fwd`` / ``::bwd`` (ops.py), which torch.compile and
    graph capture can trace."""
    from . import ops

    assert Q.dim() == 4 and K.dim() == 4 and V.dim() == 4
    q = Q.transpose(1, 2) if bhsd_input else Q
    k = K.transpose(1, 2) if bhsd_input else K
    v = V.transpose(1, 2) if bhsd_input else V
    if scale is None:
        scale = q.shape[3] ** -0.5
    _check_qkv(q, k, v)
    O = ops.attention(q, k, v, Mask, Score, float(scale), bool(is_causal), bool(use_atomic_backward))
    return O.transpose(1, 2) if bhsd_input else O


__all__ = ["flash_attention_with_4d_mask", "record_kernel_events", "KernelEventLog"]
