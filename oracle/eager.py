"""Eager fp32 reference attention (the parity oracle).  TEST INFRASTRUCTURE ONLY.

Restates ``eager_ref`` of the reference (benchmark/precision_check.py:133-180)
in this build's own code:

* GQA by ``repeat_interleave`` of K/V over the query-head group (:147-150);
* upcast to fp32 (:152-154);
* logits = (q . k^T + score) * scale, score added *before* scaling (:158-161);
* causal keep-rule ``i >= j`` with absolute, top-left aligned indices (:164-167);
* bool keep-mask AND-ed in (:168-170), dropped entries filled with -inf (:171-172);
* softmax over keys (:174), probabilities times V (:175);
* result cast back to the input dtype (:179-180); with ``ref_block`` the query
  rows are processed in chunks (:177-178).

Gradients come from torch autograd through exactly this graph, as the
reference's ``run_backward_case`` does (precision_check.py:297-304), which fixes
the dead-row policy (a row whose keys are all dropped):

* forward output row = NaN (softmax of an all -inf row);
* dQ row = exactly 0 (masked_fill's backward zeroes the whole row) and the row
  adds nothing to dK;
* dV of the whole (batch, kv-head) slice = NaN (the NaN probability row times dO
  reaches every key, and repeat_interleave's backward sums the group).

``eager_grads_chunked`` computes the same gradients in closed form, chunk by
chunk, without autograd's saved [B,H,Tq,Tk] probabilities; it is pinned against
``eager_fwd_bwd`` (autograd) in tests, dead rows included.

Pinned by: tests/test_oracle.py (float64 brute force on tiny inputs, torch SDPA
with enable_gqa on CPU, analytic invariants, finite differences for the
gradients, closed-form vs autograd).
"""

from __future__ import annotations

import math
from typing import Optional

import torch


def _expand_kv(x: torch.Tensor, groups: int) -> torch.Tensor:
    # precision_check.py:147-150
    return x if groups == 1 else x.repeat_interleave(groups, dim=1)


def _keep_for_rows(
    q_start: int,
    q_end: int,
    Tk: int,
    mask: Optional[torch.Tensor],
    is_causal: bool,
    device: torch.device,
) -> Optional[torch.Tensor]:
    """Keep-rule for query rows [q_start, q_end) (precision_check.py:163-170)."""
    keep = None
    if is_causal:
        qi = torch.arange(q_start, q_end, device=device)[:, None]
        kj = torch.arange(Tk, device=device)[None, :]
        keep = (qi >= kj).view(1, 1, q_end - q_start, Tk)
    if mask is not None:
        m = mask[:, :, q_start:q_end, :].to(device)
        keep = m if keep is None else (keep & m)
    return keep


def eager_ref(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    mask: Optional[torch.Tensor],
    score: Optional[torch.Tensor],
    *,
    scale: float,
    is_causal: bool,
    ref_block: int = 0,
    compute_dtype: torch.dtype = torch.float32,
) -> torch.Tensor:
    """Eager attention in BHSD layout; differentiable w.r.t. q, k, v.

    q: [B, Hq, Tq, D]; k, v: [B, Hk, Tk, D]; mask: bool [B|1, Hq|1, Tq, Tk];
    score: float [B|1, Hq|1, Tq, Tk].  Returns [B, Hq, Tq, D] in q.dtype.
    Follows benchmark/precision_check.py:133-180 step by step.  ``compute_dtype``
    is fp32 as in the reference; tests use float64 to pin the maths.
    """
    B, Hq, Tq, D = q.shape
    _, Hk, Tk, _ = k.shape
    if Hq % Hk != 0:
        raise ValueError(f"Hq={Hq} must be divisible by Hk={Hk}")
    groups = Hq // Hk
    cd = compute_dtype
    qf = q.to(cd)
    kf = _expand_kv(k, groups).to(cd)
    vf = _expand_kv(v, groups).to(cd)
    kt = kf.transpose(-1, -2).contiguous()

    def rows(q0: int, q1: int) -> torch.Tensor:
        logits = torch.matmul(qf[:, :, q0:q1, :], kt)
        if score is not None:
            logits = logits + score[:, :, q0:q1, :].to(cd)
        logits = logits * scale
        keep = _keep_for_rows(q0, q1, Tk, mask, is_causal, logits.device)
        if keep is not None:
            logits = logits.masked_fill(~keep, float("-inf"))
        probs = torch.softmax(logits, dim=-1)
        return torch.matmul(probs, vf)

    if ref_block and 0 < ref_block < Tq:
        parts = [rows(s, min(s + ref_block, Tq)) for s in range(0, Tq, ref_block)]
        return torch.cat(parts, dim=2).to(q.dtype)
    return rows(0, Tq).to(q.dtype)


def eager_fwd_bwd(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    mask: Optional[torch.Tensor],
    score: Optional[torch.Tensor],
    grad_out: torch.Tensor,
    *,
    scale: float,
    is_causal: bool,
    ref_block: int = 0,
    compute_dtype: torch.dtype = torch.float32,
):
    """Forward + autograd backward of :func:`eager_ref` on fresh leaf copies.

    Mirrors precision_check.py:297-304.  Returns (out, dq, dk, dv) in the
    input dtype and layout (BHSD).
    """
    qr = q.detach().clone().requires_grad_(True)
    kr = k.detach().clone().requires_grad_(True)
    vr = v.detach().clone().requires_grad_(True)
    out = eager_ref(qr, kr, vr, mask, score, scale=scale, is_causal=is_causal, ref_block=ref_block,
                    compute_dtype=compute_dtype)
    out.backward(grad_out)
    return out.detach(), qr.grad, kr.grad, vr.grad


def eager_grads_chunked(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    mask: Optional[torch.Tensor],
    score: Optional[torch.Tensor],
    grad_out: torch.Tensor,
    *,
    scale: float,
    is_causal: bool,
    block: int = 128,
    compute_dkdv: bool = True,
    compute_dtype: torch.dtype = torch.float32,
):
    """Closed-form forward + gradients of :func:`eager_ref`, chunked over query rows.

    Same values as :func:`eager_fwd_bwd` (including the dead-row policy) but
    holds only one [B, Hq, block, Tk] slab at a time, so the headline shapes fit
    in host or device memory.  All maths in fp32; results cast to q.dtype.

    Per chunk: P = softmax(logits); O = P V; dP = dO V^T; Delta_i = sum_j P_ij dP_ij;
    dS = P (dP - Delta) * scale with dropped entries' gradient zeroed (the
    masked_fill backward); dQ = dS K; dK += dS^T Q; dV += P^T dO, where P of a
    dead row is NaN everywhere (softmax of all -inf), as in autograd.
    Returns (out, dq, dk, dv).
    """
    B, Hq, Tq, D = q.shape
    _, Hk, Tk, _ = k.shape
    groups = Hq // Hk
    dev = q.device
    cd = compute_dtype
    qf = q.to(cd)
    kf = _expand_kv(k, groups).to(cd)
    vf = _expand_kv(v, groups).to(cd)
    kt = kf.transpose(-1, -2).contiguous()
    vt = vf.transpose(-1, -2).contiguous()
    gf = grad_out.to(cd)
    out = torch.empty((B, Hq, Tq, D), dtype=cd, device=dev)
    dq = torch.empty((B, Hq, Tq, D), dtype=cd, device=dev)
    dk = torch.zeros((B, Hq, Tk, D), dtype=cd, device=dev) if compute_dkdv else None
    dv = torch.zeros((B, Hq, Tk, D), dtype=cd, device=dev) if compute_dkdv else None
    for q0 in range(0, Tq, block):
        q1 = min(q0 + block, Tq)
        qc = qf[:, :, q0:q1, :]
        logits = torch.matmul(qc, kt)
        if score is not None:
            logits = logits + score[:, :, q0:q1, :].to(cd)
        logits = logits * scale
        keep = _keep_for_rows(q0, q1, Tk, mask, is_causal, dev)
        if keep is not None:
            logits = logits.masked_fill(~keep, float("-inf"))
        p = torch.softmax(logits, dim=-1)  # NaN rows where every key is dropped
        o = torch.matmul(p, vf)
        out[:, :, q0:q1, :] = o
        g = gf[:, :, q0:q1, :]
        dp = torch.matmul(g, vt)
        delta = (p * dp).sum(dim=-1, keepdim=True)
        ds = p * (dp - delta)
        if keep is not None:
            ds = ds.masked_fill(~keep, 0.0)
        ds = ds * scale
        dq[:, :, q0:q1, :] = torch.matmul(ds, kf)
        if compute_dkdv:
            dk += torch.matmul(ds.transpose(-1, -2), qc)
            dv += torch.matmul(p.transpose(-1, -2), g)
    if compute_dkdv:
        dk = dk.view(B, Hk, groups, Tk, D).sum(dim=2)
        dv = dv.view(B, Hk, groups, Tk, D).sum(dim=2)
        dk = dk.to(q.dtype)
        dv = dv.to(q.dtype)
    return out.to(q.dtype), dq.to(q.dtype), dk, dv


def eager_rows(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    mask: Optional[torch.Tensor],
    score: Optional[torch.Tensor],
    grad_out: Optional[torch.Tensor],
    rows: torch.Tensor,
    *,
    scale: float,
    is_causal: bool,
):
    """Oracle output (and dQ if grad_out is given) for a subset of query rows.

    Row i of O and dQ depends only on q_i, dO_i and all of K/V, so a row subset
    is exact for those rows (used for the full-size configs, where the whole
    oracle would take minutes on the host).  Returns (out_rows, dq_rows) with
    rows on dim 2, in q.dtype; dq_rows is None without grad_out.
    """
    B, Hq, Tq, D = q.shape
    _, Hk, Tk, _ = k.shape
    groups = Hq // Hk
    rows = rows.to(torch.long)
    qf = q[:, :, rows, :].float()
    kf = _expand_kv(k, groups).float()
    vf = _expand_kv(v, groups).float()
    logits = torch.matmul(qf, kf.transpose(-1, -2).contiguous())
    if score is not None:
        logits = logits + score[:, :, rows, :].float()
    logits = logits * scale
    keep = None
    if is_causal:
        keep = (rows[:, None].to(logits.device) >= torch.arange(Tk, device=logits.device)[None, :]).view(1, 1, -1, Tk)
    if mask is not None:
        m = mask[:, :, rows, :].to(logits.device)
        keep = m if keep is None else (keep & m)
    if keep is not None:
        logits = logits.masked_fill(~keep, float("-inf"))
    p = torch.softmax(logits, dim=-1)
    o = torch.matmul(p, vf)
    if grad_out is None:
        return o.to(q.dtype), None
    g = grad_out[:, :, rows, :].float()
    dp = torch.matmul(g, vf.transpose(-1, -2).contiguous())
    delta = (p * dp).sum(dim=-1, keepdim=True)
    ds = p * (dp - delta)
    if keep is not None:
        ds = ds.masked_fill(~keep, 0.0)
    dq = torch.matmul(ds * scale, kf)
    return o.to(q.dtype), dq.to(q.dtype)


# ---------------------------------------------------------------------------
# statistics and pass rules
# ---------------------------------------------------------------------------

def diff_stats(actual: torch.Tensor, expected: torch.Tensor) -> dict:
    """max/mean absolute and relative error (precision_check.py:183-194)."""
    af = actual.float()
    ef = expected.float()
    diff = (af - ef).abs()
    rel = diff / ef.abs().clamp_min(1e-6)
    return {
        "max_abs": diff.max().item(),
        "mean_abs": diff.mean().item(),
        "max_rel": rel.max().item(),
        "mean_rel": rel.mean().item(),
    }


def finite_diff_stats(actual: torch.Tensor, expected: torch.Tensor) -> dict:
    """diff_stats over the entries where the oracle is finite, plus NaN agreement.

    Used where the dead-row policy puts NaN into the oracle: those positions
    must be NaN in ``actual`` too (``nan_match``), and the rest is compared
    numerically.
    """
    ef = expected.float()
    af = actual.float()
    fin = torch.isfinite(ef)
    nan_match = bool(torch.equal(torch.isnan(af), torch.isnan(ef)))
    if fin.any():
        s = diff_stats(af[fin], ef[fin])
    else:
        s = {"max_abs": 0.0, "mean_abs": 0.0, "max_rel": 0.0, "mean_rel": 0.0}
    s["nan_match"] = nan_match
    return s


def case_passed(stats: dict, atol: float = 5e-2, rtol: float = 5e-2) -> bool:
    """The reference's own loose rule: max_abs <= atol OR mean_rel <= rtol
    (precision_check.py:205-206, defaults :371-372)."""
    return stats["max_abs"] <= atol or stats["mean_rel"] <= rtol


# The north-star bar for bf16/fp16: max_abs <= 2e-2 AND mean_abs <= 1e-4.
NORTH_STAR_MAX_ABS = 2e-2
NORTH_STAR_MEAN_ABS = 1e-4


def north_star_passed(stats: dict, max_abs: float = NORTH_STAR_MAX_ABS, mean_abs: float = NORTH_STAR_MEAN_ABS) -> bool:
    return stats["max_abs"] <= max_abs and stats["mean_abs"] <= mean_abs and stats.get("nan_match", True)


def estimate_tflops(B: int, Tq: int, Tk: int, Hq: int, D: int, is_causal: bool, ms: float, mode: str) -> float:
    """FLOP convention of benchmark/throughput_check.py:85-92: fwd 4*B*Hq*Tq*Tk*D,
    fwd+bwd 14*..., times 0.5 when causal; masks never reduce it."""
    return conv_flops(B, Tq, Tk, Hq, D, is_causal, mode) * 1e-12 / (ms * 1e-3)


def conv_flops(B: int, Tq: int, Tk: int, Hq: int, D: int, is_causal: bool, mode: str) -> float:
    mult = 4.0 if mode == "fwd" else 14.0
    return mult * (0.5 if is_causal else 1.0) * B * Hq * Tq * Tk * D


def lse2_reference(q, k, mask, score, *, scale: float, is_causal: bool) -> torch.Tensor:
    """log2-sum-exp2 of the scaled logits per row, [B, Hq, Tq] fp32.

    LSE2 = log2(e) * logsumexp(scale * (q k^T + score)) over kept keys; +inf for
    a dead row (the kernels' convention for "no kept key").  Internal fwd->bwd
    contract only; not user visible.
    """
    B, Hq, Tq, D = q.shape
    Hk = k.shape[1]
    kf = _expand_kv(k, Hq // Hk).float()
    logits = torch.matmul(q.float(), kf.transpose(-1, -2).contiguous())
    if score is not None:
        logits = logits + score.float()
    logits = logits * scale
    keep = _keep_for_rows(0, Tq, k.shape[2], mask, is_causal, logits.device)
    if keep is not None:
        logits = logits.masked_fill(~keep, float("-inf"))
    lse = torch.logsumexp(logits, dim=-1) * (1.0 / math.log(2.0))
    return torch.where(torch.isneginf(lse), torch.full_like(lse, float("inf")), lse)
