"""Attention with the reference kernel's 16-bit rounding points.  TEST INFRASTRUCTURE ONLY.

The eager oracle (``eager.py``) computes in fp32 throughout and rounds only its
outputs.  The reference's TileLang kernels (and this build's HIP kernels)
round two intermediates to the input dtype before a matrix product:

* forward: the probabilities P, copied to ``sP`` in dtype before ``O += P V``
  (python/fa2.py:128-129), while the row sum ``l`` adds the unrounded fp32 P
  (:124);
* backward: P before ``dV += P^T dO`` (:287) and dS before ``dK += dS^T Q``
  and ``dQ = dS K`` (:291-295); Delta is taken from the output O in dtype
  (bwd_preprocess, :166-176).

This module restates the attention forward and backward in float64 with
exactly those roundings and nothing else, so that the error a 16-bit kernel
cannot avoid (its "floor") can be measured against the eager oracle, and a
kernel can be compared against the restatement entry by entry.

Two choices fix which values get rounded, both as this build's kernels make
them (the error they leave is the same in distribution as the reference
kernel's; tests/test_oracle.py checks the mean errors agree):

* the softmax maximum in base 2 (y = s * scale * log2(e)) is the maximum m0
  of the row's first 64-key tile holding a kept key, raised in whole steps:
  m = m0 + ceil(max_j y_j - m0), p_j = 2^(y_j - m).  The rounded p_j is then
  round(2^frac(y_j - m0)) times a power of two for every m0 + k, so it does
  not depend on which running maximum an online softmax over 64-key tiles had
  when it rounded, and a row whose maximum lies in its first tile rounds its
  largest weight exactly (1).  The reference takes the fractional running
  maximum of every tile (:116-122);
* dS is rounded before the factor ``scale``, which is applied after the
  products (the reference rounds the scaled value, :291).

With a mask or a score the kernels carry each of those values as two 16-bit
parts, the rounded value plus its rounded residual, P for dV as three
(``split=True``), and the forward stores O's residual for Delta.

Pinned by tests/test_oracle.py: entry by entry against the scalar float64
loops of ``bruteforce.attention_bruteforce_rounded`` (single and split
roundings, bf16 and fp16), and planted placement mistakes in this function's
own source (P rounded after normalising, P or dS not rounded, Delta from the
unrounded O, dS rounded after the scale, the row's own maximum instead of the
first-tile grid) each fail that comparison; with the roundings off it equals
the eager oracle in float64 (forward, LSE and all three gradients, dead rows
included); the integer-maximum property of the rounded P; the floor each
rounding alone leaves at the BASELINE configs P and S.
"""

from __future__ import annotations

import math
from typing import Optional

import torch

from .eager import _expand_kv, _keep_for_rows

LOG2E = 1.0 / math.log(2.0)


def _round(x: torch.Tensor, dtype: Optional[torch.dtype]) -> torch.Tensor:
    return x if dtype is None else x.to(dtype).to(x.dtype)


def _round_split(x: torch.Tensor, dtype: Optional[torch.dtype], terms: int = 2) -> torch.Tensor:
    """x as ``terms`` 16-bit values: x rounded (through fp32, as a kernel
    rounds its fp32 values), then the fp32 residual rounded, and so on."""
    if dtype is None:
        return x
    r = x.to(torch.float32)
    out = torch.zeros_like(x)
    for _ in range(terms):
        part = r.to(dtype).to(torch.float32)
        out = out + part.to(x.dtype)
        r = r - part   # exact in fp32
    return out


def _first_tile_grid_max(y: torch.Tensor, ymax: torch.Tensor, tile_keys: int) -> torch.Tensor:
    """m0 + ceil(ymax - m0), m0 = max of the row's first ``tile_keys``-key tile
    holding a finite y (-inf for a row with none)."""
    Tk = y.shape[-1]
    nt = -(-Tk // tile_keys)
    pad = nt * tile_keys - Tk
    yt = torch.nn.functional.pad(y, (0, pad), value=float("-inf")) if pad else y
    tmax = yt.view(*y.shape[:-1], nt, tile_keys).amax(dim=-1)
    live = torch.isfinite(tmax) | (tmax == float("inf"))
    first = live.to(torch.int8).argmax(dim=-1, keepdim=True)
    m0 = torch.gather(tmax, -1, first)
    m0 = torch.where(live.any(dim=-1, keepdim=True), m0, torch.full_like(m0, float("-inf")))
    return torch.where(torch.isfinite(m0), m0 + torch.ceil(ymax - m0), ymax)


def rounded_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    mask: Optional[torch.Tensor],
    score: Optional[torch.Tensor],
    grad_out: Optional[torch.Tensor],
    *,
    scale: float,
    is_causal: bool,
    round_dtype: Optional[torch.dtype],
    round_p_fwd: bool = True,
    round_p_bwd: bool = True,
    round_ds: bool = True,
    delta_from_output: bool = True,
    scale_ds_before_round: bool = False,
    max_mode: str = "first_tile",
    tile_keys: int = 64,
    block: int = 128,
    compute_dtype: torch.dtype = torch.float64,
    split: bool = False,
):
    """Forward (and backward when ``grad_out`` is given) of attention in BHSD
    layout with the 16-bit roundings listed in the module docstring.

    q: [B, Hq, Tq, D]; k, v: [B, Hk, Tk, D]; mask bool / score float
    [B|1, Hq|1, Tq, Tk]; grad_out like q.  ``round_dtype`` is the dtype the
    intermediates are rounded to (None: no rounding).  The ``round_*`` flags
    switch single rounding points off; ``delta_from_output`` takes Delta from
    the output rounded to ``round_dtype`` (else Delta = sum_j P dP exactly);
    ``scale_ds_before_round`` and ``max_mode="row"`` (the row's fractional
    maximum) give the reference's own placements; ``max_mode="first_tile"``
    is the grid of the module docstring, over ``tile_keys``-key tiles.
    ``split``: every rounding point carries its value as two 16-bit parts,
    the rounded value plus its rounded residual, and P for dV as three (the
    second residual too) -- what the kernels do with a mask or a score; Delta
    then takes O plus the residual the forward stores.

    Returns a dict with ``out`` (compute dtype, before the final cast), ``lse``
    (base 2, [B, Hq, Tq]) and, with ``grad_out``, ``dq``, ``dk``, ``dv``
    (compute dtype; dk/dv summed over the query-head group).  Dead rows follow
    the eager oracle: a row whose kept logits are all -inf gives NaN in O,
    NaN in dV of its kv-head, dQ 0 when it keeps no key and NaN otherwise.
    """
    B, Hq, Tq, D = q.shape
    _, Hk, Tk, _ = k.shape
    G = Hq // Hk
    cd = compute_dtype
    dev = q.device
    rd = round_dtype
    R = (lambda x: _round_split(x, rd)) if split else (lambda x: _round(x, rd))
    R3 = (lambda x: _round_split(x, rd, terms=3)) if split else R   # P for dV
    qf = q.to(cd)
    kf = _expand_kv(k, G).to(cd)
    vf = _expand_kv(v, G).to(cd)
    kt = kf.transpose(-1, -2).contiguous()
    vt = vf.transpose(-1, -2).contiguous()
    out = torch.empty((B, Hq, Tq, D), dtype=cd, device=dev)
    lse = torch.empty((B, Hq, Tq), dtype=cd, device=dev)
    bwd = grad_out is not None
    if bwd:
        gf = grad_out.to(cd)
        dq = torch.empty((B, Hq, Tq, D), dtype=cd, device=dev)
        dk = torch.zeros((B, Hq, Tk, D), dtype=cd, device=dev)
        dv = torch.zeros((B, Hq, Tk, D), dtype=cd, device=dev)
    for q0 in range(0, Tq, block):
        q1 = min(q0 + block, Tq)
        qc = qf[:, :, q0:q1]
        y = torch.matmul(qc, kt)
        if score is not None:
            y = y + score[:, :, q0:q1].to(cd)
        y = y * (scale * LOG2E)
        keep = _keep_for_rows(q0, q1, Tk, mask, is_causal, dev)
        if keep is not None:
            y = y.masked_fill(~keep, float("-inf"))
        m = y.amax(dim=-1, keepdim=True)
        if max_mode == "first_tile":
            m = _first_tile_grid_max(y, m, tile_keys)
        elif max_mode != "row":
            raise ValueError(max_mode)
        pu = torch.exp2(y - m)                       # NaN rows where every logit is -inf
        l = pu.sum(dim=-1, keepdim=True)
        pr = R(pu) if round_p_fwd else pu
        o = torch.matmul(pr, vf) / l
        out[:, :, q0:q1] = o
        lse[:, :, q0:q1] = (m + torch.log2(l)).squeeze(-1)
        if not bwd:
            continue
        p = torch.exp2(y - m - torch.log2(l))        # normalised probabilities
        g = gf[:, :, q0:q1]
        dp = torch.matmul(g, vt)
        if delta_from_output:
            delta = (R(o) * g).sum(dim=-1, keepdim=True)
        else:
            delta = (p * dp).sum(dim=-1, keepdim=True)
        ds = p * (dp - delta)
        if keep is not None:
            ds = ds.masked_fill(~keep, 0.0)
        if scale_ds_before_round:
            dsr = R(ds * scale) if round_ds else ds * scale
            ds_scale = 1.0
        else:
            dsr = R(ds) if round_ds else ds
            ds_scale = scale
        pb = R3(p) if round_p_bwd else p
        dq[:, :, q0:q1] = torch.matmul(dsr, kf) * ds_scale
        dk += torch.matmul(dsr.transpose(-1, -2), qc) * ds_scale
        dv += torch.matmul(pb.transpose(-1, -2), g)
    res = {"out": out, "lse": lse}
    if bwd:
        res["dq"] = dq
        res["dk"] = dk.view(B, Hk, G, Tk, D).sum(dim=2)
        res["dv"] = dv.view(B, Hk, G, Tk, D).sum(dim=2)
    return res
