"""Scalar float64 attention for tiny inputs.  TEST INFRASTRUCTURE ONLY.

A loop-level statement of the maths the reference's eager path computes
(benchmark/precision_check.py:133-180), with no torch kernels involved, used to
pin :mod:`oracle.eager`:

    l_ij = (q_i . k_{g(h),j} + score_ij) * scale
    keep_ij = (not causal or i >= j) and mask_ij
    p_ij = exp(l_ij - max_j l_ij) / sum_j exp(...)   over kept j
    o_i = sum_j p_ij v_j

and the analytic gradients

    dp_ij = dO_i . v_j,  D_i = sum_j p_ij dp_ij,  ds_ij = p_ij (dp_ij - D_i) scale
    dq_i = sum_j ds_ij k_j,  dk_j = sum_{h in group, i} ds_ij q_i,  dv_j = sum p_ij dO_i

A row with no kept key gives NaN output, zero dq and NaN dv for its kv-head
(see oracle/eager.py for why).
"""

from __future__ import annotations

import math


def attention_bruteforce(q, k, v, mask, score, dout, scale, is_causal):
    """q: [B][Hq][Tq][D] nested lists (floats), k/v: [B][Hk][Tk][D],
    mask: None or [B][Hq][Tq][Tk] bools, score: None or [B][Hq][Tq][Tk],
    dout: None or like q.  Returns (o, dq, dk, dv) as nested lists."""
    B, Hq, Tq, D = len(q), len(q[0]), len(q[0][0]), len(q[0][0][0])
    Hk, Tk = len(k[0]), len(k[0][0])
    G = Hq // Hk
    nan = float("nan")
    o = [[[[0.0] * D for _ in range(Tq)] for _ in range(Hq)] for _ in range(B)]
    dq = [[[[0.0] * D for _ in range(Tq)] for _ in range(Hq)] for _ in range(B)]
    dk = [[[[0.0] * D for _ in range(Tk)] for _ in range(Hk)] for _ in range(B)]
    dv = [[[[0.0] * D for _ in range(Tk)] for _ in range(Hk)] for _ in range(B)]
    for b in range(B):
        for h in range(Hq):
            g = h // G
            for i in range(Tq):
                logits = []
                for j in range(Tk):
                    keep = (not is_causal or i >= j) and (mask is None or bool(mask[b][h][i][j]))
                    if not keep:
                        logits.append(None)
                        continue
                    s = sum(q[b][h][i][d] * k[b][g][j][d] for d in range(D))
                    if score is not None:
                        s += score[b][h][i][j]
                    logits.append(s * scale)
                kept = [x for x in logits if x is not None]
                if not kept:
                    for d in range(D):
                        o[b][h][i][d] = nan
                    if dout is not None:
                        for j in range(Tk):
                            for d in range(D):
                                dv[b][g][j][d] = nan
                    continue
                m = max(kept)
                e = [0.0 if x is None else math.exp(x - m) for x in logits]
                z = sum(e)
                p = [x / z for x in e]
                for d in range(D):
                    o[b][h][i][d] = sum(p[j] * v[b][g][j][d] for j in range(Tk))
                if dout is None:
                    continue
                dp = [sum(dout[b][h][i][d] * v[b][g][j][d] for d in range(D)) for j in range(Tk)]
                delta = sum(p[j] * dp[j] for j in range(Tk))
                ds = [0.0 if logits[j] is None else p[j] * (dp[j] - delta) * scale for j in range(Tk)]
                for d in range(D):
                    dq[b][h][i][d] = sum(ds[j] * k[b][g][j][d] for j in range(Tk))
                for j in range(Tk):
                    for d in range(D):
                        dk[b][g][j][d] += ds[j] * q[b][h][i][d]
                        dv[b][g][j][d] += p[j] * dout[b][h][i][d]
    return o, dq, dk, dv
