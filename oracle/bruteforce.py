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
import struct


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


# ---------------------------------------------------------------------------
# The same loops with the 16-bit roundings of the kernels (pins
# oracle/rounding.py; TEST INFRASTRUCTURE ONLY)
# ---------------------------------------------------------------------------

def _f32(x: float) -> float:
    """x rounded to the nearest float32 (ties to even), as a Python float."""
    if x != x or x in (math.inf, -math.inf):
        return x
    return struct.unpack("<f", struct.pack("<f", x))[0]


def round16(x: float, dtype: str) -> float:
    """x rounded to fp32 and then to bf16 / fp16, nearest with ties to even --
    the conversions a kernel makes from its fp32 values (and torch's
    ``.to(dtype)`` of a float64 tensor).  bf16 by the bit pattern of the fp32
    value (keep the top 16 bits, round on the lower 16); fp16 by struct's
    IEEE half packing of the fp32 value."""
    x = _f32(x)
    if x != x or x in (math.inf, -math.inf):
        return x
    if dtype == "fp16":
        return struct.unpack("<e", struct.pack("<e", x))[0] if abs(x) < 65520.0 else math.copysign(math.inf, x)
    if dtype != "bf16":
        raise ValueError(dtype)
    bits = struct.unpack("<I", struct.pack("<f", x))[0]
    lower = bits & 0xFFFF
    upper = bits >> 16
    if lower > 0x8000 or (lower == 0x8000 and (upper & 1)):
        upper += 1
    return struct.unpack("<f", struct.pack("<I", (upper & 0xFFFF) << 16))[0]


def round16_split(x: float, dtype: str, terms: int = 2) -> float:
    """x carried as ``terms`` 16-bit values: the rounded value, then its
    rounding residual (the fp32 difference, itself rounded), and so on --
    what the kernels feed the matrix products with a mask or a score."""
    r = _f32(x)
    total = 0.0
    for _ in range(terms):
        part = round16(r, dtype)
        if part != part or part in (math.inf, -math.inf):
            return part
        total += part
        r = _f32(r - part)
    return total


def attention_bruteforce_rounded(q, k, v, mask, score, dout, scale, is_causal, dtype="bf16", split=False,
                                 tile_keys=64):
    """Scalar float64 loops of the attention forward and backward with the
    16-bit roundings of the kernels (the points ``oracle/rounding.py``
    restates with tensor operations):

    * base-2 logits y_j = (q . k_j + score_j) scale log2(e) over kept keys;
      the softmax maximum is the maximum m0 of the row's first ``tile_keys``
      key tile that holds a kept key, raised in whole steps:
      m = m0 + ceil(max_j y_j - m0); p_j = 2^(y_j - m), l = sum_j p_j (not
      rounded), LSE = m + log2 l;
    * O = sum_j R(p_j) v_j / l, R = rounding to ``dtype`` (with ``split``:
      the rounded value plus its rounded residual);
    * backward: P_j = 2^(y_j - LSE) (not rounded), dP_j = dO . v_j,
      Delta = sum_d R(O_d) dO_d (O from the forward, as stored, plus its
      residual with ``split``), dS_j = P_j (dP_j - Delta) (0 for dropped
      keys), dQ = scale sum_j R(dS_j) k_j, dK_j += scale R(dS_j) q,
      dV_j += R3(P_j) dO -- dS rounded before the factor scale; R3 = R,
      except with ``split`` three parts (the second residual too).

    Scores of -inf are not supported here (oracle/eager.py covers them).
    Same arguments and nested-list layout as :func:`attention_bruteforce`,
    plus ``dtype`` ("bf16" / "fp16"; None: no rounding) and ``split``.  Returns (o, lse, dq, dk,
    dv); lse is base 2, [B][Hq][Tq], +inf for a row with no kept key.  Dead
    rows follow :func:`attention_bruteforce` (NaN O, zero dQ, NaN dV of the
    kv-head)."""
    if dtype is None:
        R = lambda x: x   # noqa: E731  (no rounding: the plain maths)
    else:
        R = (lambda x: round16_split(x, dtype)) if split else (lambda x: round16(x, dtype))
    R3 = (lambda x: round16_split(x, dtype, terms=3)) if split and dtype is not None else R   # P for dV
    B, Hq, Tq, D = len(q), len(q[0]), len(q[0][0]), len(q[0][0][0])
    Hk, Tk = len(k[0]), len(k[0][0])
    G = Hq // Hk
    nan, inf = float("nan"), float("inf")
    log2e = 1.0 / math.log(2.0)
    o = [[[[0.0] * D for _ in range(Tq)] for _ in range(Hq)] for _ in range(B)]
    lse = [[[inf] * Tq for _ in range(Hq)] for _ in range(B)]
    dq = [[[[0.0] * D for _ in range(Tq)] for _ in range(Hq)] for _ in range(B)]
    dk = [[[[0.0] * D for _ in range(Tk)] for _ in range(Hk)] for _ in range(B)]
    dv = [[[[0.0] * D for _ in range(Tk)] for _ in range(Hk)] for _ in range(B)]
    for b in range(B):
        for h in range(Hq):
            g = h // G
            for i in range(Tq):
                y = []
                for j in range(Tk):
                    keep = (not is_causal or i >= j) and (mask is None or bool(mask[b][h][i][j]))
                    if not keep:
                        y.append(None)
                        continue
                    s = sum(q[b][h][i][d] * k[b][g][j][d] for d in range(D))
                    if score is not None:
                        s += score[b][h][i][j]
                    y.append(s * scale * log2e)
                kept = [x for x in y if x is not None]
                if not kept:
                    for d in range(D):
                        o[b][h][i][d] = nan
                    if dout is not None:
                        for j in range(Tk):
                            for d in range(D):
                                dv[b][g][j][d] = nan
                    continue
                first = min(j for j in range(Tk) if y[j] is not None and y[j] > -inf) // tile_keys
                m0 = max(y[j] for j in range(first * tile_keys, min(Tk, (first + 1) * tile_keys)) if y[j] is not None)
                m = m0 + math.ceil(max(kept) - m0)
                p = [0.0 if x is None else 2.0 ** (x - m) for x in y]
                l = sum(p)
                row_o = [sum(R(p[j]) * v[b][g][j][d] for j in range(Tk)) / l for d in range(D)]
                o[b][h][i] = row_o
                L = m + math.log2(l)
                lse[b][h][i] = L
                if dout is None:
                    continue
                P = [0.0 if x is None else 2.0 ** (x - L) for x in y]
                dp = [sum(dout[b][h][i][d] * v[b][g][j][d] for d in range(D)) for j in range(Tk)]
                delta = sum(R(row_o[d]) * dout[b][h][i][d] for d in range(D))
                ds = [0.0 if y[j] is None else P[j] * (dp[j] - delta) for j in range(Tk)]
                dsr = [R(x) for x in ds]
                for d in range(D):
                    dq[b][h][i][d] = sum(dsr[j] * k[b][g][j][d] for j in range(Tk)) * scale
                for j in range(Tk):
                    pr = R3(P[j])
                    for d in range(D):
                        dk[b][g][j][d] += dsr[j] * q[b][h][i][d] * scale
                        dv[b][g][j][d] += pr * dout[b][h][i][d]
    return o, lse, dq, dk, dv
