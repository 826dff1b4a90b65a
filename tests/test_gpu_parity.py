"""GPU parity: the HIP kernels (through the product API and the C ABI) against
the eager oracle on identical seeded inputs.

Small and medium shapes are checked against the CPU oracle (oracle/eager.py,
autograd through the reference's eager graph).  The BASELINE configs at full
size are checked against the same oracle's closed-form chunked variant run in
fp32 on the device (the CPU would take minutes), plus size-independent
properties.

Tolerances (bf16/fp16, every output O, dQ, dK, dV):
  * the north-star bar max_abs <= 2e-2 and mean_abs <= 1e-4 at the BASELINE
    shapes;
  * on the small shapes outputs are larger (fewer keys to average over), so the
    mean bar scales with the output magnitude: mean_abs <= max(1e-4, 2^-8 *
    mean|ref|), i.e. about one bf16 rounding step of the typical entry;
  * NaN positions must match the oracle exactly (dead-row policy) and a dead
    row's dQ must be exactly 0.
"""

import ctypes
import math

import pytest
import torch

from oracle import eager as E
from oracle import inputs as I

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2


def _api():
    import tilelang_fa2_4d_mask as api

    return api


def _one_unit_limit(cfg):
    """dS workspace bytes of one (batch, kv-head) unit: the group's Hq/Hk planes
    of 32x32 16-bit tiles (causal: tiles on or below the diagonal)."""
    nq, nk = -(-cfg.Tq // 32), -(-cfg.Tk // 32)
    plane = sum(min(s + 1, nk) for s in range(nq)) if cfg.is_causal else nq * nk
    return 2 * (cfg.Hq // cfg.Hk) * plane * 1024


def _rows_limit(cfg):
    """dS workspace bytes of the largest 512-row range of every (batch, head)
    plane: below one unit (Tq > 512 B Hk) the backward then runs one range of
    query rows per launch pair; otherwise it slices by units."""
    nq, nk = -(-cfg.Tq // 32), -(-cfg.Tk // 32)
    parts = 2 if (cfg.mask is not None or cfg.score is not None) else 1
    tiles = [min(s + 1, nk) if cfg.is_causal else nk for s in range(nq)]
    best = max(sum(tiles[c:c + 16]) for c in range(0, nq, 16))
    return 2 * parts * cfg.B * cfg.Hq * best * 1024


def _one_plane_limit(cfg):
    """dS workspace bytes of one (batch, head) plane, tile pairs included (a
    mask or a score): below one unit, a masked backward splits each head
    group into parts of one head."""
    nq, nk = -(-cfg.Tq // 32), -(-cfg.Tk // 32)
    plane = sum(min(s + 1, nk) for s in range(nq)) if cfg.is_causal else nq * nk
    parts = 2 if (cfg.mask is not None or cfg.score is not None) else 1
    return 2 * parts * plane * 1024


def run_ours(case, cfg, *, atomic=True, scale=None, attention_mask=None, backward=True, ds_limit=0):
    """ds_limit: dS workspace limit of the backward (0 = default, dQ from the
    stored dS tiles; -1 = no workspace: dQ recomputed, in both modes;
    "unit" = one (batch, kv-head) unit: the dS kernels run once
    per unit; "rows" = one 512-row range of every unit, see _rows_limit;
    "plane" = one (batch, head) plane, see _one_plane_limit)."""
    api = _api()
    import tilelang_fa2_4d_mask.fa2 as fa2mod

    fa2mod.DS_LIMIT_BYTES = {"unit": _one_unit_limit, "rows": _rows_limit, "plane": _one_plane_limit}[ds_limit](
        cfg) if isinstance(
        ds_limit, str) else ds_limit
    dev = torch.device("cuda:0")
    q = case["q"].to(dev).detach().requires_grad_(backward)
    k = case["k"].to(dev).detach().requires_grad_(backward)
    v = case["v"].to(dev).detach().requires_grad_(backward)
    mask = None if case["mask"] is None else case["mask"].to(dev)
    score = None if case["score"] is None else case["score"].to(dev)
    am = None if attention_mask is None else attention_mask.to(dev)
    out = api.tilelang_flash_attention(
        q, k, v, mask=mask, score=score, attention_mask=am, scale=scale, is_causal=cfg.is_causal,
        layout=cfg.layout, use_atomic_backward=atomic,
    )
    res = {"out": out.detach()}
    try:
        if backward:
            out.backward(case["grad"].to(dev))
            res.update(dq=q.grad, dk=k.grad, dv=v.grad)
        torch.cuda.synchronize()
    finally:
        fa2mod.DS_LIMIT_BYTES = 0
    if cfg.layout == "bshd":
        res = {n: t.transpose(1, 2) for n, t in res.items()}
    return {n: t.float().cpu() for n, t in res.items()}


def run_oracle_cpu(case, cfg, *, scale=None, backward=True):
    s = cfg.D ** -0.5 if scale is None else scale
    q, k, v = (case[n].cpu() for n in ("q_bhsd", "k_bhsd", "v_bhsd"))
    mask = case["mask"]
    score = case["score"]
    if not backward:
        return {"out": E.eager_ref(q, k, v, mask, score, scale=s, is_causal=cfg.is_causal).float()}
    o, dq, dk, dv = E.eager_fwd_bwd(q, k, v, mask, score, case["grad_bhsd"].cpu(), scale=s, is_causal=cfg.is_causal)
    return {"out": o.float(), "dq": dq.float(), "dk": dk.float(), "dv": dv.float()}


def run_exact_cpu(case, cfg):
    """Output and gradients of the oracle's graph in float64 from the same
    inputs (leaves upcast first, so no rounding to the input dtype anywhere)."""
    q, k, v = (case[n].cpu().double().requires_grad_(True) for n in ("q_bhsd", "k_bhsd", "v_bhsd"))
    o = E.eager_ref(q, k, v, case["mask"], case["score"], scale=cfg.D ** -0.5, is_causal=cfg.is_causal,
                    compute_dtype=torch.float64)
    o.backward(case["grad_bhsd"].cpu().double())
    return {"out": o.detach().float(), "dq": q.grad.float(), "dk": k.grad.float(), "dv": v.grad.float()}


def check(ours, ref, *, label, mean_floor=1e-4, small_shape=True, mean_rel=2.0 ** -8, abs_bar=MAX_ABS,
          rel_bar=2.0 ** -6):
    """small_shape: per-entry |ours - ref| <= 2e-2 + 2^-6 |ref| (the absolute bar,
    or two bf16 ulps of the entry, whichever is larger: gradient entries of a few
    units exist at small T and one bf16 ulp there is already 0.03) and
    mean_abs <= max(1e-4, mean_rel * mean|ref|).  Otherwise the north-star bar:
    max_abs <= 2e-2 and mean_abs <= 1e-4."""
    report = {}
    for name in ref:
        st = E.finite_diff_stats(ours[name], ref[name])
        r = ref[name]
        fin = torch.isfinite(r)
        mag = r[fin].abs().mean().item() if fin.any() else 0.0
        mean_tol = max(mean_floor, mean_rel * mag) if small_shape else mean_floor
        if fin.any():
            err = (ours[name][fin].float() - r[fin].float()).abs()
            bound = abs_bar + rel_bar * r[fin].float().abs() if small_shape else torch.full_like(err, MAX_ABS)
            worst = (err - bound).max().item()
        else:
            worst = -1.0
        report[name] = (st, mean_tol, worst)
        print(f"[{label}] {name}: max_abs={st['max_abs']:.3e} mean_abs={st['mean_abs']:.3e} "
              f"(tol {mean_tol:.1e}) mag={mag:.3e} nan_match={st['nan_match']} bound_margin={-worst:.2e}", flush=True)
    for name, (st, mean_tol, worst) in report.items():
        assert st["nan_match"], f"{label} {name}: NaN positions differ from the oracle"
        assert worst <= 0.0, f"{label} {name}: max_abs {st['max_abs']:.3e} exceeds the bound by {worst:.3e}"
        assert st["mean_abs"] <= mean_tol, f"{label} {name}: mean_abs {st['mean_abs']:.3e} > {mean_tol:.1e}"


C = I.AttnConfig
SMALL = [
    C("mha_d128", 2, 256, 256, 4, 4, 128),
    C("gqa_d128_causal", 1, 384, 384, 8, 2, 128, is_causal=True),
    C("gqa_d64", 2, 256, 256, 8, 2, 64),
    C("mqa_d64_causal", 1, 320, 320, 8, 1, 64, is_causal=True),
    C("ragged_noncausal", 1, 200, 333, 4, 2, 128),
    C("ragged_causal_tq_lt_tk", 1, 130, 333, 4, 2, 128, is_causal=True),
    C("ragged_causal_tq_gt_tk", 1, 333, 130, 4, 2, 64, is_causal=True),
    C("fp16_gqa", 1, 256, 256, 8, 4, 128, torch.float16),
    C("fp16_causal_d64", 1, 256, 256, 4, 4, 64, torch.float16, is_causal=True),
    C("bshd_mqa", 1, 192, 512, 8, 1, 64, layout="bshd"),
    C("mask_full_heads", 2, 256, 256, 4, 2, 128, mask="bernoulli"),
    C("mask_head_bcast", 2, 256, 256, 4, 2, 128, mask="bernoulli", mask_heads=1),
    C("mask_causal_ragged", 1, 257, 257, 4, 2, 64, is_causal=True, mask="bernoulli"),
    C("score", 1, 256, 256, 4, 2, 128, score="normal"),
    C("score_mask_causal", 1, 256, 256, 4, 4, 128, is_causal=True, mask="bernoulli", score="normal"),
    C("packed_docs", 1, 512, 512, 4, 2, 128, mask="packed_docs", mask_heads=1,
      extra={"packed": {"lo": 40, "hi": 160}}),
    C("alibi_sparse", 1, 256, 256, 4, 4, 128, mask="sparse_diag", mask_heads=4, score="alibi_noise"),
    C("fp16_mask_score_d64", 1, 200, 200, 4, 2, 64, torch.float16, mask="bernoulli", score="normal"),
    # score rows of 203 floats (not 16-byte aligned), a partial last key tile
    C("score_unaligned_ragged", 1, 200, 203, 4, 2, 128, mask="bernoulli", score="normal"),
    C("score_causal_ragged", 1, 333, 203, 4, 2, 128, is_causal=True, score="normal"),
    # BASELINE configs[0] (C) at its shape, B1 Hq4 Hk2 T256 D64 causal, in the
    # GPU dtypes (its fp32 form is the CPU oracle's own plumbing case)
    C("C_shape_bf16", 1, 256, 256, 4, 2, 64, is_causal=True),
    C("C_shape_fp16", 1, 256, 256, 4, 2, 64, torch.float16, is_causal=True),
]


# backward modes: fp32-atomic dQ over key ranges of the stored dS (default);
# atomic mode without a dS workspace (dQ recomputed, as in the deterministic
# mode); deterministic with dQ from the stored dS tiles; deterministic with dQ
# recomputed (no dS workspace allowed); both dS modes with a workspace of one (batch, kv-head)
# unit, so that the dS kernels run slice by slice (sized without the tile
# pairs of a mask or score: half a unit there, so a masked group splits in
# two); both with a workspace of one 512-row range of every unit (ranges of
# rows where Tq > 512 B Hk without a mask; unit slices or recompute
# otherwise); both with a workspace of one (batch, head) plane (a masked
# head group then splits into one-head parts)
MODES = {"atomic": (True, 0), "atomic_no_ws": (True, -1), "det_ds": (False, 0), "det_recompute": (False, -1),
         "atomic_sliced": (True, "unit"), "det_sliced": (False, "unit"),
         "atomic_rows": (True, "rows"), "det_rows": (False, "rows"),
         "atomic_parts": (True, "plane"), "det_parts": (False, "plane")}


@pytest.mark.parametrize("mode", list(MODES))
@pytest.mark.parametrize("cfg", SMALL, ids=[c.name for c in SMALL])
def test_small_vs_oracle(cuda, cfg, mode):
    case = I.make_case(cfg, seed=0)
    print(f"case {cfg.name} mode={mode}", flush=True)
    atomic, ds_limit = MODES[mode]
    ours = run_ours(case, cfg, atomic=atomic, ds_limit=ds_limit)
    ref = run_oracle_cpu(case, cfg)
    check(ours, ref, label=f"{cfg.name}/{mode}")


# Shapes with enough 512-row query blocks (B Hq ceil(Tq / 512) >= 256) that
# the dQ kernel runs its 8-wave workgroups (head dim 128, no mask), in atomic
# mode too (row blocks enough for every CU: written directly, no atomics);
# ragged Tq and Tk, causal with Tq != Tk, fp16
WIDE_DQ = [
    C("wide_dq_ragged", 2, 1000, 900, 64, 8, 128),
    C("wide_dq_causal", 1, 700, 760, 128, 16, 128, is_causal=True),
    C("wide_dq_fp16_bshd", 1, 520, 520, 128, 32, 128, torch.float16, layout="bshd"),
]


@pytest.mark.parametrize("mode", ["det_ds", "atomic"])
@pytest.mark.parametrize("cfg", WIDE_DQ, ids=[c.name for c in WIDE_DQ])
def test_wide_dq_vs_oracle(cuda, cfg, mode):
    case = I.make_case(cfg, seed=5)
    print(f"case {cfg.name} mode={mode}", flush=True)
    atomic, ds_limit = MODES[mode]
    ours = run_ours(case, cfg, atomic=atomic, ds_limit=ds_limit)
    ref = run_oracle_cpu(case, cfg)
    check(ours, ref, label=f"{cfg.name}/{mode}")


# The backward over ranges of query rows (Tq > 512 B Hk, no mask, head dim
# <= 128): 2-5 ranges, so the dK/dV sums are written, added to and finished;
# MQA and GQA, causal with Tq > Tk, a score (dS tile pairs), fp16 bshd, head
# dim 64.
ROWS = [
    C("rows_mqa", 1, 1500, 1100, 4, 1, 128),
    C("rows_mqa_causal", 1, 1500, 1100, 4, 1, 128, is_causal=True),
    C("rows_gqa_ragged", 1, 2100, 600, 4, 2, 128),
    C("rows_score_d64", 1, 1100, 700, 2, 1, 64, score="normal"),
    C("rows_fp16_bshd_causal", 1, 1200, 1000, 8, 1, 128, torch.float16, layout="bshd", is_causal=True),
    # causal with Tq < Tk: key blocks past the last row get no step in any
    # range (their sums stay 0 and dK/dV come out 0)
    C("rows_causal_tq_lt_tk", 1, 1100, 1700, 4, 1, 128, is_causal=True),
]


def _plan_of(cfg, limit, atomic):
    from tilelang_fa2_4d_mask import _ext

    p = _ext.FaBwdParams()
    p.batch, p.seqlen_q, p.seqlen_k, p.heads_q, p.heads_k, p.head_dim = cfg.B, cfg.Tq, cfg.Tk, cfg.Hq, cfg.Hk, cfg.D
    p.scale, p.is_causal, p.atomic_dq, p.dtype = cfg.D ** -0.5, int(cfg.is_causal), int(atomic), 0
    p.ds_limit_bytes = limit
    p.score = 16 if cfg.score is not None else None
    p.mask = 16 if cfg.mask is not None else None
    plan = _ext.FaBwdPlan()
    lib = _ext.load_library()
    assert lib.fa_bwd_plan(ctypes.byref(p), ctypes.byref(plan)) == 0
    return plan


@pytest.mark.parametrize("mode", ["det_rows", "atomic_rows"])
@pytest.mark.parametrize("cfg", ROWS, ids=[c.name for c in ROWS])
def test_row_ranges_vs_oracle(cuda, cfg, mode):
    atomic, ds_limit = MODES[mode]
    plan = _plan_of(cfg, _rows_limit(cfg), atomic)
    # the route really is the ranged one: dS tiles, the fp32 sums (one per
    # head-group part; causal launches split the group), no dQ atomics
    assert plan.ds_elems > 0 and plan.dkv_accum_elems == plan.kv_split * cfg.B * cfg.Tk * cfg.Hk * cfg.D
    assert plan.needs_dq_accum == 0 and (plan.kv_split == 1 or cfg.is_causal)
    case = I.make_case(cfg, seed=7)
    print(f"case {cfg.name} mode={mode}", flush=True)
    ours = run_ours(case, cfg, atomic=atomic, ds_limit=ds_limit)
    ref = run_oracle_cpu(case, cfg)
    check(ours, ref, label=f"{cfg.name}/{mode}")
    # dQ of a row comes from the same dS tiles in the same key order as the
    # unranged launch: bitwise equal to it
    one = run_ours(case, cfg, atomic=False, ds_limit=0)
    assert torch.equal(ours["dq"], one["dq"]) and torch.equal(ours["out"], one["out"])


# The masked backward over parts of head groups (one (batch, head) plane of
# workspace, below one unit): GQA with batch 2, packed documents with a score
# in MQA causal, a group of three heads (split 3) with a head-broadcast mask in
# fp16 bshd.
PARTS = [
    C("parts_mask_gqa", 2, 700, 600, 8, 2, 128, mask="bernoulli"),
    C("parts_docs_mqa_causal_score", 1, 512, 512, 4, 1, 64, is_causal=True, mask="packed_docs", mask_heads=1,
      score="normal"),
    C("parts_mask_g3_fp16_bshd", 1, 300, 333, 6, 2, 128, torch.float16, layout="bshd", mask="bernoulli",
      mask_heads=1),
    # causal with Tq < Tk and a per-head mask: key blocks without a live step
    C("parts_mask_causal_tq_lt_tk", 1, 200, 450, 4, 2, 64, is_causal=True, mask="bernoulli"),
]


@pytest.mark.parametrize("mode", ["det_parts", "atomic_parts"])
@pytest.mark.parametrize("cfg", PARTS, ids=[c.name for c in PARTS])
def test_head_group_parts_vs_oracle(cuda, cfg, mode):
    atomic, ds_limit = MODES[mode]
    plan = _plan_of(cfg, _one_plane_limit(cfg), atomic)
    # the route really is the one of parts: one head per part, dS tiles, a slab
    # per part, no dQ atomics
    assert plan.ds_elems > 0 and plan.kv_split == cfg.Hq // cfg.Hk and plan.dq_split == 1
    assert plan.needs_dq_accum == 0 and plan.dkv_accum_elems == plan.kv_split * cfg.B * cfg.Tk * cfg.Hk * cfg.D
    case = I.make_case(cfg, seed=9)
    print(f"case {cfg.name} mode={mode}", flush=True)
    ours = run_ours(case, cfg, atomic=atomic, ds_limit=ds_limit)
    ref = run_oracle_cpu(case, cfg)
    check(ours, ref, label=f"{cfg.name}/{mode}")
    # dQ of a head comes from the same dS tiles in the same key order as the
    # unsliced launch: bitwise equal to it
    one = run_ours(case, cfg, atomic=False, ds_limit=0)
    assert torch.equal(ours["dq"], one["dq"]) and torch.equal(ours["out"], one["out"])


@pytest.mark.parametrize("mode", ["atomic", "det_ds"])
@pytest.mark.parametrize("scale", [0.05, -0.08, 0.0], ids=["small", "negative", "zero"])
def test_scale_values(cuda, scale, mode):
    cfg = C("scale", 1, 200, 260, 4, 2, 128, mask="bernoulli", score="normal")
    case = I.make_case(cfg, seed=1)
    atomic, ds_limit = MODES[mode]
    ours = run_ours(case, cfg, scale=scale, atomic=atomic, ds_limit=ds_limit)
    ref = run_oracle_cpu(case, cfg, scale=scale)
    check(ours, ref, label=f"scale={scale}/{mode}")


@pytest.mark.parametrize("d", [64, 256])
def test_dead_rows_policy(cuda, d):
    """Rows with no kept key: O row NaN, dQ row exactly 0, dV of that kv-head NaN."""
    cfg = C("dead", 2, 256, 256, 4, 2, d, mask="bernoulli")
    case = I.make_case(cfg, seed=2)
    m = case["mask"].clone()
    m[0, 1, 17, :] = False     # batch 0, head 1 (kv-head 0)
    m[1, 3, 200, :] = False    # batch 1, head 3 (kv-head 1)
    m[1, 3, 0:64, :] = False   # a fully dead leading q tile
    case["mask"] = m
    for mode, (atomic, ds_limit) in MODES.items():
        ours = run_ours(case, cfg, atomic=atomic, ds_limit=ds_limit)
        ref = run_oracle_cpu(case, cfg)
        assert torch.isnan(ref["out"][0, 1, 17]).all() and torch.isnan(ref["dv"][0, 0]).all()
        check(ours, ref, label=f"dead/{mode}")
        assert torch.isnan(ours["out"][0, 1, 17]).all()
        assert (ours["dq"][0, 1, 17] == 0).all() and (ours["dq"][1, 3, 200] == 0).all()
        assert (ours["dq"][1, 3, 0:64] == 0).all()
        assert torch.isnan(ours["dv"][0, 0]).all() and torch.isnan(ours["dv"][1, 1]).all()
        assert torch.isfinite(ours["dv"][0, 1]).all() and torch.isfinite(ours["dv"][1, 0]).all()
        assert torch.isfinite(ours["dk"]).all()


SCORE_DEAD = [
    C("score_dead_mask", 2, 256, 256, 4, 2, 64, mask="bernoulli", score="normal"),
    C("score_dead_mask_causal_d256", 1, 200, 200, 4, 2, 256, is_causal=True, mask="bernoulli", score="normal"),
    C("score_dead_mask_causal", 1, 320, 320, 4, 2, 128, is_causal=True, mask="bernoulli", score="normal"),
    C("score_dead_nomask", 2, 256, 200, 4, 2, 128, score="normal"),
    C("score_dead_nomask_causal", 1, 300, 300, 4, 1, 64, is_causal=True, score="normal"),
    C("score_dead_rows", 1, 1100, 700, 4, 1, 64, score="normal"),   # ranges of rows in the *_rows modes
]


@pytest.mark.parametrize("cfg", SCORE_DEAD, ids=[c.name for c in SCORE_DEAD])
def test_dead_rows_from_scores(cuda, cfg):
    """Rows whose kept logits are all -inf because of the score (HF's float
    padding masks reach this: finfo.min / scale overflows to -inf) follow eager
    autograd: O row NaN, dQ row NaN, dK NaN at exactly the keys the row keeps
    (mask and causality), dV of the kv-head NaN; rows with no kept key at all
    keep dQ = 0.  Every backward mode, against the CPU oracle (autograd through
    the eager graph), NaN positions compared exactly."""
    case = I.make_case(cfg, seed=11)
    s = case["score"].clone()
    s[0, 1, 17, :] = float("-inf")                # b0 h1 (kv-head 0): every key -inf
    s[cfg.B - 1, 3, 100, : cfg.Tk // 3] = float("-inf")   # partly -inf: an ordinary row
    if cfg.mask is not None:
        m = case["mask"].clone()
        m[0, 0, 30, :] = False
        m[0, 0, 30, 3:12] = True                  # b0 h0 keeps keys 3..11 only ...
        s[0, 0, 30, 3:12] = float("-inf")         # ... whose scores are -inf
        m[cfg.B - 1, 2, 40, :] = False            # a row with no kept key: dQ row 0
        case["mask"] = m
    if cfg.is_causal:
        s[0, 2, 5, :] = float("-inf")             # causal row 5 keeps keys 0..5
    case["score"] = s
    for mode, (atomic, ds_limit) in MODES.items():
        print(f"case {cfg.name} mode={mode}", flush=True)
        ours = run_ours(case, cfg, atomic=atomic, ds_limit=ds_limit)
        ref = run_oracle_cpu(case, cfg)
        assert torch.isnan(ref["dq"][0, 1, 17]).all() and torch.isnan(ref["out"][0, 1, 17]).all()
        check(ours, ref, label=f"{cfg.name}/{mode}")
        assert torch.isnan(ours["dq"][0, 1, 17]).all()
        if cfg.mask is not None:
            dk_nan = torch.isnan(ours["dk"][0, 0]).any(-1)
            assert dk_nan[3:12].all() and torch.isnan(ours["dq"][0, 0, 30]).all()
            assert (ours["dq"][cfg.B - 1, 2, 40] == 0).all()
        elif not cfg.is_causal:
            assert torch.isnan(ours["dk"][0, 0]).all()   # every key is kept by row 17


SDPA_CASES = [
    C("sdpa_mha_d128", 2, 256, 256, 4, 4, 128),
    C("sdpa_gqa_causal_d64", 1, 384, 384, 8, 2, 64, is_causal=True),
    C("sdpa_mask_d128", 1, 200, 300, 4, 2, 128, mask="bernoulli"),
]


@pytest.mark.parametrize("cfg", SDPA_CASES, ids=[c.name for c in SDPA_CASES])
def test_sdpa_cross_check(cuda, cfg):
    """The reference's SDPA comparison (precision_check.py:89-107, 247-263) on
    the GPU: torch's scaled_dot_product_attention (math backend, float32 on the
    device, K/V repeated over the query-head group, a bool mask as keep mask)
    against ours through autograd, output and gradients at the small-shape bar.
    A second, independent reference beside the eager oracle."""
    from torch.nn.attention import SDPBackend, sdpa_kernel

    dev = torch.device("cuda:0")
    case = I.make_case(cfg, seed=11)
    ours = run_ours(case, cfg, atomic=False)
    G = cfg.Hq // cfg.Hk
    q = case["q_bhsd"].to(dev).float().requires_grad_(True)
    k = case["k_bhsd"].to(dev).float().requires_grad_(True)
    v = case["v_bhsd"].to(dev).float().requires_grad_(True)
    kk, vv = (x.repeat_interleave(G, dim=1) for x in (k, v))
    mask = None if case["mask"] is None else case["mask"].to(dev)
    assert not torch.backends.cuda.matmul.allow_tf32
    with sdpa_kernel(SDPBackend.MATH):
        o = torch.nn.functional.scaled_dot_product_attention(q, kk, vv, attn_mask=mask, is_causal=cfg.is_causal,
                                                             scale=cfg.D ** -0.5)
    o.backward(case["grad_bhsd"].to(dev).float())
    ref = {"out": o.detach().cpu(), "dq": q.grad.cpu(), "dk": k.grad.cpu(), "dv": v.grad.cpu()}
    check(ours, ref, label=f"sdpa {cfg.name}")


# head dims the kernels are not built for: zero-padded to 64 / 128 by the host
PADDED_D = [
    C("d32_gqa", 1, 192, 256, 4, 2, 32),
    C("d80_causal", 1, 256, 256, 4, 4, 80, is_causal=True),
    C("d96_mask", 2, 200, 200, 4, 2, 96, mask="bernoulli"),
    C("d112_score_fp16", 1, 160, 224, 4, 2, 112, torch.float16, score="normal"),
    C("d96_bshd_causal", 1, 257, 257, 8, 2, 96, layout="bshd", is_causal=True),
]


@pytest.mark.parametrize("mode", ["atomic", "det_ds"])
@pytest.mark.parametrize("cfg", PADDED_D, ids=[c.name for c in PADDED_D])
def test_padded_head_dims(cuda, cfg, mode):
    """Head dims other than 64 and 128 (the reference compiles any D,
    python/fa2.py:33) through the zero-padded kernels: output and gradients
    against the CPU oracle at the small-shape bar, gradients shaped like the
    inputs."""
    atomic, ds_limit = MODES[mode]
    case = I.make_case(cfg, seed=7)
    ours = run_ours(case, cfg, atomic=atomic, ds_limit=ds_limit)
    ref = run_oracle_cpu(case, cfg)
    for name in ("dq", "dk", "dv", "out"):
        assert ours[name].shape == ref[name].shape, name
    check(ours, ref, label=f"padded-D {cfg.name}/{mode}")


RAMP = [
    C("ramp_d128_ragged", 1, 320, 200, 4, 2, 128),
    C("ramp_d64_causal", 1, 256, 256, 4, 4, 64, is_causal=True),
]


@pytest.mark.parametrize("cfg", RAMP, ids=[c.name for c in RAMP])
def test_rising_row_maximum(cuda, cfg):
    """Logits that rise along the keys by about 100 (D 128) or 140 (D 64) base-2
    steps per 64-key tile: every row's running maximum is raised again and again,
    each time far above the forward's fast-path allowance (O rescaled by powers
    of two of up to 2^-140).  O against the oracle's forward, LSE (base 2)
    against a float64 logsumexp of the same 16-bit inputs within 1e-3 (the fp32
    row sum of up to 200 terms).  Gradients are left to the other tests: keys of
    size ~300 make one 16-bit step of dS worth more than the gradient bar."""
    case = I.make_case(cfg, seed=6, with_grad=False)
    q, k = case["q_bhsd"], case["k_bhsd"]   # views of the tensors the API receives
    q[..., 0] = 8.0
    k[..., 0] = (1.5 * torch.arange(cfg.Tk, dtype=torch.float32)).to(k.dtype)
    ours = run_ours(case, cfg, backward=False)
    ref = run_oracle_cpu(case, cfg, backward=False)
    check(ours, ref, label=f"rising-max {cfg.name}")
    dev = torch.device("cuda:0")
    scale = cfg.D ** -0.5
    with torch.no_grad():
        q_t, k_t, v_t = (case[n + "_bhsd"].transpose(1, 2).to(dev) for n in ("q", "k", "v"))   # [B, T, H, D]
        _, lse, _, _ = torch.ops.tilelang_fa2_4d_mask.fwd(q_t, k_t, v_t, None, None, scale, cfg.is_causal, False,
                                                          False)
    kk = case["k_bhsd"].double().repeat_interleave(cfg.Hq // cfg.Hk, dim=1)
    logits = (case["q_bhsd"].double() @ kk.transpose(-1, -2)) * scale
    if cfg.is_causal:
        keep = torch.arange(cfg.Tk)[None, :] <= torch.arange(cfg.Tq)[:, None]
        logits = logits.masked_fill(~keep, float("-inf"))
    want = torch.logsumexp(logits, dim=-1) / math.log(2.0)
    err = (lse.cpu().double() - want).abs().max().item()
    print(f"[rising-max {cfg.name}] lse max_abs={err:.3e} (|lse| up to {want.abs().max().item():.1f})", flush=True)
    assert err <= 1e-3


def test_leading_masked_tiles_are_not_nan(cuda):
    """A row whose first key tiles are all dropped but later keys are kept must be
    finite (the reference TileLang kernel turns such rows into NaN; eager does not)."""
    cfg = C("lead", 1, 128, 512, 2, 2, 128, mask="bernoulli")
    case = I.make_case(cfg, seed=3)
    m = case["mask"].clone()
    m[:, :, :, :300] = False
    case["mask"] = m
    ours = run_ours(case, cfg)
    ref = run_oracle_cpu(case, cfg)
    assert torch.isfinite(ours["out"]).all()
    check(ours, ref, label="leading-masked")


def test_float_attention_mask_matches_score(cuda):
    """attention_mask (float, scaled convention) equals score = am / scale."""
    cfg = C("am", 1, 192, 192, 4, 2, 64)
    case = I.make_case(cfg, seed=4)
    am = torch.randn((1, 1, 192, 192), generator=I.make_generator(9)) * 0.5
    ours = run_ours(case, cfg, attention_mask=am)
    case2 = dict(case)
    case2["score"] = (am / (64 ** -0.5)).expand(1, 4, 192, 192)
    ref = run_oracle_cpu(case2, cfg)
    check(ours, ref, label="float-attention-mask")


def test_bhsd_contiguous_inputs(cuda):
    """BHSD-contiguous (not BTHD-backed) tensors take the strided path, no copy."""
    api = _api()
    cfg = C("bhsdc", 1, 256, 256, 4, 2, 128, is_causal=True)
    case = I.make_case(cfg, seed=5)
    dev = torch.device("cuda:0")
    q = case["q_bhsd"].contiguous().to(dev).requires_grad_(True)
    k = case["k_bhsd"].contiguous().to(dev).requires_grad_(True)
    v = case["v_bhsd"].contiguous().to(dev).requires_grad_(True)
    out = api.tilelang_flash_attention(q, k, v, is_causal=True)
    out.backward(case["grad_bhsd"].to(dev))
    ours = {"out": out.detach().float().cpu(), "dq": q.grad.float().cpu(), "dk": k.grad.float().cpu(),
            "dv": v.grad.float().cpu()}
    check(ours, run_oracle_cpu(case, cfg), label="bhsd-contiguous")


@pytest.mark.parametrize("mode", ["atomic", "det_ds", "atomic_no_ws", "det_recompute"])
def test_tiny_lengths(cuda, mode):
    # Boundary/indexing test (an indexing bug gives O(1) errors).  With a few
    # hundred entries per output the mean is dominated by single bf16 rounding
    # steps (mean bar: one ulp of the typical entry, 2^-7), and with 3 keys each
    # dK entry sums 70 terms of bf16-rounded dS (rounded as in the reference
    # kernel, python/fa2.py:291-292) that are larger than the result, so the
    # per-entry bar is 4e-2 + 2^-5 |ref|.
    shapes = [(1, 1, False, 64, None), (1, 7, False, 64, None), (5, 1, True, 64, None), (3, 65, True, 64, None),
              (70, 3, False, 64, None), (1, 40, False, 128, "bernoulli"), (33, 2, True, 128, "bernoulli"),
              (2, 300, False, 128, None)]
    for (tq, tk, causal, d, mask) in shapes:
        cfg = C("tiny", 1, tq, tk, 2, 1, d, is_causal=causal, mask=mask, keep_prob=0.9)
        case = I.make_case(cfg, seed=6)
        atomic, ds_limit = MODES[mode]
        check(run_ours(case, cfg, atomic=atomic, ds_limit=ds_limit), run_oracle_cpu(case, cfg),
              label=f"tiny {tq}x{tk} causal={causal} {mode}",
              mean_rel=2.0 ** -7, abs_bar=4e-2, rel_bar=2.0 ** -5)


def test_atomic_mode_on_a_full_grid_writes_dq_once(cuda):
    """Atomic mode where the 256-row query blocks give every CU a workgroup:
    dQ is written per block (no atomics), so it is bitwise repeatable and
    equal to the deterministic mode's (the same kernel and row blocks)."""
    import ctypes

    from tilelang_fa2_4d_mask import _ext

    cfg = WIDE_DQ[0]
    lib = _ext.load_library()
    p = _ext.FaBwdParams()
    p.batch, p.seqlen_q, p.seqlen_k, p.heads_q, p.heads_k, p.head_dim = cfg.B, cfg.Tq, cfg.Tk, cfg.Hq, cfg.Hk, cfg.D
    p.scale, p.atomic_dq = cfg.D ** -0.5, 1
    plan = _ext.FaBwdPlan()
    assert lib.fa_bwd_plan(ctypes.byref(p), ctypes.byref(plan)) == 0
    assert plan.dq_split == 1 and plan.needs_dq_accum == 0
    case = I.make_case(cfg, seed=8)
    a = run_ours(case, cfg, atomic=True)
    b = run_ours(case, cfg, atomic=True)
    c = run_ours(case, cfg, atomic=False)
    for n in a:
        assert torch.equal(a[n], b[n]) and torch.equal(a[n], c[n]), n


@pytest.mark.parametrize("ds_limit", [0, -1], ids=["det_ds", "det_recompute"])
def test_deterministic_path_is_bitwise_repeatable(cuda, ds_limit):
    cfg = C("det", 1, 512, 512, 8, 2, 128, is_causal=True, mask="bernoulli")
    case = I.make_case(cfg, seed=7)
    a = run_ours(case, cfg, atomic=False, ds_limit=ds_limit)
    b = run_ours(case, cfg, atomic=False, ds_limit=ds_limit)
    for n in a:
        assert torch.equal(a[n], b[n]), n


# ---------------------------------------------------------------------------
# Seeded random sweep over the configuration space: shape (ragged lengths,
# GQA/MQA, head dims 64/128 and padded ones), dtype, layout, causality, mask
# kind and density, score, and backward route -- each case against the CPU
# oracle with the small-shape bar (the tiny-length bar when a length is below
# 16: see test_tiny_lengths).
# ---------------------------------------------------------------------------
def _random_case(seed):
    import random

    r = random.Random(1000 + seed)
    hk = r.choice([1, 1, 2, 3])
    g = r.choice([1, 2, 4])
    d = r.choice([64, 64, 128, 128, 128, 80, 112])
    tq = r.choice([r.randint(1, 64), r.randint(65, 640)])
    tk = tq if r.random() < 0.4 else r.choice([r.randint(1, 64), r.randint(65, 640)])
    causal = r.random() < 0.3
    mask, mask_heads, keep = None, 0, 0.75
    u = r.random()
    if u < 0.35:
        mask, mask_heads, keep = "bernoulli", r.choice([1, hk * g]), r.choice([0.3, 0.6, 0.9])
    elif u < 0.5 and tq == tk and tq >= 32:
        mask, mask_heads = "packed_docs", 1
    score = "normal" if r.random() < 0.4 else None
    cfg = C(f"rand{seed}", r.choice([1, 2]), tq, tk, hk * g, hk, d,
            torch.float16 if r.random() < 0.3 else torch.bfloat16, is_causal=causal, mask=mask,
            mask_heads=mask_heads, score=score, keep_prob=keep, layout=r.choice(["bhsd", "bshd"]),
            extra={"packed": {"lo": 16, "hi": 128}} if mask == "packed_docs" else {})
    return cfg, r.choice(list(MODES))


RANDOM_SEEDS = list(range(100))


@pytest.mark.parametrize("seed", RANDOM_SEEDS)
def test_random_configs_vs_oracle(cuda, seed):
    cfg, mode = _random_case(seed)
    print(f"case {cfg.name} B{cfg.B} Tq{cfg.Tq} Tk{cfg.Tk} Hq{cfg.Hq} Hk{cfg.Hk} D{cfg.D} {cfg.dtype} "
          f"{cfg.layout} causal={cfg.is_causal} mask={cfg.mask}/{cfg.mask_heads}/{cfg.keep_prob} "
          f"score={cfg.score} mode={mode}", flush=True)
    case = I.make_case(cfg, seed=seed)
    atomic, ds_limit = MODES[mode]
    ours = run_ours(case, cfg, atomic=atomic, ds_limit=ds_limit)
    bars = dict(mean_rel=2.0 ** -7, abs_bar=4e-2, rel_bar=2.0 ** -5) if min(cfg.Tq, cfg.Tk) < 16 else {}
    check(ours, run_oracle_cpu(case, cfg), label=f"{cfg.name} {mode}", **bars)
    # The oracle is the reference's eager graph, whose autograd rounds each query
    # head's dK/dV to the input dtype before repeat_interleave's backward sums the
    # group (several ulps at large |dV|).  The same bar against the exact
    # gradients (float64 throughout, same inputs) pins that the kernels' own
    # error is no larger.
    check(ours, run_exact_cpu(case, cfg), label=f"{cfg.name} {mode} vs float64", **bars)


# ---------------------------------------------------------------------------
# Head dims above 128 (the reference compiles any D, python/fa2.py:33): kernels
# at 256 (fa_wide.hip; dQ recomputed in both backward modes), other head dims
# in (128, 256] zero-padded to 256 by the host.
# ---------------------------------------------------------------------------
WIDE_D = [
    C("d256_mha", 2, 200, 200, 4, 4, 256),
    C("d256_gqa_causal", 1, 300, 300, 8, 2, 256, is_causal=True),
    C("d256_causal_tq_gt_tk", 1, 333, 130, 4, 2, 256, is_causal=True),
    C("d256_tq_lt_tk_mqa", 1, 130, 333, 4, 1, 256),
    C("d256_mask", 2, 200, 200, 4, 2, 256, mask="bernoulli", mask_heads=4, keep_prob=0.5),
    C("d256_packed_docs", 1, 256, 256, 4, 2, 256, mask="packed_docs", mask_heads=1,
      extra={"packed": {"lo": 16, "hi": 128}}),
    C("d256_score_fp16", 1, 160, 224, 4, 2, 256, torch.float16, score="normal"),
    C("d256_mask_score_causal_bshd", 1, 257, 257, 8, 2, 256, layout="bshd", is_causal=True, mask="bernoulli",
      score="normal"),
    C("d256_causal_tq_lt_tk_mask", 1, 100, 300, 4, 2, 256, is_causal=True, mask="bernoulli", mask_heads=4),
    C("d192_padded", 1, 200, 240, 4, 2, 192),
    C("d160_causal_fp16", 1, 180, 180, 4, 4, 160, torch.float16, is_causal=True),
]


@pytest.mark.parametrize("mode", ["atomic", "det_ds", "atomic_no_ws"])
@pytest.mark.parametrize("cfg", WIDE_D, ids=[c.name for c in WIDE_D])
def test_head_dim_256(cuda, cfg, mode):
    """Output and gradients at head dims above 128 against the CPU oracle and
    against the same graph in float64, at the small-shape bar; gradients shaped
    like the inputs."""
    print(f"case {cfg.name} mode={mode}", flush=True)
    atomic, ds_limit = MODES[mode]
    case = I.make_case(cfg, seed=5)
    ours = run_ours(case, cfg, atomic=atomic, ds_limit=ds_limit)
    ref = run_oracle_cpu(case, cfg)
    for name in ("dq", "dk", "dv", "out"):
        assert ours[name].shape == ref[name].shape, name
    check(ours, ref, label=f"{cfg.name}/{mode}")
    check(ours, run_exact_cpu(case, cfg), label=f"{cfg.name}/{mode} vs float64")


def test_head_dim_256_modes_agree_bitwise(cuda):
    """At head dim 256 both backward modes run the deterministic recompute route:
    repeated calls and the two modes give the same bits."""
    cfg = C("d256_det", 1, 384, 384, 8, 2, 256, is_causal=True, mask="bernoulli", score="normal")
    case = I.make_case(cfg, seed=9)
    a = run_ours(case, cfg, atomic=False)
    b = run_ours(case, cfg, atomic=False)
    c = run_ours(case, cfg, atomic=True)
    for n in a:
        assert torch.equal(a[n], b[n]) and torch.equal(a[n], c[n]), n


def _random_case_wide(seed):
    import random

    r = random.Random(5000 + seed)
    hk = r.choice([1, 2, 3])
    g = r.choice([1, 2, 4])
    d = r.choice([256, 256, 256, 192, 160, 144])
    tq = r.choice([r.randint(1, 48), r.randint(49, 400)])
    tk = tq if r.random() < 0.4 else r.choice([r.randint(1, 48), r.randint(49, 400)])
    causal = r.random() < 0.3
    mask, mask_heads, keep = None, 0, 0.75
    u = r.random()
    if u < 0.35:
        mask, mask_heads, keep = "bernoulli", r.choice([1, hk * g]), r.choice([0.3, 0.6, 0.9])
    elif u < 0.5 and tq == tk and tq >= 32:
        mask, mask_heads = "packed_docs", 1
    score = "normal" if r.random() < 0.4 else None
    cfg = C(f"wide{seed}", r.choice([1, 2]), tq, tk, hk * g, hk, d,
            torch.float16 if r.random() < 0.3 else torch.bfloat16, is_causal=causal, mask=mask,
            mask_heads=mask_heads, score=score, keep_prob=keep, layout=r.choice(["bhsd", "bshd"]),
            extra={"packed": {"lo": 16, "hi": 128}} if mask == "packed_docs" else {})
    return cfg, r.choice(list(MODES))


@pytest.mark.parametrize("seed", list(range(24)))
def test_random_wide_configs_vs_oracle(cuda, seed):
    cfg, mode = _random_case_wide(seed)
    print(f"case {cfg.name} B{cfg.B} Tq{cfg.Tq} Tk{cfg.Tk} Hq{cfg.Hq} Hk{cfg.Hk} D{cfg.D} {cfg.dtype} "
          f"{cfg.layout} causal={cfg.is_causal} mask={cfg.mask}/{cfg.mask_heads}/{cfg.keep_prob} "
          f"score={cfg.score} mode={mode}", flush=True)
    case = I.make_case(cfg, seed=seed)
    atomic, ds_limit = MODES[mode]
    ours = run_ours(case, cfg, atomic=atomic, ds_limit=ds_limit)
    bars = dict(mean_rel=2.0 ** -7, abs_bar=4e-2, rel_bar=2.0 ** -5) if min(cfg.Tq, cfg.Tk) < 16 else {}
    check(ours, run_oracle_cpu(case, cfg), label=f"{cfg.name} {mode}", **bars)
    check(ours, run_exact_cpu(case, cfg), label=f"{cfg.name} {mode} vs float64", **bars)
