"""GPU parity at the BASELINE configs, full size (H, P, S, M).

The oracle is the closed-form, row-chunked restatement of the eager reference
(oracle/eager.py ``eager_grads_chunked``, pinned against autograd through the
eager graph in tests/test_oracle.py), run in fp32 on the device: the CPU would
take minutes per config.  Inputs are the seeded BASELINE inputs
(oracle/inputs.py CONFIGS).

Bar, per output (O, dQ, dK, dV) over the entries where the oracle is finite,
with NaN positions identical: |ours - oracle| <= 2e-2 + 2^-6 |oracle| per entry
and mean_abs <= max(1e-4, 2^-8 mean|oracle|) -- the rule of the small-shape
suite (tests/test_gpu_parity.py).  The strict north-star bar (max_abs <= 2e-2
and mean_abs <= 1e-4) is printed beside it.  It holds at H and M; where
outputs are large it is below bf16 resolution: one bf16 ulp is 2^-5 at |x| >= 4
(the causal configs' first keys reach |dV| ~ 10), and at P (short documents,
mean|dV| ~ 0.17, ulp 2^-10) P and dS rounded to bf16 inside the GEMMs -- as the
reference kernel does, python/fa2.py:287, 291 -- move a fraction of the bf16
outputs to the neighbouring value, a mean error of about 0.3 ulp of the typical
entry.  Every config runs the atomic-dQ backward (the reference default) and
the deterministic one (dQ from the stored dS tiles).

Size-independent properties checked beside the oracle:
  * the deterministic backward is bitwise repeatable at full size;
  * bhsd and bshd inputs of the same data give identical outputs (config M).
"""

import pytest
import torch

from oracle import eager as E
from oracle import inputs as I

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
MEAN_ABS = 1e-4


def _api():
    import tilelang_fa2_4d_mask as api

    return api


def run_ours(case, cfg, *, atomic):
    api = _api()
    q = case["q"].detach().requires_grad_(True)
    k = case["k"].detach().requires_grad_(True)
    v = case["v"].detach().requires_grad_(True)
    out = api.tilelang_flash_attention(q, k, v, mask=case["mask"], score=case["score"], is_causal=cfg.is_causal,
                                       layout=cfg.layout, use_atomic_backward=atomic)
    out.backward(case["grad"])
    torch.cuda.synchronize()
    res = {"out": out.detach(), "dq": q.grad, "dk": k.grad, "dv": v.grad}
    if cfg.layout == "bshd":
        res = {n: t.transpose(1, 2) for n, t in res.items()}
    return res


def run_oracle(case, cfg):
    out, dq, dk, dv = E.eager_grads_chunked(case["q_bhsd"], case["k_bhsd"], case["v_bhsd"], case["mask"],
                                           case["score"], case["grad_bhsd"], scale=cfg.D ** -0.5,
                                           is_causal=cfg.is_causal, block=128)
    torch.cuda.synchronize()
    return {"out": out, "dq": dq, "dk": dk, "dv": dv}


def check(ours, ref, label):
    failures = []
    for name in ref:
        st = E.finite_diff_stats(ours[name], ref[name])
        r = ref[name].float()
        fin = torch.isfinite(r)
        err = (ours[name].float()[fin] - r[fin]).abs()
        mag = r[fin].abs().mean().item() if err.numel() else 0.0
        margin = (err - (MAX_ABS + 2.0 ** -6 * r[fin].abs())).max().item() if err.numel() else -1.0
        mean_tol = max(MEAN_ABS, 2.0 ** -8 * mag)
        strict = st["max_abs"] <= MAX_ABS and st["mean_abs"] <= MEAN_ABS
        print(f"[{label}] {name}: max_abs={st['max_abs']:.3e} mean_abs={st['mean_abs']:.3e} (tol {mean_tol:.2e}) "
              f"mean|ref|={mag:.3e} entries>2e-2: {int((err > MAX_ABS).sum().item())} of {err.numel()} "
              f"nan_match={st['nan_match']} strict_north_star={strict}", flush=True)
        if not st["nan_match"]:
            failures.append(f"{name}: NaN positions differ")
        if margin > 0:
            failures.append(f"{name}: an entry exceeds 2e-2 + 2^-6 |ref| by {margin:.3e}")
        if st["mean_abs"] > mean_tol:
            failures.append(f"{name}: mean_abs {st['mean_abs']:.3e} > {mean_tol:.2e}")
    assert not failures, f"{label}: " + "; ".join(failures)


CASES = [("H", True), ("H", False), ("H_causal", True), ("H_causal", False),
         ("P", True), ("P", False), ("S", True), ("S", False), ("M", True), ("M", False)]


@pytest.mark.parametrize("name,atomic", CASES, ids=[f"{n}-{'atomic' if a else 'det'}" for n, a in CASES])
def test_fullsize_vs_oracle(cuda, name, atomic):
    cfg = I.CONFIGS[name]
    print(f"case {name} atomic={atomic} B{cfg.B} Tq{cfg.Tq} Tk{cfg.Tk} Hq{cfg.Hq} Hk{cfg.Hk} D{cfg.D} "
          f"{cfg.layout} causal={cfg.is_causal} mask={cfg.mask} score={cfg.score}", flush=True)
    case = I.make_case(cfg, seed=0, device=cuda)
    ours = run_ours(case, cfg, atomic=atomic)
    ref = run_oracle(case, cfg)
    check(ours, ref, f"{name}/{'atomic' if atomic else 'det'}")


def test_fullsize_deterministic_repeatable(cuda):
    cfg = I.CONFIGS["H_causal"]
    print("case H_causal deterministic twice", flush=True)
    case = I.make_case(cfg, seed=1, device=cuda)
    a = run_ours(case, cfg, atomic=False)
    b = run_ours(case, cfg, atomic=False)
    for n in a:
        assert torch.equal(a[n], b[n]), n


def test_fullsize_layouts_agree(cuda):
    cfg = I.CONFIGS["M"]
    print("case M bshd vs bhsd", flush=True)
    case = I.make_case(cfg, seed=2, device=cuda)
    a = run_ours(case, cfg, atomic=False)
    cfg2 = cfg.scaled(layout="bhsd")
    case2 = dict(case, q=case["q_bhsd"], k=case["k_bhsd"], v=case["v_bhsd"], grad=case["grad_bhsd"])
    b = run_ours(case2, cfg2, atomic=False)
    for n in a:
        assert torch.equal(a[n], b[n]), n


# ---------------------------------------------------------------------------
# The reference's scripted regression (precision_check.sh: B1 Tq=Tk=8191 Hq32
# Hk8 D128 bf16, cases no_causal / causal / random_mask, --check-backward):
# a length that is not a multiple of any tile, at the headline heads.  The
# random_mask case is precision_check.py:110-117's per-head Bernoulli mask
# (keep 0.75, key min(i, Tk-1) forced) -- [1, 32, 8191, 8191], drawn on the
# device with a seeded generator (2 GiB; the same tensor goes to the oracle).
# It runs the prepared-mask paths that small shapes never reach: per-head
# lists of more than 128 steps (dK/dV list cursor across heads, dQ positions
# past 128).
# ---------------------------------------------------------------------------
def _device_case(cfg, seed, dev, mask_heads=None):
    """Seeded inputs drawn on the device (the CPU would need 8 GiB of floats
    for a full-head mask of this size)."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)

    def rnd(shape):
        return torch.randn(shape, generator=g, device=dev, dtype=torch.float32).to(cfg.dtype)

    q = rnd((cfg.B, cfg.Tq, cfg.Hq, cfg.D))
    k = rnd((cfg.B, cfg.Tk, cfg.Hk, cfg.D))
    v = rnd((cfg.B, cfg.Tk, cfg.Hk, cfg.D))
    mask = None
    if cfg.mask == "bernoulli":
        mh = mask_heads or cfg.Hq
        mask = torch.rand((cfg.B, mh, cfg.Tq, cfg.Tk), generator=g, device=dev) < cfg.keep_prob
        qi = torch.arange(cfg.Tq, device=dev)
        mask[:, :, qi, torch.clamp(qi, max=cfg.Tk - 1)] = True
    grad = rnd((cfg.B, cfg.Tq, cfg.Hq, cfg.D))
    case = {"q_bhsd": q.transpose(1, 2), "k_bhsd": k.transpose(1, 2), "v_bhsd": v.transpose(1, 2),
            "grad_bhsd": grad.transpose(1, 2), "mask": mask, "score": None}
    case.update(q=case["q_bhsd"], k=case["k_bhsd"], v=case["v_bhsd"], grad=case["grad_bhsd"])
    return case


REGRESSION = {
    "no_causal": I.AttnConfig("R_no_causal", 1, 8191, 8191, 32, 8, 128),
    "causal": I.AttnConfig("R_causal", 1, 8191, 8191, 32, 8, 128, is_causal=True),
    "random_mask": I.AttnConfig("R_random_mask", 1, 8191, 8191, 32, 8, 128, mask="bernoulli", keep_prob=0.75),
}
REG_CASES = [(n, a) for n in REGRESSION for a in (True, False)]


@pytest.mark.parametrize("name,atomic", REG_CASES, ids=[f"{n}-{'atomic' if a else 'det'}" for n, a in REG_CASES])
def test_reference_regression_T8191(cuda, name, atomic):
    cfg = REGRESSION[name]
    print(f"case precision_check.sh {name} atomic={atomic} B1 T8191 Hq32 Hk8 D128", flush=True)
    case = _device_case(cfg, seed=0, dev=cuda)
    ours = run_ours(case, cfg, atomic=atomic)
    ref = run_oracle(case, cfg)
    check(ours, ref, f"T8191/{name}/{'atomic' if atomic else 'det'}")


def test_long_keys_head_broadcast_mask(cuda):
    """Tk 16384 with a head-broadcast mask: the forward's list of live 64-key
    tiles runs to 256 positions (entries past 128 come from memory, not the
    list registers); both backward modes."""
    cfg = I.AttnConfig("long_keys_mask", 1, 2048, 16384, 8, 2, 128, mask="bernoulli", keep_prob=0.75)
    case = _device_case(cfg, seed=3, dev=cuda, mask_heads=1)
    for atomic in (True, False):
        print(f"case long_keys_mask atomic={atomic} B1 Tq2048 Tk16384 Hq8 Hk2 D128, mask [1,1,T,T]", flush=True)
        ours = run_ours(case, cfg, atomic=atomic)
        ref = run_oracle(case, cfg)
        check(ours, ref, f"long_keys_mask/{'atomic' if atomic else 'det'}")
