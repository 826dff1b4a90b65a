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
