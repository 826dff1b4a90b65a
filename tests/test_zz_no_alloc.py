"""fa_bwd_noalloc: the backward with its scratch in the library's device array.

Called through the C ABI (ctypes) on the forward's outputs, against the
existing backward entry points on the same inputs:

* bitwise equal to fa_bwd_preprocess + fa_bwd + fa_bwd_finalize with caller
  workspaces on the same route (deterministic, no dS workspace so dQ is
  recomputed, head-group split 1: the same kernels);
* within the parity bar of the default route (dQ from the stored dS tiles);
* two calls in a row on one GPU, the second on a smaller problem without dead
  rows after a first one with dead rows in every kv-head: the flags the first
  call raised in the shared scratch must not leak into the second (its dV
  would turn NaN); then a third at head dim 256 (its own kernels, the same
  route).
"""

import ctypes

import pytest
import torch

from oracle import inputs as I

pytestmark = pytest.mark.gpu


def _bwd_params(q, k, v, O, LSE, do, dQ, dK, dV, mask, score, mask_ws, mst, sst, scale, causal, O_lo):
    import tilelang_fa2_4d_mask.fa2 as F
    from tilelang_fa2_4d_mask import _ext

    B, Tq, Hq, D = q.shape
    _, Tk, Hk, _ = k.shape
    p = _ext.FaBwdParams()
    p.batch, p.seqlen_q, p.seqlen_k, p.heads_q, p.heads_k, p.head_dim = B, Tq, Tk, Hq, Hk, D
    p.scale, p.is_causal, p.dtype = scale, int(causal), _ext.dtype_code(q.dtype)
    p.q, p.k, p.v, p.o, p.dout = q.data_ptr(), k.data_ptr(), v.data_ptr(), O.data_ptr(), do.data_ptr()
    p.lse = LSE.data_ptr()
    p.mask, p.score, p.mask_ws = _ext.ptr(mask), _ext.ptr(score), _ext.ptr(mask_ws)
    p.dq, p.dk, p.dv = dQ.data_ptr(), dK.data_ptr(), dV.data_ptr()
    for pre, t in (("q", q), ("k", k), ("v", v), ("o", O), ("do", do), ("dq", dQ), ("dk", dK), ("dv", dV)):
        sb, st, sh = F._bthd_strides(t)
        setattr(p, f"{pre}_stride_b", sb)
        setattr(p, f"{pre}_stride_t", st)
        setattr(p, f"{pre}_stride_h", sh)
    p.mask_stride_b, p.mask_stride_h, p.mask_stride_q = mst
    p.score_stride_b, p.score_stride_h, p.score_stride_q = sst
    if O_lo is not None:   # the forward's rounding residual of O (mask or score)
        p.o_lo = O_lo.data_ptr()
        p.o_lo_stride_b, p.o_lo_stride_t, p.o_lo_stride_h = F._bthd_strides(O_lo)
    p.stream = torch.cuda.current_stream().cuda_stream
    return p


def _run(cfg, seed, dev, dead_rows):
    import tilelang_fa2_4d_mask.fa2 as F
    from tilelang_fa2_4d_mask import _ext

    case = I.make_case(cfg, seed=seed, device=dev)
    if dead_rows:
        m = case["mask"].clone()
        for h in range(0, cfg.Hq, cfg.Hq // cfg.Hk):   # one row with no kept key in every kv-head
            m[0, h, 5, :] = False
        case["mask"] = m
    q, k, v = (case[n].transpose(1, 2) for n in ("q", "k", "v"))   # logical [B, T, H, D]
    do = case["grad"].transpose(1, 2)
    scale = cfg.D ** -0.5
    O, LSE, mask_ws, O_lo, (q, k, v, mask, score, mst, sst) = F._forward_impl(
        q, k, v, case["mask"], case["score"], scale, cfg.is_causal, residual=True)
    do = F._kernel_operand(do)
    # the new entry point
    dQ, dK, dV = (torch.full_like(t, float("nan")) for t in (q, k, v))
    p = _bwd_params(q, k, v, O, LSE, do, dQ, dK, dV, mask, score, mask_ws, mst, sst, scale, cfg.is_causal, O_lo)
    lib = _ext.load_library()
    print(f"case noalloc {cfg.name} dead_rows={dead_rows}", flush=True)
    _ext.check(lib.fa_bwd_noalloc(ctypes.byref(p)), "fa_bwd_noalloc", lib)
    torch.cuda.synchronize()
    ours = (dQ.clone(), dK.clone(), dV.clone())
    ref = {}
    # the existing entry points on the same route (caller workspaces, no dS
    # tiles, deterministic, head-group split 1): the same kernels
    rQ, rK, rV = (torch.full_like(t, float("nan")) for t in (q, k, v))
    B, Tq, Hq, _ = q.shape
    Hk = k.shape[2]
    delta = torch.empty((2, B, Hq, Tq), dtype=torch.float32, device=dev)
    dead = torch.zeros((B * Hk,), dtype=torch.int32, device=dev)
    p2 = _bwd_params(q, k, v, O, LSE, do, rQ, rK, rV, mask, score, mask_ws, mst, sst, scale, cfg.is_causal, O_lo)
    p2.delta, p2.dead_flags = delta.data_ptr(), dead.data_ptr()
    p2.ds_limit_bytes, p2.atomic_dq, p2.kv_split = -1, 0, 1
    for entry in ("fa_bwd_preprocess", "fa_bwd", "fa_bwd_finalize"):
        _ext.check(getattr(lib, entry)(ctypes.byref(p2)), entry, lib)
    ref["same_route"] = (rQ, rK, rV)
    # the default route of the product backward (dQ from the stored dS tiles)
    ref["default"] = F._backward_impl(do, q, k, v, O, LSE, mask, score, mask_ws, mst, sst, scale, cfg.is_causal,
                                      False, O_lo)
    torch.cuda.synchronize()
    return ours, ref


def test_noalloc_backward_matches_the_workspace_backward(cuda):
    C = I.AttnConfig
    first = C("noalloc_big", 2, 300, 400, 8, 2, 128, is_causal=True, mask="bernoulli", score="normal")
    second = C("noalloc_small", 1, 100, 150, 4, 1, 64, mask="bernoulli")
    third = C("noalloc_d256", 1, 160, 200, 4, 2, 256, is_causal=True, mask="bernoulli", score="normal")
    for cfg, dead in ((first, True), (second, False), (third, False)):
        ours, ref = _run(cfg, seed=4, dev=cuda, dead_rows=dead)
        for name, a, b, c in zip(("dq", "dk", "dv"), ours, ref["same_route"], ref["default"]):
            assert torch.equal(torch.isnan(a), torch.isnan(b)), (cfg.name, name)
            assert torch.equal(a[~torch.isnan(a)], b[~torch.isnan(b)]), (cfg.name, name)
            assert torch.equal(torch.isnan(a), torch.isnan(c)), (cfg.name, name)
            fin = torch.isfinite(c)
            err = (a[fin].float() - c[fin].float()).abs()
            ref_mag = c[fin].float().abs()
            print(f"  {cfg.name} {name}: vs default route max={err.max().item():.3e} mean={err.mean().item():.3e}",
                  flush=True)
            assert (err <= 2e-2 + 2.0 ** -6 * ref_mag).all(), (cfg.name, name)
            assert err.mean().item() <= max(1e-4, 2.0 ** -8 * ref_mag.mean().item()), (cfg.name, name)
        if dead:   # batch 0 has a dead row in every kv-head, batch 1 none
            assert torch.isnan(ours[2][0]).all() and torch.isfinite(ours[2][1]).all()
        else:
            assert torch.isfinite(ours[2]).all(), "stale dead-row flags from the previous call"
