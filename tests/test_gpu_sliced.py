"""The sliced backward at long sequences.

At T = 16384 with the headline's heads (B1 Hq32 Hk8 D128) the dS tiles of all
units (17 GB, 8.6 GB causal) exceed the default 4 GiB workspace.  The
non-causal backward then runs the dK/dV and dQ kernels once per slice of
(batch, kv-head) units (csrc/fa_api.cpp ``ds_slice_units``); the causal one
once per range of query rows over every unit (``row_ranges``: dK/dV added to
fp32 sums across the ranges).  The same call with a limit that holds every
unit runs them once.  Checks:

* non-causal, deterministic: the sliced and the single-launch gradients are
  bitwise equal (the same workgroups do the same arithmetic; only the launch
  they belong to differs);
* causal, deterministic: dQ is bitwise equal (the same dS tiles, summed in
  the same key order); dK and dV are sums over the ranges in fp32 and may
  round to the neighbouring bf16 value: within one bf16 step of the single
  launch;
* atomic mode, non-causal: sliced and single-launch dQ agree within fp32
  summation order (dK/dV bitwise).

At T = 32768 one unit's tiles (8 GiB) exceed the default limit: both modes
run over row ranges there (16 ranges of 2048 rows non-causal), checked
against the single launch (an 80 GiB limit: 64 GiB of tiles, 34 GB causal).

The route, the slices and the head-group split depend on the problem and the
limit only (the default limit is a constant): the deterministic backward is
bitwise repeatable whatever the allocator holds, and two limits that give the
same head-group split give the same bits.

The parity of the slicing itself against the oracle runs at small shapes in
tests/test_gpu_parity.py (modes ``det_sliced``, ``atomic_sliced``).
"""

import pytest
import torch

pytestmark = pytest.mark.gpu


def _grads(q, k, v, do, *, causal, atomic, limit):
    import tilelang_fa2_4d_mask as api
    import tilelang_fa2_4d_mask.fa2 as fa2mod

    fa2mod.DS_LIMIT_BYTES = limit
    try:
        qq, kk, vv = (x.detach().requires_grad_(True) for x in (q, k, v))
        api.tilelang_flash_attention(qq, kk, vv, is_causal=causal, use_atomic_backward=atomic).backward(do)
        torch.cuda.synchronize()
        return qq.grad, kk.grad, vv.grad
    finally:
        fa2mod.DS_LIMIT_BYTES = 0


@pytest.mark.parametrize("causal,atomic", [(False, False), (True, False), (False, True)],
                         ids=["det", "det_causal", "atomic"])
def test_sliced_backward_matches_single_launch(cuda, causal, atomic):
    T = 16384
    g = torch.Generator().manual_seed(11)
    q, k, v, do = (torch.randn(1, T, h, 128, generator=g).to(torch.bfloat16).to(cuda).transpose(1, 2)
                   for h in (32, 8, 8, 32))
    print(f"case T={T} causal={causal} atomic={atomic}: sliced (default limit) vs one launch", flush=True)
    sliced = _grads(q, k, v, do, causal=causal, atomic=atomic, limit=0)
    single = _grads(q, k, v, do, causal=causal, atomic=atomic, limit=64 << 30)
    for name, a, b in zip(("dq", "dk", "dv"), sliced, single):
        assert torch.isfinite(a).all(), name
        if (name == "dq" and not atomic) or (name != "dq" and not causal):
            assert torch.equal(a, b), name
        else:
            # one bf16 step of the value (fp32 sums in another order, rounded
            # once); entries near zero after cancellation get an absolute floor
            bf = b.float()
            step = bf.abs() * 2.0 ** -7 + 1e-5 * bf.abs().max()
            diff = (a.float() - bf).abs()
            assert (diff <= step).all(), f"{name}: max diff {diff.max().item():.3e}"
        del a, b
    del sliced, single
    torch.cuda.empty_cache()


@pytest.mark.parametrize("causal", [False, True], ids=["noncausal", "causal"])
def test_row_ranges_match_single_launch_at_32k(cuda, causal):
    T = 32768
    g = torch.Generator().manual_seed(13)
    q, k, v, do = (torch.randn(1, T, h, 128, generator=g).to(torch.bfloat16).to(cuda).transpose(1, 2)
                   for h in (32, 8, 8, 32))
    print(f"case T={T} causal={causal}: row ranges (default limit) vs one launch (80 GiB)", flush=True)
    ranged = _grads(q, k, v, do, causal=causal, atomic=False, limit=0)
    single = _grads(q, k, v, do, causal=causal, atomic=False, limit=80 << 30)
    for name, a, b in zip(("dq", "dk", "dv"), ranged, single):
        assert torch.isfinite(a).all(), name
        if name == "dq":
            assert torch.equal(a, b), name
        else:
            bf = b.float()
            step = bf.abs() * 2.0 ** -7 + 1e-5 * bf.abs().max()
            diff = (a.float() - bf).abs()
            assert (diff <= step).all(), f"{name}: max diff {diff.max().item():.3e}"
    del ranged, single
    torch.cuda.empty_cache()


def test_default_limit_is_stable_and_equal_split_limits_agree(cuda):
    """T 4096 at the headline's heads, deterministic: two calls under the
    default limit with 24 GiB allocated in between (a different allocator
    state) are bitwise equal; a 512 MiB limit (two slices of four units) and a
    1 GiB one (one launch) both split each head group in two and give the
    same bits; causal likewise under the default limit."""
    import tilelang_fa2_4d_mask.fa2 as fa2mod

    assert fa2mod.ds_limit_bytes() == fa2mod.DS_LIMIT_DEFAULT
    T = 4096
    g = torch.Generator().manual_seed(12)
    q, k, v, do = (torch.randn(1, T, h, 128, generator=g).to(torch.bfloat16).to(cuda).transpose(1, 2)
                   for h in (32, 8, 8, 32))
    for causal in (False, True):
        print(f"case T={T} causal={causal}: default limit twice around a 24 GiB allocation", flush=True)
        a = _grads(q, k, v, do, causal=causal, atomic=False, limit=0)
        hog = torch.empty(24 << 30, dtype=torch.uint8, device=cuda)
        b = _grads(q, k, v, do, causal=causal, atomic=False, limit=0)
        del hog
        torch.cuda.empty_cache()
        for name, x, y in zip(("dq", "dk", "dv"), a, b):
            assert torch.equal(x, y), (causal, name)
    print(f"case T={T}: 512 MiB (sliced) vs 1 GiB (one launch), equal head-group split", flush=True)
    a = _grads(q, k, v, do, causal=False, atomic=False, limit=512 << 20)
    b = _grads(q, k, v, do, causal=False, atomic=False, limit=1 << 30)
    for name, x, y in zip(("dq", "dk", "dv"), a, b):
        assert torch.equal(x, y), name
