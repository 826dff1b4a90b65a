"""The custom ops' fake (meta) implementations on the CPU (no GPU, no kernel
runs): output shapes and dtypes, and the prepared-mask workspace size, which
must equal what fa_mask_plan reports for the same mask view."""

import ctypes

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode


def _mods():
    from tilelang_fa2_4d_mask import _ext, fa2, ops  # noqa: F401

    return _ext, fa2, ops


@pytest.mark.parametrize("mask_heads,mask_batch", [(1, 1), (1, 2), (8, 2)])
def test_fake_shapes(mask_heads, mask_batch):
    _ext, fa2, _ = _mods()
    B, Hq, Hk, Tq, Tk, D = 2, 8, 2, 300, 500, 64
    with FakeTensorMode():
        q = torch.empty(B, Tq, Hq, D, dtype=torch.bfloat16, device="cuda")
        k = torch.empty(B, Tk, Hk, D, dtype=torch.bfloat16, device="cuda")
        mask = torch.empty(mask_batch, mask_heads, Tq, Tk, dtype=torch.bool, device="cuda")
        O, L, ws, lo = torch.ops.tilelang_fa2_4d_mask.fwd(q, k, k, mask, None, 0.125, True, True, True)
        assert O.shape == (B, Tq, Hq, D) and O.dtype == torch.bfloat16
        assert L.shape == (B, Hq, Tq) and L.dtype == torch.float32
        assert lo.shape == O.shape and lo.dtype == O.dtype   # O's rounding residual (mask present)
        nws = ws.shape[0]
        dq, dk, dv = torch.ops.tilelang_fa2_4d_mask.bwd(O, q, k, k, O, L, mask, None, ws, lo, 0.125, True, False)
        assert dq.shape == q.shape and dk.shape == k.shape and dv.shape == k.shape
        O2, _, ws2, lo2 = torch.ops.tilelang_fa2_4d_mask.fwd(q, k, k, None, None, 0.125, False, True, True)
        assert ws2.shape == (0,) and lo2.shape == (0,)   # no mask, no score: no residual
        _, _, _, lo3 = torch.ops.tilelang_fa2_4d_mask.fwd(q, k, k, mask, None, 0.125, True, True, False)
        assert lo3.shape == (0,)   # not asked for
    # same size from the C ABI for the same broadcast
    lib = _ext.load_library()
    mp = _ext.FaMaskParams()
    mp.mask = 256
    mp.mask_stride_b = 0 if mask_batch == 1 else mask_heads * Tq * Tk
    mp.mask_stride_h = 0 if mask_heads == 1 else Tq * Tk
    mp.mask_stride_q = Tk
    mp.batch, mp.seqlen_q, mp.seqlen_k, mp.heads_q, mp.is_causal = B, Tq, Tk, Hq, 1
    n = ctypes.c_int64(0)
    assert lib.fa_mask_plan(ctypes.byref(mp), ctypes.byref(n)) == 0
    assert nws == n.value


def test_public_wrapper_routes_through_the_op():
    _, fa2, ops = _mods()
    import inspect

    src = inspect.getsource(fa2.flash_attention_with_4d_mask)
    assert "ops.attention" in src
    sig = inspect.signature(fa2.flash_attention_with_4d_mask)
    assert list(sig.parameters) == ["Q", "K", "V", "Mask", "Score", "scale", "is_causal", "use_atomic_backward",
                                    "bhsd_input"]


def test_backward_without_an_output_gradient():
    """LSE, the mask workspace and O's rounding residual get no materialised
    zero gradients (no fill kernels before every backward); when O does not
    reach the loss either, the backward returns no gradients and launches
    nothing."""
    _, _, ops = _mods()

    class Ctx:
        materialize = True

        def save_for_backward(self, *t):
            self.saved_tensors = t

        def set_materialize_grads(self, value):
            self.materialize = value

    ctx = Ctx()
    q = torch.empty((1, 4, 2, 64), device="meta")
    ops._setup_context(ctx, (q, q, q, None, None, 0.125, False, True, True), (q, q, q, q))
    assert ctx.materialize is False
    assert ops._backward(ctx, None, None, None, None) == (None,) * 9


def test_default_ds_limit_is_a_constant():
    """The backward's dS workspace limit does not depend on the device's
    memory state (the route, slices and head-group split, hence the bits of
    the deterministic backward, depend on the problem alone); DS_LIMIT_BYTES
    overrides it."""
    _, fa2, _ = _mods()
    assert fa2.DS_LIMIT_BYTES == 0 and fa2.ds_limit_bytes() == fa2.DS_LIMIT_DEFAULT == 4 << 30
    old = fa2.DS_LIMIT_BYTES
    try:
        fa2.DS_LIMIT_BYTES = 1 << 30
        assert fa2.ds_limit_bytes() == 1 << 30
        fa2.DS_LIMIT_BYTES = -1
        assert fa2.ds_limit_bytes() == -1
    finally:
        fa2.DS_LIMIT_BYTES = old
