"""The registered custom ops (tilelang_fa2_4d_mask::fwd / ::bwd) on the GPU:

* ``torch.library.opcheck``: schema, fake (meta) implementation, autograd
  registration and the dispatcher's own consistency tests;
* ``torch.compile(fullgraph=True)`` of a function calling the public wrapper
  (mask, score, causal) traces it without a graph break, and its forward and
  gradients equal the eager calls bit for bit (deterministic backward);
* HIP-graph capture (``torch.cuda.graph``) of the forward and of forward +
  backward: every replay, with new inputs copied into the static tensors and
  eager work plus a synchronisation between replays, equals the eager call bit
  for bit (the same kernels run; the deterministic backward is repeatable).
"""

import pytest
import torch

pytestmark = pytest.mark.gpu


def _api():
    import tilelang_fa2_4d_mask as api

    return api


def _inputs(dev, seed, B=2, Hq=4, Hk=2, Tq=200, Tk=330, D=64, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn((B, Hq, Tq, D), generator=g).to(dtype).to(dev)
    k = torch.randn((B, Hk, Tk, D), generator=g).to(dtype).to(dev)
    v = torch.randn((B, Hk, Tk, D), generator=g).to(dtype).to(dev)
    do = torch.randn((B, Hq, Tq, D), generator=g).to(dtype).to(dev)
    mask = (torch.rand((B, 1, Tq, Tk), generator=g) < 0.7).to(dev)
    mask[..., 0] = True
    score = (0.1 * torch.randn((B, Hq, Tq, Tk), generator=g)).to(dev)
    return q, k, v, do, mask, score


def test_opcheck(cuda):
    q, k, v, do, mask, score = _inputs(cuda, 0)
    qt, kt, vt = (x.transpose(1, 2).detach().requires_grad_(True) for x in (q, k, v))
    print("case opcheck fwd with mask+score, causal", flush=True)
    torch.library.opcheck(torch.ops.tilelang_fa2_4d_mask.fwd, (qt, kt, vt, mask, score, 0.125, True, False, True),
                          test_utils=("test_schema", "test_faketensor", "test_autograd_registration"))
    print("case opcheck fwd, no mask", flush=True)
    torch.library.opcheck(torch.ops.tilelang_fa2_4d_mask.fwd, (qt, kt, vt, None, None, 0.125, False, True, True),
                          test_utils=("test_schema", "test_faketensor", "test_autograd_registration"))
    with torch.no_grad():
        O, L, ws, lo = torch.ops.tilelang_fa2_4d_mask.fwd(qt, kt, vt, mask, score, 0.125, True, False, True)
    assert lo.shape == O.shape
    print("case opcheck bwd", flush=True)
    torch.library.opcheck(torch.ops.tilelang_fa2_4d_mask.bwd,
                          (do.transpose(1, 2), qt.detach(), kt.detach(), vt.detach(), O, L, mask, score, ws, lo,
                           0.125, True, False), test_utils=("test_schema", "test_faketensor"))


def _fwd_bwd(fn, q, k, v, do, **kw):
    q, k, v = (x.detach().requires_grad_(True) for x in (q, k, v))
    out = fn(q, k, v, **kw)
    out.backward(do)
    return out.detach(), q.grad, k.grad, v.grad


def test_torch_compile_fullgraph(cuda):
    api = _api()
    q, k, v, do, mask, score = _inputs(cuda, 1)

    def f(q, k, v, mask, score):
        return api.tilelang_flash_attention(q, k, v, mask=mask, score=score, is_causal=True, use_atomic_backward=False)

    print("case torch.compile(aot_eager, fullgraph) fwd+bwd", flush=True)
    cf = torch.compile(f, backend="aot_eager", fullgraph=True)
    eager = _fwd_bwd(f, q, k, v, do, mask=mask, score=score)
    comp = _fwd_bwd(cf, q, k, v, do, mask=mask, score=score)
    for name, a, b in zip(("out", "dq", "dk", "dv"), comp, eager):
        assert torch.equal(a, b), name


@pytest.mark.parametrize("d", [64, 256])
@pytest.mark.parametrize("backward", [False, True], ids=["fwd", "fwd_bwd"])
def test_graph_capture_replays(cuda, backward, d):
    api = _api()
    q0, k0, v0, do0, mask0, score0 = _inputs(cuda, 2, D=d)
    sq, sk, sv, sdo, smask, sscore = (x.clone() for x in (q0, k0, v0, do0, mask0, score0))
    if backward:
        sq, sk, sv = (x.requires_grad_(True) for x in (sq, sk, sv))

    def step():
        out = api.tilelang_flash_attention(sq, sk, sv, mask=smask, score=sscore, is_causal=True,
                                           use_atomic_backward=False)
        if backward:
            out.backward(sdo)
        return out

    # warm up on a side stream (library load, allocator), as torch.cuda.graph requires
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            if backward:
                sq.grad = sk.grad = sv.grad = None
            step()
    torch.cuda.current_stream().wait_stream(s)
    if backward:
        sq.grad = sk.grad = sv.grad = None
    print(f"case graph capture backward={backward} D={d}", flush=True)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        static_out = step()
    for rep in range(3):
        q, k, v, do, mask, score = _inputs(cuda, 10 + rep, D=d)
        with torch.no_grad():
            for dst, src in ((sq, q), (sk, k), (sv, v), (sdo, do), (smask, mask), (sscore, score)):
                dst.copy_(src)
        g.replay()
        torch.cuda.synchronize()
        ref = _fwd_bwd(lambda a, b, c: api.tilelang_flash_attention(a, b, c, mask=mask, score=score, is_causal=True,
                                                                    use_atomic_backward=False), q, k, v, do)
        torch.cuda.synchronize()
        print(f"  replay {rep}", flush=True)
        assert torch.equal(static_out.detach(), ref[0]), f"out replay {rep}"
        if backward:
            for name, a, b in zip(("dq", "dk", "dv"), (sq.grad, sk.grad, sv.grad), ref[1:]):
                assert torch.equal(a, b), f"{name} replay {rep}"
