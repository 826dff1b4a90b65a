#!/usr/bin/env python3
"""Headline benchmark: FA2 fwd and fwd+bwd TFLOPS at B1 T8192 Hq32 Hk8 D128 bf16.

One step = one fwd+bwd pass (non-causal) of ``tilelang_flash_attention`` over
the BASELINE headline config: Q/K/V/dO ~ N(0,1) bf16, BHSD views
over BTHD storage, scale D^-0.5 -- what the reference's throughput_check.py
times (fwd+bwd = zero grads, forward, backward(dO),
benchmark/throughput_check.py:206-211).  ``value`` uses the deterministic
backward (use_atomic_backward=False: dK/dV kernel that also stores dS, then
dQ = dS K); the reference's default atomic-dQ backward is timed in the same run
(``breakdown``), as are fwd and fwd+bwd with is_causal=True.

FLOP convention (benchmark/throughput_check.py:85-92): fwd 4*B*Hq*Tq*Tk*D,
fwd+bwd 14*..., x0.5 when causal.  Peak: MI355X dense bf16 MFMA 2.5 PFLOP/s.

Timing (the reference's do_bench protocol, throughput_check.py:216, 248-256):
after W untimed steps, each of K steps is timed with its own HIP event pair
on the launch stream, with a 512 MiB write before it (outside the events) so
that L2 and the 256 MB Infinity Cache hold none of its inputs; ``ms_per_step``
is the median, with the 20/80 % quantiles beside it, and
``ms_per_step_window`` the synchronised wall time of the whole loop per step
(flushes included).  ``peak_mem_mib`` is the peak device memory one step
allocates beyond what is live before it (throughput_check.py:218-243);
``ds_limit_bytes`` the dS workspace limit in force (the library default,
4 GiB, unless ``--ds-limit`` sets one).  ``breakdown`` also times the headline
fwd and fwd+bwd replayed from a captured HIP graph (the reference's
``--cudagraph`` mode, benchmark/throughput_check.py:249-250): the same kernels
without the host work of the Python and autograd layers between launches;
and the deterministic fwd+bwd under a 1 GiB dS workspace (``*_ds1g``:
non-causal in slices of (batch, kv-head) units, causal in ranges of query
rows), the cost of a bounded backward workspace.

``roofline`` is for the dominant kernel of the step, the dK/dV kernel launched
by ``fa_bwd`` on the deterministic path: 4 GEMMs (S, dP, dV, dK), i.e.
8*B*Hq*Tq*Tk*D algorithmic FLOPs per launch, timed with HIP events on the
launch stream inside the timed region.  ``traffic`` (HBM bytes per launch) is
read from profiles/traffic_H_S.json, written from rocprofv3 FETCH_SIZE /
WRITE_SIZE runs of ``bench.py --traffic-pass`` scaled by a copy-kernel
calibration.  ``cpu_baseline`` times
this repository's eager fp32 oracle on the host cores on a bounded sample.

The other BASELINE configs (P: packed-document mask, S: score + sparse mask,
M: MQA long KV, bshd) are timed after the headline and reported under
``configs`` with dense-convention TFLOPS and GB/s against their algorithmic
bytes (each tensor once; mask at its passed head count), the HBM fraction of
8 TB/s, and for the masked ones the live TFLOPS (dense convention times the
kept fraction of pairs) and its fraction of peak instead of a dense fraction;
each also replays its fwd and deterministic fwd+bwd from captured graphs
(``fwd_graph``, ``fwd_bwd_graph``: eager minus graph is the host time the
GPU waits for).  ``cpu_baseline`` also times BASELINE configs[0] (C) on the
host.

Usage: python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-cpu-baseline] [--no-side-configs]
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (str(ROOT), str(ROOT / "fa2-with-4d-mask_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "fwd and fwd+bwd TFLOPS (and % bf16 MFMA peak) at B1 T8192 Hq32 Hk8 D128"
PEAK_TFLOPS = 2500.0          # MI355X dense bf16 MFMA
PUBLISHED_FWD_BWD = 169.43    # reference README.md:136 (TileLang fwd+bwd, non-causal, RTX PRO 5000)
B, T, HQ, HK, D = 1, 8192, 32, 8, 128


def conv_flops(mode: str, causal: bool) -> float:
    return (4.0 if mode == "fwd" else 14.0) * (0.5 if causal else 1.0) * B * HQ * T * T * D


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_inputs(torch, dev):
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    q = torch.randn((B, T, HQ, D), generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
    k = torch.randn((B, T, HK, D), generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
    v = torch.randn((B, T, HK, D), generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
    do = torch.randn((B, T, HQ, D), generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
    return q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), do.transpose(1, 2)


def packed_docs_mask(torch, dev, batch: int, t: int, gen, lo: int = 128, hi: int = 1024):
    """[batch, 1, t, t] block-diagonal causal keep-mask of packed documents
    segment lengths uniform in [lo, hi], last one truncated."""
    seg = torch.empty((batch, t), dtype=torch.int32)
    for bi in range(batch):
        pos, sid = 0, 0
        while pos < t:
            n = int(torch.randint(lo, hi + 1, (1,), generator=gen).item())
            seg[bi, pos:pos + n] = sid
            pos, sid = pos + n, sid + 1
    seg = seg.to(dev)
    keep = (seg[:, :, None] == seg[:, None, :]) & torch.ones((t, t), dtype=torch.bool, device=dev).tril()
    return keep.unsqueeze(1).contiguous()


def side_configs(torch, dev):
    """The other BASELINE configs as bench lines: P (packed-document mask), S
    (score + sparse mask), M (MQA, long KV, bshd); then D256, head dim 256 at
    config H's FLOPs per head pair (not a BASELINE config: the reference takes
    any head dim, python/fa2.py:33).  Yields (name, inputs)."""
    g = torch.Generator(device="cpu")
    g.manual_seed(0)

    def rnd(shape):
        return torch.randn(shape, generator=g).to(torch.bfloat16).to(dev)

    # P: B2 T4096 Hq32 Hk8 D128, mask [2, 1, T, T]
    b, t, hq, hk, d = 2, 4096, 32, 8, 128
    q, k, v, do = rnd((b, t, hq, d)), rnd((b, t, hk, d)), rnd((b, t, hk, d)), rnd((b, t, hq, d))
    mask = packed_docs_mask(torch, dev, b, t, g)
    yield "P", dict(q=q.transpose(1, 2), k=k.transpose(1, 2), v=v.transpose(1, 2), do=do.transpose(1, 2),
                    mask=mask, score=None, layout="bhsd", dims=(b, t, t, hq, hk, d))
    del q, k, v, do, mask
    # S: B1 T4096 Hq=Hk=16 D128, score [1,16,T,T] fp32 (ALiBi + N(0, 0.1)), mask [1,16,T,T] (p_drop 0.1, diag kept)
    b, t, hq, hk, d = 1, 4096, 16, 16, 128
    q, k, v, do = rnd((b, t, hq, d)), rnd((b, t, hk, d)), rnd((b, t, hk, d)), rnd((b, t, hq, d))
    slopes = torch.tensor([2.0 ** (-8.0 * (h + 1) / hq) for h in range(hq)], device=dev).view(1, hq, 1, 1)
    idx = torch.arange(t, device=dev, dtype=torch.float32)
    score = -slopes * (idx[:, None] - idx[None, :]).abs() + 0.1 * torch.randn((b, hq, t, t), generator=g).to(dev)
    mask = torch.rand((b, hq, t, t), generator=g).to(dev) >= 0.1
    mask[:, :, torch.arange(t), torch.arange(t)] = True
    yield "S", dict(q=q.transpose(1, 2), k=k.transpose(1, 2), v=v.transpose(1, 2), do=do.transpose(1, 2),
                    mask=mask.contiguous(), score=score.contiguous(), layout="bhsd", dims=(b, t, t, hq, hk, d))
    del q, k, v, do, mask, score
    # M: B1 Tq2048 Tk16384 Hq32 Hk1 D64, bshd
    b, tq, tk, hq, hk, d = 1, 2048, 16384, 32, 1, 64
    yield "M", dict(q=rnd((b, tq, hq, d)), k=rnd((b, tk, hk, d)), v=rnd((b, tk, hk, d)), do=rnd((b, tq, hq, d)),
                    mask=None, score=None, layout="bshd", dims=(b, tq, tk, hq, hk, d))
    # D256: B1 T4096 Hq16 Hk4 D256, bhsd
    b, t, hq, hk, d = 1, 4096, 16, 4, 256
    q, k, v, do = rnd((b, t, hq, d)), rnd((b, t, hk, d)), rnd((b, t, hk, d)), rnd((b, t, hq, d))
    yield "D256", dict(q=q.transpose(1, 2), k=k.transpose(1, 2), v=v.transpose(1, 2), do=do.transpose(1, 2),
                       mask=None, score=None, layout="bhsd", dims=(b, t, t, hq, hk, d))


def side_bytes(x, mode: str) -> float:
    """Algorithmic HBM bytes: every tensor once (Q, K, V, O, LSE, mask at its
    passed head count, score); fwd+bwd adds dO, dQ, dK, dV, Delta and a second
    read of mask/score."""
    b, tq, tk, hq, hk, d = x["dims"]
    side = (x["mask"].numel() if x["mask"] is not None else 0) + 4 * (x["score"].numel() if x["score"] is not None else 0)
    fwd = 2 * d * (2 * b * tq * hq + 2 * b * tk * hk) + 4 * b * hq * tq + side
    if mode == "fwd":
        return float(fwd)
    return float(fwd + 2 * d * (2 * b * tq * hq + 2 * b * tk * hk) + 4 * b * hq * tq + side)


FLUSH_BYTES = 512 << 20   # > the 256 MB Infinity Cache (MALL) and every XCD's L2


class Flusher:
    """Writes a 512 MiB buffer between timed steps (outside their events), so
    that no step finds its inputs in L2 or the MALL, as the reference's
    do_bench clears the cache before every repetition
    (benchmark/throughput_check.py:248-256)."""

    def __init__(self, torch, dev):
        self.buf = torch.empty(FLUSH_BYTES // 4, dtype=torch.float32, device=dev)
        self.n = 0

    def __call__(self):
        self.n += 1
        self.buf.fill_(float(self.n))


def time_steps(torch, fn, steps: int, warmup: int, record_events, flush):
    """Times each of ``steps`` steps with a HIP event pair on the launch stream
    (torch's current stream), after ``warmup`` untimed steps, with the cache
    flushed before every step outside the events.  Returns the median and the
    20/80 % quantiles of the per-step times (the reference's do_bench
    statistics, throughput_check.py:216, 248-256), the synchronised wall time
    of the whole timed loop per step (flushes included), and each library
    call's mean time."""
    for _ in range(warmup):
        flush()
        fn()
    torch.cuda.synchronize()
    ev0 = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ev1 = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    with record_events() as ev:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(steps):
            flush()
            ev0[i].record()
            fn()
            ev1[i].record()
        torch.cuda.synchronize()
        t1 = time.perf_counter()
    per = sorted(a.elapsed_time(b) for a, b in zip(ev0, ev1))
    q = statistics.quantiles(per, n=10, method="inclusive") if len(per) > 1 else [per[0]] * 9
    per_kernel = {name: statistics.mean(v) for name, v in ev.elapsed_ms().items()}
    return {"ms": statistics.median(per), "ms_p20": q[1], "ms_p80": q[7],
            "ms_window": (t1 - t0) * 1e3 / steps}, per_kernel


def graph_of(torch, fn):
    """``fn`` captured into a HIP graph (after two warm-up calls on a side
    stream, as torch.cuda.graph requires); returns the graph's replay."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def peak_extra_mib(torch, fn, dev) -> float:
    """Peak device memory one step allocates beyond what is live before it
    (benchmark/throughput_check.py:218-243)."""
    torch.cuda.empty_cache()
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats(dev)
    base = torch.cuda.memory_allocated(dev)
    fn()
    torch.cuda.synchronize()
    return round((torch.cuda.max_memory_allocated(dev) - base) / 2 ** 20, 1)


def cpu_config_c(seconds: float) -> dict:
    """BASELINE configs[0] (C): the eager fp32 oracle's fwd+bwd at B1 Hq4 Hk2
    T256 D64, causal, fp32 Q/K/V/dO ~ N(0,1), on the host cores."""
    import torch

    from oracle import eager as E

    g = torch.Generator(device="cpu")
    g.manual_seed(0)
    q = torch.randn((1, 256, 4, 64), generator=g).transpose(1, 2)
    k = torch.randn((1, 256, 2, 64), generator=g).transpose(1, 2)
    v = torch.randn((1, 256, 2, 64), generator=g).transpose(1, 2)
    do = torch.randn((1, 256, 4, 64), generator=g).transpose(1, 2)
    E.eager_fwd_bwd(q, k, v, None, None, do, scale=64 ** -0.5, is_causal=True)   # warm-up
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        E.eager_fwd_bwd(q, k, v, None, None, do, scale=64 ** -0.5, is_causal=True)
        times.append(time.perf_counter() - t0)
    ms = statistics.median(times) * 1e3
    flops = 14.0 * 0.5 * 1 * 4 * 256 * 256 * 64
    return {"workload": "C (BASELINE configs[0]): B1 Hq4 Hk2 T256 D64 fp32 causal, fwd+bwd", "ms": round(ms, 4),
            "tflops": round(flops / (ms * 1e-3) * 1e-12, 5), "runs": len(times)}


def cpu_baseline(seconds: float) -> dict:
    """The fp32 oracle (oracle/eager.py) on the host cores at the whole headline
    workload (B1 T8192 Hq32 Hk8 D128, non-causal): fwd+bwd by the closed-form
    chunked gradients (``eager_grads_chunked``: the eager graph's gradients,
    pinned against autograd in the CPU suite, one [B, Hq, 128, T] slab at a
    time instead of autograd's saved [B, Hq, T, T] probabilities), the forward
    by ``eager_ref`` in chunks of 128 query rows; BASELINE configs[0] (C)
    beside them.  Each runs at least once and repeats until ``seconds`` (the
    forward ``seconds / 3``) have passed."""
    import torch

    from oracle import eager as E

    g = torch.Generator(device="cpu")
    g.manual_seed(0)
    q = torch.randn((B, T, HQ, D), generator=g).to(torch.bfloat16).transpose(1, 2)
    k = torch.randn((B, T, HK, D), generator=g).to(torch.bfloat16).transpose(1, 2)
    v = torch.randn((B, T, HK, D), generator=g).to(torch.bfloat16).transpose(1, 2)
    do = torch.randn((B, T, HQ, D), generator=g).to(torch.bfloat16).transpose(1, 2)
    flops = 14.0 * B * HQ * T * T * D
    runs, t0 = 0, time.perf_counter()
    while True:
        E.eager_grads_chunked(q, k, v, None, None, do, scale=D ** -0.5, is_causal=False, block=128)
        runs += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    tflops = flops * runs / el * 1e-12
    fruns, t1 = 0, time.perf_counter()
    with torch.no_grad():
        while True:
            E.eager_ref(q, k, v, None, None, scale=D ** -0.5, is_causal=False, ref_block=128)
            fruns += 1
            fel = time.perf_counter() - t1
            if fel >= seconds / 3:
                break
    fwd_tflops = 4.0 * B * HQ * T * T * D * fruns / fel * 1e-12
    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count()
    return {
        "value": round(tflops, 4),
        "unit": "TFLOPS",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"the whole headline workload (B1 T8192 Hq32 Hk8 D128 bf16 inputs, fp32 maths, non-causal): "
                   f"oracle fwd+bwd by closed-form chunked gradients (block 128), {runs} run(s) in {el:.1f} s; "
                   f"host affinity {cores} cores"),
        "ms_per_step": round(el / runs * 1e3, 1),
        "fwd": {"value": round(fwd_tflops, 4), "unit": "TFLOPS", "ms": round(fel / fruns * 1e3, 1),
                "sample": f"oracle eager forward (ref_block 128), same inputs, {fruns} run(s) in {fel:.1f} s"},
        "config_C": cpu_config_c(min(5.0, seconds / 3)),
    }


def traffic_pass(torch, api, dev) -> int:
    """One untimed launch of each kernel whose counters are reported (what the
    rocprofv3 --pmc passes count), after a 1 GiB copy whose FETCH_SIZE /
    WRITE_SIZE reading calibrates those counters: the H forward and
    deterministic fwd+bwd, non-causal and causal; the P, S and M fwd+bwd
    (deterministic)."""
    x = torch.empty(2 ** 28, dtype=torch.float32, device=dev)
    y = torch.empty_like(x)
    y.copy_(x)
    torch.cuda.synchronize()
    del x, y
    q0, k0, v0, do = make_inputs(torch, dev)
    for causal in (False, True):
        log(f"profile pass: H causal={causal}")
        q, k, v = (t.detach().requires_grad_(True) for t in (q0, k0, v0))
        with torch.no_grad():
            api.tilelang_flash_attention(q0, k0, v0, is_causal=causal)
        api.tilelang_flash_attention(q, k, v, is_causal=causal, use_atomic_backward=False).backward(do)
        torch.cuda.synchronize()
        del q, k, v
    del q0, k0, v0, do
    for n, c in side_configs(torch, dev):
        log(f"profile pass: {n}")
        q, k, v = (c[t].detach().requires_grad_(True) for t in ("q", "k", "v"))
        api.tilelang_flash_attention(q, k, v, mask=c["mask"], score=c["score"], layout=c["layout"],
                                     use_atomic_backward=False).backward(c["do"])
        torch.cuda.synchronize()
        del q, k, v, c
    log("traffic pass done")
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-side-configs", action="store_true",
                    help="skip the P / S / M config lines (mask, score+mask, MQA)")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--ds-limit", type=int, default=None,
                    help="dS workspace limit in bytes for the backward (tilelang_fa2_4d_mask.fa2.DS_LIMIT_BYTES); "
                         "default: the library's")
    ap.add_argument("--traffic-pass", action="store_true",
                    help="run once, untimed, what the rocprofv3 --pmc passes count: a 1 GiB fp32 copy "
                         "(calibration), the H forward and deterministic fwd+bwd (non-causal and causal), "
                         "the P, S and M deterministic fwd+bwd")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}): this build has no multi-GPU "
              "path; the op shards over (batch x kv-head) with no communication.", file=sys.stderr)
        return 2

    import torch

    import tilelang_fa2_4d_mask as api
    from tilelang_fa2_4d_mask.fa2 import record_kernel_events

    if not torch.cuda.is_available():
        log("no GPU visible")
        return 1
    dev = torch.device("cuda:0")
    if args.ds_limit is not None:
        import tilelang_fa2_4d_mask.fa2 as fa2mod
        fa2mod.DS_LIMIT_BYTES = args.ds_limit
    if args.traffic_pass:
        return traffic_pass(torch, api, dev)
    q0, k0, v0, do = make_inputs(torch, dev)
    q = q0.detach().requires_grad_(True)
    k = k0.detach().requires_grad_(True)
    v = v0.detach().requires_grad_(True)

    def fwd(causal):
        def f():
            with torch.no_grad():
                api.tilelang_flash_attention(q0, k0, v0, is_causal=causal)
        return f

    def fwd_bwd(causal, atomic):
        def f():
            q.grad = k.grad = v.grad = None
            out = api.tilelang_flash_attention(q, k, v, is_causal=causal, use_atomic_backward=atomic)
            out.backward(do)
        return f

    import tilelang_fa2_4d_mask.fa2 as fa2mod

    def fwd_bwd_limited(causal, limit):
        # deterministic fwd+bwd with the dS workspace capped at `limit` bytes
        inner = fwd_bwd(causal, False)

        def f():
            prev = fa2mod.DS_LIMIT_BYTES
            fa2mod.DS_LIMIT_BYTES = limit
            try:
                inner()
            finally:
                fa2mod.DS_LIMIT_BYTES = prev
        return f

    log(f"device: {torch.cuda.get_device_name(dev)}; workload B{B} T{T} Hq{HQ} Hk{HK} D{D} bf16")
    flush = Flusher(torch, dev)
    from tilelang_fa2_4d_mask.fa2 import ds_limit_bytes
    ds_limit = ds_limit_bytes(dev)
    results = {}
    for name, fn, mode, causal in (
        ("fwd_bwd", fwd_bwd(False, False), "fwd_bwd", False),
        ("fwd", fwd(False), "fwd", False),
        ("fwd_causal", fwd(True), "fwd", True),
        ("fwd_bwd_causal", fwd_bwd(True, False), "fwd_bwd", True),
        ("fwd_bwd_atomic", fwd_bwd(False, True), "fwd_bwd", False),
        ("fwd_bwd_causal_atomic", fwd_bwd(True, True), "fwd_bwd", True),
        ("fwd_bwd_ds1g", fwd_bwd_limited(False, 1 << 30), "fwd_bwd", False),
        ("fwd_bwd_causal_ds1g", fwd_bwd_limited(True, 1 << 30), "fwd_bwd", True),
    ):
        tm, kern = time_steps(torch, fn, args.steps, args.warmup, record_kernel_events, flush)
        ms = tm["ms"]
        tf = conv_flops(mode, causal) / (ms * 1e-3) * 1e-12
        results[name] = {"ms": round(ms, 4), "ms_p20": round(tm["ms_p20"], 4), "ms_p80": round(tm["ms_p80"], 4),
                         "ms_window": round(tm["ms_window"], 4), "tflops": round(tf, 2),
                         "tflops_p20_p80": [round(conv_flops(mode, causal) / (tm[k] * 1e-3) * 1e-12, 2)
                                            for k in ("ms_p80", "ms_p20")],
                         "frac_of_peak": round(tf / PEAK_TFLOPS, 4),
                         "peak_extra_mib": peak_extra_mib(torch, fn, dev),
                         "kernel_ms": {k2: round(v2, 4) for k2, v2 in kern.items()}}
        q.grad = k.grad = v.grad = None
        log(f"{name:22s} {ms:8.3f} ms (p20 {tm['ms_p20']:.3f}, p80 {tm['ms_p80']:.3f})  {tf:8.1f} TFLOPS  "
            f"({100 * tf / PEAK_TFLOPS:5.1f}% of peak)  peak extra {results[name]['peak_extra_mib']} MiB  kernels {kern}")

    # the headline fwd and fwd+bwd replayed from captured graphs
    for name, mode in (("fwd_graph", "fwd"), ("fwd_bwd_graph", "fwd_bwd")):
        if mode == "fwd":
            step = fwd(False)
        else:
            def step():
                q.grad = k.grad = v.grad = None
                api.tilelang_flash_attention(q, k, v, is_causal=False, use_atomic_backward=False).backward(do)
        g = graph_of(torch, step)
        tm, _ = time_steps(torch, g.replay, args.steps, args.warmup, record_kernel_events, flush)
        ms = tm["ms"]
        tf = conv_flops(mode, False) / (ms * 1e-3) * 1e-12
        eager = results["fwd" if mode == "fwd" else "fwd_bwd"]["ms"]
        results[name] = {"ms": round(ms, 4), "ms_p20": round(tm["ms_p20"], 4), "ms_p80": round(tm["ms_p80"], 4),
                         "tflops": round(tf, 2), "frac_of_peak": round(tf / PEAK_TFLOPS, 4),
                         "eager_minus_graph_ms": round(eager - ms, 4)}
        log(f"{name:22s} {ms:8.3f} ms  {tf:8.1f} TFLOPS ({100 * tf / PEAK_TFLOPS:5.1f}% of peak), eager - graph "
            f"{eager - ms:+.3f} ms")
        del g
        q.grad = k.grad = v.grad = None
        torch.cuda.empty_cache()

    side = {}
    if not args.no_side_configs:
        del q, k, v
        for name, x in side_configs(torch, dev):
            bq, tq, tk, hq, hk, d = x["dims"]
            flops_fwd = 4.0 * bq * hq * tq * tk * d
            xq = x["q"].detach().requires_grad_(True)
            xk = x["k"].detach().requires_grad_(True)
            xv = x["v"].detach().requires_grad_(True)
            kw = dict(mask=x["mask"], score=x["score"], layout=x["layout"])

            def sfwd():
                with torch.no_grad():
                    api.tilelang_flash_attention(x["q"], x["k"], x["v"], **kw)

            def sfb(atomic):
                def f():
                    xq.grad = xk.grad = xv.grad = None
                    api.tilelang_flash_attention(xq, xk, xv, use_atomic_backward=atomic, **kw).backward(x["do"])
                return f

            entry = {}
            # kept fraction of (row, key) pairs: the work a kernel that skips
            # dropped entries has to do (the dense convention overstates it)
            keep = x["mask"].float().mean().item() if x["mask"] is not None else 1.0
            for mode, fn in (("fwd", sfwd), ("fwd_bwd", sfb(False)), ("fwd_bwd_atomic", sfb(True))):
                tm, kern = time_steps(torch, fn, max(3, args.steps // 2), max(1, args.warmup // 2),
                                      record_kernel_events, flush)
                ms = tm["ms"]
                fl = flops_fwd * (1.0 if mode == "fwd" else 3.5)
                nbytes = side_bytes(x, "fwd" if mode == "fwd" else "fwd_bwd")
                gbps = nbytes / (ms * 1e-3) * 1e-9
                e = {"ms": round(ms, 4), "ms_p20": round(tm["ms_p20"], 4), "ms_p80": round(tm["ms_p80"], 4),
                     "ms_window": round(tm["ms_window"], 4),
                     "tflops_dense_conv": round(fl / (ms * 1e-3) * 1e-12, 2),
                     "alg_bytes": nbytes, "gbps": round(gbps, 1), "hbm_frac": round(gbps / 8000.0, 4),
                     "peak_extra_mib": peak_extra_mib(torch, fn, dev),
                     "kernel_ms": {k2: round(v2, 4) for k2, v2 in kern.items()}}
                if x["mask"] is None:
                    e["frac_of_peak"] = round(e["tflops_dense_conv"] / PEAK_TFLOPS, 4)
                else:
                    e["tflops_live"] = round(e["tflops_dense_conv"] * keep, 2)
                    e["live_frac_of_peak"] = round(e["tflops_live"] / PEAK_TFLOPS, 4)
                xq.grad = xk.grad = xv.grad = None
                entry[mode] = e
                log(f"{name} {mode:15s} {ms:8.3f} ms  {e['tflops_dense_conv']:8.1f} TFLOPS (dense conv.)"
                    f"  {e['gbps']:8.1f} GB/s of {nbytes / 1e9:.3f} GB algorithmic  peak extra {e['peak_extra_mib']} MiB"
                    f"  kernels {kern}")
            # the same steps replayed from captured graphs: what the host adds
            # per call (eager minus graph)
            for mode, fn in (("fwd_graph", sfwd), ("fwd_bwd_graph", sfb(False))):
                g = graph_of(torch, fn)
                tm, _ = time_steps(torch, g.replay, max(3, args.steps // 2), max(1, args.warmup // 2),
                                   record_kernel_events, flush)
                ms = tm["ms"]
                eager = entry["fwd" if mode == "fwd_graph" else "fwd_bwd"]["ms"]
                entry[mode] = {"ms": round(ms, 4), "ms_p20": round(tm["ms_p20"], 4), "ms_p80": round(tm["ms_p80"], 4),
                               "eager_minus_graph_ms": round(eager - ms, 4)}
                log(f"{name} {mode:15s} {ms:8.3f} ms  eager - graph {eager - ms:+.3f} ms")
                del g
                xq.grad = xk.grad = xv.grad = None
                torch.cuda.empty_cache()
            if x["mask"] is not None:
                entry["mask_keep_fraction"] = round(keep, 4)
            entry["config"] = {"B": bq, "Tq": tq, "Tk": tk, "Hq": hq, "Hk": hk, "D": d, "layout": x["layout"],
                               "mask": None if x["mask"] is None else list(x["mask"].shape),
                               "score": None if x["score"] is None else list(x["score"].shape)}
            side[name] = entry
            del x, xq, xk, xv
            torch.cuda.empty_cache()

    main_res = results["fwd_bwd"]
    # dominant kernel: dK/dV (fa_bwd on the deterministic path), 4 GEMMs
    dkdv_ms = main_res["kernel_ms"]["fa_bwd"]
    dkdv_flops = 8.0 * B * HQ * T * T * D
    achieved = dkdv_flops / (dkdv_ms * 1e-3) * 1e-12
    # dQ = dS K (fa_bwd_finalize on the deterministic path): streams the 16-bit dS tiles
    dq_ms = main_res["kernel_ms"]["fa_bwd_finalize"]
    dq_bytes = 2.0 * B * HQ * T * T + 2.0 * B * HQ * T * D * 2   # dS tiles + K rows (L2) + dQ out
    fwd_kernel_ms = results["fwd"]["kernel_ms"]["fa_fwd"]
    fwd_achieved = 4.0 * B * HQ * T * T * D / (fwd_kernel_ms * 1e-3) * 1e-12
    for name, r in results.items():
        causal = "causal" in name
        km = r.get("kernel_ms", {})
        if "fa_fwd" in km:
            r["fwd_kernel_tflops"] = round(conv_flops("fwd", causal) / (km["fa_fwd"] * 1e-3) * 1e-12, 2)
        if "fa_bwd" in km:
            bwd_ms = km["fa_bwd"] + km.get("fa_bwd_finalize", 0.0)
            r["bwd_tflops"] = round(10.0 * (0.5 if causal else 1.0) * B * HQ * T * T * D / (bwd_ms * 1e-3) * 1e-12, 2)
    traffic = traffic_fwd = traffic_dq = None
    tpath = ROOT / "profiles" / "traffic_H_S.json"
    if tpath.exists():
        try:
            kern = json.loads(tpath.read_text())["kernels"]
            traffic = kern["dkdv2_kernel<bf16,128> H (fa_bwd, deterministic)"]["bytes_per_launch"]
            traffic_fwd = kern["fwd_kernel<bf16,128> H (fa_fwd, non-causal)"]["bytes_per_launch"]
            traffic_dq = kern["dq_ds_kernel<bf16,128> H (fa_bwd_finalize, deterministic)"]["bytes_per_launch"]
        except (OSError, ValueError, KeyError):
            traffic = traffic_fwd = traffic_dq = None

    line = {
        "metric": METRIC,
        "value": main_res["tflops"],
        "unit": "TFLOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": main_res["ms"],
        "ms_per_step_p20_p80": [main_res["ms_p20"], main_res["ms_p80"]],
        "ms_per_step_window": main_res["ms_window"],
        "peak_mem_mib": main_res["peak_extra_mib"],
        "ds_limit_bytes": ds_limit,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(main_res["tflops"] / PUBLISHED_FWD_BWD, 3),
        "dtype": "bf16",
        "data": "synthetic: Q/K/V/dO ~ N(0,1) bf16, seeded, BHSD views over BTHD storage",
        "config": {
            "workload": "H (BASELINE configs[1]): fwd+bwd non-causal per step, deterministic backward "
                        "(use_atomic_backward=False); atomic-dQ default in breakdown",
            "batch": B, "seq_len_q": T, "seq_len_k": T, "heads_q": HQ, "heads_k": HK, "head_dim": D,
            "layout": "bhsd", "scale": "D^-0.5", "parallelism": "single GPU",
        },
        "breakdown": results,
        "configs": side,
        "roofline": {
            "kernel": "dkdv2_kernel<bf16,128> via fa_bwd (dK/dV + dS tiles, deterministic path)",
            "bound": "mfma",
            "achieved": round(achieved, 2),
            "peak": PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_TFLOPS, 4),
            "traffic": traffic,
            "avg_launch_ms": round(dkdv_ms, 4),
            "flops_per_launch": dkdv_flops,
            "fwd_kernel": {"achieved": round(fwd_achieved, 2), "frac": round(fwd_achieved / PEAK_TFLOPS, 4),
                           "avg_launch_ms": round(fwd_kernel_ms, 4), "unit": "TFLOP/s", "traffic": traffic_fwd},
            "dq_kernel": {"bound": "hbm", "achieved": round(dq_bytes / (dq_ms * 1e-3) * 1e-9, 1), "peak": 8000.0,
                          "unit": "GB/s", "frac": round(dq_bytes / (dq_ms * 1e-3) * 1e-9 / 8000.0, 4),
                          "avg_launch_ms": round(dq_ms, 4), "bytes_per_launch": dq_bytes, "traffic": traffic_dq},
        },
    }
    if not args.no_cpu_baseline:
        log("timing the CPU baseline ...")
        line["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
        log(f"cpu baseline: {line['cpu_baseline']}")
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
