"""C ABI of libfa2_4d_mask.so, without a GPU.

* the library loads and exports every function include/fa2_4d_mask.h declares;
* the ctypes mirror of the parameter structs has exactly the C layout (a small
  C program compiled with gcc against the header prints sizeof/offsetof);
* every validation path returns its FA_ERR_* code before any HIP call;
* fa_bwd_plan's head-group split and workspace sizes.
"""

import ctypes
import math
import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "fa2_4d_mask.h"


def _ext():
    from tilelang_fa2_4d_mask import _ext

    return _ext


@pytest.fixture(scope="module")
def lib():
    ext = _ext()
    if not ext.LIB_PATH.exists():
        import importlib.util

        spec = importlib.util.spec_from_file_location("fa_build_ext", ROOT / "fa2-with-4d-mask_amd" / "build_ext.py")
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        mod.build(jobs=4)
    return ext.load_library()


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(fa_\w+)\s*\(", text, flags=re.M)))


def test_exports_every_declared_function(lib):
    names = declared_functions()
    assert {"fa_fwd", "fa_bwd_preprocess", "fa_bwd", "fa_bwd_finalize", "fa_bwd_plan", "fa_last_error",
            "fa_abi_version"} <= set(names)
    for n in names:
        assert hasattr(lib, n), n
    assert set(_ext().EXPORTED) == set(names)
    assert lib.fa_abi_version() == _ext().ABI_VERSION


def test_struct_layout_matches_header(tmp_path):
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    ext = _ext()
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', "int main(void) {"]
    for cname, cls in (("FaFwdParams", ext.FaFwdParams), ("FaBwdParams", ext.FaBwdParams),
                       ("FaBwdPlan", ext.FaBwdPlan), ("FaMaskParams", ext.FaMaskParams)):
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for fname, _ in cls._fields_:
            lines.append(f'printf("{cname} {fname} %zu\\n", offsetof({cname}, {fname}));')
    lines += ["return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run([gcc, "-std=c99", str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    got = {}
    for line in out:
        if line.strip():
            parts = line.split()
            got[(parts[0], parts[1])] = int(parts[2])
    for cname, cls in (("FaFwdParams", ext.FaFwdParams), ("FaBwdParams", ext.FaBwdParams),
                       ("FaBwdPlan", ext.FaBwdPlan), ("FaMaskParams", ext.FaMaskParams)):
        assert got[(cname, "size")] == ctypes.sizeof(cls), cname
        for fname, _ in cls._fields_:
            assert got[(cname, fname)] == getattr(cls, fname).offset, (cname, fname)


FAKE = 0x100000  # 16-byte aligned, never dereferenced: validation fails first


def fwd_params(**over):
    ext = _ext()
    p = ext.FaFwdParams()
    p.q = p.k = p.v = p.o = p.lse = FAKE
    p.q_stride_b, p.q_stride_t, p.q_stride_h = 8192 * 32 * 128, 32 * 128, 128
    p.k_stride_b, p.k_stride_t, p.k_stride_h = 8192 * 8 * 128, 8 * 128, 128
    p.v_stride_b, p.v_stride_t, p.v_stride_h = 8192 * 8 * 128, 8 * 128, 128
    p.o_stride_b, p.o_stride_t, p.o_stride_h = 8192 * 32 * 128, 32 * 128, 128
    p.batch, p.seqlen_q, p.seqlen_k, p.heads_q, p.heads_k, p.head_dim = 1, 8192, 8192, 32, 8, 128
    p.scale = 128 ** -0.5
    p.dtype = 0
    for k, v in over.items():
        setattr(p, k, v)
    return p


def bwd_params(**over):
    ext = _ext()
    p = ext.FaBwdParams()
    for n in ("q", "k", "v", "o", "dout", "lse", "delta", "dead_flags", "dq_accum", "dq", "dk", "dv"):
        setattr(p, n, FAKE)
    for pre, h in (("q", 32), ("o", 32), ("do", 32), ("dq", 32), ("k", 8), ("v", 8), ("dk", 8), ("dv", 8)):
        setattr(p, f"{pre}_stride_b", 8192 * h * 128)
        setattr(p, f"{pre}_stride_t", h * 128)
        setattr(p, f"{pre}_stride_h", 128)
    p.batch, p.seqlen_q, p.seqlen_k, p.heads_q, p.heads_k, p.head_dim = 1, 8192, 8192, 32, 8, 128
    p.scale = 128 ** -0.5
    p.atomic_dq = 1
    for k, v in over.items():
        setattr(p, k, v)
    return p


FWD_ERRORS = [
    (dict(head_dim=96), 3, "head_dim 96"),
    (dict(head_dim=192), 3, "head_dim 192"),
    (dict(head_dim=512), 3, "head_dim 512"),
    (dict(dtype=5), 4, "dtype"),
    (dict(heads_k=5), 2, "divisible"),
    (dict(batch=0), 2, "sizes must be"),
    (dict(seqlen_k=0), 2, "sizes must be"),
    (dict(scale=float("nan")), 6, "finite"),
    (dict(scale=float("inf")), 6, "finite"),
    (dict(q=FAKE + 8), 5, "not 16-byte aligned"),
    (dict(k_stride_t=8 * 128 + 4), 5, "multiples of 8"),
    (dict(v=None), 1, "v is NULL"),
    (dict(lse=None), 1, "lse is NULL"),
    (dict(mask=FAKE, mask_stride_q=-1), 5, "non-negative"),
    (dict(score=FAKE, score_stride_h=-4), 5, "non-negative"),
    (dict(score=FAKE, score_stride_q=1 << 26), 5, "32 score rows"),
    (dict(mask=FAKE), 8, "prepared workspace"),
    (dict(mask=FAKE, mask_ws=FAKE + 16), 5, "mask_ws must be 256-byte aligned"),
    # rows of every head below 2^31 - 2^16 (a tile round-up must not overflow)
    (dict(heads_q=8, heads_k=8, seqlen_k=(1 << 28) - 64), 2, "32-bit row indices"),
    (dict(heads_q=8, heads_k=8, seqlen_q=(1 << 28) - 64), 2, "32-bit row indices"),
]


@pytest.mark.parametrize("over,code,msg", FWD_ERRORS, ids=[e[2] for e in FWD_ERRORS])
def test_fwd_validation(lib, over, code, msg):
    assert lib.fa_fwd(ctypes.byref(fwd_params(**over))) == code
    assert msg in lib.fa_last_error().decode()


def test_null_params(lib):
    assert lib.fa_fwd(None) == 1
    assert lib.fa_bwd(None) == 1
    assert lib.fa_bwd_preprocess(None) == 1
    assert lib.fa_bwd_finalize(None) == 1
    assert lib.fa_bwd_plan(None, None) == 1
    assert lib.fa_mask_plan(None, None) == 1
    assert lib.fa_mask_prepare(None) == 1
    assert lib.fa_bwd_noalloc(None) == 1


NOALLOC_ERRORS = [
    (dict(seqlen_q=1 << 21), 8, "device scratch"),        # 2^26 rows: 512 MiB of Delta/LSE > 16 MiB
    (dict(q=None), 1, "q is NULL"),
    (dict(dq=None), 1, "dq is NULL"),
    (dict(head_dim=32), 3, "head_dim 32"),
    (dict(mask=FAKE), 8, "prepared workspace"),
    (dict(score=FAKE, score_stride_q=1 << 26), 5, "32 score rows"),
]


@pytest.mark.parametrize("over,code,msg", NOALLOC_ERRORS, ids=[e[2] for e in NOALLOC_ERRORS])
def test_noalloc_validation(lib, over, code, msg):
    """The allocation-free backward rejects what it cannot run before any HIP
    call; it needs none of the workspaces (they are NULL here)."""
    over = dict(dict(delta=None, dead_flags=None, dq_accum=None, ds_tiles=None), **over)
    assert lib.fa_bwd_noalloc(ctypes.byref(bwd_params(**over))) == code
    assert msg in lib.fa_last_error().decode()


BWD_ERRORS = [
    (dict(dq_accum=None, seqlen_q=2048, seqlen_k=2048, heads_q=16, heads_k=2), 8, "needs dq_accum"),   # dq_split 8
    (dict(dq_accum=None, seqlen_q=1024, seqlen_k=1024, heads_q=16, heads_k=2), 8, "needs dq_accum"),
    (dict(kv_split=3), 2, "must divide"),
    (dict(kv_split=2), 8, "needs dk_accum"),
    (dict(dout=None), 1, "dout is NULL"),
    (dict(delta=None), 1, "delta is NULL"),
    (dict(dead_flags=None), 1, "dead_flags is NULL"),
    (dict(dk_stride_h=100), 5, "multiples of 8"),
    (dict(score=FAKE, score_stride_q=1 << 26), 5, "32 score rows"),
    (dict(head_dim=32), 3, "head_dim 32"),
    (dict(mask=FAKE, ds_tiles=FAKE, ds_tiles_elems=1 << 40), 8, "prepared workspace"),
    (dict(ds_tiles=None), 8, "needs ds_tiles"),
    (dict(ds_tiles=FAKE, ds_tiles_elems=1024), 8, "the plan needs"),
    # a workspace sized by a plan made without the mask: half the tile pairs
    (dict(mask=FAKE, mask_ws=FAKE, ds_tiles=FAKE, ds_tiles_elems=32 * 256 * 256 * 1024, ds_limit_bytes=8 << 30), 8,
     "pair of tiles"),
]


@pytest.mark.parametrize("over,code,msg", BWD_ERRORS, ids=[e[2] for e in BWD_ERRORS])
@pytest.mark.parametrize("entry", ["fa_bwd_preprocess", "fa_bwd", "fa_bwd_finalize"])
def test_bwd_validation(lib, entry, over, code, msg):
    assert getattr(lib, entry)(ctypes.byref(bwd_params(**over))) == code
    assert msg in lib.fa_last_error().decode()


def _plan(lib, **over):
    ext = _ext()
    plan = ext.FaBwdPlan()
    assert lib.fa_bwd_plan(ctypes.byref(bwd_params(**over)), ctypes.byref(plan)) == 0
    return plan


def test_plan_headline_needs_no_split(lib):
    # atomic mode at the headline: 1024 dQ row blocks (>= one per CU) each
    # own their rows, so no fp32 accumulator; without a dS workspace dQ is
    # recomputed in both modes, no accumulator either
    plan = _plan(lib)
    assert plan.kv_split == 1 and plan.needs_dq_accum == 0 and plan.dq_split == 1
    assert plan.dq_accum_elems == 0 and plan.dkv_accum_elems == 0
    plan = _plan(lib, ds_limit_bytes=-1)
    assert plan.needs_dq_accum == 0 and plan.dq_accum_elems == 0 and plan.ds_elems == 0
    plan = _plan(lib, atomic_dq=0)
    assert plan.needs_dq_accum == 0 and plan.dq_accum_elems == 0


def test_plan_ds_tiles(lib):
    # causal 8192 x 8192: 256 query steps x 256 key steps, lower triangle with
    # the diagonal = 256 * 257 / 2 tiles of 32 x 32 per head
    # both modes hand dS over when it fits (the default limit, 4 GiB, holds the
    # headline's 4 GiB exactly); the atomic one splits the key
    # range (fp32 atomics) only below one 256-row block per CU: 2 x 8 heads x
    # 8 blocks = 128 -> 8 ranges (1024 workgroups)
    plan = _plan(lib)
    assert plan.ds_elems == 32 * 256 * 256 * 1024 and plan.dq_split == 1
    small = dict(seqlen_q=2048, seqlen_k=2048, heads_q=16, heads_k=2)
    plan = _plan(lib, **small)
    assert plan.dq_split == 8 and plan.needs_dq_accum == 1 and plan.dq_accum_elems == 2048 * 16 * 128
    assert _plan(lib, atomic_dq=0, **small).dq_split == 1
    assert _plan(lib, atomic_dq=0).dq_split == 1
    # ... and recomputes dQ when it does not
    plan = _plan(lib, ds_limit_bytes=-1)
    assert plan.ds_elems == 0 and plan.dq_split == 1
    plan = _plan(lib, atomic_dq=0, is_causal=1)
    assert plan.ds_elems == 32 * (256 * 257 // 2) * 1024
    plan = _plan(lib, atomic_dq=0)
    assert plan.ds_elems == 32 * 256 * 256 * 1024
    # ragged causal, Tq > Tk: steps past the last key step keep nk32 tiles
    plan = _plan(lib, atomic_dq=0, is_causal=1, seqlen_q=333, seqlen_k=130, heads_q=4, heads_k=2)
    nq, nk = 11, 5
    assert plan.ds_elems == 4 * (nk * (nk + 1) // 2 + (nq - nk) * nk) * 1024
    # caller limits below the need: the workspace holds as many (batch,
    # kv-head) units (the group's 4 planes, 512 MiB here) as fit, and the dS
    # kernels run slice by slice; below one unit, or none at all -> dQ
    # recomputed
    unit = 4 * 256 * 256 * 1024
    assert _plan(lib, atomic_dq=0, ds_limit_bytes=1 << 29).ds_elems == unit
    assert _plan(lib, atomic_dq=0, ds_limit_bytes=1 << 30).ds_elems == 2 * unit
    # 5 units would fit: 8 units run as 2 slices of 4 (balanced)
    assert _plan(lib, atomic_dq=0, ds_limit_bytes=(3 << 30) - 1).ds_elems == 4 * unit
    assert _plan(lib, ds_limit_bytes=1 << 29).ds_elems == unit   # atomic mode slices too
    # below one unit: ranges of query rows over every unit (next test); below
    # one 512-row range of them, or none at all -> dQ recomputed
    assert _plan(lib, atomic_dq=0, ds_limit_bytes=(1 << 28) - 2).ds_elems == 0
    assert _plan(lib, atomic_dq=0, is_causal=1, ds_limit_bytes=-1).ds_elems == 0
    assert _plan(lib, atomic_dq=0, is_causal=1, ds_limit_bytes=3 << 30).ds_elems > 0
    # with a mask or a score every stored block is a pair of tiles (dS and
    # its rounding residual): twice the elements, and slices of half the units
    for side in (dict(mask=FAKE), dict(score=FAKE), dict(mask=FAKE, score=FAKE)):
        assert _plan(lib, ds_limit_bytes=8 << 30, **side).ds_elems == 2 * 32 * 256 * 256 * 1024
        assert _plan(lib, atomic_dq=0, ds_limit_bytes=1 << 30, **side).ds_elems == 2 * unit
        # the default 4 GiB holds half of them: two slices of four units
        assert _plan(lib, **side).ds_elems == 4 * 2 * unit


def test_plan_row_ranges(lib):
    """Without a mask, a limit below one (batch, kv-head) unit's tiles runs
    the dS kernels over ranges of query rows, every unit in each launch:
    512-row chunks (16 steps), as few ranges as the limit allows, balanced;
    dQ written per range (no fp32 atomics, in atomic mode too).  Non-causal:
    head-group split 1, one fp32 sum each for dK and dV; causal: the group
    split of a sliced causal launch (1024 workgroups), one fp32 slab per part,
    summed by fa_bwd_finalize."""
    chunk = 32 * 16 * 256 * 1024   # tiles of 512 rows x 8192 keys over the 32 heads (256 MiB)
    for atomic in (0, 1):
        plan = _plan(lib, atomic_dq=atomic, ds_limit_bytes=(1 << 29) - 2)   # 1 chunk fits: 16 ranges
        assert plan.ds_elems == chunk and plan.kv_split == 1 and plan.dq_split == 1
        assert plan.needs_dq_accum == 0 and plan.dq_accum_elems == 0
        assert plan.dkv_accum_elems == 8192 * 8 * 128 and plan.dkv_accum_zeroed == 0
    # MQA (Hk 1: one unit is all 16 chunks): 9 chunks fit, two ranges of 8 (not 9 + 7)
    assert _plan(lib, atomic_dq=0, heads_k=1, ds_limit_bytes=9 * chunk * 2).ds_elems == 8 * chunk
    # causal (one unit: 269 MB; the last 512-row chunk of every head: 260 MB):
    # ranges balanced by tile count (later rows hold more tiles), the largest
    # within the limit; below the last chunk, dQ recomputed
    for limit in (1 << 28, 265_000_000):
        plan = _plan(lib, atomic_dq=0, is_causal=1, ds_limit_bytes=limit)
        assert 0 < 2 * plan.ds_elems <= limit and plan.kv_split == 2, limit
        assert plan.dkv_accum_elems == 2 * 8192 * 8 * 128 and plan.dkv_accum_zeroed == 0, limit
    assert _plan(lib, atomic_dq=0, is_causal=1, ds_limit_bytes=250_000_000).ds_elems == 0
    # causal problems take ranges whenever they slice at all (unit slices would
    # split each head group through fp32 slabs): 2.2 GB of tiles under 1 GiB
    for atomic in (0, 1):
        plan = _plan(lib, atomic_dq=atomic, is_causal=1, ds_limit_bytes=1 << 30)
        assert 0 < 2 * plan.ds_elems <= 1 << 30 and plan.kv_split == 2 and plan.dq_split == 1
        assert plan.dkv_accum_elems == 2 * 8192 * 8 * 128
    # ... but not when every tile fits (the headline's causal 2.2 GB under the default)
    plan = _plan(lib, atomic_dq=0, is_causal=1)
    assert plan.ds_elems == 32 * (256 * 257 // 2) * 1024 and plan.dkv_accum_elems == 0
    # T 32768 under the default 4 GiB: one unit is 8 GiB, 4 chunks of 1 GiB fit
    long = dict(seqlen_q=32768, seqlen_k=32768)
    plan = _plan(lib, atomic_dq=0, **long)
    assert plan.ds_elems == 4 * 32 * 16 * 1024 * 1024 and plan.kv_split == 1
    # with a mask, below one unit: parts of the head group (next test)
    assert _plan(lib, atomic_dq=0, ds_limit_bytes=(1 << 29) - 2, mask=FAKE).kv_split == 4
    # the row ranges need the fp32 sums; a caller's split gives one slab per part
    p = bwd_params(atomic_dq=0, ds_limit_bytes=(1 << 29) - 2, ds_tiles=FAKE, ds_tiles_elems=chunk)
    assert lib.fa_bwd(ctypes.byref(p)) == 8
    assert "needs dk_accum and dv_accum" in lib.fa_last_error().decode()
    plan = _plan(lib, atomic_dq=0, ds_limit_bytes=(1 << 29) - 2, kv_split=4)
    assert plan.kv_split == 4 and plan.dkv_accum_elems == 4 * 8192 * 8 * 128 and plan.ds_elems == chunk


def test_plan_head_group_parts(lib):
    """With a mask, a limit below one (batch, kv-head) unit's tiles (the
    group's planes, pairs of tiles with a mask) splits the head group into
    one-head parts (or the caller's split), each slice as many parts of one
    unit as fit, balanced; one fp32 slab per part (fully written), dQ written
    per launch."""
    plane = 256 * 256 * 1024 * 2          # one head's tile pairs at T 8192 (256 MiB of elements x 2 B)
    for atomic in (0, 1):
        # 1 GiB per unit: 600 MiB holds two planes -> split 4, two parts per slice
        plan = _plan(lib, atomic_dq=atomic, mask=FAKE, ds_limit_bytes=600 << 20)
        assert plan.kv_split == 4 and plan.ds_elems == 2 * plane and plan.dq_split == 1
        assert plan.needs_dq_accum == 0 and plan.dkv_accum_elems == 4 * 8192 * 8 * 128
        assert plan.dkv_accum_zeroed == 0
    # 300 MiB: one plane -> split 4
    plan = _plan(lib, atomic_dq=0, mask=FAKE, ds_limit_bytes=300 << 20)
    assert plan.kv_split == 4 and plan.ds_elems == plane and plan.dkv_accum_elems == 4 * 8192 * 8 * 128
    # below one plane: dQ recomputed
    assert _plan(lib, atomic_dq=0, mask=FAKE, ds_limit_bytes=200 << 20).ds_elems == 0
    # mask and score at T 20000 under the default 4 GiB: a unit's four planes
    # take 6.4 GB, two of them 3.2 GB -> split 4, two parts per slice
    big = dict(seqlen_q=20000, seqlen_k=20000, mask=FAKE, score=FAKE)
    plan = _plan(lib, atomic_dq=0, **big)
    assert plan.kv_split == 4 and plan.ds_elems == 2 * 625 * 625 * 1024 * 2
    # the caller's split is kept when a part fits, refused (dQ recomputed) when not
    plan = _plan(lib, atomic_dq=0, mask=FAKE, ds_limit_bytes=600 << 20, kv_split=2)
    assert plan.kv_split == 2 and plan.ds_elems == 2 * plane
    assert _plan(lib, atomic_dq=0, mask=FAKE, ds_limit_bytes=300 << 20, kv_split=2).ds_elems == 0


def test_det_path_needs_ds_tiles(lib):
    p = bwd_params(atomic_dq=0)
    assert lib.fa_bwd(ctypes.byref(p)) == 8
    assert "needs ds_tiles" in lib.fa_last_error().decode()
    p = bwd_params(atomic_dq=0, ds_tiles=FAKE + 8, ds_tiles_elems=1 << 40)
    assert lib.fa_bwd(ctypes.byref(p)) == 5
    assert "ds_tiles must be 16-byte aligned" in lib.fa_last_error().decode()


def test_plan_mqa_splits_the_group(lib):
    # BASELINE config M: B1 Tq2048 Tk16384 Hq32 Hk1 D64 -> 128 key tiles; split 4 -> 512 workgroups
    m = dict(seqlen_q=2048, seqlen_k=16384, heads_q=32, heads_k=1, head_dim=64)
    for atomic in (0, 1):   # pipelined dK/dV kernel: one slab per split, no zeroing
        plan = _plan(lib, atomic_dq=atomic, **m)
        assert plan.kv_split == 4 and plan.dkv_accum_elems == 4 * 16384 * 64 and plan.dkv_accum_zeroed == 0
    assert _plan(lib, **m).dq_split == 1   # 256 dQ row blocks: one per CU, rows owned, no atomics
    # no dS workspace (dQ recomputed): the same split and slabs, nothing to zero
    plan = _plan(lib, ds_limit_bytes=-1, **m)
    assert plan.kv_split == 4 and plan.dkv_accum_elems == 4 * 16384 * 64 and plan.dkv_accum_zeroed == 0
    plan = _plan(lib, kv_split=8, **m)
    assert plan.kv_split == 8


def test_plan_head_dim_256_recomputes_dq(lib):
    # head dim 256: dQ recomputed in both modes (no dS tiles, no fp32 dQ
    # atomics); dK/dV over 128-key blocks, the group split while a launch has
    # fewer than 512 workgroups (fp32 slabs, fully overwritten)
    w = dict(seqlen_q=4096, seqlen_k=4096, heads_q=32, heads_k=8, head_dim=256)
    for atomic in (0, 1):
        for limit in (0, -1, 8 << 30):
            plan = _plan(lib, atomic_dq=atomic, ds_limit_bytes=limit, **w)
            assert plan.ds_elems == 0 and plan.needs_dq_accum == 0 and plan.dq_accum_elems == 0, (atomic, limit)
            assert plan.dq_split == 1 and plan.kv_split == 2 and plan.dkv_accum_zeroed == 0
            assert plan.dkv_accum_elems == 2 * 4096 * 8 * 256
    plan = _plan(lib, atomic_dq=1, seqlen_q=8192, seqlen_k=8192, heads_q=8, heads_k=8, head_dim=256)
    assert plan.kv_split == 1 and plan.dkv_accum_elems == 0


def test_plans_of_shapes_past_any_device(lib):
    """Shapes just inside the row bound, whose dS tiles (2^62 bytes and more)
    no device holds, still plan with defined arithmetic (the size products
    saturate instead of overflowing): the recompute route under the default
    and a negative limit; under a limit beyond any device (clamped to 2^58
    bytes) a workspace within that clamp."""
    big = dict(batch=1, heads_q=2, heads_k=1, seqlen_q=(1 << 30) - (1 << 16), seqlen_k=(1 << 31) - (1 << 17))
    for causal in (0, 1):
        for atomic in (0, 1):
            for limit in (0, -1, 1 << 62):
                plan = _plan(lib, is_causal=causal, atomic_dq=atomic, ds_limit_bytes=limit, **big)
                if limit <= 0:
                    assert plan.ds_elems == 0, (causal, atomic, limit)
                else:
                    assert 0 <= 2 * plan.ds_elems <= 1 << 58, (causal, atomic, plan.ds_elems)
                assert plan.dq_accum_elems >= 0 and plan.dkv_accum_elems >= 0 and plan.kv_split >= 1


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(RuntimeError, match="not built"):
        _ext().load_library(tmp_path / "nope.so")


def test_library_path_override(tmp_path):
    """FA2_4D_MASK_LIB names the build to load; a missing one raises, with no
    fallback to the in-tree library (checked in a fresh interpreter, since the
    path is read at import)."""
    import os
    import sys
    pkg = Path(__file__).resolve().parents[1] / "fa2-with-4d-mask_amd"
    code = ("import sys; sys.path.insert(0, %r)\n"
            "from tilelang_fa2_4d_mask import _ext\n"
            "print(_ext.LIB_PATH)\n"
            "try:\n    _ext.load_library()\nexcept RuntimeError as e:\n    print('raised', 'not built' in str(e))\n") % str(pkg)
    env = dict(os.environ, FA2_4D_MASK_LIB=str(tmp_path / "other.so"))
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    lines = r.stdout.strip().splitlines()
    assert lines[-2] == str(tmp_path / "other.so") and lines[-1] == "raised True", r.stdout


def mask_params(**over):
    ext = _ext()
    p = ext.FaMaskParams()
    p.mask = FAKE
    p.mask_stride_b, p.mask_stride_h, p.mask_stride_q = 0, 0, 4096
    p.batch, p.seqlen_q, p.seqlen_k, p.heads_q = 2, 4096, 4096, 32
    for k, v in over.items():
        setattr(p, k, v)
    return p


def _mask_bytes(lib, **over):
    n = ctypes.c_int64(-1)
    assert lib.fa_mask_plan(ctypes.byref(mask_params(**over)), ctypes.byref(n)) == 0
    return n.value


def _a256(x):
    return (x + 255) // 256 * 256


def test_mask_plan_sizes(lib):
    # config P: mask [2, 1, 4096, 4096] -> batch kept (stride != 0), heads broadcast: 2 planes
    T = 4096
    per = dict(bits=T * 128 * 4, bitsT=128 * 128 * 32 * 4, blk=128 * 128, lfwd=16 * 65 * 4, lkv=32 * 129 * 4,
               ldq=16 * 129 * 4, ord=(16 + 32 + 16) * 4, hist=(65 + 129 + 129) * 4)
    off = 0
    for k in ("bits", "bitsT", "blk", "lfwd", "lkv", "ldq", "ord", "hist"):
        off = _a256(off + 2 * per[k])
    assert _mask_bytes(lib, mask_stride_b=T * T) == off
    # broadcast over batch too: one plane; full head extent: 64 planes
    assert _mask_bytes(lib) < _mask_bytes(lib, mask_stride_b=T * T)
    assert _mask_bytes(lib, mask_stride_b=32 * T * T, mask_stride_h=T * T) > 30 * _mask_bytes(lib, mask_stride_b=T * T)
    # ragged sizes: words padded to 16 bytes per row
    n = _mask_bytes(lib, batch=1, seqlen_q=33, seqlen_k=65, heads_q=1)
    bits = 33 * 4 * 4          # nk32 = 3 -> wk = 4
    bitsT = _a256(bits) + 3 * 4 * 32 * 4   # nk32 = 3 key blocks x wq = 4 words x 32 keys
    assert n >= bitsT


MASK_ERRORS = [
    (dict(batch=0), 2, "sizes must be"),
    (dict(seqlen_k=0), 2, "sizes must be"),
    (dict(mask=None), 1, "mask is NULL"),
    (dict(mask_stride_q=-1), 5, "non-negative"),
]


@pytest.mark.parametrize("over,code,msg", MASK_ERRORS, ids=[e[2] for e in MASK_ERRORS])
def test_mask_validation(lib, over, code, msg):
    n = ctypes.c_int64(0)
    assert lib.fa_mask_plan(ctypes.byref(mask_params(**over)), ctypes.byref(n)) == code
    assert msg in lib.fa_last_error().decode()
    assert lib.fa_mask_prepare(ctypes.byref(mask_params(**over))) == code


def test_mask_prepare_needs_aligned_workspace(lib):
    assert lib.fa_mask_prepare(ctypes.byref(mask_params())) == 8
    assert "workspace is NULL" in lib.fa_last_error().decode()
    assert lib.fa_mask_prepare(ctypes.byref(mask_params(workspace=FAKE + 64))) == 5
    assert "256-byte aligned" in lib.fa_last_error().decode()


def test_mask_plan_beyond_one_grid_dimension(lib):
    """The preparation walks planes and 32-row blocks with grid strides: more
    than 65535 of either plans (and prepares) like any other mask; planes
    that overflow 32-bit plane indices are refused."""
    # 70000 batches of a per-batch mask [70000, 1, 64, 64]: 70000 planes
    n = _mask_bytes(lib, batch=70000, heads_q=1, seqlen_q=64, seqlen_k=64, mask_stride_b=64 * 64, mask_stride_q=64)
    one = _mask_bytes(lib, batch=1, heads_q=1, seqlen_q=64, seqlen_k=64, mask_stride_b=64 * 64, mask_stride_q=64)
    assert n > 60000 * one // 2
    # 2^21 + 64 query rows: 65538 row blocks of 32
    assert _mask_bytes(lib, batch=1, heads_q=1, seqlen_q=(1 << 21) + 64, seqlen_k=64, mask_stride_q=64) > 0
    # 2^16 batches x 2^15 heads, per-head mask: 2^31 planes
    nb = ctypes.c_int64(0)
    p = mask_params(batch=1 << 16, heads_q=1 << 15, seqlen_q=32, seqlen_k=32, mask_stride_b=(1 << 15) * 1024,
                    mask_stride_h=1024, mask_stride_q=32)
    assert lib.fa_mask_plan(ctypes.byref(p), ctypes.byref(nb)) == 2
    assert "32-bit plane indices" in lib.fa_last_error().decode()
