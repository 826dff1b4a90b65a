"""ctypes binding of libfa2_4d_mask.so (the C ABI in include/fa2_4d_mask.h).

The library is loaded lazily on first use and must have been built in-tree
(``python fa2-with-4d-mask_amd/build_ext.py``).  There is no fallback: a
missing or unloadable library raises ``RuntimeError``.  The environment
variable ``FA2_4D_MASK_LIB`` names another build of the same library to load
instead (for instance the host-sanitized one that ``build_ext.py
--host-sanitize`` writes).

torch is imported before the library is loaded so that the library binds to
the HIP runtime torch already holds (same SONAME), which keeps torch's stream
handles and device pointers valid on both sides.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch  # noqa: F401  (must be loaded before the HIP library, see above)

LIB_PATH = (Path(os.environ["FA2_4D_MASK_LIB"]) if os.environ.get("FA2_4D_MASK_LIB")
            else Path(__file__).resolve().parent / "_lib" / "libfa2_4d_mask.so")
ABI_VERSION = 6

FA_DTYPE_BF16 = 0
FA_DTYPE_FP16 = 1

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32


def _fields(*groups):
    out = []
    for names, typ in groups:
        out += [(n, typ) for n in names.split()]
    return out


class FaFwdParams(ctypes.Structure):
    _fields_ = _fields(
        ("q k v o lse mask score", _vp),
        ("q_stride_b q_stride_t q_stride_h k_stride_b k_stride_t k_stride_h "
         "v_stride_b v_stride_t v_stride_h o_stride_b o_stride_t o_stride_h "
         "mask_stride_b mask_stride_h mask_stride_q score_stride_b score_stride_h score_stride_q", _i64),
        ("batch seqlen_q seqlen_k heads_q heads_k head_dim", _i32),
        ("scale", ctypes.c_float),
        ("is_causal dtype", _i32),
        ("stream mask_ws o_lo", _vp),
        ("o_lo_stride_b o_lo_stride_t o_lo_stride_h", _i64),
    )


class FaBwdParams(ctypes.Structure):
    _fields_ = _fields(
        ("q k v o dout lse delta dead_flags mask score dq_accum dk_accum dv_accum dq dk dv", _vp),
        ("q_stride_b q_stride_t q_stride_h k_stride_b k_stride_t k_stride_h "
         "v_stride_b v_stride_t v_stride_h o_stride_b o_stride_t o_stride_h "
         "do_stride_b do_stride_t do_stride_h dq_stride_b dq_stride_t dq_stride_h "
         "dk_stride_b dk_stride_t dk_stride_h dv_stride_b dv_stride_t dv_stride_h "
         "mask_stride_b mask_stride_h mask_stride_q score_stride_b score_stride_h score_stride_q", _i64),
        ("batch seqlen_q seqlen_k heads_q heads_k head_dim", _i32),
        ("scale", ctypes.c_float),
        ("is_causal atomic_dq kv_split dtype", _i32),
        ("stream ds_tiles", _vp),
        ("ds_limit_bytes", _i64),
        ("mask_ws o_lo", _vp),
        ("o_lo_stride_b o_lo_stride_t o_lo_stride_h ds_tiles_elems", _i64),
    )


class FaMaskParams(ctypes.Structure):
    _fields_ = _fields(
        ("mask", _vp),
        ("mask_stride_b mask_stride_h mask_stride_q", _i64),
        ("batch seqlen_q seqlen_k heads_q is_causal", _i32),
        ("workspace stream", _vp),
    )


class FaBwdPlan(ctypes.Structure):
    _fields_ = [
        ("kv_split", _i32),
        ("needs_dq_accum", _i32),
        ("dq_accum_elems", _i64),
        ("dkv_accum_elems", _i64),
        ("ds_elems", _i64),
        ("dkv_accum_zeroed", _i32),
        ("dq_split", _i32),
    ]


EXPORTED = ("fa_fwd", "fa_bwd_preprocess", "fa_bwd", "fa_bwd_finalize", "fa_bwd_plan", "fa_mask_plan",
            "fa_mask_prepare", "fa_last_error", "fa_abi_version", "fa_bwd_noalloc")

_lib = None
_lock = threading.Lock()


def load_library(path: os.PathLike | None = None) -> ctypes.CDLL:
    """Loads (once) and returns the library; raises RuntimeError if it is absent."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = Path(path) if path is not None else LIB_PATH
        if not p.exists():
            raise RuntimeError(
                f"{p} is not built: run `python fa2-with-4d-mask_amd/build_ext.py` "
                "(the HIP kernels are required; there is no fallback path)"
            )
        lib = ctypes.CDLL(str(p))
        lib.fa_fwd.argtypes = [ctypes.POINTER(FaFwdParams)]
        lib.fa_fwd.restype = ctypes.c_int
        lib.fa_bwd_preprocess.argtypes = [ctypes.POINTER(FaBwdParams)]
        lib.fa_bwd_preprocess.restype = ctypes.c_int
        lib.fa_bwd.argtypes = [ctypes.POINTER(FaBwdParams)]
        lib.fa_bwd.restype = ctypes.c_int
        lib.fa_bwd_finalize.argtypes = [ctypes.POINTER(FaBwdParams)]
        lib.fa_bwd_finalize.restype = ctypes.c_int
        lib.fa_bwd_noalloc.argtypes = [ctypes.POINTER(FaBwdParams)]
        lib.fa_bwd_noalloc.restype = ctypes.c_int
        lib.fa_bwd_plan.argtypes = [ctypes.POINTER(FaBwdParams), ctypes.POINTER(FaBwdPlan)]
        lib.fa_bwd_plan.restype = ctypes.c_int
        lib.fa_mask_plan.argtypes = [ctypes.POINTER(FaMaskParams), ctypes.POINTER(ctypes.c_int64)]
        lib.fa_mask_plan.restype = ctypes.c_int
        lib.fa_mask_prepare.argtypes = [ctypes.POINTER(FaMaskParams)]
        lib.fa_mask_prepare.restype = ctypes.c_int
        lib.fa_last_error.argtypes = []
        lib.fa_last_error.restype = ctypes.c_char_p
        lib.fa_abi_version.argtypes = []
        lib.fa_abi_version.restype = ctypes.c_int
        if lib.fa_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{p}: ABI version {lib.fa_abi_version()} != {ABI_VERSION}, rebuild it")
        if path is None:
            _lib = lib
        return lib


class FaError(RuntimeError):
    def __init__(self, code: int, where: str, msg: str):
        super().__init__(f"{where} failed with status {code}: {msg}")
        self.code = code


def check(status: int, where: str, lib: ctypes.CDLL | None = None) -> None:
    if status != 0:
        lib = lib or load_library()
        raise FaError(status, where, lib.fa_last_error().decode(errors="replace"))


def dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.bfloat16:
        return FA_DTYPE_BF16
    if dtype == torch.float16:
        return FA_DTYPE_FP16
    raise ValueError(f"unsupported dtype {dtype} (bf16 / fp16 only)")


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()
