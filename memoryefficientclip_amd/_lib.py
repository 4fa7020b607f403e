"""ctypes binding of the C ABI declared in ``include/mec.h``.

The shared library is built in-tree (``memoryefficientclip_amd/lib/libmec.so``)
by ``memoryefficientclip_amd.build``.  There is no fallback: if the library is
missing or fails to load, every entry point raises.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libmec.so"

MEC_OK = 0
MEC_ERR_INVALID = -1
MEC_ERR_UNSUPPORTED = -2
MEC_ERR_HIP = -3

DTYPE_F32 = 0
DTYPE_BF16 = 1
DTYPE_F16 = 2
DTYPE_F32_BF16X3 = 3  # fp32 data, products as three bf16 MFMA terms
DTYPE_F32_BF16 = 4  # fp32 data, bf16 products
MODE_CLIP = 0
MODE_LIT = 1
FLAG_DETERMINISTIC = 0x100  # OR into the mode of mec_sumexp / mec_forward
FLAG_KEEP_EXP = 0x200  # OR into the mode of mec_forward and the matching backward
KEEP_EXP_MAX_N = 2048  # MEC_KEEP_EXP_MAX_N
SIDE_X = 1  # MEC_SIDE_X: the x side of the backward (acc_x, dx)
SIDE_Y = 2  # MEC_SIDE_Y: the y side (CLIP only)

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_f32 = ctypes.c_float

# name -> (restype, argtypes); mirrors include/mec.h one to one.
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "mec_last_error": (ctypes.c_char_p, []),
    "mec_version": (ctypes.c_char_p, []),
    "mec_workspace_floats": (_i64, [_i64]),
    "mec_workspace_floats_for": (_i64, [_i64, _i64, _int]),
    "mec_workspace_floats_mode": (_i64, [_i64, _i64, _int, _int]),
    "mec_keep_exp_supported": (_int, [_vp, _i64, _vp, _i64, _i64, _i64, _int]),
    "mec_grad_scratch_bytes": (_i64, [_i64, _i64, _int]),
    "mec_grad_scratch_bytes_for": (_i64, [_i64, _i64, _int, _int, _int]),
    "mec_backward_plan": (_int, [_i64, _i64, _int, _int, _int, _int, _vp]),
    "mec_grad_blocking": (_int, [_i64, _i64, _int, _vp, _vp]),
    "mec_prepass": (_int, [_vp, _i64, _vp, _i64, _i64, _i64, _int, _int, _vp, _vp]),
    "mec_sumexp": (_int, [_vp, _i64, _vp, _i64, _i64, _i64, _int, _int, _int, _f32, _vp, _vp]),
    "mec_finalize": (_int, [_i64, _int, _f32, _vp, _vp, _vp]),
    "mec_forward": (_int, [_vp, _i64, _vp, _i64, _i64, _i64, _int, _int, _int, _f32, _vp, _vp, _vp]),
    "mec_grad": (_int, [_vp, _i64, _vp, _i64, _i64, _i64, _int, _int, _int, _f32, _vp, _vp, _i64, _vp, _vp,
                        _vp]),
    "mec_grad_step": (_int, [_vp, _i64, _vp, _i64, _i64, _i64, _int, _int, _int, _f32, _vp, _i64, _vp, _i64,
                             _vp, _vp, _vp]),
    "mec_postpass": (_int, [_vp, _i64, _vp, _i64, _i64, _i64, _int, _int, _int, _f32, _vp, _vp, _vp, _vp, _vp,
                            _vp, _vp]),
    "mec_backward": (_int, [_vp, _i64, _vp, _i64, _i64, _i64, _int, _int, _int, _f32, _f32, _vp, _vp, _vp, _i64,
                            _vp, _vp, _vp, _vp, _vp]),
    "mec_backward_noalloc": (_int, [_vp, _i64, _vp, _i64, _i64, _i64, _int, _int, _int, _f32, _f32, _vp, _vp,
                                    _vp, _vp, _vp, _vp, _vp]),
}
NOALLOC_SCRATCH_BYTES = 256 << 20  # MEC_NOALLOC_SCRATCH_BYTES


class BackwardPlan(ctypes.Structure):
    """mec_backward_plan_t (include/mec.h)."""
    _fields_ = [("block_rows", ctypes.c_int64), ("num_blocks", ctypes.c_int64), ("scratch_bytes", ctypes.c_int64),
                ("noalloc_block_rows", ctypes.c_int64), ("noalloc_scratch_bytes", ctypes.c_int64),
                ("contract_tile_rows", ctypes.c_int32), ("contract_tile_features", ctypes.c_int32),
                ("narrow_tiles", ctypes.c_int32), ("reserved", ctypes.c_int32)]

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class MecError(RuntimeError):
    """A C-ABI call returned a non-zero status."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed ({code}): {msg}")
        self.code = code


def load(path: str | os.PathLike | None = None) -> ctypes.CDLL:
    """Load (once) and return the library with argtypes set."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = Path(path) if path is not None else LIB_PATH
        if not p.exists():
            raise RuntimeError(
                f"HIP library {p} is not built; run `python -m memoryefficientclip_amd.build` "
                "(or __graft_entry__.build()) first")
        lib = ctypes.CDLL(str(p))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if path is None:
            _lib = lib
        return lib


def grad_blocking(n: int, d: int, dtype: int) -> tuple[int, int]:
    """(block_rows, num_blocks) of the backward's block decomposition."""
    bs, nb = ctypes.c_int64(), ctypes.c_int64()
    call("mec_grad_blocking", n, d, dtype, ctypes.byref(bs), ctypes.byref(nb))
    return bs.value, nb.value


def backward_plan(n: int, d: int, dtype: int, mode: int = MODE_CLIP, sides: int = SIDE_X | SIDE_Y,
                  compute_units: int = 0) -> BackwardPlan:
    """The backward's plan (blocking, scratch, contraction tiles, what
    mec_backward_noalloc would use) for (n, d, dtype, mode, sides) on a device
    of `compute_units` CUs (0: the current device)."""
    plan = BackwardPlan()
    call("mec_backward_plan", n, d, dtype, mode, sides, compute_units, ctypes.byref(plan))
    return plan


def last_error() -> str:
    return load().mec_last_error().decode()


def call(name: str, *args) -> int:
    """Call an int-returning entry point, raising MecError on failure."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != MEC_OK:
        raise MecError(name, rc, lib.mec_last_error().decode())
    return rc
