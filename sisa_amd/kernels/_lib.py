"""ctypes binding of ``libsisa_hip.so`` (the C ABI declared in ``include/sisa_hip.h``).

The library is built in-tree by :func:`sisa_amd.build.build` (``hipcc --offload-arch=gfx950``). Loading fails loudly:
there is no CPU or Python fallback behind these functions. Tensors cross the boundary as raw device pointers plus
element strides; every launch goes on the current HIP stream of the tensors' device (torch's ``cuda`` device type is
the HIP device on ROCm builds).
"""
from __future__ import annotations

import ctypes
import os
import threading
from ctypes import POINTER, Structure, c_char_p, c_float, c_int, c_int32, c_int64, c_void_p

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "libsisa_hip.so")
ABI_VERSION = 4

F32, BF16, F16, F64 = 0, 1, 2, 3
_DTYPES = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16, torch.float64: F64}


class View(Structure):
    _fields_ = [("ptr", c_void_p), ("sb", c_int64), ("sh", c_int64), ("sl", c_int64)]


class FactorsArgs(Structure):
    _fields_ = [("B", c_int32), ("H", c_int32), ("L", c_int32), ("g", View), ("rowf", c_void_p),
                ("colf", c_void_p), ("mono", c_void_p)]


class AttnFwdArgs(Structure):
    _fields_ = [("B", c_int32), ("H", c_int32), ("L", c_int32), ("dtype", c_int32),
                ("q", View), ("k", View), ("v", View), ("c", View), ("b", View), ("g", View), ("f", View),
                ("lam", c_void_p), ("s_lam", c_int64), ("rowf", c_void_p), ("colf", c_void_p),
                ("o", View), ("lse", c_void_p), ("o32", c_void_p)]


class AttnBwdArgs(Structure):
    _fields_ = [("B", c_int32), ("H", c_int32), ("L", c_int32), ("dtype", c_int32), ("dcb_dtype", c_int32),
                ("q", View), ("k", View), ("v", View), ("c", View), ("b", View), ("g", View), ("f", View),
                ("lam", c_void_p), ("s_lam", c_int64), ("rowf", c_void_p), ("colf", c_void_p),
                ("o", View), ("o32", c_void_p), ("lse", c_void_p), ("dout", View),
                ("dq", View), ("dk", View), ("dv", View), ("dc", View), ("db", View),
                ("dg", c_void_p), ("df", c_void_p), ("dlam", c_void_p), ("workspace", c_void_p),
                ("exact", c_int32)]


class PrepFwdArgs(Structure):
    _fields_ = [("B", c_int32), ("L", c_int32), ("H", c_int32), ("dtype", c_int32),
                ("proj", c_void_p), ("s_pb", c_int64), ("s_pl", c_int64),
                ("z", c_void_p), ("s_zb", c_int64), ("s_zl", c_int64),
                ("cr", c_void_p), ("br", c_void_p), ("g", c_void_p), ("f", c_void_p), ("rowf", c_void_p),
                ("colf", c_void_p), ("tot", c_void_p)]


class PrepBwdArgs(Structure):
    _fields_ = [("B", c_int32), ("L", c_int32), ("H", c_int32), ("dtype", c_int32),
                ("proj", c_void_p), ("s_pb", c_int64), ("s_pl", c_int64),
                ("z", c_void_p), ("s_zb", c_int64), ("s_zl", c_int64),
                ("tot", c_void_p), ("dg", c_void_p), ("df", c_void_p), ("dcr", c_void_p), ("dbr", c_void_p),
                ("dproj", c_void_p), ("s_db", c_int64), ("s_dl", c_int64),
                ("dz", c_void_p), ("s_dzb", c_int64), ("s_dzl", c_int64), ("workspace", c_void_p)]


class LmceRowsArgs(Structure):
    _fields_ = [("T", c_int64), ("V", c_int64), ("Vp", c_int64), ("stride", c_int64), ("dtype", c_int32),
                ("compute_grad", c_int32), ("logits", c_void_p), ("labels", c_void_p), ("ignore_index", c_int64),
                ("inv_n", c_void_p), ("gscale", c_float), ("loss_rows", c_void_p), ("lse", c_void_p)]


class RmsNormArgs(Structure):
    _fields_ = [("N", c_int64), ("D", c_int32), ("dtype", c_int32), ("eps", c_float),
                ("x", c_void_p), ("sx", c_int64), ("w", c_void_p), ("y", c_void_p), ("sy", c_int64),
                ("rstd", c_void_p), ("dy", c_void_p), ("sdy", c_int64), ("dx", c_void_p), ("sdx", c_int64),
                ("dw", c_void_p), ("dw_partial", c_void_p)]


class NormArgs(Structure):
    _fields_ = [("N", c_int64), ("D", c_int32), ("H", c_int32), ("xdtype", c_int32), ("ydtype", c_int32),
                ("eps", c_float), ("reserved", c_int32), ("x", c_void_p), ("sx", c_int64), ("w", c_void_p),
                ("wf", c_void_p), ("bf", c_void_p), ("y", c_void_p), ("sy", c_int64), ("rstd", c_void_p),
                ("z", c_void_p), ("dy", c_void_p), ("sdy", c_int64), ("dz", c_void_p), ("dx", c_void_p),
                ("sdx", c_int64), ("dw", c_void_p), ("dwf", c_void_p), ("dbf", c_void_p), ("workspace", c_void_p),
                ("res", c_void_p), ("sres", c_int64), ("h", c_void_p), ("sh", c_int64), ("dh", c_void_p),
                ("sdh", c_int64)]


class SwigluArgs(Structure):
    _fields_ = [("n", c_int64), ("dtype", c_int32), ("pairs", c_int32), ("a", c_void_p), ("b", c_void_p),
                ("h", c_void_p), ("dh", c_void_p), ("da", c_void_p), ("db", c_void_p)]


class WgradArgs(Structure):
    _fields_ = [("M", c_int64), ("N", c_int32), ("K", c_int32), ("dtype", c_int32), ("nsplit", c_int32),
                ("m_per_split", c_int64), ("a", c_void_p), ("lda", c_int64), ("b", c_void_p), ("ldb", c_int64),
                ("c", c_void_p), ("ldc", c_int64), ("workspace", c_void_p)]


class LmceFwdArgs(Structure):
    _fields_ = [("N", c_int64), ("V", c_int64), ("Vp", c_int64), ("D", c_int32), ("dtype", c_int32),
                ("x", c_void_p), ("ldx", c_int64), ("w", c_void_p), ("ldw", c_int64), ("labels", c_void_p),
                ("ignore_index", c_int64), ("lse", c_void_p), ("loss_rows", c_void_p), ("workspace", c_void_p)]


class DecodeArgs(Structure):
    _fields_ = [("B", c_int32), ("H", c_int32), ("M", c_int32), ("N", c_int32), ("dtype", c_int32),
                ("q_start", c_int32), ("q", View), ("k", View), ("v", View), ("c", View), ("b", View),
                ("gq", View), ("gk", View), ("fq", View), ("fk", View), ("lam", c_void_p), ("s_lam", c_int64),
                ("out", c_void_p), ("workspace", c_void_p)]


class LmceTrainArgs(Structure):
    _fields_ = [("N", c_int64), ("V", c_int64), ("Vp", c_int64), ("D", c_int32), ("dtype", c_int32),
                ("x", c_void_p), ("ldx", c_int64), ("w", c_void_p), ("ldw", c_int64), ("labels", c_void_p),
                ("ignore_index", c_int64), ("inv_n", c_void_p), ("gscale", c_float), ("loss_rows", c_void_p),
                ("lse", c_void_p), ("dx", c_void_p), ("lddx", c_int64), ("dw", c_void_p), ("lddw", c_int64),
                ("dw_accumulate", c_int32), ("dx_splits", c_int32), ("workspace", c_void_p)]


class Round16Args(Structure):
    _fields_ = [("n", c_int64), ("dtype", c_int32), ("x", c_void_p), ("y", c_void_p), ("back", c_void_p)]


# exported symbol -> (argument types, return type); the same list the header declares
SIGNATURES = {
    "sisa_abi_version": ([], c_int),
    "sisa_last_error": ([], c_char_p),
    "sisa_factors": ([POINTER(FactorsArgs), c_void_p], c_int),
    "sisa_attn_fwd": ([POINTER(AttnFwdArgs), c_void_p], c_int),
    "sisa_attn_bwd_workspace_bytes": ([c_int32, c_int32, c_int32], c_int64),
    "sisa_attn_bwd": ([POINTER(AttnBwdArgs), c_void_p], c_int),
    "sisa_attn_bwd_noalloc": ([POINTER(AttnBwdArgs), c_void_p], c_int),
    "sisa_lmce_fwd_workspace_bytes": ([c_int64, c_int64], c_int64),
    "sisa_lmce_fwd": ([POINTER(LmceFwdArgs), c_void_p], c_int),
    "sisa_lmce_train_workspace_bytes": ([c_int64, c_int64, c_int32, c_int32], c_int64),
    "sisa_lmce_train": ([POINTER(LmceTrainArgs), c_void_p], c_int),
    "sisa_prep_fwd": ([POINTER(PrepFwdArgs), c_void_p], c_int),
    "sisa_prep_bwd_workspace_bytes": ([c_int32, c_int32, c_int32], c_int64),
    "sisa_finite_sum": ([c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p], c_int),
    "sisa_prep_bwd": ([POINTER(PrepBwdArgs), c_void_p], c_int),
    "sisa_lmce_rows": ([POINTER(LmceRowsArgs), c_void_p], c_int),
    "sisa_rmsnorm_bwd_workspace_bytes": ([c_int64, c_int32], c_int64),
    "sisa_rmsnorm_fwd": ([POINTER(RmsNormArgs), c_void_p], c_int),
    "sisa_rmsnorm_bwd": ([POINTER(RmsNormArgs), c_void_p], c_int),
    "sisa_norm_bwd_workspace_bytes": ([c_int64, c_int32, c_int32], c_int64),
    "sisa_norm_fwd": ([POINTER(NormArgs), c_void_p], c_int),
    "sisa_norm_bwd": ([POINTER(NormArgs), c_void_p], c_int),
    "sisa_swiglu_fwd": ([POINTER(SwigluArgs), c_void_p], c_int),
    "sisa_swiglu_bwd": ([POINTER(SwigluArgs), c_void_p], c_int),
    "sisa_wgrad_splits": ([c_int64, c_int32, c_int32], c_int32),
    "sisa_wgrad_workspace_bytes": ([c_int64, c_int32, c_int32, c_int32], c_int64),
    "sisa_wgrad": ([POINTER(WgradArgs), c_void_p], c_int),
    "sisa_decode_workspace_bytes": ([c_int32, c_int32, c_int32, c_int32], c_int64),
    "sisa_decode_attn": ([POINTER(DecodeArgs), c_void_p], c_int),
    "sisa_round16": ([POINTER(Round16Args), c_void_p], c_int),
}

_LOCK = threading.Lock()
_LIB = None


def load() -> ctypes.CDLL:
    """Load ``libsisa_hip.so`` once. Raises ``RuntimeError`` when it is missing or incompatible."""
    global _LIB
    if _LIB is not None:
        return _LIB
    with _LOCK:
        if _LIB is not None:
            return _LIB
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"SISA HIP library not built: {LIB_PATH} is missing (run sisa_amd.build.build())")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (argtypes, restype) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = restype
        if lib.sisa_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH}: ABI version {lib.sisa_abi_version()} != {ABI_VERSION}")
        _LIB = lib
        return lib


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DTYPES[dt]
    except KeyError:
        raise TypeError(f"unsupported dtype {dt}") from None


def view(t: torch.Tensor | None) -> View:
    """(B,H,L,.) or (B,H,L) tensor -> View (pointer + batch/head/sequence strides). None -> null view."""
    if t is None:
        return View(None, 0, 0, 0)
    return View(t.data_ptr(), t.stride(0), t.stride(1), t.stride(2))


def ptr(t: torch.Tensor | None):
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def call(name: str, args, dev_tensor: torch.Tensor) -> None:
    lib = load()
    with torch.cuda.device(dev_tensor.device):
        rc = getattr(lib, name)(ctypes.byref(args), stream_of(dev_tensor))
    if rc != 0:
        msg = lib.sisa_last_error().decode(errors="replace")
        raise RuntimeError(f"{name} failed (code {rc}): {msg}")


def workspace_bytes(name: str, *dims: int) -> int:
    return int(getattr(load(), name)(*[int(d) for d in dims]))
