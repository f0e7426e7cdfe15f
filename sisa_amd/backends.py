"""Which SISA attention implementation runs, and how the HIP paths check their inputs.

Implementations of one function (the reference's ``attn_impl`` values, src/sisa/backends.py:47, with its Triton
backends replaced by this build's HIP library):

* ``"torch"``: the exact blocked PyTorch path (:func:`sisa_amd.functional.sisa_attention_torch`), any device/dtype.
* ``"hip"``: projections etc. in torch, attention on the gfx950 kernels (:mod:`sisa_amd.kernels.attention`).
* ``"hip_fused"``: one projection GEMM, the HIP preparation kernels and the HIP attention kernels
  (:mod:`sisa_amd.kernels.fused_prep`).

Selection is a table lookup: every HIP implementation has a list of requirements (a GPU that loads the library, the
kernels' head/state sizes, a compute dtype from its set), and :func:`select_impl` collects the unmet ones. A forced
implementation with an unmet requirement raises ``ValueError`` naming all of them; ``"auto"`` takes the first HIP
implementation in preference order with none unmet, and otherwise the torch path, warning once per device and
reason when that happens on a GPU. Nothing falls back silently.
"""
from __future__ import annotations

import threading
import warnings
from functools import lru_cache
from typing import TYPE_CHECKING, Union

import torch

from .config import HIP_D_HEAD, HIP_D_STATE

if TYPE_CHECKING:  # pragma: no cover
    from .config import SISAConfig

DeviceLike = Union[torch.device, str, int]

__all__ = ["IMPLS", "CHECK_MODES", "hip_status", "fused_eligible", "set_check_mode", "get_check_mode", "describe",
           "select_impl", "device_info", "attention_config", "compute_dtype", "warn_fallback",
           "reset_fallback_warnings"]

IMPLS = ("auto", "torch", "hip", "hip_fused")
#: gfx targets the library is compiled for.
HIP_ARCHS = ("gfx950",)
#: Compute dtypes each HIP implementation takes, in the order "auto" tries the implementations.
_HIP_DTYPES: dict[str, tuple[torch.dtype, ...]] = {
    "hip_fused": (torch.bfloat16, torch.float16),
    "hip": (torch.bfloat16, torch.float16, torch.float32),
}

#: Check modes of the HIP paths and what each one does.
CHECK_MODES: dict[str, str] = {
    "async": "device-side asserts (torch._assert_async), no host synchronisation; a failed check poisons the HIP "
             "context and the next GPU call raises",
    "sync": "one host synchronisation per call; a failed check raises at once (ValueError for a decay g that "
            "increases, FloatingPointError for a non-finite score input of the fused layer)",
    "off": "no checks (for timing)",
}
_mode = ["async"]


# ------------------------------------------------------------------------------------------------------ check mode
def set_check_mode(mode: str) -> None:
    """Choose how the HIP paths validate inputs: one of :data:`CHECK_MODES` (default ``"async"``).

    What is checked: the unfused attention's ``g`` does not increase along the sequence (the fused layer builds it
    monotone), and the fused layer's score inputs (q, k, c, b, lambda, g, F) are finite. Same modes and meanings as
    the reference (src/sisa/backends.py:75-89).
    """
    if mode not in CHECK_MODES:
        raise ValueError(f"unknown check mode {mode!r}; choose one of: {', '.join(CHECK_MODES)}")
    _mode[0] = mode


def get_check_mode() -> str:
    """The check mode in force (a key of :data:`CHECK_MODES`)."""
    return _mode[0]


# ------------------------------------------------------------------------------------------------------ device facts
def _device_index(device: DeviceLike | None) -> int:
    if device is None:
        return torch.cuda.current_device()
    dev = torch.device(device)
    if dev.type != "cuda":
        raise ValueError(f"{dev} is not a GPU device")
    return torch.cuda.current_device() if dev.index is None else dev.index


@lru_cache(maxsize=None)
def _properties(index: int) -> tuple:
    p = torch.cuda.get_device_properties(index)
    arch = (getattr(p, "gcnArchName", "") or "").split(":")[0]
    return (("index", index), ("name", p.name), ("arch", arch), ("cu_count", int(p.multi_processor_count)),
            ("lds_per_block", int(getattr(p, "shared_memory_per_block", 0) or 0)),
            ("total_memory", int(p.total_memory)))


def device_info(device: DeviceLike | None = None) -> dict:
    """Name, gfx architecture, CU count, LDS per workgroup and memory of a GPU (default: the current one)."""
    return dict(_properties(_device_index(device)))


def attention_config(device: DeviceLike | None, dtype: torch.dtype) -> dict:
    """The attention kernels' fixed launch geometry (no autotuning) and the MFMA instruction used for ``dtype``.

    Forward and dq kernel: 8 waves x 16 query rows = 128 queries (two 64-row decay blocks) per workgroup; dkv
    kernel: 4 waves x 16 rows = one 64-row decay block of keys (dk, dv, db) per workgroup; the other operand streams
    through LDS in 64-position tiles; decay factors are anchored per 64-row block (``T``). The geometry does not
    depend on the device.
    """
    mfma = {torch.bfloat16: "v_mfma_f32_16x16x32_bf16", torch.float16: "v_mfma_f32_16x16x32_f16",
            torch.float32: "v_mfma_f32_16x16x4_f32"}.get(dtype)
    if mfma is None:
        raise ValueError(f"the attention kernels take bf16, fp16 or fp32 inputs, not {dtype}")
    return dict(T=64, tile=64, rows_per_wave=16, fwd_waves=8, fwd_rows_per_wg=128, dq_waves=8, dq_rows_per_wg=128,
                dkv_waves=4, dkv_rows_per_wg=64, mfma=mfma)


# ------------------------------------------------------------------------------------------------------ requirements
def hip_status(device: DeviceLike | None = None) -> tuple[bool, str]:
    """``(True, summary)`` if the HIP library runs on ``device`` (default: the current GPU), else ``(False, why)``.

    The counterpart of the reference's ``triton_status`` (src/sisa/backends.py:205-250): ROCm PyTorch, a visible
    gfx950 GPU, and ``libsisa_hip.so`` loading with the ABI version this package expects. Cached per device.
    """
    if not getattr(torch.version, "hip", None):
        return False, "this PyTorch is not a ROCm build"
    if not torch.cuda.is_available():
        return False, "PyTorch sees no GPU"
    if device is not None and torch.device(device).type != "cuda":
        return False, f"{torch.device(device)} is not a GPU device"
    return _status_of(_device_index(device))


_status_lock = threading.Lock()


@lru_cache(maxsize=None)
def _status_of(index: int) -> tuple[bool, str]:
    with _status_lock:      # one library load at a time
        info = device_info(index)
        if info["arch"] not in HIP_ARCHS:
            return False, f"{info['name']} is {info['arch'] or 'an unknown architecture'}; the library is built " \
                          f"for {', '.join(HIP_ARCHS)}"
        try:
            from .kernels import _lib
            _lib.load()
        except Exception as e:  # noqa: BLE001 - any load failure is the answer
            return False, f"libsisa_hip.so does not load ({type(e).__name__}: {e})"
        return True, f"{info['name']}: {info['arch']}, {info['cu_count']} CUs, libsisa_hip.so loaded"


def compute_dtype(x: torch.Tensor) -> torch.dtype:
    """The dtype a layer's matrix products see for input ``x``: autocast's dtype when autocast is on for ``x``'s
    device type, else ``x.dtype``."""
    kind = x.device.type
    if kind in ("cuda", "cpu") and torch.is_autocast_enabled(kind):
        return torch.get_autocast_dtype(kind)
    return x.dtype


def _unmet(impl: str, x: torch.Tensor, cfg: SISAConfig | None) -> list[str]:
    """The requirements of HIP implementation ``impl`` that layer input ``x`` and config ``cfg`` do not meet."""
    if not isinstance(x, torch.Tensor):
        return [f"the layer input is a {type(x).__name__}, not a tensor"]
    unmet = []
    if x.device.type != "cuda":
        unmet.append(f"the input is on the {x.device.type}, not a GPU")
    else:
        ok, why = hip_status(x.device)
        if not ok:
            unmet.append(why)
    if cfg is not None:
        d_head = cfg.d_model // cfg.n_head
        if (d_head, cfg.d_state) != (HIP_D_HEAD, HIP_D_STATE):
            unmet.append(f"the kernels are built for d_head {HIP_D_HEAD} and d_state {HIP_D_STATE}, this model has "
                         f"{d_head} and {cfg.d_state}")
    dt = compute_dtype(x)
    if dt not in _HIP_DTYPES[impl]:
        names = "/".join(str(d).replace("torch.", "") for d in _HIP_DTYPES[impl])
        hint = " (run under autocast or with low-precision parameters)" if impl == "hip_fused" else ""
        unmet.append(f"{impl} computes in {names}, the compute dtype here is {dt}{hint}")
    return unmet


def fused_eligible(x: torch.Tensor) -> bool:
    """Whether ``hip_fused`` can run for layer input ``x`` as far as device and dtype go (the head/state sizes are
    :func:`select_impl`'s part)."""
    return not _unmet("hip_fused", x, None)


_warned: set = set()


def warn_fallback(device: torch.device, reason: str) -> None:
    """Warn, once per (device, reason), that the torch attention path runs on a GPU in place of a HIP one."""
    key = (str(device), reason)
    if key not in _warned:
        _warned.add(key)
        warnings.warn(f"SISA: the torch attention implementation runs on {device}: {reason}", stacklevel=3)


def reset_fallback_warnings() -> None:
    """Forget which fallback warnings were given (tests use this to see them again)."""
    _warned.clear()


def select_impl(requested: str, x: torch.Tensor, cfg: SISAConfig | None) -> str:
    """The implementation that runs for ``requested`` (one of :data:`IMPLS`) on layer input ``x``.

    ``cfg`` supplies ``d_model``, ``n_head`` and ``d_state`` (``None`` skips the size requirement). ``"torch"`` is
    returned as is; a forced HIP implementation is returned if every requirement holds and raises ``ValueError``
    listing the unmet ones otherwise; ``"auto"`` takes ``hip_fused``, then ``hip``, then ``torch``.
    """
    if requested not in IMPLS:
        raise ValueError(f"unknown attn_impl {requested!r}; expected one of {IMPLS}")
    if requested == "torch":
        return "torch"
    if requested != "auto":
        unmet = _unmet(requested, x, cfg)
        if unmet:
            raise ValueError(f"attn_impl={requested!r} is not available: {'; '.join(unmet)}")
        return requested
    unmet = {}
    for impl in _HIP_DTYPES:
        unmet[impl] = _unmet(impl, x, cfg)
        if not unmet[impl]:
            return impl
    if isinstance(x, torch.Tensor) and x.device.type == "cuda":
        warn_fallback(x.device, "; ".join(unmet["hip"]))
    return "torch"


def describe() -> str:
    """A report of PyTorch, the check mode, and per GPU the HIP status and what ``attn_impl="auto"`` picks."""
    out = [f"torch {torch.__version__}, HIP {getattr(torch.version, 'hip', None)}",
           f"check mode {get_check_mode()!r}: {CHECK_MODES[get_check_mode()]}"]
    gpus = torch.cuda.device_count() if torch.cuda.is_available() else 0
    if not gpus:
        out.append("no GPU: attn_impl='auto' runs 'torch'")
    for i in range(gpus):
        ok, why = hip_status(i)
        out.append(f"cuda:{i}: {why}")
        out.append("  auto: 'hip_fused' for bf16/fp16 compute, 'hip' for fp32" if ok else "  auto: 'torch'")
    return "\n".join(out)
