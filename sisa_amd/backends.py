"""Backend selection, device checks, launch configuration and the runtime check mode.

SISA attention has three implementations of the same function:

* ``"torch"``: the exact blocked reference in plain PyTorch (:func:`sisa_amd.functional.sisa_attention_torch`).
  Works on any device and dtype.
* ``"hip"``: torch glue (projections, cumulative sums, rotation) plus the gfx950 HIP attention kernels
  (:func:`sisa_amd.kernels.attention.sisa_attention_hip`).
* ``"hip_fused"``: one projection GEMM, then the HIP preparation kernels plus the HIP attention kernels
  (:func:`sisa_amd.kernels.fused_prep.sisa_fused`).

``"auto"`` picks ``hip_fused`` when eligible, else ``hip``, else ``torch``. Forcing a HIP implementation on an input
it cannot handle raises ``ValueError``; nothing ever falls back silently. This mirrors the reference's
``sisa.backends`` (src/sisa/backends.py:1-20, 47, 284-336) with the Triton backends replaced by the HIP library.

HIP requirements: a ROCm build of PyTorch, an AMD Instinct MI355X-class GPU (gfx950; the kernels use
``v_mfma_f32_16x16x32_{bf16,f16}`` and ``v_cvt_pk_bf16_f32``), the in-tree library ``libsisa_hip.so``,
``d_head == 64`` and ``d_state == 32``. The fused path additionally needs a bf16/fp16 compute dtype.
"""
from __future__ import annotations

import threading
import warnings
from typing import TYPE_CHECKING, Union

import torch

if TYPE_CHECKING:  # pragma: no cover
    from .config import SISAConfig

DeviceLike = Union[torch.device, str, int]

__all__ = [
    "IMPLS",
    "hip_status",
    "fused_eligible",
    "set_check_mode",
    "get_check_mode",
    "describe",
    "select_impl",
    "device_info",
    "attention_config",
]

IMPLS = ("auto", "torch", "hip", "hip_fused")
SUPPORTED_ARCHS = ("gfx950",)

# Launch configuration of the attention kernels (fixed, no autotuning): the forward runs 128 queries per workgroup of
# 8 waves (16 query rows per wave), the backward kernels 64 queries (dq) or keys (dk/dv/db) per workgroup of 4 waves;
# 64-position tiles staged in LDS; decay factors over 64-row blocks (T).
_ATTN_CFG_ALL = dict(T=64, tile=64, rows_per_wave=16, fwd_rows_per_wg=128, fwd_waves=8, bwd_rows_per_wg=64,
                     bwd_waves=4)

_CHECK_MODES = ("async", "sync", "off")
_STATE = {"check": "async"}
_LOCK = threading.Lock()
_DEVICE_INFO: dict[int, dict] = {}
_HIP_STATUS: dict[int, tuple[bool, str]] = {}
_WARNED: set = set()


# ---------------------------------------------------------------------------------------------------- check mode
def set_check_mode(mode: str) -> None:
    """Set how the HIP paths check their inputs at run time.

    ``"async"`` (default): device-side asserts (``torch._assert_async``), no host synchronisation; a failed check
    stops the device context. ``"sync"``: the check synchronises once per call and raises a Python exception right
    away (``ValueError`` for a non-monotone decay ``g``, ``FloatingPointError`` for non-finite values in the fused
    layer). ``"off"``: no checks (benchmarks only). Semantics of the reference (src/sisa/backends.py:75-89).
    """
    if mode not in _CHECK_MODES:
        raise ValueError(f"check mode must be one of {_CHECK_MODES}, got {mode!r}")
    _STATE["check"] = mode


def get_check_mode() -> str:
    """The current check mode (``"async"``, ``"sync"`` or ``"off"``)."""
    return _STATE["check"]


# ---------------------------------------------------------------------------------------------------- device facts
def _cuda_index(device: DeviceLike | None = None) -> int:
    if device is None:
        return torch.cuda.current_device()
    dev = torch.device(device)
    if dev.type != "cuda":
        raise ValueError(f"not a HIP/CUDA device: {dev}")
    return dev.index if dev.index is not None else torch.cuda.current_device()


def device_info(device: DeviceLike | None = None) -> dict:
    """Facts about a GPU that the launch configuration depends on (cached per device)."""
    idx = _cuda_index(device)
    info = _DEVICE_INFO.get(idx)
    if info is not None:
        return dict(info)
    p = torch.cuda.get_device_properties(idx)
    arch = str(getattr(p, "gcnArchName", "") or "")
    info = dict(
        index=idx,
        name=p.name,
        arch=arch.split(":")[0],
        cu_count=int(p.multi_processor_count),
        lds_per_block=int(getattr(p, "shared_memory_per_block", 0) or 0),
        total_memory=int(p.total_memory),
    )
    _DEVICE_INFO[idx] = info
    return dict(info)


def attention_config(device: DeviceLike | None, dtype: torch.dtype) -> dict:
    """Launch configuration of the attention kernels (identical for every dtype; fp32 uses fp32 MFMA)."""
    if dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise ValueError(f"unsupported attention dtype {dtype}")
    cfg = dict(_ATTN_CFG_ALL)
    cfg["mfma"] = "v_mfma_f32_16x16x4_f32" if dtype == torch.float32 else "v_mfma_f32_16x16x32_" + (
        "bf16" if dtype == torch.bfloat16 else "f16")
    return cfg


# ---------------------------------------------------------------------------------------------------- eligibility
def hip_status(device: DeviceLike | None = None) -> tuple[bool, str]:
    """Whether the HIP kernels can run on ``device`` (default: the current GPU), with the reason.

    Returns ``(True, summary)`` or ``(False, why_not)``; cached per device. The counterpart of the reference's
    ``triton_status`` (src/sisa/backends.py:205-250).
    """
    if not getattr(torch.version, "hip", None):
        return False, "PyTorch is not a ROCm build"
    if not torch.cuda.is_available():
        return False, "no HIP device is available"
    if device is not None and torch.device(device).type != "cuda":
        return False, f"device {torch.device(device)} is not a GPU device"
    idx = _cuda_index(device)
    hit = _HIP_STATUS.get(idx)
    if hit is not None:
        return hit
    with _LOCK:
        hit = _HIP_STATUS.get(idx)
        if hit is not None:
            return hit
        res = _hip_status_uncached(idx)
        _HIP_STATUS[idx] = res
        return res


def _hip_status_uncached(idx: int) -> tuple[bool, str]:
    info = device_info(idx)
    if info["arch"] not in SUPPORTED_ARCHS:
        return False, f"{info['name']}: architecture {info['arch'] or '?'} is not gfx950"
    try:
        from .kernels import _lib
        _lib.load()
    except Exception as e:  # noqa: BLE001 - report any load failure as the reason
        return False, f"loading libsisa_hip.so failed: {type(e).__name__}: {e}"
    return True, f"HIP kernels on {info['name']} ({info['arch']}, {info['cu_count']} CUs)"


def _compute_dtype(x: torch.Tensor) -> torch.dtype:
    dt = x.device.type
    try:
        if torch.is_autocast_enabled(dt):
            return torch.get_autocast_dtype(dt)
    except (TypeError, RuntimeError):  # device types without autocast support
        pass
    return x.dtype


def fused_eligible(x: torch.Tensor) -> bool:
    """Whether the fused HIP layer path can run for layer input ``x`` (shape checks are done by select_impl)."""
    if not isinstance(x, torch.Tensor) or x.device.type != "cuda":
        return False
    if _compute_dtype(x) not in (torch.bfloat16, torch.float16):
        return False
    return hip_status(x.device)[0]


def _shape_problem(cfg) -> str | None:
    if cfg is None:
        return None
    d_model, n_head = int(cfg.d_model), int(cfg.n_head)
    d_head = getattr(cfg, "d_head", None)
    d_head = int(d_head) if d_head is not None else d_model // n_head
    d_state = int(cfg.d_state)
    if d_head != 64 or d_state != 32:
        return f"the HIP kernels need d_head == 64 and d_state == 32 (got d_head={d_head}, d_state={d_state})"
    return None


def select_impl(requested: str, x: torch.Tensor, cfg: SISAConfig | None) -> str:
    """Resolve ``requested`` (one of ``IMPLS``) to the implementation used for layer input ``x``.

    ``"auto"`` returns ``"hip_fused"`` if eligible, else ``"hip"``, else ``"torch"`` (with a one-time warning on a
    GPU). A forced HIP implementation on an ineligible input raises ``ValueError`` with the reason.
    """
    if requested not in IMPLS:
        raise ValueError(f"attn_impl must be one of {IMPLS}, got {requested!r}")
    if requested == "torch":
        return "torch"
    on_gpu = isinstance(x, torch.Tensor) and x.device.type == "cuda"
    if on_gpu:
        ok, why = hip_status(x.device)
    else:
        ok, why = False, f"input is on {x.device.type if isinstance(x, torch.Tensor) else type(x).__name__}, not a GPU"
    shape = _shape_problem(cfg)
    cdt = _compute_dtype(x) if isinstance(x, torch.Tensor) else None
    hip_dtype_ok = cdt in (torch.bfloat16, torch.float16, torch.float32)
    fused_dtype_ok = cdt in (torch.bfloat16, torch.float16)

    if requested == "hip_fused":
        if not ok:
            raise ValueError(f"attn_impl='hip_fused' is not available: {why}")
        if shape:
            raise ValueError(f"attn_impl='hip_fused' is not available: {shape}")
        if not fused_dtype_ok:
            raise ValueError(f"attn_impl='hip_fused' needs a bf16/fp16 compute dtype (enable autocast or use "
                             f"low-precision parameters); got {cdt}")
        return "hip_fused"
    if requested == "hip":
        if not ok:
            raise ValueError(f"attn_impl='hip' is not available: {why}")
        if shape:
            raise ValueError(f"attn_impl='hip' is not available: {shape}")
        if not hip_dtype_ok:
            raise ValueError(f"attn_impl='hip' supports bf16, fp16 and fp32 compute dtypes; got {cdt}")
        return "hip"
    # auto
    if ok and not shape:
        if fused_dtype_ok:
            return "hip_fused"
        if hip_dtype_ok:
            return "hip"
    if on_gpu:
        reason = why if not ok else (shape or f"compute dtype {cdt}")
        key = (x.device.index, reason)
        if key not in _WARNED:
            _WARNED.add(key)
            warnings.warn(f"SISA: using the torch attention implementation on the GPU because {reason}", stacklevel=2)
    return "torch"


def describe() -> str:
    """Human-readable summary of the environment, the HIP status and the default backend choice."""
    lines = [f"torch {torch.__version__} (HIP {getattr(torch.version, 'hip', None)})", f"check mode: {get_check_mode()}"]
    if not torch.cuda.is_available():
        lines.append("GPU: not available -> attn_impl='auto' uses 'torch'")
        return "\n".join(lines)
    for idx in range(torch.cuda.device_count()):
        info = device_info(idx)
        ok, why = hip_status(idx)
        lines.append(f"cuda:{idx} {info['name']} ({info['arch']}, {info['cu_count']} CUs)")
        lines.append(f"  hip kernels: {'available' if ok else 'unavailable'} - {why}")
        if ok:
            lines.append("  attn_impl='auto': 'hip_fused' under bf16/fp16 autocast, 'hip' for fp32 inputs")
        else:
            lines.append("  attn_impl='auto': 'torch'")
    return "\n".join(lines)
