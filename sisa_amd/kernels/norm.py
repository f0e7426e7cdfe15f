"""RMSNorm and the SwiGLU activation on the HIP kernels (``sisa_rmsnorm_*``, ``sisa_swiglu_*`` in
``include/sisa_hip.h``): autograd functions with the semantics of the reference's eager modules
(src/sisa/modeling.py:26-50): RMSNorm in float32 with the output in the input dtype and a float32 weight gradient;
``silu(a) * b`` with fp32 arithmetic and one rounding to the input dtype.
"""
from __future__ import annotations

import torch
from torch import Tensor

from . import _lib

__all__ = ["rms_norm_hip", "swiglu_hip"]


def _rows(x: Tensor) -> Tensor:
    """``x`` as a 2-D ``(N, D)`` view with a unit last stride (copying only when the rows are not addressable)."""
    x2 = x.reshape(-1, x.shape[-1])
    if x2.stride(-1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    return x2


class _RMSNormFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x: Tensor, weight: Tensor, eps: float) -> Tensor:
        x2 = _rows(x)
        w = weight.detach().float().contiguous()
        N, D = x2.shape
        y = torch.empty((N, D), device=x.device, dtype=x.dtype)
        rstd = torch.empty(N, device=x.device, dtype=torch.float32)
        args = _lib.RmsNormArgs(N, D, _lib.dtype_code(x.dtype), float(eps), x2.data_ptr(), x2.stride(0), w.data_ptr(),
                                y.data_ptr(), y.stride(0), rstd.data_ptr(), None, 0, None, 0, None, None)
        _lib.call("sisa_rmsnorm_fwd", args, x)
        ctx.save_for_backward(x2, w, rstd)
        ctx.eps, ctx.shape, ctx.wdtype = eps, x.shape, weight.dtype
        return y.view(x.shape)

    @staticmethod
    def backward(ctx, dy: Tensor):
        x2, w, rstd = ctx.saved_tensors
        N, D = x2.shape
        dy2 = _rows(dy.to(x2.dtype))
        dx = torch.empty((N, D), device=x2.device, dtype=x2.dtype)
        dw = torch.empty(D, device=x2.device, dtype=torch.float32)
        ws = torch.empty(_lib.workspace_bytes("sisa_rmsnorm_bwd_workspace_bytes", N, D) // 4, device=x2.device,
                         dtype=torch.float32)
        args = _lib.RmsNormArgs(N, D, _lib.dtype_code(x2.dtype), float(ctx.eps), x2.data_ptr(), x2.stride(0),
                                w.data_ptr(), None, 0, rstd.data_ptr(), dy2.data_ptr(), dy2.stride(0), dx.data_ptr(),
                                dx.stride(0), dw.data_ptr(), ws.data_ptr())
        _lib.call("sisa_rmsnorm_bwd", args, x2)
        return dx.view(ctx.shape), dw.to(ctx.wdtype), None


def rms_norm_hip(x: Tensor, weight: Tensor, eps: float) -> Tensor:
    """``(x * rsqrt(mean(x^2, -1) + eps)) * weight`` in float32, returned in ``x.dtype`` (bf16, fp16 or fp32;
    last dimension a multiple of 8, at most 4096)."""
    if x.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise TypeError(f"rms_norm_hip: unsupported dtype {x.dtype}")
    return _RMSNormFn.apply(x, weight, eps)


class _SwiGLUFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, a: Tensor, b: Tensor) -> Tensor:
        a_, b_ = a.contiguous(), b.contiguous()
        h = torch.empty_like(a_)
        args = _lib.SwigluArgs(a_.numel(), _lib.dtype_code(a_.dtype), a_.data_ptr(), b_.data_ptr(), h.data_ptr(),
                               None, None, None)
        _lib.call("sisa_swiglu_fwd", args, a_)
        ctx.save_for_backward(a_, b_)
        return h

    @staticmethod
    def backward(ctx, dh: Tensor):
        a_, b_ = ctx.saved_tensors
        dh_ = dh.to(a_.dtype).contiguous()
        da, db = torch.empty_like(a_), torch.empty_like(b_)
        args = _lib.SwigluArgs(a_.numel(), _lib.dtype_code(a_.dtype), a_.data_ptr(), b_.data_ptr(), None,
                               dh_.data_ptr(), da.data_ptr(), db.data_ptr())
        _lib.call("sisa_swiglu_bwd", args, a_)
        return da, db


def swiglu_hip(a: Tensor, b: Tensor) -> Tensor:
    """``silu(a) * b`` (same shape and dtype; bf16, fp16 or fp32; element count a multiple of 8)."""
    if a.shape != b.shape or a.dtype != b.dtype:
        raise ValueError(f"swiglu_hip: a {tuple(a.shape)} {a.dtype} and b {tuple(b.shape)} {b.dtype} must match")
    if a.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise TypeError(f"swiglu_hip: unsupported dtype {a.dtype}")
    if a.numel() % 8:
        raise ValueError(f"swiglu_hip: element count {a.numel()} must be a multiple of 8")
    return _SwiGLUFn.apply(a, b)
