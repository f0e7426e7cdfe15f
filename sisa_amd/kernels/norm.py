"""RMSNorm (optionally with the fused fp32 forget-gate projection of the attention sublayer) and the SwiGLU
activation on the HIP kernels (``sisa_norm_*``, ``sisa_swiglu_*`` in ``include/sisa_hip.h``): autograd functions with
the semantics of the reference's eager modules (src/sisa/modeling.py:26-50, 166-169): RMSNorm in float32 with the
output in the input dtype (optionally already cast to the consuming GEMM's autocast dtype) and float32 weight
gradients; ``silu(a) * b`` with fp32 arithmetic and one rounding to the input dtype.
"""
from __future__ import annotations

import torch
from torch import Tensor

from . import _lib

__all__ = ["rms_norm_hip", "rms_norm_add_hip", "rms_norm_forget_hip", "rms_norm_forget_add_hip", "swiglu_hip",
           "swiglu_pairs_hip", "interleave_gate_up"]


def _rows(x: Tensor) -> Tensor:
    """``x`` as a 2-D ``(N, D)`` view with a unit last stride (copying only when the rows are not addressable)."""
    x2 = x.reshape(-1, x.shape[-1])
    if x2.stride(-1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    return x2


_HALF = (torch.bfloat16, torch.float16)


class _NormFn(torch.autograd.Function):
    """RMSNorm of the rows of ``x`` with the output in ``out_dtype`` and, when ``wf`` is given, the fp32 projection
    ``z = n W_f^T + b_f`` of the normalised rows ``n`` (in ``x``'s dtype) -- one ``sisa_norm_fwd`` launch; the backward
    is one ``sisa_norm_bwd`` call (row pass, dw reduction, dW_f/db_f)."""

    @staticmethod
    def forward(ctx, x: Tensor, weight: Tensor, wf, bf, eps: float, out_dtype: torch.dtype):
        x2 = _rows(x)
        w = weight.detach().float().contiguous()
        N, D = x2.shape
        H = 0 if wf is None else wf.shape[0]
        wf32 = None if wf is None else wf.detach().float().contiguous()
        bf32 = None if bf is None else bf.detach().float().contiguous()
        y = torch.empty((N, D), device=x.device, dtype=out_dtype)
        rstd = torch.empty(N, device=x.device, dtype=torch.float32)
        z = torch.empty((N, H), device=x.device, dtype=torch.float32) if H else None
        args = _lib.NormArgs(N, D, H, _lib.dtype_code(x.dtype), _lib.dtype_code(out_dtype), float(eps), 0,
                             x2.data_ptr(), x2.stride(0), w.data_ptr(), _lib.ptr(wf32), _lib.ptr(bf32),
                             y.data_ptr(), y.stride(0), rstd.data_ptr(), _lib.ptr(z))
        _lib.call("sisa_norm_fwd", args, x)
        ctx.save_for_backward(x2, w, rstd, wf32, bf32)
        ctx.eps, ctx.shape, ctx.wdtype, ctx.out_dtype = eps, x.shape, weight.dtype, out_dtype
        ctx.fdtypes = (None, None) if wf is None else (wf.dtype, bf.dtype)
        y = y.view(x.shape)
        if H:
            return y, z.view(*x.shape[:-1], H)
        return y

    @staticmethod
    def backward(ctx, dy: Tensor, dz: Tensor | None = None):
        x2, w, rstd, wf32, bf32 = ctx.saved_tensors
        N, D = x2.shape
        H = 0 if wf32 is None else wf32.shape[0]
        if dy is None:
            dy = torch.zeros((N, D), device=x2.device, dtype=ctx.out_dtype)
        dy2 = _rows(dy.to(ctx.out_dtype))
        dz2 = None
        if H:
            dz2 = (torch.zeros((N, H), device=x2.device, dtype=torch.float32) if dz is None
                   else dz.reshape(N, H).float().contiguous())
        dx = torch.empty((N, D), device=x2.device, dtype=x2.dtype)
        dw = torch.empty(D, device=x2.device, dtype=torch.float32)
        dwf = torch.empty((H, D), device=x2.device, dtype=torch.float32) if H else None
        dbf = torch.empty(H, device=x2.device, dtype=torch.float32) if H else None
        ws = torch.empty(_lib.workspace_bytes("sisa_norm_bwd_workspace_bytes", N, D, H) // 4, device=x2.device,
                         dtype=torch.float32)
        args = _lib.NormArgs(N, D, H, _lib.dtype_code(x2.dtype), _lib.dtype_code(ctx.out_dtype), float(ctx.eps), 0,
                             x2.data_ptr(), x2.stride(0), w.data_ptr(), _lib.ptr(wf32), _lib.ptr(bf32), None, 0,
                             rstd.data_ptr(), None, dy2.data_ptr(), dy2.stride(0), _lib.ptr(dz2), dx.data_ptr(),
                             dx.stride(0), dw.data_ptr(), _lib.ptr(dwf), _lib.ptr(dbf), ws.data_ptr())
        _lib.call("sisa_norm_bwd", args, x2)
        dwf_out = None if dwf is None else dwf.to(ctx.fdtypes[0])
        dbf_out = None if dbf is None else dbf.to(ctx.fdtypes[1])
        return dx.view(ctx.shape), dw.to(ctx.wdtype), dwf_out, dbf_out, None, None


class _AddNormFn(torch.autograd.Function):
    """The residual add and the RMSNorm that follows it in one pass: ``h = x + res`` (in ``x``'s dtype) and
    ``y = RMSNorm(h)`` in ``out_dtype``, with the fp32 forget projection ``z`` of the normalised rows when ``wf`` is
    given -- one ``sisa_norm_fwd`` launch. The backward sums the gradient of ``h`` from the residual stream into the
    norm's dx inside the ``sisa_norm_bwd`` row pass; ``res`` receives that sum in its own dtype, as autograd gives it
    to the operand of the add."""

    @staticmethod
    def forward(ctx, x: Tensor, res: Tensor, weight: Tensor, wf, bf, eps: float, out_dtype: torch.dtype):
        x2, r2 = _rows(x), _rows(res)
        w = weight.detach().float().contiguous()
        N, D = x2.shape
        H = 0 if wf is None else wf.shape[0]
        wf32 = None if wf is None else wf.detach().float().contiguous()
        bf32 = None if bf is None else bf.detach().float().contiguous()
        h = torch.empty((N, D), device=x.device, dtype=x.dtype)
        y = torch.empty((N, D), device=x.device, dtype=out_dtype)
        rstd = torch.empty(N, device=x.device, dtype=torch.float32)
        z = torch.empty((N, H), device=x.device, dtype=torch.float32) if H else None
        args = _lib.NormArgs(N, D, H, _lib.dtype_code(x.dtype), _lib.dtype_code(out_dtype), float(eps), 0,
                             x2.data_ptr(), x2.stride(0), w.data_ptr(), _lib.ptr(wf32), _lib.ptr(bf32), y.data_ptr(),
                             y.stride(0), rstd.data_ptr(), _lib.ptr(z), None, 0, None, None, 0, None, None, None,
                             None, r2.data_ptr(), r2.stride(0), h.data_ptr(), h.stride(0))
        _lib.call("sisa_norm_fwd", args, x)
        ctx.save_for_backward(h, w, rstd, wf32, bf32)
        ctx.eps, ctx.shape, ctx.wdtype, ctx.out_dtype, ctx.rdtype = eps, x.shape, weight.dtype, out_dtype, res.dtype
        ctx.fdtypes = (None, None) if wf is None else (wf.dtype, bf.dtype)
        if H:
            return h.view(x.shape), y.view(x.shape), z.view(*x.shape[:-1], H)
        return h.view(x.shape), y.view(x.shape)

    @staticmethod
    def backward(ctx, dh: Tensor | None, dy: Tensor | None, dz: Tensor | None = None):
        h2, w, rstd, wf32, bf32 = ctx.saved_tensors
        N, D = h2.shape
        H = 0 if wf32 is None else wf32.shape[0]
        if dy is None:
            dy = torch.zeros((N, D), device=h2.device, dtype=ctx.out_dtype)
        dy2 = _rows(dy.to(ctx.out_dtype))
        dh2 = None if dh is None else _rows(dh.to(h2.dtype))
        dz2 = None
        if H:
            dz2 = (torch.zeros((N, H), device=h2.device, dtype=torch.float32) if dz is None
                   else dz.reshape(N, H).float().contiguous())
        dx = torch.empty((N, D), device=h2.device, dtype=h2.dtype)
        dw = torch.empty(D, device=h2.device, dtype=torch.float32)
        dwf = torch.empty((H, D), device=h2.device, dtype=torch.float32) if H else None
        dbf = torch.empty(H, device=h2.device, dtype=torch.float32) if H else None
        ws = torch.empty(_lib.workspace_bytes("sisa_norm_bwd_workspace_bytes", N, D, H) // 4, device=h2.device,
                         dtype=torch.float32)
        args = _lib.NormArgs(N, D, H, _lib.dtype_code(h2.dtype), _lib.dtype_code(ctx.out_dtype), float(ctx.eps), 0,
                             h2.data_ptr(), h2.stride(0), w.data_ptr(), _lib.ptr(wf32), _lib.ptr(bf32), None, 0,
                             rstd.data_ptr(), None, dy2.data_ptr(), dy2.stride(0), _lib.ptr(dz2), dx.data_ptr(),
                             dx.stride(0), dw.data_ptr(), _lib.ptr(dwf), _lib.ptr(dbf), ws.data_ptr(), None, 0, None,
                             0, _lib.ptr(dh2), 0 if dh2 is None else dh2.stride(0))
        _lib.call("sisa_norm_bwd", args, h2)
        dx = dx.view(ctx.shape)
        dwf_out = None if dwf is None else dwf.to(ctx.fdtypes[0])
        dbf_out = None if dbf is None else dbf.to(ctx.fdtypes[1])
        return dx, dx.to(ctx.rdtype), dw.to(ctx.wdtype), dwf_out, dbf_out, None, None


def _check_norm(x: Tensor, out_dtype: torch.dtype, H: int) -> None:
    if x.dtype not in (torch.float32, *_HALF):
        raise TypeError(f"rms_norm_hip: unsupported dtype {x.dtype}")
    if out_dtype != x.dtype and not (x.dtype == torch.float32 and out_dtype in _HALF):
        raise TypeError(f"rms_norm_hip: output dtype {out_dtype} needs an fp32 input (got {x.dtype})")
    D = x.shape[-1]
    if D % 8 or D > 4096 or D < 8:
        raise ValueError(f"rms_norm_hip: row length {D} must be a multiple of 8 in [8, 4096]")
    if H > 64:
        raise ValueError(f"rms_norm_hip: at most 64 projection outputs, got {H}")


def rms_norm_hip(x: Tensor, weight: Tensor, eps: float, out_dtype: torch.dtype | None = None) -> Tensor:
    """``(x * rsqrt(mean(x^2, -1) + eps)) * weight`` in float32, rounded to ``x.dtype`` and returned in ``out_dtype``
    (default ``x.dtype``; a 16-bit ``out_dtype`` needs an fp32 ``x``, as the reference's RMSNorm output followed by
    the autocast cast of the consuming GEMM). bf16, fp16 or fp32; last dimension a multiple of 8, at most 4096."""
    out_dtype = out_dtype or x.dtype
    _check_norm(x, out_dtype, 0)
    return _NormFn.apply(x, weight, None, None, eps, out_dtype)


def rms_norm_add_hip(x: Tensor, res: Tensor, weight: Tensor, eps: float,
                     out_dtype: torch.dtype | None = None) -> tuple[Tensor, Tensor]:
    """``h = x + res`` followed by :func:`rms_norm_hip` of ``h``, in one kernel pass each way: the residual add of a
    pre-norm block and the next sublayer's norm (src/sisa/modeling.py:288-291). ``res`` must have ``out_dtype``
    (the consuming GEMM's autocast dtype, as the sublayer outputs under autocast) and ``x``'s shape; ``h`` is in
    ``x.dtype``, rounded once as ``x + res`` is. Returns ``(h, y)``."""
    out_dtype = out_dtype or x.dtype
    _check_norm(x, out_dtype, 0)
    if res.shape != x.shape or res.dtype != out_dtype:
        raise ValueError(f"rms_norm_add_hip: residual {tuple(res.shape)} {res.dtype} must match x {tuple(x.shape)} "
                         f"and have the output dtype {out_dtype}")
    return _AddNormFn.apply(x, res, weight, None, None, eps, out_dtype)


def rms_norm_forget_add_hip(x: Tensor, res: Tensor, weight: Tensor, eps: float, wf: Tensor, bf: Tensor,
                            out_dtype: torch.dtype | None = None) -> tuple[Tensor, Tensor, Tensor]:
    """``h = x + res`` followed by :func:`rms_norm_forget_hip` of ``h`` in one pass each way: the residual add that
    ends a decoder block and the next block's attention norm with its forget-gate projection. Returns
    ``(h, y, z)``; ``res`` as in :func:`rms_norm_add_hip`."""
    out_dtype = out_dtype or x.dtype
    if wf.dim() != 2 or wf.shape[1] != x.shape[-1] or bf.shape != (wf.shape[0],):
        raise ValueError(f"rms_norm_forget_add_hip: projection {tuple(wf.shape)} / bias {tuple(bf.shape)} do not "
                         f"match rows of {x.shape[-1]}")
    _check_norm(x, out_dtype, wf.shape[0])
    if res.shape != x.shape or res.dtype != out_dtype:
        raise ValueError(f"rms_norm_forget_add_hip: residual {tuple(res.shape)} {res.dtype} must match x "
                         f"{tuple(x.shape)} and have the output dtype {out_dtype}")
    return _AddNormFn.apply(x, res, weight, wf, bf, eps, out_dtype)


def rms_norm_forget_hip(x: Tensor, weight: Tensor, eps: float, wf: Tensor, bf: Tensor,
                        out_dtype: torch.dtype | None = None) -> tuple[Tensor, Tensor]:
    """RMSNorm as :func:`rms_norm_hip` plus the fp32 forget-gate logits ``z = n W_f^T + b_f`` of the normalised rows
    ``n`` (in ``x.dtype``), as ``SISAAttention._forget_logits`` computes them from the normalised input
    (src/sisa/modeling.py:166-169). Returns ``(y, z)`` with ``z`` of shape ``(..., H)`` float32."""
    out_dtype = out_dtype or x.dtype
    if wf.dim() != 2 or wf.shape[1] != x.shape[-1] or bf.shape != (wf.shape[0],):
        raise ValueError(f"rms_norm_forget_hip: projection {tuple(wf.shape)} / bias {tuple(bf.shape)} do not match "
                         f"rows of {x.shape[-1]}")
    _check_norm(x, out_dtype, wf.shape[0])
    return _NormFn.apply(x, weight, wf, bf, eps, out_dtype)


class _SwiGLUFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, a: Tensor, b: Tensor) -> Tensor:
        a_, b_ = a.contiguous(), b.contiguous()
        h = torch.empty_like(a_)
        args = _lib.SwigluArgs(a_.numel(), _lib.dtype_code(a_.dtype), 0, a_.data_ptr(), b_.data_ptr(), h.data_ptr(),
                               None, None, None)
        _lib.call("sisa_swiglu_fwd", args, a_)
        ctx.save_for_backward(a_, b_)
        return h

    @staticmethod
    def backward(ctx, dh: Tensor):
        a_, b_ = ctx.saved_tensors
        dh_ = dh.to(a_.dtype).contiguous()
        da, db = torch.empty_like(a_), torch.empty_like(b_)
        args = _lib.SwigluArgs(a_.numel(), _lib.dtype_code(a_.dtype), 0, a_.data_ptr(), b_.data_ptr(), None,
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


class _SwiGLUPairsFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, ab: Tensor) -> Tensor:
        ab_ = ab.contiguous()
        n = ab_.numel() // 2
        h = torch.empty((*ab_.shape[:-1], ab_.shape[-1] // 2), device=ab_.device, dtype=ab_.dtype)
        args = _lib.SwigluArgs(n, _lib.dtype_code(ab_.dtype), 1, ab_.data_ptr(), None, h.data_ptr(), None, None, None)
        _lib.call("sisa_swiglu_fwd", args, ab_)
        ctx.save_for_backward(ab_)
        return h

    @staticmethod
    def backward(ctx, dh: Tensor):
        (ab_,) = ctx.saved_tensors
        dh_ = dh.to(ab_.dtype).contiguous()
        dab = torch.empty_like(ab_)
        args = _lib.SwigluArgs(ab_.numel() // 2, _lib.dtype_code(ab_.dtype), 1, ab_.data_ptr(), None, None,
                               dh_.data_ptr(), dab.data_ptr(), None)
        _lib.call("sisa_swiglu_bwd", args, ab_)
        return dab


def interleave_gate_up(w_gate: Tensor, w_up: Tensor) -> Tensor:
    """``(2F, D)`` weight whose rows alternate 8-row chunks of ``w_gate`` and ``w_up`` (F a multiple of 8): one GEMM
    against it yields, per row, the interleaved chunks :func:`swiglu_pairs_hip` takes."""
    F_, D = w_gate.shape
    return torch.stack((w_gate.reshape(F_ // 8, 8, D), w_up.reshape(F_ // 8, 8, D)), dim=1).reshape(2 * F_, D)


def swiglu_pairs_hip(ab: Tensor) -> Tensor:
    """``silu(a) * b`` where the last dimension of ``ab`` (2F) holds the interleaved 8-element chunks of a and b (the
    output of ``F.linear(x, interleave_gate_up(w_gate, w_up))``); returns ``(..., F)``."""
    if ab.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise TypeError(f"swiglu_pairs_hip: unsupported dtype {ab.dtype}")
    if ab.shape[-1] % 16:
        raise ValueError(f"swiglu_pairs_hip: last dimension {ab.shape[-1]} must be a multiple of 16")
    return _SwiGLUPairsFn.apply(ab)
