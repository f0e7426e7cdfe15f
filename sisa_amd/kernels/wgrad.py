"""Weight gradients of linear layers on the HIP kernel ``sisa_wgrad`` (``include/sisa_hip.h``): ``dW = dY^T X`` in
fp32 from bf16/fp16 operands, and ``linear_hip``, a linear layer whose forward and input gradient stay on the
library GEMMs and whose weight gradient uses the kernel (the weight-gradient products autograd runs for the
nn.Linear projections of src/sisa/modeling.py:79-291, written in fp32 without the bf16 rounding and cast pass).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import Tensor

from . import _lib

__all__ = ["wgrad_hip", "linear_hip", "row_pieces"]

TM = 64


def _rows16(t: Tensor) -> Tensor:
    t2 = t.reshape(-1, t.shape[-1])
    if t2.stride(-1) != 1 or t2.stride(0) % 8 or t2.data_ptr() % 16:
        t2 = t2.contiguous()
    return t2


# One launch addresses each operand through a 32-bit byte offset: a row range of an operand stays below 2 GiB.
OPERAND_LIMIT = 1 << 31


def row_pieces(M: int, lda: int, ldb: int, elem: int = 2) -> list[tuple[int, int]]:
    """Row ranges [r0, r1) of the reduction axis, each small enough for one launch (both operands' ranges below
    2 GiB), every range but the last a multiple of 64 rows."""
    per_row = max(lda, ldb) * elem
    cap = (OPERAND_LIMIT - 1) // per_row
    cap = max(TM, cap // TM * TM)
    return [(r, min(M, r + cap)) for r in range(0, M, cap)] if M > 0 else []


def wgrad_hip(dy: Tensor, x: Tensor, out: Tensor | None = None, nsplit: int | None = None) -> Tensor:
    """``dy^T x`` in fp32 for ``dy`` ``(..., N)`` and ``x`` ``(..., K)`` of one 16-bit dtype (the leading dims are
    the reduction); returns ``(N, K)`` float32 (written into ``out`` when given). Operands of 2 GiB or more are
    reduced in row ranges (see :func:`row_pieces`) whose fp32 results are added in range order."""
    if dy.dtype != x.dtype or dy.dtype not in (torch.bfloat16, torch.float16):
        raise TypeError(f"wgrad_hip: dy {dy.dtype} and x {x.dtype} must be one of bf16/fp16")
    a, b = _rows16(dy), _rows16(x)
    if a.shape[0] != b.shape[0]:
        raise ValueError(f"wgrad_hip: {a.shape[0]} rows of dy vs {b.shape[0]} of x")
    pieces = row_pieces(a.shape[0], a.stride(0), b.stride(0), a.element_size())
    if len(pieces) > 1:
        out = _wgrad_launch(a[pieces[0][0]:pieces[0][1]], b[pieces[0][0]:pieces[0][1]], out, nsplit)
        part = torch.empty_like(out)
        for r0, r1 in pieces[1:]:
            out += _wgrad_launch(a[r0:r1], b[r0:r1], part, nsplit)
        return out
    return _wgrad_launch(a, b, out, nsplit)


def _wgrad_launch(a: Tensor, b: Tensor, out: Tensor | None, nsplit: int | None) -> Tensor:
    M, N = a.shape
    K = b.shape[1]
    lib = _lib.load()
    s = int(lib.sisa_wgrad_splits(M, N, K)) if nsplit is None else int(nsplit)
    per = -(-M // s)
    per = -(-per // TM) * TM
    if out is None:
        out = torch.empty((N, K), device=a.device, dtype=torch.float32)
    elif out.shape != (N, K) or out.dtype != torch.float32 or out.stride(1) != 1:
        raise ValueError("wgrad_hip: out must be an (N, K) float32 tensor with unit column stride")
    ws_bytes = int(lib.sisa_wgrad_workspace_bytes(M, N, K, s))
    ws = torch.empty(max(ws_bytes // 4, 1), device=a.device, dtype=torch.float32) if ws_bytes else None
    args = _lib.WgradArgs(M, N, K, _lib.dtype_code(a.dtype), s, per, a.data_ptr(), a.stride(0), b.data_ptr(),
                          b.stride(0), out.data_ptr(), out.stride(0), _lib.ptr(ws))
    _lib.call("sisa_wgrad", args, a)
    return out


class _LinearFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x: Tensor, weight: Tensor, bias: Tensor | None, cd: torch.dtype, bias_cols) -> Tensor:
        w16 = weight.detach().to(cd)
        x16 = x.detach().to(cd)
        b16 = None if bias is None else bias.detach().to(cd)
        ctx.save_for_backward(x16, w16)
        ctx.has_bias, ctx.wdtype, ctx.bdtype = bias is not None, weight.dtype, None if bias is None else bias.dtype
        ctx.xdtype, ctx.bias_cols = x.dtype, bias_cols
        return F.linear(x16, w16, b16)

    @staticmethod
    def backward(ctx, dy: Tensor):
        x16, w16 = ctx.saved_tensors
        dy16 = dy.to(w16.dtype)
        dx = (dy16 @ w16).to(ctx.xdtype) if ctx.needs_input_grad[0] else None
        dw = wgrad_hip(dy16, x16).to(ctx.wdtype) if ctx.needs_input_grad[1] else None
        db = None
        if ctx.has_bias and ctx.needs_input_grad[2]:
            d2 = dy16.reshape(-1, dy16.shape[-1])
            if ctx.bias_cols is None:
                db = d2.sum(0, dtype=torch.float32).to(ctx.bdtype)
            else:                       # only these bias entries reach a parameter: sum just their columns
                c0, c1 = ctx.bias_cols
                db = torch.zeros(d2.shape[1], device=d2.device, dtype=ctx.bdtype)
                db[c0:c1] = d2[:, c0:c1].sum(0, dtype=torch.float32).to(ctx.bdtype)
        return dx, dw, db, None, None


def linear_hip(x: Tensor, weight: Tensor, bias: Tensor | None = None, bias_cols: tuple[int, int] | None = None
               ) -> Tensor:
    """``F.linear(x, weight, bias)`` in the autocast dtype (bf16/fp16; the weights' dtype without autocast) with the
    weight gradient from :func:`wgrad_hip` (fp32 accumulation, no rounding to 16 bits before the parameter's
    dtype). The input gradient and the forward stay on the library GEMMs. ``bias_cols = (c0, c1)``: only bias entries
    c0..c1-1 lead to parameters (the rest is constant padding), so the backward sums only those columns of dy."""
    cd = torch.get_autocast_dtype("cuda") if torch.is_autocast_enabled("cuda") else weight.dtype
    if cd not in (torch.bfloat16, torch.float16):
        raise TypeError(f"linear_hip: compute dtype {cd} is not bf16/fp16")
    return _LinearFn.apply(x, weight, bias, cd, bias_cols)
