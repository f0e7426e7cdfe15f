"""Chunked linear + cross-entropy for a tied LM head on MI355X, without materialising the full logits.

Mirrors ``src/sisa/kernels/linear_ce.py`` of the reference: the same public functions (``linear_cross_entropy``,
``reference_linear_cross_entropy``), arguments, loss/gradient definitions, ``grad_scale`` promise, eager fallback for
CPU tensors or an fp32 compute dtype, and error behaviour (``ValueError`` for a bad weight shape or label count).

Per token chunk (gradients are produced during forward, as in the reference, linear_ce.py:167-191):

  1. ``logits = x_c @ W_pad^T`` -- hipBLASLt through ``torch.mm``, compute-dtype output with fp32 accumulation
     (the autocast formula). W is padded with zero rows to a multiple of 128 (50,277 -> 50,304).
  2. ``sisa_lmce_rows`` (HIP, ``csrc/lmce.hip``): per row lse, loss row and, when a gradient is needed,
     G = (softmax - onehot) * (1/N_valid) * gscale rounded once to the compute dtype, written over the logits. A
     row of up to 65,536 columns is read from HBM once and written once.
  3. ``dx_c = G @ W_pad`` with fp32 output; 4. ``dW (+)= G^T @ x_c`` with fp32 output and accumulation.

Backward multiplies the stored dx / dW by the incoming seed, or, with ``grad_scale`` promised, only checks the promise
on the device. The chunk budget is 4 GiB of logits (MI355X has 288 GB of HBM; the reference uses 1 GiB), so the
16,384-token benchmark case runs as one chunk.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from . import _lib

__all__ = ["linear_cross_entropy", "reference_linear_cross_entropy", "lmce_rows", "flops"]

VOCAB_PAD = 128
CHUNK_BYTES = 4 << 30
_HAS_OUT_DTYPE = hasattr(torch.ops.aten.mm, "dtype") and hasattr(torch.ops.aten.addmm, "dtype_out")


def _compute_dtype(x: torch.Tensor) -> torch.dtype:
    """The autocast dtype when autocast is on for x's device type, else x.dtype (linear_ce.py:107-113)."""
    try:
        if torch.is_autocast_enabled(x.device.type):
            return torch.get_autocast_dtype(x.device.type)
    except (TypeError, RuntimeError):
        pass
    return x.dtype


def _pick_chunk(N: int, Vp: int, chunk_tokens: int | None, elt: int, budget: int = CHUNK_BYTES) -> int:
    """Rows per chunk: ``chunk_tokens`` when given (clamped to [1, N]); otherwise the fewest chunks whose logits fit
    the budget, balanced and rounded up to a multiple of 128 rows (linear_ce.py:116-124)."""
    if N <= 0:
        return 1
    if chunk_tokens:
        return max(1, min(N, int(chunk_tokens)))
    rows_max = max(128, budget // (Vp * elt))
    n_chunks = -(-N // rows_max)
    rows = -(-N // n_chunks)
    return min(N, -(-rows // 128) * 128)


def _padded_lowp_weight(w: torch.Tensor, dtype: torch.dtype, vocab_pad: int = VOCAB_PAD) -> torch.Tensor:
    """(Vp, D) copy of w in ``dtype`` (RNE, as autocast) with zero rows V..Vp-1 (linear_ce.py:127-135)."""
    V, D = w.shape
    Vp = -(-V // vocab_pad) * vocab_pad
    out = torch.empty((Vp, D), dtype=dtype, device=w.device)
    out[:V].copy_(w.detach())
    out[V:].zero_()
    return out


def lmce_rows(logits: torch.Tensor, labels: torch.Tensor, loss_rows: torch.Tensor, V: int, ignore_index: int,
              inv_n: torch.Tensor | None = None, gscale: float = 1.0, lse: torch.Tensor | None = None) -> None:
    """Row pass over one chunk of logits (T, Vp) bf16/fp16 with unit column stride: writes ``loss_rows`` (T,) fp32
    (and ``lse`` if given) and, when ``inv_n`` (a device scalar 1/N_valid) is given, overwrites the logits with G.
    Replaces ``_launch_rows`` / ``_lmce_row_kernel`` (linear_ce.py:60-104)."""
    T, Vp = logits.shape
    if T == 0:
        return
    if logits.stride(1) != 1:
        raise ValueError("lmce_rows: logits need a unit column stride")
    if labels.dtype != torch.int64 or not labels.is_contiguous() or labels.numel() != T:
        raise ValueError("lmce_rows: labels must be a contiguous int64 tensor with one entry per row")
    args = _lib.LmceRowsArgs(T, int(V), Vp, logits.stride(0), _lib.dtype_code(logits.dtype), int(inv_n is not None),
                             logits.data_ptr(), labels.data_ptr(), int(ignore_index), _lib.ptr(inv_n), float(gscale),
                             loss_rows.data_ptr(), _lib.ptr(lse))
    _lib.call("sisa_lmce_rows", args, logits)


def _check_seed(g: torch.Tensor, grad_scale: float) -> None:
    """G already carries the promised seed: check the promise where g lives (a device-side assert on the GPU, no
    host sync; a RuntimeError on the CPU) (linear_ce.py:202-206)."""
    torch._assert_async(g.to(torch.float32) == float(grad_scale),
                        "linear_cross_entropy: backward seed differs from the promised grad_scale")


class _LinearCrossEntropyFn(torch.autograd.Function):
    """Autograd wrapper of the chunk loop (linear_ce.py:138-217)."""

    @staticmethod
    def forward(ctx, h, w, labels, opts):
        ignore_index, chunk_tokens, cdtype, need_dh, need_dw, grad_scale = opts
        D = h.shape[-1]
        V = w.shape[0]
        dev = h.device
        x = h.reshape(-1, D)
        N = x.shape[0]
        lab = labels.reshape(-1).to(torch.int64).contiguous()
        xb = x.to(cdtype).contiguous()
        wp = _padded_lowp_weight(w, cdtype)
        Vp = wp.shape[0]
        n_valid = (lab != ignore_index).sum()
        inv_n = torch.reciprocal(n_valid.to(torch.float32)).reshape(1)
        loss_rows = torch.empty(N, dtype=torch.float32, device=dev)
        rows = _pick_chunk(N, Vp, chunk_tokens, wp.element_size())
        need_g = need_dh or need_dw
        buf = torch.empty((rows, Vp), dtype=cdtype, device=dev) if N else None
        dx = torch.empty((N, D), dtype=torch.float32, device=dev) if need_dh else None
        # dW over all Vp rows keeps the GEMM on aligned shapes; rows V.. are dropped in backward
        dw = torch.empty((Vp, D), dtype=torch.float32, device=dev) if need_dw else None
        if need_dw and N == 0:
            dw.zero_()
        gs = 1.0 if grad_scale is None else float(grad_scale)
        for s in range(0, N, rows):
            e = min(N, s + rows)
            lg = buf[:e - s]
            xc = xb[s:e]
            torch.mm(xc, wp.t(), out=lg)
            lmce_rows(lg, lab[s:e], loss_rows[s:e], V, ignore_index, inv_n if need_g else None, gs)
            if need_dh:
                if _HAS_OUT_DTYPE:
                    torch.mm(lg, wp, out_dtype=torch.float32, out=dx[s:e])
                else:
                    dx[s:e].copy_(torch.mm(lg, wp))
            if need_dw:
                if _HAS_OUT_DTYPE:
                    if s == 0:
                        torch.mm(lg.t(), xc, out_dtype=torch.float32, out=dw)
                    else:
                        torch.addmm(dw, lg.t(), xc, out_dtype=torch.float32, out=dw)
                elif s == 0:
                    dw.copy_(torch.mm(lg.t(), xc))
                else:
                    dw.add_(torch.mm(lg.t(), xc))
        del buf
        loss = loss_rows.sum() / n_valid
        ctx.h_shape, ctx.h_dtype, ctx.w_dtype, ctx.grad_scale, ctx.V = h.shape, h.dtype, w.dtype, grad_scale, V
        ctx.save_for_backward(dx, dw)
        return loss

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, g):
        dx, dw = ctx.saved_tensors
        if ctx.grad_scale is not None:
            _check_seed(g, ctx.grad_scale)
            dh = dx.view(ctx.h_shape) if dx is not None else None
            dW = dw[:ctx.V] if dw is not None else None
        else:
            g32 = g.to(torch.float32)
            dh = (dx * g32).view(ctx.h_shape) if dx is not None else None
            dW = dw[:ctx.V] * g32 if dw is not None else None
        if dh is not None and dh.dtype != ctx.h_dtype:
            dh = dh.to(ctx.h_dtype)
        if dW is not None and dW.dtype != ctx.w_dtype:
            dW = dW.to(ctx.w_dtype)
        return dh, dW, None, None


def reference_linear_cross_entropy(hidden: torch.Tensor, weight: torch.Tensor, labels: torch.Tensor,
                                   ignore_index: int = -100) -> torch.Tensor:
    """The eager formula ``F.cross_entropy(F.linear(hidden, weight).float(), labels, ignore_index)``
    (linear_ce.py:220-224)."""
    logits = F.linear(hidden, weight)
    return F.cross_entropy(logits.view(-1, logits.size(-1)).float(), labels.reshape(-1), ignore_index=ignore_index)


@torch.compiler.disable
def linear_cross_entropy(hidden: torch.Tensor, weight: torch.Tensor, labels: torch.Tensor, ignore_index: int = -100,
                         *, chunk_tokens: int | None = None, grad_scale: float | None = None) -> torch.Tensor:
    """Mean cross-entropy of ``hidden @ weight.T`` against ``labels`` without materialising the full logits
    (linear_ce.py:227-259).

    Args:
        hidden: ``(..., D)`` hidden states (fp32 under autocast, or bf16/fp16).
        weight: ``(V, D)`` LM-head weight (fp32 master or bf16/fp16); receives dL/dW.
        labels: ``(...)`` integer targets aligned with the hidden rows (no shift). Rows equal to ``ignore_index``
            get neither loss nor gradient.
        chunk_tokens: rows per chunk (default: balanced chunks under a 4 GiB logits buffer).
        grad_scale: promise that backward is seeded with exactly this value; G is then scaled in forward and a
            different seed trips a device-side assert.

    Returns the fp32 scalar loss (NaN when every row is ignored). The compute dtype is the autocast dtype when
    autocast is on, else ``hidden.dtype``; with CPU tensors or an fp32 compute dtype the eager formula is used.
    A label outside [0, V) that is not ``ignore_index`` gives a NaN loss.
    """
    cdtype = _compute_dtype(hidden)
    if cdtype not in (torch.bfloat16, torch.float16) or not hidden.is_cuda:
        return reference_linear_cross_entropy(hidden, weight, labels, ignore_index)
    if weight.dim() != 2 or weight.shape[1] != hidden.shape[-1]:
        raise ValueError(f"weight must be (V, {hidden.shape[-1]}), got {tuple(weight.shape)}")
    if labels.numel() != hidden.numel() // hidden.shape[-1]:
        raise ValueError(f"labels have {labels.numel()} elements, expected one per hidden row "
                         f"({hidden.numel() // hidden.shape[-1]})")
    ge = torch.is_grad_enabled()
    opts = (ignore_index, chunk_tokens, cdtype, bool(ge and hidden.requires_grad), bool(ge and weight.requires_grad),
            grad_scale)
    return _LinearCrossEntropyFn.apply(hidden, weight, labels, opts)


def flops(N: int, V: int, D: int) -> dict:
    """Algorithmic work of one forward (which also produces the gradients): three GEMMs of 2*N*V*D each."""
    g = 2.0 * N * V * D
    return {"logits": g, "dx": g, "dw": g, "total": 3 * g}
