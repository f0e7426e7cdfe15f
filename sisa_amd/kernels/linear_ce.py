"""Linear layer + cross-entropy for a tied LM head on MI355X without the full (tokens x vocabulary) logits.

Interface of the reference's ``sisa.kernels.linear_ce`` (src/sisa/kernels/linear_ce.py:220-259):
``linear_cross_entropy(hidden, weight, labels, ignore_index=-100, *, chunk_tokens=None, grad_scale=None)`` -> the mean
loss over the non-ignored rows, differentiable in ``hidden`` and ``weight``, and the eager formula
``reference_linear_cross_entropy``. Labels are not shifted. A label outside [0, V) makes the loss NaN. A ``weight`` of
the wrong shape or a label count that does not match the hidden rows raises ``ValueError``. CPU tensors and an fp32
compute dtype take the eager formula.

How the work is arranged here (every kernel is HIP, ``libsisa_hip.so``; no library GEMM):

* No gradient wanted (``torch.no_grad``, evaluation, or neither input requires grad): one fused launch,
  ``sisa_lmce_fwd`` (csrc/lmce_fwd.hip). An MFMA GEMM whose tiles are reduced on the fly to each row's log-sum-exp
  and label logit; no logits are stored anywhere.
* Gradients wanted: ``sisa_lmce_train`` (csrc/lmce_train.hip) per chunk of rows. The same logits GEMM also stores
  each exponential relative to its row's maximum over half a 256-column vocabulary tile (compute dtype) and those
  maxima; then one launch of MFMA tiles computes dW = G^T x and dx = G W_pad, each forming
  G = (softmax - onehot) / N_valid * gscale from the stored exponentials while staging it into LDS. Neither the logits
  nor G are ever written. The reference's chunk loop (linear_ce.py:160-191: logits GEMM, row kernel, dx and dW
  GEMMs) has the same contract; its chunk budget is 1 GiB of logits, this one 2 GiB of exponentials (one chunk at
  N = 16,384, V = 50,277), because every chunk after the first re-reads and adds the fp32 dW.

Both paths round each logit, accumulated in fp32 by the MFMAs, once to the compute dtype before the log-sum-exp, as
the reference's row kernel reads bf16/fp16 logits (linear_ce.py:166-170), so the loss has the reference's rounding
point, and the two paths give bitwise the same loss.

The vocabulary is padded with zero rows to a multiple of 128 (50,277 -> 50,304) and the hidden size with zero columns
to a multiple of 64, so that every GEMM runs on aligned shapes; the padding never enters a sum. ``grad_scale`` is the
caller's promise of the backward seed: G is then scaled in the forward pass and the backward only checks the promise
on the device.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from .. import backends
from . import _lib

__all__ = ["linear_cross_entropy", "reference_linear_cross_entropy", "lmce_rows", "lmce_fused_loss_rows",
           "lmce_train_chunk", "padded_weight", "chunk_rows", "flops"]

VOCAB_MULTIPLE = 128
HIDDEN_MULTIPLE = 64             # the CE kernels stream the hidden size in 64-wide stages
PROBS_BUDGET = 2 << 30           # bytes of one chunk of stored exponentials


# ------------------------------------------------------------------------------------------------ pieces
def padded_weight(weight: torch.Tensor, dtype: torch.dtype, cols: int | None = None) -> torch.Tensor:
    """The LM-head weight in the compute dtype (one round-to-nearest-even cast, as autocast does) with zero rows up
    to the next multiple of 128 (and zero columns up to ``cols``)."""
    V, D = weight.shape
    rows = -(-V // VOCAB_MULTIPLE) * VOCAB_MULTIPLE
    cols = D if cols is None else cols
    pad = rows > V or cols > D
    out = weight.new_zeros((rows, cols), dtype=dtype) if pad else weight.new_empty((rows, cols), dtype=dtype)
    out[:V, :D].copy_(weight.detach())
    return out


def chunk_rows(n_rows: int, vocab_rows: int, chunk_tokens: int | None, itemsize: int,
               budget: int = PROBS_BUDGET) -> int:
    """Token rows per chunk of the gradient pass: ``chunk_tokens`` if given (within [1, n_rows]); otherwise the
    smallest number of equal chunks whose stored exponentials fit ``budget`` bytes, each rounded up to whole 128-row
    GEMM tiles."""
    if n_rows <= 0:
        return 1
    if chunk_tokens:
        return min(n_rows, max(1, int(chunk_tokens)))
    fit = max(VOCAB_MULTIPLE, budget // (vocab_rows * itemsize))
    pieces = -(-n_rows // fit)
    per = -(-n_rows // pieces)
    return min(n_rows, -(-per // VOCAB_MULTIPLE) * VOCAB_MULTIPLE)


def lmce_rows(logits: torch.Tensor, labels: torch.Tensor, loss_rows: torch.Tensor, V: int, ignore_index: int,
              inv_n: torch.Tensor | None = None, gscale: float = 1.0, lse: torch.Tensor | None = None) -> None:
    """Row pass of one (T, Vp) bf16/fp16 logits chunk (``sisa_lmce_rows``): loss rows (and lse if given) and, when
    ``inv_n`` (device scalar 1/N_valid) is given, G over the logits in place."""
    T, Vp = logits.shape
    if T == 0:
        return
    if logits.stride(1) != 1:
        raise ValueError("lmce_rows: the logits chunk must have unit column stride")
    if labels.dtype != torch.int64 or not labels.is_contiguous() or labels.numel() != T:
        raise ValueError(f"lmce_rows: expected {T} contiguous int64 labels")
    args = _lib.LmceRowsArgs(T, int(V), Vp, logits.stride(0), _lib.dtype_code(logits.dtype), int(inv_n is not None),
                             logits.data_ptr(), labels.data_ptr(), int(ignore_index), _lib.ptr(inv_n), float(gscale),
                             loss_rows.data_ptr(), _lib.ptr(lse))
    _lib.call("sisa_lmce_rows", args, logits)


def lmce_fused_loss_rows(x: torch.Tensor, wpad: torch.Tensor, labels: torch.Tensor, V: int, ignore_index: int,
                         lse: torch.Tensor | None = None) -> torch.Tensor:
    """Loss rows (N,) fp32 of ``x`` (N, D) against the padded weight ``wpad`` (Vp, D) from the fused kernel
    (``sisa_lmce_fwd``): no logits buffer. D must be a multiple of 64; writes ``lse`` (natural log) if given."""
    N, D = x.shape
    out = torch.empty(N, dtype=torch.float32, device=x.device)
    if N == 0:
        return out
    ws = torch.empty(max(1, _lib.workspace_bytes("sisa_lmce_fwd_workspace_bytes", N, wpad.shape[0]) // 4),
                     dtype=torch.float32, device=x.device)
    args = _lib.LmceFwdArgs(N, int(V), wpad.shape[0], D, _lib.dtype_code(x.dtype), x.data_ptr(), x.stride(0),
                            wpad.data_ptr(), wpad.stride(0), labels.data_ptr(), int(ignore_index), _lib.ptr(lse),
                            out.data_ptr(), ws.data_ptr())
    _lib.call("sisa_lmce_fwd", args, x)
    return out


def lmce_train_chunk(x: torch.Tensor, wpad: torch.Tensor, labels: torch.Tensor, V: int, ignore_index: int,
                     inv_n: torch.Tensor, gscale: float, loss_rows: torch.Tensor, dx: torch.Tensor | None,
                     dw: torch.Tensor | None, accumulate: bool, workspace: torch.Tensor, dx_splits: int = 0,
                     lse: torch.Tensor | None = None) -> None:
    """One chunk of the training pass (``sisa_lmce_train``): x (n, D) rows, the padded weight (Vp, D), labels (n,)
    int64; writes loss_rows (n,), dx (n, D) fp32 (if given) and dW (Vp, D) fp32 (written, or added with
    ``accumulate``), for G scaled by the device scalar ``inv_n`` times ``gscale``."""
    n, D = x.shape
    if n == 0:
        return
    args = _lib.LmceTrainArgs(n, int(V), wpad.shape[0], D, _lib.dtype_code(x.dtype), x.data_ptr(), x.stride(0),
                              wpad.data_ptr(), wpad.stride(0), labels.data_ptr(), int(ignore_index), inv_n.data_ptr(),
                              float(gscale), loss_rows.data_ptr(), _lib.ptr(lse), _lib.ptr(dx),
                              dx.stride(0) if dx is not None else 0, _lib.ptr(dw), dw.stride(0) if dw is not None else 0,
                              int(bool(accumulate)), int(dx_splits), workspace.data_ptr())
    _lib.call("sisa_lmce_train", args, x)


def train_workspace(chunk_sizes, Vp: int, D: int, device, dx_splits: int = 0) -> torch.Tensor:
    """A 256-byte aligned byte buffer for ``sisa_lmce_train`` on chunks of each of the given row counts."""
    need = max(_lib.workspace_bytes("sisa_lmce_train_workspace_bytes", n, Vp, D, dx_splits) for n in chunk_sizes)
    ws = torch.empty(max(1, need) + 256, dtype=torch.uint8, device=device)
    skip = (-ws.data_ptr()) % 256
    return ws[skip:skip + max(1, need)]


class _Problem:
    """One call's operands in the compute dtype: x (N, D) contiguous, the padded weight, int64 labels, and the
    device scalars N_valid and 1/N_valid."""

    def __init__(self, hidden: torch.Tensor, weight: torch.Tensor, labels: torch.Tensor, ignore_index: int,
                 cdtype: torch.dtype):
        D = hidden.shape[-1]
        Dp = -(-D // HIDDEN_MULTIPLE) * HIDDEN_MULTIPLE
        x = hidden.reshape(-1, D).to(cdtype)
        if Dp != D:     # zero columns: the logits, and the kept columns of dx and dW, do not change
            x = F.pad(x, (0, Dp - D))
        self.x = x.contiguous()
        self.wpad = padded_weight(weight, cdtype, Dp)
        self.labels = labels.reshape(-1).to(torch.int64).contiguous()
        self.V, self.ignore_index = weight.shape[0], int(ignore_index)
        self.N, self.D = self.x.shape[0], D
        self.n_valid = (self.labels != self.ignore_index).sum()

    def loss_without_grad(self) -> torch.Tensor:
        rows = lmce_fused_loss_rows(self.x, self.wpad, self.labels, self.V, self.ignore_index)
        return rows.sum() / self.n_valid

    def loss_and_grads(self, want_dx: bool, want_dw: bool, gscale: float, chunk_tokens: int | None):
        """The chunk loop: loss and, as requested, dL/dx (N, D) and dL/dW_pad (Vp, D) in fp32 for a unit seed
        (times ``gscale``)."""
        N, Dp, dev = self.N, self.x.shape[1], self.x.device
        Vp = self.wpad.shape[0]
        rows = torch.empty(N, dtype=torch.float32, device=dev)
        dx = torch.empty((N, Dp), dtype=torch.float32, device=dev) if want_dx else None
        dw = (torch.zeros if N == 0 else torch.empty)((Vp, Dp), dtype=torch.float32, device=dev) if want_dw else None
        inv_n = torch.reciprocal(self.n_valid.to(torch.float32)).reshape(1)
        step = chunk_rows(N, Vp, chunk_tokens, self.wpad.element_size())
        if N:
            ws = train_workspace({min(step, N), N - (N - 1) // step * step}, Vp, Dp, dev)   # this loop's chunk sizes
            for r0 in range(0, N, step):
                r1 = min(N, r0 + step)
                lmce_train_chunk(self.x[r0:r1], self.wpad, self.labels[r0:r1], self.V, self.ignore_index, inv_n,
                                 gscale, rows[r0:r1], None if dx is None else dx[r0:r1], dw, r0 > 0, ws)
        if dx is not None and Dp != self.D:
            dx = dx[:, :self.D]
        if dw is not None and Dp != self.D:
            dw = dw[:, :self.D]
        return rows.sum() / self.n_valid, dx, dw


class _LinearCE(torch.autograd.Function):
    """Loss in the forward pass; the gradients, computed there too, are scaled by the seed in the backward pass."""

    @staticmethod
    def forward(ctx, hidden, weight, labels, ignore_index, chunk_tokens, grad_scale, cdtype, want_dx, want_dw):
        prob = _Problem(hidden, weight, labels, ignore_index, cdtype)
        gscale = 1.0 if grad_scale is None else float(grad_scale)
        loss, dx, dw = prob.loss_and_grads(want_dx, want_dw, gscale, chunk_tokens)
        ctx.meta = (hidden.shape, hidden.dtype, weight.dtype, prob.V, grad_scale)
        ctx.save_for_backward(dx, dw)
        return loss

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, seed):
        dx, dw = ctx.saved_tensors
        shape, h_dtype, w_dtype, V, promised = ctx.meta
        if promised is None:
            s = seed.to(torch.float32)
            dx = None if dx is None else dx * s
            dw = None if dw is None else dw[:V] * s
        else:   # G already carries the promised seed: check it on the device, no host synchronisation
            torch._assert_async(seed.to(torch.float32) == float(promised),
                                "linear_cross_entropy: the backward seed is not the promised grad_scale")
            dw = None if dw is None else dw[:V]
        dh = None if dx is None else dx.reshape(shape).to(h_dtype)
        dW = None if dw is None else dw.to(w_dtype)
        return dh, dW, None, None, None, None, None, None, None


def reference_linear_cross_entropy(hidden: torch.Tensor, weight: torch.Tensor, labels: torch.Tensor,
                                   ignore_index: int = -100) -> torch.Tensor:
    """``F.cross_entropy(F.linear(hidden, weight).float(), labels, ignore_index=ignore_index)`` over all rows (the
    reference's eager definition, linear_ce.py:220-224)."""
    logits = F.linear(hidden, weight)
    return F.cross_entropy(logits.reshape(-1, logits.shape[-1]).float(), labels.reshape(-1),
                           ignore_index=ignore_index)


@torch.compiler.disable
def linear_cross_entropy(hidden: torch.Tensor, weight: torch.Tensor, labels: torch.Tensor, ignore_index: int = -100,
                         *, chunk_tokens: int | None = None, grad_scale: float | None = None) -> torch.Tensor:
    """Mean cross-entropy of ``hidden @ weight.T`` against ``labels`` (fp32 scalar) without the full logits.

    hidden ``(..., D)``; weight ``(V, D)`` (the tied embedding; fp32 master or 16-bit); labels ``(...)`` integer
    targets, one per hidden row, not shifted; rows equal to ``ignore_index`` add neither loss nor gradient (the loss
    is NaN when all are ignored). ``chunk_tokens``: token rows per chunk of the gradient pass (default: chunks of at
    most 1 GiB of logits). ``grad_scale``: promise that the backward seed is exactly this value (G is scaled in the
    forward pass; a different seed trips a device-side assert). The compute dtype is the autocast dtype when autocast
    is on, else ``hidden.dtype``; CPU tensors and fp32 use the eager formula.
    """
    cdtype = backends.compute_dtype(hidden)
    if not hidden.is_cuda or cdtype not in (torch.bfloat16, torch.float16):
        return reference_linear_cross_entropy(hidden, weight, labels, ignore_index)
    D = hidden.shape[-1]
    if weight.dim() != 2 or weight.shape[1] != D:
        raise ValueError(f"linear_cross_entropy: weight must have shape (V, {D}); got {tuple(weight.shape)}")
    rows = hidden.numel() // D if D else 0
    if labels.numel() != rows:
        raise ValueError(f"linear_cross_entropy: {labels.numel()} labels for {rows} hidden rows")
    grads = torch.is_grad_enabled()
    want_dx, want_dw = grads and hidden.requires_grad, grads and weight.requires_grad
    if not (want_dx or want_dw):
        with torch.no_grad():
            return _Problem(hidden, weight, labels, ignore_index, cdtype).loss_without_grad()
    return _LinearCE.apply(hidden, weight, labels, ignore_index, chunk_tokens, grad_scale, cdtype, want_dx, want_dw)


def flops(N: int, V: int, D: int) -> dict:
    """Algorithmic work: the logits GEMM (also the whole of the fused no-gradient forward) and, with gradients, the
    dx and dW GEMMs -- 2 N V D flop each."""
    g = 2.0 * N * V * D
    return {"logits": g, "dx": g, "dw": g, "total": 3 * g, "forward": g}
