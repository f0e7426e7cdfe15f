"""SISA attention as a function: the exact PyTorch implementation and the dispatcher over implementations.

Per head, query ``i`` scores key ``j <= i`` as::

    s_ij = q_i . k_j / sqrt(d_head)                 content term, no positional encoding
         + lam * exp(g_i - g_j) * (c_i . b_j)       state term; c, b rotated by the cumulative phase
         + (F_i - F_j)                              forget-gate term (optional)

and ``o_i = sum_j softmax_j(s_ij) v_j``. ``g = cumsum(-softplus(alpha))`` does not increase along the sequence,
``F = cumsum(logsigmoid(z))``, and ``c``, ``b`` are rotated pairwise by ``Phi = cumsum(theta)`` (:func:`rotate_pairs`).

Public names and signatures are the reference's ``sisa.functional`` (src/sisa/functional.py:38, 106, 181); the
accelerated implementation behind ``impl="hip"`` is :func:`sisa_amd.kernels.attention.sisa_attention_hip`.
"""
from __future__ import annotations

import contextlib

import torch
from torch import Tensor
from torch.utils.checkpoint import checkpoint

from . import backends
from .config import HIP_D_HEAD, HIP_D_STATE

__all__ = ["rotate_pairs", "sisa_attention_torch", "sisa_attention"]


def rotate_pairs(z: Tensor, phi: Tensor) -> Tensor:
    """Rotate the channel pairs ``(2m, 2m+1)`` of ``z`` (``(..., d_state)``) by the angles ``phi``
    (``(..., d_state // 2)``, radians), as the complex product ``(z_2m + i z_2m+1) * exp(i phi_m)``."""
    re, im = z.unflatten(-1, (-1, 2)).unbind(-1)
    cos, sin = torch.cos(phi), torch.sin(phi)
    return torch.stack((re * cos - im * sin, im * cos + re * sin), dim=-1).flatten(-2)


def working_dtype(dtype: torch.dtype) -> torch.dtype:
    """The precision of the torch path: float64 for float64 inputs, float32 for everything else."""
    return torch.float64 if dtype == torch.float64 else torch.float32


@contextlib.contextmanager
def autocast_disabled(device_type: str):
    """Run the enclosed products in their operands' dtype even when the caller has autocast on."""
    if torch.amp.is_autocast_available(device_type):
        with torch.autocast(device_type=device_type, enabled=False):
            yield
    else:
        yield


def attend_block(rows: tuple, keys: tuple, lam: Tensor, first: int) -> Tensor:
    """Exact attention output of ``M`` consecutive queries at positions ``first .. first+M-1`` over the keys at
    positions ``0 .. N-1``, in the operands' own dtype (autocast off).

    ``rows = (q, c, g, f)`` with ``q``, ``c`` of shape ``(B, H, M, .)`` and ``g``, ``f`` ``(B, H, M)``;
    ``keys = (k, v, b, g, f)`` with positions on dim 2 (``N`` of them); ``f`` is ``None`` on both sides without a
    forget gate. Keys after a query are masked, and so is their decay exponent before ``exp`` (``g_i - g_j`` grows
    without bound for ``j > i``). Same semantics as the reference's ``_attend_rows`` (src/sisa/functional.py:69-103).
    """
    q, c, g_row, f_row = rows
    k, v, b, g_key, f_key = keys
    with autocast_disabled(q.device.type):
        visible = torch.ones(q.shape[-2], k.shape[-2], dtype=torch.bool, device=q.device).tril(first)
        decay = torch.where(visible, g_row[..., :, None] - g_key[..., None, :], 0.0).exp()
        s = (q @ k.mT) * q.shape[-1] ** -0.5 + lam[:, None, None] * decay * (c @ b.mT)
        if f_row is not None:
            s = s + (f_row[..., :, None] - f_key[..., None, :])
        return torch.where(visible, s, float("-inf")).softmax(dim=-1) @ v


def _shape_errors(q: Tensor, k: Tensor, v: Tensor, c: Tensor, b: Tensor, g: Tensor, lam: Tensor,
                  fgate: Tensor | None, block_q: int) -> list[str]:
    if q.dim() != 4:
        return [f"q has shape {tuple(q.shape)}; expected (B, H, L, d_head)"]
    bhl, n_head = tuple(q.shape[:3]), q.shape[1]
    rules = (
        (k.shape == q.shape and tuple(v.shape[:3]) == bhl, f"k {tuple(k.shape)} and v {tuple(v.shape)} do not "
                                                           f"match q {tuple(q.shape)}"),
        (tuple(c.shape[:3]) == bhl and b.shape == c.shape, f"c {tuple(c.shape)} and b {tuple(b.shape)} are not "
                                                          f"(B, H, L, d_state) for (B, H, L) = {bhl}"),
        (c.shape[-1] % 2 == 0, f"d_state {c.shape[-1]} is odd; the state channels rotate in pairs"),
        (tuple(g.shape) == bhl, f"g has shape {tuple(g.shape)}, expected {bhl}"),
        (fgate is None or tuple(fgate.shape) == bhl, f"fgate has shape {None if fgate is None else tuple(fgate.shape)},"
                                                    f" expected {bhl}"),
        (tuple(lam.shape) == (n_head,), f"lam has shape {tuple(lam.shape)}, expected ({n_head},)"),
        (block_q > 0, f"block_q = {block_q} must be positive"),
    )
    return [msg for ok, msg in rules if not ok]


def sisa_attention_torch(q: Tensor, k: Tensor, v: Tensor, c: Tensor, b: Tensor, g: Tensor, lam: Tensor,
                         fgate: Tensor | None = None, block_q: int = 256) -> Tensor:
    """Exact SISA attention in plain PyTorch: any device, any ``d_head``, any even ``d_state``.

    Computes in float32 (float64 for float64 inputs) with autocast off and returns ``(B, H, L, d_head)`` in
    ``q.dtype``. Queries go in blocks of ``block_q``, each against the keys up to its last row, so at most a
    ``(B, H, block_q, L)`` score block exists at a time; under autograd every block is recomputed in the backward
    (activation checkpointing) to keep that bound. Counterpart of src/sisa/functional.py:106-155.
    """
    errors = _shape_errors(q, k, v, c, b, g, lam, fgate, block_q)
    if errors:
        raise ValueError("sisa_attention_torch: " + "; ".join(errors))
    wd = working_dtype(q.dtype)
    x = [None if t is None else t.to(wd) for t in (q, k, v, c, b, g, lam, fgate)]
    qw, kw, vw, cw, bw, gw, lw, fw = x
    seq_len = q.shape[2]
    recompute = (seq_len > block_q and torch.is_grad_enabled()
                 and any(t is not None and t.requires_grad for t in x))
    outs = []
    for first in range(0, seq_len, block_q):
        last = min(first + block_q, seq_len)
        rows = (qw[:, :, first:last], cw[:, :, first:last], gw[:, :, first:last],
                None if fw is None else fw[:, :, first:last])
        keys = (kw[:, :, :last], vw[:, :, :last], bw[:, :, :last], gw[:, :, :last],
                None if fw is None else fw[:, :, :last])
        outs.append(checkpoint(attend_block, rows, keys, lw, first, use_reentrant=False) if recompute
                    else attend_block(rows, keys, lw, first))
    return torch.cat(outs, dim=2).to(q.dtype)


_HIP_INPUT_DTYPES = (torch.bfloat16, torch.float16, torch.float32)


def _hip_unmet(q: Tensor, k: Tensor, v: Tensor, c: Tensor, g: Tensor, fgate: Tensor | None) -> list[str]:
    """What stops the HIP attention kernels from taking these prepared inputs (empty: nothing)."""
    if q.device.type != "cuda":
        return [f"the inputs are on the {q.device.type}; the HIP kernels run on a GPU"]
    unmet = []
    ok, why = backends.hip_status(q.device)
    if not ok:
        unmet.append(why)
    if (q.shape[-1], c.shape[-1]) != (HIP_D_HEAD, HIP_D_STATE):
        unmet.append(f"d_head {q.shape[-1]} and d_state {c.shape[-1]}: the kernels are built for {HIP_D_HEAD} and "
                     f"{HIP_D_STATE}")
    if k.dtype != q.dtype or v.dtype != q.dtype or q.dtype not in _HIP_INPUT_DTYPES:
        unmet.append(f"q, k, v are {q.dtype}, {k.dtype}, {v.dtype}: the kernels take one of bf16, fp16, fp32 for "
                     f"all three")
    wide = [n for n, t in (("g", g), ("fgate", fgate)) if t is not None and t.dtype != torch.float32]
    if wide:
        unmet.append(f"{' and '.join(wide)} must be float32 (cumulative sums lose their low bits in 16-bit types)")
    return unmet


def sisa_attention(q: Tensor, k: Tensor, v: Tensor, c: Tensor, b: Tensor, g: Tensor, lam: Tensor,
                   fgate: Tensor | None = None, impl: str = "auto", block_q: int = 256) -> Tensor:
    """SISA attention of prepared inputs by ``impl``.

    ``"torch"`` is :func:`sisa_attention_torch` (``block_q`` is its query block); ``"hip"`` the gfx950 kernels
    (GPU, ``d_head`` 64, ``d_state`` 32, float32 ``g``/``fgate``), raising ``ValueError`` with the reasons when the
    inputs do not qualify; ``"auto"`` is ``"hip"`` when they qualify and ``"torch"`` otherwise (warned once per
    reason on a GPU). ``"hip_fused"`` includes the projections and is a layer-level choice only.
    Returns ``(B, H, L, d_head)`` in ``q.dtype``.
    """
    if impl == "hip_fused":
        raise ValueError("impl='hip_fused' starts from the layer input (it fuses the projections); set it through "
                         "SISAConfig.attn_impl, or pass impl='hip' for prepared inputs")
    if impl not in ("auto", "torch", "hip"):
        raise ValueError(f"unknown impl {impl!r}: sisa_attention runs 'auto', 'torch' or 'hip'")
    if impl != "torch":
        unmet = _hip_unmet(q, k, v, c, g, fgate)
        if not unmet:
            from .kernels.attention import sisa_attention_hip
            return sisa_attention_hip(q, k, v, c, b, g, lam, fgate)
        if impl == "hip":
            raise ValueError(f"impl='hip' is not available: {'; '.join(unmet)}")
        if q.device.type == "cuda":
            backends.warn_fallback(q.device, "; ".join(unmet))
    return sisa_attention_torch(q, k, v, c, b, g, lam, fgate, block_q=block_q)
