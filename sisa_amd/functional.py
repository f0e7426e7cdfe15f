"""Functional form of SISA attention: the pure-PyTorch implementation and the backend dispatcher.

For each head the score of query ``i`` and key ``j <= i`` is::

    s_ij = q_i . k_j / sqrt(d_head)                      content term (no positional encoding)
         + lam_h * exp(g_i - g_j) * (c_i . b_j)          SSM term, c and b already rotated
         + (F_i - F_j)                                   forget-gate term

and ``o_i = sum_j softmax_j(s_ij) v_j``. ``g`` is the non-increasing cumulative log-decay ``cumsum(-softplus(a))``,
``F`` the cumulative log-sigmoid forget gate and ``c``, ``b`` the SSM read/write vectors rotated pairwise by the
cumulative phase ``Phi = cumsum(theta)``.

Same public API as the reference's ``sisa.functional`` (src/sisa/functional.py:35, 38, 106, 181): ``rotate_pairs``,
``sisa_attention_torch`` and the dispatcher ``sisa_attention`` whose accelerated backend here is ``impl="hip"``.
"""
from __future__ import annotations

import contextlib
import math
import warnings

import torch
from torch import Tensor
from torch.utils.checkpoint import checkpoint

__all__ = ["rotate_pairs", "sisa_attention_torch", "sisa_attention"]

HIP_D_HEAD = 64
HIP_D_STATE = 32


def rotate_pairs(z: Tensor, phi: Tensor) -> Tensor:
    """Rotate interleaved channel pairs ``(0, 1), (2, 3), ...`` of ``z`` (``(..., d_state)``) by ``phi``
    (``(..., d_state // 2)`` radians): ``(e, o) -> (e cos - o sin, e sin + o cos)``."""
    pairs = z.unflatten(-1, (-1, 2))
    e, o = pairs[..., 0], pairs[..., 1]
    cs, sn = phi.cos(), phi.sin()
    return torch.stack((e * cs - o * sn, e * sn + o * cs), dim=-1).flatten(-2)


def _work_dtype(dtype: torch.dtype) -> torch.dtype:
    """float32, or float64 when the inputs already are float64."""
    return torch.float64 if dtype == torch.float64 else torch.float32


_AUTOCAST_DEVICE_TYPES = frozenset(d for d in ("cuda", "cpu", "xpu", "hpu", "mps") if torch.amp.is_autocast_available(d))


def _autocast_off(device_type: str):
    if device_type in _AUTOCAST_DEVICE_TYPES:
        return torch.autocast(device_type=device_type, enabled=False)
    return contextlib.nullcontext()


def _attend_rows(q: Tensor, k: Tensor, v: Tensor, c: Tensor, b: Tensor, g_q: Tensor, g_k: Tensor, lam: Tensor,
                 f_q: Tensor | None, f_k: Tensor | None, q_start: int) -> Tensor:
    """Exact attention of the query rows ``q_start .. q_start+M-1`` against keys ``0 .. N-1`` in the inputs' dtype
    (autocast disabled). The decay exponent is masked before ``exp`` so that future keys cannot overflow."""
    with _autocast_off(q.device.type):
        m, n = q.shape[-2], k.shape[-2]
        rows = torch.arange(q_start, q_start + m, device=q.device).unsqueeze(1)
        cols = torch.arange(n, device=q.device).unsqueeze(0)
        future = cols > rows                                                   # (M, N)
        logits = (q @ k.transpose(-1, -2)) / math.sqrt(q.shape[-1])
        expo = (g_q.unsqueeze(-1) - g_k.unsqueeze(-2)).masked_fill(future, 0.0)
        logits = logits + lam.view(1, -1, 1, 1) * expo.exp() * (c @ b.transpose(-1, -2))
        if f_q is not None:
            logits = logits + (f_q.unsqueeze(-1) - f_k.unsqueeze(-2))
        weights = logits.masked_fill(future, float("-inf")).softmax(dim=-1)
        return weights @ v


def sisa_attention_torch(q: Tensor, k: Tensor, v: Tensor, c: Tensor, b: Tensor, g: Tensor, lam: Tensor,
                         fgate: Tensor | None = None, block_q: int = 256) -> Tensor:
    """Exact SISA attention in plain PyTorch (any device, any ``d_head``, any even ``d_state``).

    Inputs are cast to float32 (float64 stays float64); scores, softmax and ``P @ V`` run in that precision with
    autocast disabled, and the output is cast back to ``q.dtype``. Query blocks of ``block_q`` rows attend to the keys
    up to the end of their block; with gradients each block is checkpointed, so memory stays ``O(block_q * L)``.

    Returns ``(B, H, L, d_head)`` in ``q.dtype``. Reference counterpart: src/sisa/functional.py:106-155.
    """
    if q.dim() != 4:
        raise ValueError(f"q must be (B, H, L, d_head), got shape {tuple(q.shape)}")
    bsz, n_head, seq_len, _ = q.shape
    if k.shape != q.shape or v.shape[:3] != q.shape[:3]:
        raise ValueError(f"q, k, v shapes do not match: {tuple(q.shape)}, {tuple(k.shape)}, {tuple(v.shape)}")
    if c.shape[:3] != q.shape[:3] or b.shape != c.shape or c.shape[-1] % 2 != 0:
        raise ValueError(f"c and b must be (B, H, L, d_state) with even d_state, got {tuple(c.shape)}, "
                         f"{tuple(b.shape)}")
    if g.shape != q.shape[:3] or (fgate is not None and fgate.shape != g.shape):
        raise ValueError("g and fgate must be (B, H, L)")
    if lam.shape != (n_head,):
        raise ValueError(f"lam must be ({n_head},), got {tuple(lam.shape)}")
    if block_q <= 0:
        raise ValueError("block_q must be positive")
    out_dtype = q.dtype
    wd = _work_dtype(q.dtype)
    q, k, v, c, b, g, lam = (t.to(wd) for t in (q, k, v, c, b, g, lam))
    fgate = None if fgate is None else fgate.to(wd)
    grad = torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in (q, k, v, c, b, g, lam, fgate))
    pieces = []
    for start in range(0, seq_len, block_q):
        end = min(start + block_q, seq_len)
        args = (q[:, :, start:end], k[:, :, :end], v[:, :, :end], c[:, :, start:end], b[:, :, :end],
                g[:, :, start:end], g[:, :, :end], lam,
                None if fgate is None else fgate[:, :, start:end], None if fgate is None else fgate[:, :, :end], start)
        pieces.append(checkpoint(_attend_rows, *args, use_reentrant=False) if grad and seq_len > block_q
                      else _attend_rows(*args))
    out = pieces[0] if len(pieces) == 1 else torch.cat(pieces, dim=2)
    return out.to(out_dtype)


def _hip_problem(q: Tensor, k: Tensor, v: Tensor, c: Tensor, g: Tensor, fgate: Tensor | None) -> str | None:
    """Why the HIP attention kernels cannot take these inputs, or ``None``."""
    if q.device.type != "cuda":
        return f"inputs are on {q.device.type}, the HIP kernels need a GPU"
    if q.shape[-1] != HIP_D_HEAD or c.shape[-1] != HIP_D_STATE:
        return (f"the HIP kernels need d_head={HIP_D_HEAD} and d_state={HIP_D_STATE}, "
                f"got {q.shape[-1]} and {c.shape[-1]}")
    if q.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        return f"unsupported dtype {q.dtype} (bf16, fp16 or fp32)"
    if k.dtype != q.dtype or v.dtype != q.dtype:
        return f"q, k and v must share one dtype, got {q.dtype}, {k.dtype}, {v.dtype}"
    if g.dtype != torch.float32 or (fgate is not None and fgate.dtype != torch.float32):
        return f"g and fgate must be float32, got {g.dtype} and {None if fgate is None else fgate.dtype}"
    from . import backends

    ok, why = backends.hip_status(q.device)
    return None if ok else why


def sisa_attention(q: Tensor, k: Tensor, v: Tensor, c: Tensor, b: Tensor, g: Tensor, lam: Tensor,
                   fgate: Tensor | None = None, impl: str = "auto", block_q: int = 256) -> Tensor:
    """SISA attention with a selectable backend.

    Args:
        impl: ``"torch"`` (:func:`sisa_attention_torch`), ``"hip"`` (the gfx950 HIP kernels; GPU, ``d_head`` 64,
            ``d_state`` 32) or ``"auto"`` (HIP when possible, else torch). Forcing ``"hip"`` on inputs it cannot
            take raises ``ValueError``. ``"hip_fused"`` fuses the projections and exists only at the layer level.
        block_q: Query block size of the torch backend.

    Returns:
        ``(B, H, L, d_head)`` in ``q.dtype``.
    """
    if impl == "auto":
        why = _hip_problem(q, k, v, c, g, fgate)
        impl = "hip" if why is None else "torch"
        if why is not None and q.device.type == "cuda":
            from . import backends

            key = (q.device.index, why)
            if key not in backends._WARNED:
                backends._WARNED.add(key)
                warnings.warn(f"SISA: using the torch attention implementation on the GPU because {why}",
                              stacklevel=2)
    if impl == "torch":
        return sisa_attention_torch(q, k, v, c, b, g, lam, fgate, block_q=block_q)
    if impl == "hip":
        why = _hip_problem(q, k, v, c, g, fgate)
        if why is not None:
            raise ValueError(f"impl='hip' is not available: {why}")
        from .kernels.attention import sisa_attention_hip

        return sisa_attention_hip(q, k, v, c, b, g, lam, fgate)
    if impl == "hip_fused":
        raise ValueError("impl='hip_fused' fuses the input projections and is only available through "
                         "SISAAttention / SISAConfig.attn_impl; use impl='hip' for prepared inputs")
    raise ValueError(f"unknown impl {impl!r}; expected 'auto', 'torch' or 'hip'")
