"""Decode-step attention on the HIP kernel ``sisa_decode_attn`` (``include/sisa_hip.h``): the new query rows of a
decode step against the layer's cache, with the semantics of the reference's ``_attend_rows``
(src/sisa/functional.py:69-93) in float32: inputs in the compute dtype (bf16, fp16 or fp32), g and F in float32,
the result in float32 ``(B, H, M, 64)``.
"""
from __future__ import annotations

import torch
from torch import Tensor

from . import _lib

__all__ = ["sisa_decode_hip"]


def _rows16(t: Tensor) -> Tensor:
    """A (B,H,L,w) view whose rows are 16-byte aligned with a unit last stride (copy otherwise)."""
    es = t.element_size()
    ok = (t.stride(-1) == 1 and t.data_ptr() % 16 == 0
          and all((t.stride(i) * es) % 16 == 0 for i in range(3)))
    return t if ok else t.contiguous()


@torch.no_grad()
def sisa_decode_hip(q: Tensor, k: Tensor, v: Tensor, c: Tensor, b: Tensor, g_q: Tensor, g_k: Tensor, lam: Tensor,
                    f_q: Tensor | None, f_k: Tensor | None, q_start: int) -> Tensor:
    """Exact SISA attention of the query rows ``q_start .. q_start+M-1`` against keys ``0 .. N-1``: ``q, c``
    ``(B,H,M,64|32)``, ``k, v, b`` ``(B,H,N,64|32)`` in one dtype, ``g_q, f_q`` ``(B,H,M)`` and ``g_k, f_k``
    ``(B,H,N)`` float32, ``lam`` ``(H,)``. Returns ``(B,H,M,64)`` float32 (inference only: no autograd). Any M: a
    launch takes fewer than 65,536 (batch, head, query) rows, so longer query blocks (chunked prefill into a filled
    cache) run as several launches over row ranges."""
    B, H, M, D = q.shape
    N = k.shape[2]
    if D != 64 or c.shape[-1] != 32:
        raise ValueError(f"sisa_decode_hip: d_head must be 64 and d_state 32, got {D} and {c.shape[-1]}")
    if not (q.dtype == k.dtype == v.dtype == c.dtype == b.dtype):
        raise TypeError("sisa_decode_hip: q, k, v, c, b must share one dtype")
    if q_start < 0 or q_start + M > N:
        raise ValueError(f"sisa_decode_hip: query rows {q_start}..{q_start + M - 1} outside the {N} cached positions")
    if (f_q is None) != (f_k is None):
        raise ValueError("sisa_decode_hip: f_q and f_k must be given together")
    q = q if q.stride(-1) == 1 else q.contiguous()
    c = c if c.stride(-1) == 1 else c.contiguous()
    k, v, b = _rows16(k), _rows16(v), _rows16(b)
    g_q, g_k = g_q.float(), g_k.float()
    f_q = None if f_q is None else f_q.float()
    f_k = None if f_k is None else f_k.float()
    lam = lam.float()
    rows = ROWS_PER_LAUNCH // (B * H)
    if rows < 1:
        raise ValueError(f"sisa_decode_hip: B*H = {B * H} query heads exceed one launch ({ROWS_PER_LAUNCH})")
    parts = []
    for m0 in range(0, M, rows):       # the grid holds fewer than 65,536 query rows: longer blocks go in pieces
        m1 = min(M, m0 + rows)
        parts.append(_launch(q[:, :, m0:m1], k, v, c[:, :, m0:m1], b, g_q[:, :, m0:m1], g_k,
                             None if f_q is None else f_q[:, :, m0:m1], f_k, lam, q_start + m0, N))
    return parts[0] if len(parts) == 1 else torch.cat(parts, 2)


ROWS_PER_LAUNCH = 65535


def _launch(q, k, v, c, b, g_q, g_k, f_q, f_k, lam, q_start, N):
    B, H, M, _ = q.shape
    out = torch.empty((B, H, M, 64), device=q.device, dtype=torch.float32)
    ws = torch.empty(_lib.workspace_bytes("sisa_decode_workspace_bytes", B, H, M, N) // 4, device=q.device,
                     dtype=torch.float32)
    args = _lib.DecodeArgs(B, H, M, N, _lib.dtype_code(q.dtype), int(q_start), _lib.view(q), _lib.view(k),
                           _lib.view(v), _lib.view(c), _lib.view(b), _lib.view(g_q), _lib.view(g_k), _lib.view(f_q),
                           _lib.view(f_k), lam.data_ptr(), lam.stride(0), out.data_ptr(), ws.data_ptr())
    _lib.call("sisa_decode_attn", args, q)
    return out
