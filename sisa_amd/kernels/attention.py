"""Exact SISA attention on gfx950 HIP kernels: host cores, autograd wrapper and the public entry point.

    s_ij = q_i.k_j / sqrt(D) + lam_h * exp(g_i - g_j) * (c_i.b_j) + (F_i - F_j)        (j <= i)
    o_i  = sum_j softmax_j(s_ij) v_j

Mirrors the host side of the reference's ``sisa.kernels.attention`` (src/sisa/kernels/attention.py:666-877): the
same core functions (``attn_forward``, ``attn_backward``), the same autograd contract (``_SISAAttentionFn``), the
same validation (``_prepare_inputs``) and the public ``sisa_attention_hip`` (the counterpart of
``sisa_attention_triton``). The arithmetic runs in ``libsisa_hip.so`` (sisa_amd/csrc/attention.hip).

Numerics (as the reference's notes (A)-(E), attention.py:9-78): the decay is applied in fp32 after the c.b product,
chunk-factored over 64-row blocks; differences are taken before log2(e); the backward uses the exact delta with the
self-normalised fp32 o'' stored by the forward pass and the delta-free diagonal dS_tt. Deterministic (no atomics).
"""
from __future__ import annotations

import math

import torch

from .. import backends
from . import _lib

__all__ = ["sisa_attention_hip", "attn_forward", "attn_backward"]

# Maximum allowed increase of g between neighbouring positions (fp32 cumulative sums of non-positive increments can
# rise by a few ulps). Reference: attention.py:125.
MONOTONE_TOL = 1e-3
BLOCK = 64


def _aligned(x: torch.Tensor) -> bool:
    """Rows readable with 16-byte vector loads: contiguous last axis, 16-byte aligned base and row strides."""
    es = x.element_size()
    if x.stride(-1) != 1 or x.data_ptr() % 16:
        return False
    return all((s * es) % 16 == 0 for s in x.stride()[:-1])


def _ready(x: torch.Tensor) -> torch.Tensor:
    return x if _aligned(x) else x.contiguous()


def _like(x: torch.Tensor) -> torch.Tensor:
    return torch.empty_like(x) if _aligned(x) else torch.empty(x.shape, device=x.device, dtype=x.dtype)


def _check_monotone(mono: torch.Tensor, mode: str) -> None:
    if mode == "off":
        return
    if mode == "sync":
        mx = float(mono.max())
        if not mx <= MONOTONE_TOL:
            raise ValueError(f"g must be non-increasing along the sequence (max increase {mx:.3e} > {MONOTONE_TOL})")
    else:
        torch._assert_async(mono.max() <= MONOTONE_TOL, "SISA attention: g must be non-increasing along the sequence")


def compute_factors(g: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """rowf, colf ((B,H,L) fp32 contiguous) and the per-64-block maximum increase of g."""
    B, H, L = g.shape
    nt = -(-L // BLOCK)
    rowf = torch.empty((B, H, L), device=g.device, dtype=torch.float32)
    colf = torch.empty_like(rowf)
    mono = torch.empty((B * H * nt,), device=g.device, dtype=torch.float32)
    _lib.call("sisa_factors", _lib.FactorsArgs(B, H, L, _lib.view(g), rowf.data_ptr(), colf.data_ptr(),
                                                mono.data_ptr()), g)
    return rowf, colf, mono


def attn_forward(q, k, v, c, b, g, lam, fgate, factors=None, check=None, want32=False):
    """Forward core (no autograd).

    ``factors=(rowf, colf)`` (built by the fused preparation, 64-row blocks) skips the factor kernel and the
    monotonicity check. ``check`` overrides the global check mode. ``want32=True`` also returns the self-normalised
    fp32 o'' = sum DT(pe)v / sum DT(pe) as a contiguous (B,H,L,D) tensor (fp32 inputs: o itself).

    Returns ``(o, lse, rowf, colf, cfg, o32 or None)``; o is a (B,H,L,D) tensor in (B,L,H,D) memory layout and lse
    is in log2 units. Reference: attention.py:686-727.
    """
    B, H, L, D = q.shape
    dev = q.device
    cfg = backends.attention_config(dev, q.dtype)
    has_f = fgate is not None
    if factors is None:
        rowf, colf, mono = compute_factors(g)
        if L > 1:
            _check_monotone(mono, backends.get_check_mode() if check is None else check)
    else:
        rowf, colf = factors
        assert rowf.is_contiguous() and colf.is_contiguous()
    # o in (B,L,H,D) memory layout, so the layer's transpose(1,2).reshape is a view
    o = torch.empty_strided((B, H, L, D), (L * H * D, D, H * D, 1), device=dev, dtype=q.dtype)
    lse = torch.empty((B, H, L), device=dev, dtype=torch.float32)
    store32 = bool(want32) and q.dtype != torch.float32
    o32 = torch.empty((B, H, L, D), device=dev, dtype=torch.float32) if store32 else None
    args = _lib.AttnFwdArgs(B, H, L, _lib.dtype_code(q.dtype), _lib.view(q), _lib.view(k), _lib.view(v),
                            _lib.view(c), _lib.view(b), _lib.view(g), _lib.view(fgate if has_f else None),
                            lam.data_ptr(), lam.stride(0), rowf.data_ptr(), colf.data_ptr(), _lib.view(o),
                            lse.data_ptr(), _lib.ptr(o32))
    _lib.call("sisa_attn_fwd", args, q)
    if want32 and not store32:
        o32 = o
    return o, lse, rowf, colf, cfg, o32


def attn_backward(q, k, v, c, b, g, fgate, rowf, colf, lam, o, lse, do, exact=True,
                  dq=None, dk=None, dv=None, dc=None, db=None, o32=None):
    """Backward core (no autograd); the exact-delta scheme.

    dq .. db may be caller buffers of any 16-byte-aligned strides (e.g. views of the fused layer's d proj, fp32
    dc/db). ``o32`` is the self-normalised fp32 o'' of ``attn_forward(want32=True)`` (None: delta = o.do).
    Returns ``(dq, dk, dv, dc, db, dg, dlam (H,), dF or None)``. Reference: attention.py:730-784.
    """
    B, H, L, D = q.shape
    dev = q.device
    has_f = fgate is not None
    do = _ready(do)
    dq = _like(q) if dq is None else dq
    dk = _like(k) if dk is None else dk
    dv = _like(v) if dv is None else dv
    dc = _like(c) if dc is None else dc
    db = _like(b) if db is None else db
    if dc.dtype != db.dtype or dc.dtype not in (q.dtype, torch.float32):
        raise TypeError(f"dc/db must share dtype {q.dtype} or float32, got {dc.dtype}/{db.dtype}")
    for name, t in (("dq", dq), ("dk", dk), ("dv", dv), ("dc", dc), ("db", db)):
        if not _aligned(t):
            raise ValueError(f"{name} buffer rows must be 16-byte aligned with a contiguous last axis")
    if dq.dtype != q.dtype or dk.dtype != q.dtype or dv.dtype != q.dtype:
        raise TypeError("dq/dk/dv buffers must have the dtype of q")
    f32 = dict(device=dev, dtype=torch.float32)
    dg = torch.empty((B, H, L), **f32)
    dF = torch.empty((B, H, L), **f32) if has_f else None
    dlam = torch.empty((H,), **f32)
    ws = torch.empty((_lib.workspace_bytes("sisa_attn_bwd_workspace_bytes", B, H, L) // 4,), **f32)
    has32 = bool(exact) and o32 is not None and o32 is not o
    if has32:
        assert o32.shape == (B, H, L, D) and o32.is_contiguous() and o32.dtype == torch.float32
    args = _lib.AttnBwdArgs(B, H, L, _lib.dtype_code(q.dtype), _lib.dtype_code(dc.dtype),
                            _lib.view(q), _lib.view(k), _lib.view(v), _lib.view(c), _lib.view(b), _lib.view(g),
                            _lib.view(fgate if has_f else None), lam.data_ptr(), lam.stride(0),
                            rowf.data_ptr(), colf.data_ptr(), _lib.view(o), o32.data_ptr() if has32 else None,
                            lse.data_ptr(), _lib.view(do), _lib.view(dq), _lib.view(dk), _lib.view(dv),
                            _lib.view(dc), _lib.view(db), dg.data_ptr(), _lib.ptr(dF), dlam.data_ptr(),
                            ws.data_ptr(), 1 if exact else 0)
    _lib.call("sisa_attn_bwd", args, q)
    return dq, dk, dv, dc, db, dg, dlam, dF


class _SISAAttentionFn(torch.autograd.Function):
    """Autograd wrapper of the HIP cores (exact-delta backward). Reference: attention.py:788-809."""

    @staticmethod
    def forward(ctx, q, k, v, c, b, g, lam, fgate, exact):
        need = bool(exact) and any(ctx.needs_input_grad)
        o, lse, rowf, colf, _, o32 = attn_forward(q, k, v, c, b, g, lam, fgate, want32=need)
        has_f = fgate is not None
        ctx.save_for_backward(q, k, v, c, b, g, fgate if has_f else g, rowf, colf, lam, o, lse,
                              o32 if (need and o32 is not o) else None)
        ctx.meta = (has_f, bool(exact))
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, c, b, g, Fp, rowf, colf, lam, o, lse, o32 = ctx.saved_tensors
        has_f, exact = ctx.meta
        dq, dk, dv, dc, db, dg, dlam, dF = attn_backward(q, k, v, c, b, g, Fp if has_f else None, rowf, colf, lam,
                                                         o, lse, do, exact, o32=o32)
        return dq, dk, dv, dc, db, dg, dlam, dF, None


def _prepare_inputs(q, k, v, c, b, g, lam, fgate):
    """Validation and dtype/stride normalisation (reference: attention.py:812-850)."""
    if q.dim() != 4 or q.shape[-1] != 64 or c.dim() != 4 or c.shape[-1] != 32:
        raise ValueError(f"the HIP kernels support d_head=64 and d_state=32 only; got q {tuple(q.shape)}, "
                         f"c {tuple(c.shape)}")
    if q.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise TypeError(f"q must be bf16, fp16 or fp32, got {q.dtype}")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise TypeError(f"q/k/v dtypes differ: {q.dtype}, {k.dtype}, {v.dtype}")
    if not (q.is_cuda and k.device == q.device and v.device == q.device and c.device == q.device
            and b.device == q.device and g.device == q.device and lam.device == q.device):
        raise ValueError("all inputs must be on the same GPU device")
    B, H, L, _ = q.shape
    if L < 1:
        raise ValueError("sequence length must be >= 1")
    if k.shape != q.shape or v.shape != q.shape:
        raise ValueError(f"k/v shapes {tuple(k.shape)}/{tuple(v.shape)} != q shape {tuple(q.shape)}")
    if c.shape != (B, H, L, 32) or b.shape != (B, H, L, 32):
        raise ValueError(f"c/b must have shape {(B, H, L, 32)}, got {tuple(c.shape)}/{tuple(b.shape)}")
    if g.dtype != torch.float32:
        raise TypeError(f"g must be fp32, got {g.dtype}")
    if g.shape != (B, H, L):
        raise ValueError(f"g must have shape {(B, H, L)}, got {tuple(g.shape)}")
    if fgate is not None:
        if fgate.dtype != torch.float32:
            raise TypeError(f"fgate must be fp32, got {fgate.dtype}")
        if fgate.shape != g.shape:
            raise ValueError(f"fgate shape {tuple(fgate.shape)} != g shape {tuple(g.shape)}")
        if fgate.device != q.device:
            raise ValueError("all inputs must be on the same GPU device")
    if lam.shape != (H,):
        raise ValueError(f"lam must have shape {(H,)}, got {tuple(lam.shape)}")
    if lam.dtype != torch.float32:
        lam = lam.float()
    if c.dtype != q.dtype:
        c = c.to(q.dtype)
    if b.dtype != q.dtype:
        b = b.to(q.dtype)
    q, k, v, c, b = [_ready(x) for x in (q, k, v, c, b)]
    return q, k, v, c, b, g, lam, fgate


def sisa_attention_hip(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, c: torch.Tensor, b: torch.Tensor,
                       g: torch.Tensor, lam: torch.Tensor, fgate: torch.Tensor | None = None) -> torch.Tensor:
    """Exact SISA attention (HIP, gfx950), differentiable with respect to every tensor argument.

    Computes ``o = softmax(s) v`` with, for ``j <= i``,
    ``s_ij = q_i.k_j / 8 + lam_h * exp(g_i - g_j) * (c_i.b_j) + (fgate_i - fgate_j)``.

    Args:
        q, k, v: ``(B, H, L, 64)`` bf16, fp16 or fp32. Any strides with a contiguous last dimension.
        c, b: ``(B, H, L, 32)`` rotated SSM read/write vectors (cast to ``q.dtype`` if they differ).
        g: ``(B, H, L)`` fp32 cumulative log-decay, non-increasing along L (checked per the check mode).
        lam: ``(H,)`` fp32 side-term weights ``softplus(lambda_raw)``.
        fgate: ``(B, H, L)`` fp32 cumulative log-sigmoid forget gate, or ``None``.

    Returns:
        ``(B, H, L, 64)`` in ``q.dtype``, stored in ``(B, L, H, 64)`` memory layout.

    Deterministic: two calls with the same inputs give bit-identical outputs and gradients.
    Reference counterpart: ``sisa_attention_triton`` (attention.py:853-877).
    """
    q, k, v, c, b, g, lam, fgate = _prepare_inputs(q, k, v, c, b, g, lam, fgate)
    return _SISAAttentionFn.apply(q, k, v, c, b, g, lam, fgate, True)


def flops(B: int, H: int, L: int, d_head: int = 64, d_state: int = 32) -> dict:
    """Algorithmic MFMA work (FlashAttention convention, causal pairs P = B*H*L^2/2)."""
    pairs = B * H * L * L / 2.0
    fwd = pairs * (4 * d_head + 2 * d_state)
    bwd = pairs * (10 * d_head + 6 * d_state)
    return dict(pairs=pairs, fwd=fwd, bwd=bwd, total=fwd + bwd, scale=1.0 / math.sqrt(d_head))
