"""Exact SISA attention on the gfx950 kernels of ``libsisa_hip.so``: the launch cores, the autograd function and the
public entry point.

    s_ij = q_i.k_j / 8 + lam_h exp(g_i - g_j) (c_i.b_j) + (F_i - F_j)        (j <= i),    o_i = sum_j softmax_j(s_ij) v_j

Public names and contracts are those of the reference's ``sisa.kernels.attention`` host half
(src/sisa/kernels/attention.py:686-877): ``attn_forward`` / ``attn_backward`` (no autograd; the fused layer calls them
with its own factor tables and gradient buffers) and ``sisa_attention_hip`` in place of ``sisa_attention_triton``.

The work per call is one C call each way. Forward: ``sisa_factors`` (per-64-row-block decay anchors rowf/colf and the
largest rise of ``g`` in each block) unless the caller brings factors, then ``sisa_attn_fwd``, which writes ``o`` in
(B, L, H, D) memory order, the row log-sum-exp (log2 units) and, for the exact backward, the self-normalised fp32
output o''. Backward: ``sisa_attn_bwd`` (two launches: dq with the fp64 dlambda sums of 16-row groups, then
dk/dv/db, in which one workgroup adds each head's group sums in a fixed order; deterministic). All numerics live in
csrc/attention.hip, csrc/attention_dq.hip and csrc/attention_bwd.hip.
"""
from __future__ import annotations

import math
from typing import NamedTuple

import torch

from .. import backends
from ..config import HIP_D_HEAD, HIP_D_STATE
from . import _lib

__all__ = ["sisa_attention_hip", "attn_forward", "attn_backward", "kernel_operands", "Forward", "Grads"]

#: Largest rise of ``g`` between neighbours that still counts as non-increasing: fp32 cumulative sums of non-positive
#: steps can go up by a few ulps (the reference allows 1e-3, src/sisa/kernels/attention.py:125).
MONOTONE_TOL = 1e-3
#: Decay-factor block of the kernels (rows per rowf/colf anchor).
BLOCK = 64
_INPUT_DTYPES = (torch.bfloat16, torch.float16, torch.float32)


class Forward(NamedTuple):
    """Result of :func:`attn_forward`: ``o`` (B, H, L, D) in (B, L, H, D) memory order, ``lse`` (B, H, L) fp32 in log2
    units, the decay factors ``rowf``/``colf`` (B, H, L) fp32, and ``o32`` -- the fp32 self-normalised output for the
    exact backward (``o`` itself for fp32 inputs) or ``None`` when not asked for."""
    o: torch.Tensor
    lse: torch.Tensor
    rowf: torch.Tensor
    colf: torch.Tensor
    o32: torch.Tensor | None


class Grads(NamedTuple):
    """Result of :func:`attn_backward`; ``dlam`` is (H,) and ``dF`` is ``None`` without a forget gate."""
    dq: torch.Tensor
    dk: torch.Tensor
    dv: torch.Tensor
    dc: torch.Tensor
    db: torch.Tensor
    dg: torch.Tensor
    dlam: torch.Tensor
    dF: torch.Tensor | None


def _vector_rows(x: torch.Tensor) -> bool:
    """Rows of ``x`` can be read with 16-byte loads: unit last stride, 16-byte aligned base and outer strides."""
    if x.stride(-1) != 1 or x.data_ptr() % 16:
        return False
    return all(s * x.element_size() % 16 == 0 for s in x.stride()[:-1])


def _readable(x: torch.Tensor) -> torch.Tensor:
    return x if _vector_rows(x) else x.contiguous()


def _output_like(x: torch.Tensor) -> torch.Tensor:
    """A gradient buffer for ``x``: its strides when those are vector-readable, else contiguous."""
    return torch.empty_like(x) if _vector_rows(x) else torch.empty(x.shape, device=x.device, dtype=x.dtype)


def _enforce_monotone(rise: torch.Tensor, mode: str) -> None:
    """Check the per-block maxima of ``g[t+1] - g[t]`` written by the factor kernel against MONOTONE_TOL."""
    if mode == "sync":
        worst = rise.max().item()
        if not worst <= MONOTONE_TOL:     # also catches NaN
            raise ValueError(f"sisa_attention_hip: g rises by {worst:.3e} between neighbouring positions (more than "
                             f"{MONOTONE_TOL}); the cumulative log-decay must not increase along the sequence")
    elif mode == "async":
        torch._assert_async(rise.max() <= MONOTONE_TOL,
                            "sisa_attention_hip: the cumulative log-decay g increases along the sequence")


def compute_factors(g: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """``rowf``, ``colf`` ((B, H, L) fp32) and the largest rise of ``g`` in each 64-row block (B*H*ceil(L/64))."""
    B, H, L = g.shape
    rowf = torch.empty((B, H, L), device=g.device, dtype=torch.float32)
    colf = torch.empty_like(rowf)
    rise = torch.empty((B * H * -(-L // BLOCK),), device=g.device, dtype=torch.float32)
    _lib.call("sisa_factors", _lib.FactorsArgs(B, H, L, _lib.view(g), rowf.data_ptr(), colf.data_ptr(),
                                                rise.data_ptr()), g)
    return rowf, colf, rise


def attn_forward(q, k, v, c, b, g, lam, fgate, factors=None, check=None, want32=False) -> Forward:
    """Forward launch on kernel-ready operands (see :func:`kernel_operands`); no autograd.

    ``factors=(rowf, colf)``: anchors the caller already has (the fused layer builds them in its preparation pass);
    then neither the factor kernel nor the monotonicity check runs. ``check``: a check mode for this call in place of
    :func:`sisa_amd.backends.get_check_mode`. ``want32``: also produce the fp32 self-normalised output o''.
    """
    B, H, L, D = q.shape
    backends.attention_config(q.device, q.dtype)          # rejects dtypes the kernels do not take
    if factors is None:
        rowf, colf, rise = compute_factors(g)
        if L > 1:
            _enforce_monotone(rise, backends.get_check_mode() if check is None else check)
    else:
        rowf, colf = factors
        if not (rowf.is_contiguous() and colf.is_contiguous()):
            raise ValueError("attn_forward: factor tables must be contiguous (B, H, L) fp32")
    # (B, L, H, D) memory order: the layer's transpose(1, 2).reshape(B, L, H*D) is then a view
    o = torch.empty_strided((B, H, L, D), (L * H * D, D, H * D, 1), device=q.device, dtype=q.dtype)
    lse = torch.empty((B, H, L), device=q.device, dtype=torch.float32)
    separate32 = want32 and q.dtype != torch.float32
    o32 = torch.empty((B, H, L, D), device=q.device, dtype=torch.float32) if separate32 else None
    _lib.call("sisa_attn_fwd", _lib.AttnFwdArgs(
        B, H, L, _lib.dtype_code(q.dtype), _lib.view(q), _lib.view(k), _lib.view(v), _lib.view(c), _lib.view(b),
        _lib.view(g), _lib.view(fgate), lam.data_ptr(), lam.stride(0), rowf.data_ptr(), colf.data_ptr(),
        _lib.view(o), lse.data_ptr(), _lib.ptr(o32)), q)
    return Forward(o, lse, rowf, colf, o if want32 and not separate32 else o32)


def attn_backward(q, k, v, c, b, g, fgate, rowf, colf, lam, o, lse, do, exact=True,
                  dq=None, dk=None, dv=None, dc=None, db=None, o32=None) -> Grads:
    """Backward launch; no autograd.

    ``dq`` .. ``db``: optional caller buffers with vector-readable rows (the fused layer passes views of its
    projection gradient, and fp32 ``dc``/``db``). ``exact=True`` is the exact-delta backward, using ``o32`` (the o''
    of ``attn_forward(want32=True)``) when given; ``exact=False`` is the FlashAttention-standard backward
    (delta = o.do, no diagonal correction), kept for comparisons.
    """
    B, H, L, D = q.shape
    do = _readable(do)
    dq, dk, dv, dc, db = (_output_like(ref) if buf is None else buf
                          for ref, buf in ((q, dq), (k, dk), (v, dv), (c, dc), (b, db)))
    if not (dq.dtype == dk.dtype == dv.dtype == q.dtype):
        raise TypeError(f"attn_backward: dq/dk/dv buffers must be {q.dtype}")
    if dc.dtype != db.dtype or dc.dtype not in (q.dtype, torch.float32):
        raise TypeError(f"attn_backward: dc/db buffers must both be {q.dtype} or both float32, got {dc.dtype}/"
                        f"{db.dtype}")
    unreadable = [n for n, t in zip(("dq", "dk", "dv", "dc", "db"), (dq, dk, dv, dc, db)) if not _vector_rows(t)]
    if unreadable:
        raise ValueError(f"attn_backward: buffers {unreadable} need a unit last stride and 16-byte aligned rows")
    use32 = bool(exact) and o32 is not None and o32 is not o
    if use32 and not (o32.shape == (B, H, L, D) and o32.is_contiguous() and o32.dtype == torch.float32):
        raise ValueError("attn_backward: o32 must be a contiguous (B, H, L, D) float32 tensor")
    rows = dict(device=q.device, dtype=torch.float32)
    dg = torch.empty((B, H, L), **rows)
    dF = None if fgate is None else torch.empty((B, H, L), **rows)
    dlam = torch.empty((H,), **rows)
    workspace = torch.empty((_lib.workspace_bytes("sisa_attn_bwd_workspace_bytes", B, H, L) // 4,), **rows)
    _lib.call("sisa_attn_bwd", _lib.AttnBwdArgs(
        B, H, L, _lib.dtype_code(q.dtype), _lib.dtype_code(dc.dtype), _lib.view(q), _lib.view(k), _lib.view(v),
        _lib.view(c), _lib.view(b), _lib.view(g), _lib.view(fgate), lam.data_ptr(), lam.stride(0), rowf.data_ptr(),
        colf.data_ptr(), _lib.view(o), o32.data_ptr() if use32 else None, lse.data_ptr(), _lib.view(do),
        _lib.view(dq), _lib.view(dk), _lib.view(dv), _lib.view(dc), _lib.view(db), dg.data_ptr(), _lib.ptr(dF),
        dlam.data_ptr(), workspace.data_ptr(), int(bool(exact))), q)
    return Grads(dq, dk, dv, dc, db, dg, dlam, dF)


class _SISAAttentionFn(torch.autograd.Function):
    """Autograd over the two launches. Arguments are kernel-ready operands plus ``exact`` (the public entry passes
    True; False selects the FlashAttention-standard backward for comparisons)."""

    @staticmethod
    def forward(ctx, q, k, v, c, b, g, lam, fgate, exact):
        keep32 = bool(exact) and any(ctx.needs_input_grad)
        fw = attn_forward(q, k, v, c, b, g, lam, fgate, want32=keep32)
        extra32 = fw.o32 if keep32 and fw.o32 is not fw.o else None
        ctx.save_for_backward(q, k, v, c, b, g, fgate, fw.rowf, fw.colf, lam, fw.o, fw.lse, extra32)
        ctx.exact = bool(exact)
        return fw.o

    @staticmethod
    def backward(ctx, do):
        q, k, v, c, b, g, fgate, rowf, colf, lam, o, lse, o32 = ctx.saved_tensors
        gr = attn_backward(q, k, v, c, b, g, fgate, rowf, colf, lam, o, lse, do, ctx.exact, o32=o32)
        return gr.dq, gr.dk, gr.dv, gr.dc, gr.db, gr.dg, gr.dlam, gr.dF, None


def kernel_operands(q, k, v, c, b, g, lam, fgate):
    """Check prepared attention inputs against what the kernels take and return them kernel-ready.

    Shapes: q, k, v (B, H, L, 64); c, b (B, H, L, 32); g and fgate (B, H, L); lam (H,); L >= 1 (``ValueError``
    otherwise). Dtypes: q, k, v one of bf16/fp16/fp32, g and fgate fp32 (``TypeError`` otherwise). Everything on one
    GPU. c and b are cast to q's dtype and lam to fp32; tensors whose rows are not vector-readable are copied.
    Same contract as the reference's ``_prepare_inputs`` (src/sisa/kernels/attention.py:812-850).
    """
    if q.dim() != 4:
        raise ValueError(f"sisa_attention_hip: q must be (B, H, L, {HIP_D_HEAD}), got {tuple(q.shape)}")
    B, H, L, _ = q.shape
    want = {"q": (q, (B, H, L, HIP_D_HEAD)), "k": (k, (B, H, L, HIP_D_HEAD)), "v": (v, (B, H, L, HIP_D_HEAD)),
            "c": (c, (B, H, L, HIP_D_STATE)), "b": (b, (B, H, L, HIP_D_STATE)), "g": (g, (B, H, L)),
            "lam": (lam, (H,))}
    if fgate is not None:
        want["fgate"] = (fgate, (B, H, L))
    misfits = [f"{n} {tuple(t.shape)} (expected {shape})" for n, (t, shape) in want.items() if tuple(t.shape) != shape]
    if misfits:
        raise ValueError(f"sisa_attention_hip: the kernels take d_head {HIP_D_HEAD} and d_state {HIP_D_STATE}; "
                         f"wrong shapes: {', '.join(misfits)}")
    if L < 1:
        raise ValueError("sisa_attention_hip: the sequence is empty")
    if q.dtype not in _INPUT_DTYPES or k.dtype != q.dtype or v.dtype != q.dtype:
        raise TypeError(f"sisa_attention_hip: q, k, v must share one of bf16/fp16/fp32, got {q.dtype}, {k.dtype}, "
                        f"{v.dtype}")
    wide = {n: t.dtype for n, t in (("g", g), ("fgate", fgate)) if t is not None and t.dtype != torch.float32}
    if wide:
        raise TypeError(f"sisa_attention_hip: the cumulative gates are read as float32; got {wide}")
    places = {t.device for t, _ in want.values()}
    if len(places) != 1 or not q.is_cuda:
        raise ValueError(f"sisa_attention_hip: all inputs must be on one GPU, got {sorted(map(str, places))}")
    q, k, v = (_readable(t) for t in (q, k, v))
    c, b = (_readable(t.to(q.dtype)) for t in (c, b))
    return q, k, v, c, b, g, lam.to(torch.float32), fgate


def sisa_attention_hip(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, c: torch.Tensor, b: torch.Tensor,
                       g: torch.Tensor, lam: torch.Tensor, fgate: torch.Tensor | None = None) -> torch.Tensor:
    """Exact SISA attention on the HIP kernels, differentiable in every tensor argument.

    ``q, k, v``: (B, H, L, 64) bf16/fp16/fp32, any strides with a unit last one; ``c, b``: (B, H, L, 32) rotated
    state vectors (cast to q's dtype; their gradients return in their own dtype); ``g``: (B, H, L) fp32 cumulative
    log-decay, non-increasing (checked per :func:`sisa_amd.backends.set_check_mode`); ``lam``: (H,) state-term
    weights; ``fgate``: (B, H, L) fp32 cumulative log-sigmoid forget gate or ``None``.

    Returns (B, H, L, 64) in q's dtype, laid out as (B, L, H, 64). Bitwise deterministic, gradients included; the
    backward is the exact-delta one. Counterpart of the reference's ``sisa_attention_triton``
    (src/sisa/kernels/attention.py:853-877).
    """
    return _SISAAttentionFn.apply(*kernel_operands(q, k, v, c, b, g, lam, fgate), True)


def flops(B: int, H: int, L: int, d_head: int = 64, d_state: int = 32) -> dict:
    """Algorithmic MFMA work (FlashAttention convention, causal pairs P = B*H*L^2/2)."""
    pairs = B * H * L * L / 2.0
    fwd = pairs * (4 * d_head + 2 * d_state)
    bwd = pairs * (10 * d_head + 6 * d_state)
    return dict(pairs=pairs, fwd=fwd, bwd=bwd, total=fwd + bwd, scale=1.0 / math.sqrt(d_head))
