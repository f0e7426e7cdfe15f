"""The SISA attention sublayer: the caller of the hot path.

``SISAAttention`` mirrors the reference's layer (src/sisa/modeling.py:79-255): the same parameters and
initialisation, the same unfused glue (``_prepare``: cumsums, softplus, log-sigmoid and the pair rotation in fp32),
and the same dispatch, with the Triton paths replaced by ``"hip"`` (glue + HIP attention) and ``"hip_fused"`` (one
projection GEMM + HIP prep + HIP attention). Decoding caches are not part of this build.
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch import Tensor

from .config import ATTN_IMPLS, SISAConfig
from .functional import _autocast_off, rotate_pairs, sisa_attention

__all__ = ["SISAAttention"]


def _compute_dtype(x: Tensor) -> torch.dtype:
    try:
        if torch.is_autocast_enabled(x.device.type):
            return torch.get_autocast_dtype(x.device.type)
    except (TypeError, RuntimeError):
        pass
    return x.dtype


def _resolve_impl(requested: str, x: Tensor, config: SISAConfig) -> str:
    """Map a requested attention implementation to a concrete one for input ``x`` (modeling.py:60-76)."""
    if requested not in ATTN_IMPLS:
        raise ValueError(f"attn_impl must be one of {ATTN_IMPLS}, got {requested!r}")
    if requested == "torch":
        return "torch"
    if x.device.type != "cuda":
        if requested == "auto":
            return "torch"
        raise ValueError(f"attn_impl={requested!r} needs a GPU tensor, got one on {x.device.type}; "
                         "use attn_impl='torch' or 'auto'")
    from . import backends

    impl = backends.select_impl(requested, x, config)
    if impl not in ("torch", "hip", "hip_fused"):
        raise RuntimeError(f"backend selection returned an unknown implementation {impl!r}")
    return impl


class SISAAttention(nn.Module):
    """SISA attention sublayer: projections, recurrences, attention and output projection.

    Parameters: ``W_Q, W_K, W_V, W_O`` (``d -> d``); ``W_B, W_C`` (``d -> H*d_state``); ``alpha_proj`` (``d -> H``,
    decay, with bias); ``theta_proj`` (``d -> H*d_state/2``); ``forget_proj`` (``d -> H``, with bias);
    ``lambda_raw`` (``H``, kept in fp32 under dtype casts).
    """

    def __init__(self, config: SISAConfig, layer_idx: int = 0):
        super().__init__()
        self.config = config
        self.layer_idx = layer_idx
        d, h, s = config.d_model, config.n_head, config.d_state
        self.W_Q = nn.Linear(d, d, bias=False)
        self.W_K = nn.Linear(d, d, bias=False)
        self.W_V = nn.Linear(d, d, bias=False)
        self.W_O = nn.Linear(d, d, bias=False)
        self.W_B = nn.Linear(d, h * s, bias=False)
        self.W_C = nn.Linear(d, h * s, bias=False)
        self.alpha_proj = nn.Linear(d, h, bias=True)
        self.theta_proj = nn.Linear(d, h * (s // 2), bias=False)
        self.forget_proj = nn.Linear(d, h, bias=True)
        self.lambda_raw = nn.Parameter(torch.full((h,), float(config.lambda_raw_init)))
        self.reset_parameters()

    @torch.no_grad()
    def reset_parameters(self) -> None:
        """SISA initialisation: weights ~ N(0, init_std), W_C = 0 (zero_init_c), theta ~ N(0, theta_init_std),
        decay bias, forget bias and lambda_raw constants (modeling.py:122-141)."""
        cfg = self.config
        for lin in (self.W_Q, self.W_K, self.W_V, self.W_O, self.W_B, self.alpha_proj, self.forget_proj):
            nn.init.normal_(lin.weight, std=cfg.init_std)
        if cfg.zero_init_c:
            nn.init.zeros_(self.W_C.weight)
        else:
            nn.init.normal_(self.W_C.weight, std=cfg.init_std)
        nn.init.normal_(self.theta_proj.weight, std=cfg.theta_init_std)
        nn.init.constant_(self.alpha_proj.bias, cfg.decay_bias_init)
        nn.init.constant_(self.forget_proj.bias, cfg.forget_bias_init)
        self.lambda_raw.fill_(cfg.lambda_raw_init)

    def _apply(self, fn, recurse: bool = True) -> "SISAAttention":
        # keep lambda_raw in float32 when the module is cast to bf16/fp16 (modeling.py:144-160)
        low = (torch.float16, torch.bfloat16)
        old = self.lambda_raw
        old_data = old.data
        old_grad = None if old.grad is None else old.grad.data
        super()._apply(fn, recurse)
        p = self.lambda_raw
        if p.dtype in low:
            src = old_data if old_data.dtype not in low else p.data
            p.data = src.to(device=p.device, dtype=torch.float32)
            if p.grad is not None:
                gsrc = old_grad if old_grad is not None and old_grad.dtype not in low else p.grad
                p.grad = gsrc.to(device=p.device, dtype=torch.float32)
        return self

    def lam(self) -> Tensor:
        """Per-head SSM weight ``softplus(lambda_raw)`` as float32, shape ``(H,)``."""
        return F.softplus(self.lambda_raw).float()

    def _forget_logits(self, x: Tensor) -> Tensor:
        """Forget-gate pre-activations ``(B, L, H)`` in float32 with autocast disabled."""
        with _autocast_off(x.device.type):
            return F.linear(x.float(), self.forget_proj.weight.float(), self.forget_proj.bias.float())

    def _prepare(self, x: Tensor):
        """Projections and recurrences of the unfused paths: ``q, k, v, c~, b~`` in the compute dtype and ``g, F,
        Phi`` in float32 (modeling.py:171-199)."""
        bsz, seq_len, _ = x.shape
        h, dh, s = self.config.n_head, self.config.d_head, self.config.d_state

        def heads(t, w):
            return t.view(bsz, seq_len, h, w).transpose(1, 2)
        q, k, v = heads(self.W_Q(x), dh), heads(self.W_K(x), dh), heads(self.W_V(x), dh)
        b, c = heads(self.W_B(x), s), heads(self.W_C(x), s)
        a = self.alpha_proj(x).transpose(1, 2)
        theta = heads(self.theta_proj(x), s // 2)
        g = torch.cumsum(-F.softplus(a.float()), dim=2)
        phi = torch.cumsum(theta.float(), dim=2)
        z = self._forget_logits(x)
        with _autocast_off(x.device.type):
            fgate = torch.cumsum(F.logsigmoid(z).transpose(1, 2), dim=2)
        c = rotate_pairs(c.float(), phi)
        b = rotate_pairs(b.float(), phi)
        cd = _compute_dtype(x)
        return q.to(cd), k.to(cd), v.to(cd), c.to(cd), b.to(cd), g, fgate, phi

    def _attend(self, q, k, v, c, b, g, fgate, impl: str) -> Tensor:
        return sisa_attention(q, k, v, c, b, g, self.lam(), fgate, impl=impl, block_q=self.config.torch_block_q)

    def _output(self, y: Tensor) -> Tensor:
        bsz, h, seq_len, dh = y.shape
        return self.W_O(y.transpose(1, 2).reshape(bsz, seq_len, h * dh))

    def _forward_fused(self, x: Tensor) -> Tensor:
        from .kernels.fused_prep import concat_fused_weights, sisa_fused

        bsz, seq_len, d = x.shape
        weight, bias = concat_fused_weights(self.W_Q.weight, self.W_K.weight, self.W_V.weight, self.W_B.weight,
                                            self.W_C.weight, self.theta_proj.weight, self.alpha_proj.weight,
                                            self.alpha_proj.bias)
        proj = F.linear(x, weight, bias)                  # (B, L, NPAD), autocast dtype
        y = sisa_fused(proj, self._forget_logits(x), self.lam(), self.config.n_head)
        return self.W_O(y.reshape(bsz, seq_len, d))

    def forward(self, x: Tensor, *, impl: str | None = None) -> Tensor:
        """Apply the sublayer to the normalised input ``x`` ``(B, L, d_model)``; returns ``(B, L, d_model)``.
        ``impl`` overrides ``config.attn_impl`` for this call."""
        requested = impl or self.config.attn_impl
        impl = _resolve_impl(requested, x, self.config)
        if impl == "hip_fused":
            return self._forward_fused(x)
        q, k, v, c, b, g, fgate, _ = self._prepare(x)
        return self._output(self._attend(q, k, v, c, b, g, fgate, impl))
