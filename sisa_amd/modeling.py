"""The SISA causal language model as PyTorch modules, with the gfx950 HIP kernels behind its hot operations.

Module tree, parameter names and shapes, initial values and loss conventions are the reference's
(src/sisa/modeling.py), so state dicts and checkpoints interchange; the state-dict manifest is
:meth:`SISAConfig.parameter_shapes`. How the computation is organised is this build's:

* :class:`SISAAttention` turns a normalised input into the attention output along one of three routes, picked per
  call by :func:`sisa_amd.backends.select_impl`: the *unfused* route (separate projections, recurrences and pair
  rotation in fp32, then :func:`sisa_amd.functional.sisa_attention` with ``impl`` "torch" or "hip"), the *fused*
  route (one GEMM against the concatenated projection weights, then :func:`sisa_amd.kernels.fused_prep.sisa_fused`),
  and the *cached* route of generation (prefill unfused, then one-token steps on the HIP decode kernel).
* :class:`SISABlock` runs a whole pre-norm block on HIP kernels when the fused route is selected: RMSNorm plus the
  fp32 forget-gate projection in one pass, the fused sublayer, residual add plus the FFN norm in one pass, and the
  SwiGLU activation on interleaved gate/up columns. Consecutive such blocks hand the FFN output to the next block's
  norm instead of adding it (:data:`DEFER_RESIDUAL`).
* :class:`SISAForCausalLM` adds the tied LM head; its loss is eager or, with ``fused_ce``, the HIP linear
  cross-entropy, which never holds the full logits.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import TYPE_CHECKING, Any, Iterable, NamedTuple

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch import Tensor
from torch.utils.checkpoint import checkpoint

from . import backends
from .config import SISAConfig
from .functional import attend_block, autocast_disabled, rotate_pairs, sisa_attention, working_dtype

if TYPE_CHECKING:  # pragma: no cover
    from .generation import SISACache

__all__ = ["RMSNorm", "SwiGLU", "SISAAttention", "SISABlock", "SISAModel", "SISAForCausalLM", "SISAOutput"]

IGNORE_INDEX = -100
_LOW_PRECISION = (torch.float16, torch.bfloat16)


def _kernels_on(x: Tensor, config: SISAConfig | None) -> bool:
    """Whether the norm / SwiGLU / decode kernels serve input ``x``: a GPU tensor, an attention implementation other
    than "torch", and a loadable library. A forced HIP implementation without the library raises."""
    if config is None or x.device.type != "cuda" or config.attn_impl == "torch":
        return False
    ok, why = backends.hip_status(x.device)
    if not ok and config.attn_impl != "auto":
        raise ValueError(f"attn_impl={config.attn_impl!r} is not available: {why}")
    return ok


def _linear(x: Tensor, weight: Tensor, bias: Tensor | None = None, bias_cols: tuple[int, int] | None = None
            ) -> Tensor:
    """``F.linear`` of the HIP block path: with a 16-bit compute dtype on the GPU the weight gradient comes from the
    HIP weight-gradient kernel (fp32, split-K over the tokens) instead of the library GEMM and its cast."""
    if x.is_cuda and backends.compute_dtype(x) in _LOW_PRECISION and x.shape[-1] % 8 == 0 \
            and weight.shape[0] % 8 == 0:
        from .kernels.wgrad import linear_hip

        return linear_hip(x, weight, bias, bias_cols)
    return F.linear(x, weight, bias)


class RMSNorm(nn.Module):
    """Root-mean-square normalisation in float32 with a learned gain; the output keeps the input's dtype.
    ``config`` (optional) lets the module use the HIP norm kernel on the GPU."""

    def __init__(self, dim: int, eps: float = 1e-6, config: SISAConfig | None = None):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps
        self._config = config

    def forward(self, x: Tensor) -> Tensor:
        width = x.shape[-1]
        if width % 8 == 0 and width <= 4096 and x.numel() and _kernels_on(x, self._config):
            from .kernels.norm import rms_norm_hip

            return rms_norm_hip(x, self.weight, self.eps)
        return F.rms_norm(x.float(), (width,), self.weight.float(), self.eps).to(x.dtype)


class SwiGLU(nn.Module):
    """The gated feed-forward ``w_down(silu(w_gate x) * (w_up x))`` without biases. On the GPU the gate and up
    projections run as one GEMM against their rows interleaved in 8-row chunks, followed by the HIP activation
    kernel on the chunk pairs (the same dot products as two separate projections)."""

    def __init__(self, d_model: int, d_ff: int, config: SISAConfig | None = None):
        super().__init__()
        self.w_gate = nn.Linear(d_model, d_ff, bias=False)
        self.w_up = nn.Linear(d_model, d_ff, bias=False)
        self.w_down = nn.Linear(d_ff, d_model, bias=False)
        self._config = config

    def forward(self, x: Tensor) -> Tensor:
        if self.w_gate.out_features % 8 == 0 and x.shape[-1] % 8 == 0 and x.numel() and _kernels_on(x, self._config):
            from .kernels.norm import interleave_gate_up, swiglu_pairs_hip

            cd = backends.compute_dtype(x)
            gate_up = F.linear(x, interleave_gate_up(self.w_gate.weight.to(cd), self.w_up.weight.to(cd)))
            return _linear(swiglu_pairs_hip(gate_up), self.w_down.weight)
        gate, up = self.w_gate(x), self.w_up(x)
        return self.w_down(up * F.silu(gate))


class Prepared(NamedTuple):
    """Inputs of the attention function for one call of the unfused route: ``q, k, v`` ``(B, H, L, d_head)`` and the
    rotated ``c, b`` ``(B, H, L, d_state)`` in the compute dtype; ``g, fgate`` ``(B, H, L)`` and the cumulative phase
    ``phi`` ``(B, H, L, d_state/2)`` in float32."""
    q: Tensor
    k: Tensor
    v: Tensor
    c: Tensor
    b: Tensor
    g: Tensor
    fgate: Tensor
    phi: Tensor


class SISAAttention(nn.Module):
    """The SISA attention sublayer: input projections, the decay / phase / forget recurrences, SISA attention and the
    output projection.

    Parameters: ``W_Q, W_K, W_V, W_O`` (``d -> d``); ``W_B, W_C`` (``d -> H*d_state``, write and read vectors, row
    ``h*d_state + s``); ``theta_proj`` (``d -> H*d_state/2``, rotation rates); ``alpha_proj`` (``d -> H`` with bias,
    decay); ``forget_proj`` (``d -> H`` with bias, forget gate); ``lambda_raw`` (``H``; ``lam = softplus(lambda_raw)``
    weights the state term). ``lambda_raw`` stays float32, with its full value, when the module is cast to a 16-bit
    dtype: in bf16 its updates would round away.
    """

    def __init__(self, config: SISAConfig, layer_idx: int = 0):
        super().__init__()
        self.config = config
        self.layer_idx = layer_idx
        d, h, s = config.d_model, config.n_head, config.d_state

        def proj(rows: int, bias: bool = False) -> nn.Linear:
            return nn.Linear(d, rows, bias=bias)

        self.W_Q, self.W_K, self.W_V, self.W_O = proj(d), proj(d), proj(d), proj(d)       # content path
        self.W_B, self.W_C, self.theta_proj = proj(h * s), proj(h * s), proj(h * s // 2)  # state path
        self.alpha_proj, self.forget_proj = proj(h, bias=True), proj(h, bias=True)      # per-head gates
        self.lambda_raw = nn.Parameter(torch.empty(h))
        self.reset_parameters()

    @torch.no_grad()
    def reset_parameters(self) -> None:
        """Initial values of the reference (src/sisa/modeling.py:122-141): weights N(0, init_std), except ``W_C`` (0
        when ``zero_init_c``) and ``theta_proj`` (N(0, theta_init_std)); the decay and forget biases and
        ``lambda_raw`` constants from the config."""
        cfg = self.config
        gaussian = [self.W_Q, self.W_K, self.W_V, self.W_O, self.W_B, self.alpha_proj, self.forget_proj]
        if not cfg.zero_init_c:
            gaussian.append(self.W_C)
        for lin in gaussian:
            lin.weight.normal_(0.0, cfg.init_std)
        if cfg.zero_init_c:
            self.W_C.weight.zero_()
        self.theta_proj.weight.normal_(0.0, cfg.theta_init_std)
        self.alpha_proj.bias.fill_(cfg.decay_bias_init)
        self.forget_proj.bias.fill_(cfg.forget_bias_init)
        self.lambda_raw.fill_(cfg.lambda_raw_init)

    def _apply(self, fn, recurse: bool = True) -> "SISAAttention":
        # Module casts go through _apply. Keep the float32 value (and gradient) of lambda_raw from before a cast to a
        # 16-bit dtype, moved to wherever the cast put the parameter.
        p = self.lambda_raw
        kept = (p.data, None if p.grad is None else p.grad.data)
        super()._apply(fn, recurse)
        p = self.lambda_raw
        if p.dtype in _LOW_PRECISION:
            def widened(now: Tensor, before: Tensor | None) -> Tensor:
                src = before if before is not None and before.dtype not in _LOW_PRECISION else now
                return src.to(device=p.device, dtype=torch.float32)
            p.data = widened(p.data, kept[0])
            if p.grad is not None:
                p.grad = widened(p.grad, kept[1])
        return self

    def lam(self) -> Tensor:
        """``softplus(lambda_raw)`` in float32, shape ``(H,)``."""
        return F.softplus(self.lambda_raw).to(torch.float32)

    def _forget_logits(self, x: Tensor) -> Tensor:
        """The forget-gate logits ``(B, L, H)``, always float32 (autocast off), as the reference computes them."""
        with autocast_disabled(x.device.type):
            return F.linear(x.float(), self.forget_proj.weight.float(), self.forget_proj.bias.float())

    def _unfused_inputs(self, x: Tensor, state: Any = None) -> Prepared:
        """The attention inputs of ``x`` ``(B, L, d)`` on the unfused route (src/sisa/modeling.py:171-199 semantics):
        projections in the compute dtype, recurrences and rotation in float32. ``state``, a decode cache entry,
        continues the recurrences from its last position."""
        cfg = self.config

        def heads(t: Tensor, width: int) -> Tensor:                 # (B, L, H*width) -> (B, H, L, width)
            return t.unflatten(-1, (cfg.n_head, width)).transpose(1, 2)

        q, k, v = (heads(lin(x), cfg.d_head) for lin in (self.W_Q, self.W_K, self.W_V))
        c_raw, b_raw = heads(self.W_C(x), cfg.d_state), heads(self.W_B(x), cfg.d_state)
        decay = self.alpha_proj(x).float().transpose(1, 2)             # (B, H, L)
        rate = heads(self.theta_proj(x), cfg.d_state // 2).float()
        z = self._forget_logits(x).transpose(1, 2)
        with autocast_disabled(x.device.type):
            g = (-F.softplus(decay)).cumsum(dim=2)
            phi = rate.cumsum(dim=2)
            fgate = F.logsigmoid(z).cumsum(dim=2)
        if state is not None:
            g, phi, fgate = g + state.g[..., -1:], phi + state.phi[:, :, None], fgate + state.fgate[..., -1:]
        cd = backends.compute_dtype(x)
        c, b = rotate_pairs(c_raw.float(), phi), rotate_pairs(b_raw.float(), phi)
        return Prepared(q.to(cd), k.to(cd), v.to(cd), c.to(cd), b.to(cd), g, fgate, phi)

    def _attention(self, p: Prepared, impl: str) -> Tensor:
        return sisa_attention(p.q, p.k, p.v, p.c, p.b, p.g, self.lam(), p.fgate, impl=impl,
                              block_q=self.config.torch_block_q)

    def _output(self, y: Tensor) -> Tensor:
        """``W_O`` applied to the heads ``(B, H, L, d_head)`` laid side by side: ``(B, L, d)``."""
        return self.W_O(y.transpose(1, 2).flatten(2))

    def _fused_weights(self) -> tuple[Tensor, Tensor]:
        from .kernels.fused_prep import concat_fused_weights

        return concat_fused_weights(self.W_Q.weight, self.W_K.weight, self.W_V.weight, self.W_B.weight,
                                    self.W_C.weight, self.theta_proj.weight, self.alpha_proj.weight,
                                    self.alpha_proj.bias)

    def _forward_fused(self, x: Tensor, z: Tensor | None = None) -> Tensor:
        """The fused route. ``z``: forget-gate logits already produced by the decoder block's norm kernel; with it
        the projections use the HIP weight-gradient GEMM path of the block, without it (the sublayer called on its
        own) plain ``F.linear``."""
        from .kernels.fused_prep import fused_layout, sisa_fused

        weight, bias = self._fused_weights()
        n_head = self.config.n_head
        if z is None:
            y = sisa_fused(F.linear(x, weight, bias), self._forget_logits(x), self.lam(), n_head)
            return self.W_O(y)                         # y: (B, L, d), heads side by side
        a0 = fused_layout(n_head)["A"]                 # the bias is a parameter on the alpha columns only
        y = sisa_fused(_linear(x, weight, bias, (a0, a0 + n_head)), z, self.lam(), n_head)
        return _linear(y, self.W_O.weight)

    def _forward_cached(self, x: Tensor, cache: "SISACache", requested: str) -> Tensor:
        """Generation. An empty layer entry means prefill: the unfused route (the fused one keeps no k, v, b, g, F to
        cache) with "hip" standing in for "hip_fused". Otherwise a step: the new rows attend to the whole cache, on
        the HIP decode kernel on the GPU, else exactly in float32 torch."""
        state = cache.get(self.layer_idx)
        p = self._unfused_inputs(x, state)
        if state is None:
            impl = backends.select_impl("hip" if requested == "hip_fused" else requested, x, self.config)
            y = self._attention(p, "hip" if impl == "hip_fused" else impl)
            cache.update(self.layer_idx, k=p.k, v=p.v, b=p.b, g=p.g, fgate=p.fgate, phi=p.phi[:, :, -1])
            return self._output(y)
        first = state.length
        state = cache.update(self.layer_idx, k=p.k, v=p.v, b=p.b, g=p.g, fgate=p.fgate, phi=p.phi[:, :, -1])
        if _kernels_on(x, self.config) and p.q.dtype in (torch.bfloat16, torch.float16, torch.float32):
            from .kernels.decode import sisa_decode_hip

            y = sisa_decode_hip(p.q, state.k, state.v, p.c, state.b, p.g, state.g, self.lam(), p.fgate,
                                state.fgate, first)
            return self._output(y.to(p.q.dtype))
        wd = working_dtype(p.q.dtype)
        rows = (p.q.to(wd), p.c.to(wd), p.g.to(wd), p.fgate.to(wd))
        keys = (state.k.to(wd), state.v.to(wd), state.b.to(wd), state.g.to(wd), state.fgate.to(wd))
        return self._output(attend_block(rows, keys, self.lam().to(wd), first).to(p.q.dtype))

    def forward(self, x: Tensor, *, cache: "SISACache | None" = None, impl: str | None = None) -> Tensor:
        """The sublayer on the normalised input ``x`` ``(B, L, d_model)``, returning ``(B, L, d_model)``. ``cache``:
        a :class:`sisa_amd.generation.SISACache` to fill (prefill) or extend (decode step); ``impl`` overrides
        ``config.attn_impl`` for this call."""
        requested = impl or self.config.attn_impl
        if cache is not None:
            return self._forward_cached(x, cache, requested)
        chosen = backends.select_impl(requested, x, self.config)
        if chosen == "hip_fused":
            return self._forward_fused(x)
        return self._output(self._attention(self._unfused_inputs(x), chosen))


class SISABlock(nn.Module):
    """Pre-norm block: ``x + attn(attn_norm(x))``, then ``x + ffn(ffn_norm(x))``. Constructed initialised."""

    def __init__(self, config: SISAConfig, layer_idx: int = 0):
        super().__init__()
        self.config = config
        self.attn_norm = RMSNorm(config.d_model, config.norm_eps, config)
        self.attn = SISAAttention(config, layer_idx)
        self.ffn_norm = RMSNorm(config.d_model, config.norm_eps, config)
        self.ffn = SwiGLU(config.d_model, config.d_ff, config)
        self.fuse_norm = True          # run the whole block on HIP kernels where _fused_norm_ok allows
        self._init_ffn_and_norms()

    @torch.no_grad()
    def _init_ffn_and_norms(self) -> None:
        for lin in (self.ffn.w_gate, self.ffn.w_up, self.ffn.w_down):
            lin.weight.normal_(0.0, self.config.init_std)
        self.attn_norm.weight.fill_(1.0)
        self.ffn_norm.weight.fill_(1.0)

    @torch.no_grad()
    def reset_parameters(self) -> None:
        """Initial values again: FFN weights N(0, init_std), norm gains 1, and the attention sublayer's."""
        self._init_ffn_and_norms()
        self.attn.reset_parameters()

    def _fused_norm_ok(self, x: Tensor) -> bool:
        """The HIP block path applies: GPU input, the fused HIP attention selected for it, and rows the norm
        kernels take."""
        if not self.fuse_norm or x.device.type != "cuda" or x.dim() != 3 or x.numel() == 0:
            return False
        d, h = x.shape[-1], self.config.n_head
        if d % 8 or d > 4096 or h > 64 or x.dtype not in (torch.float32, torch.bfloat16, torch.float16):
            return False
        return backends.select_impl(self.config.attn_impl, x, self.config) == "hip_fused"

    def _forward_hip(self, x: Tensor, res: Tensor | None = None, defer: bool = False):
        """The block on the HIP kernels: the attention norm and the fp32 forget-gate projection in one pass that
        also emits the normalised rows in the dtype of the projection GEMM (the reference casts them under autocast),
        the fused attention sublayer, the residual add and the FFN norm in one pass, SwiGLU.

        ``res``: the previous block's FFN output, whose residual add (``x + res``) runs in this block's attention
        norm. ``defer=True`` returns ``(h, f)`` -- the stream before the FFN residual and the FFN output -- for the
        next block to add the same way (``(h + f, None)`` when ``f`` cannot be passed on); otherwise ``h + f``."""
        from .kernels.norm import rms_norm_add_hip, rms_norm_forget_add_hip, rms_norm_forget_hip, rms_norm_hip

        cd = backends.compute_dtype(x)
        out_dtype = cd if x.dtype == torch.float32 else x.dtype
        at = self.attn
        nw, eps, wf, bf = self.attn_norm.weight, self.attn_norm.eps, at.forget_proj.weight, at.forget_proj.bias
        if res is not None and res.dtype == out_dtype and res.shape == x.shape:
            x, n, z = rms_norm_forget_add_hip(x, res, nw, eps, wf, bf, out_dtype)
        else:
            if res is not None:
                x = x + res
            n, z = rms_norm_forget_hip(x, nw, eps, wf, bf, out_dtype)
        a = at._forward_fused(n, z)
        if a.dtype == out_dtype and a.shape == x.shape:   # residual add fused into the FFN norm
            x, m = rms_norm_add_hip(x, a, self.ffn_norm.weight, self.ffn_norm.eps, out_dtype)
        else:
            x = x + a
            m = rms_norm_hip(x, self.ffn_norm.weight, self.ffn_norm.eps, out_dtype)
        f = self.ffn(m)
        if defer:
            return (x, f) if (f.dtype == out_dtype and f.shape == x.shape) else (x + f, None)
        return x + f

    def forward(self, x: Tensor, cache: "SISACache | None" = None) -> Tensor:
        if cache is None and self._fused_norm_ok(x):
            return self._forward_hip(x)
        h = x + self.attn(self.attn_norm(x), cache=cache)
        return h + self.ffn(self.ffn_norm(h))


@dataclass
class SISAOutput:
    """What :meth:`SISAForCausalLM.forward` returns: the mean loss (with labels) and the logits (when kept)."""

    loss: Tensor | None = None
    logits: Tensor | None = None


def _token_ce(logits: Tensor, targets: Tensor) -> Tensor:
    """Mean float32 cross-entropy of ``logits`` ``(..., V)`` against ``targets`` ``(...)``, ignoring IGNORE_INDEX."""
    return F.cross_entropy(logits.flatten(0, -2).float(), targets.flatten(), ignore_index=IGNORE_INDEX)


def _lm_head_loss(hidden: Tensor, weight: Tensor, labels: Tensor) -> Tensor:
    """Tied-head loss for aligned ``hidden`` / ``labels``, through full logits."""
    return _token_ce(F.linear(hidden, weight), labels)


def _lm_head_loss_chunked(hidden: Tensor, weight: Tensor, labels: Tensor) -> Tensor:
    """Tied-head loss for aligned ``hidden`` / ``labels`` through :func:`sisa_amd.kernels.linear_ce.
    linear_cross_entropy`: on the GPU in 16 bits without a logits buffer, elsewhere the eager formula."""
    from .kernels.linear_ce import linear_cross_entropy

    return linear_cross_entropy(hidden.flatten(0, -2), weight, labels.flatten(), ignore_index=IGNORE_INDEX)


# Consecutive fused HIP blocks pass the FFN output on to the next block's attention norm (SISAModel.forward); False
# adds it in each block instead (same results bit for bit).
DEFER_RESIDUAL = True

_TIMESCALE_BIASES = ("alpha_proj.bias", "forget_proj.bias")


class SISAModel(nn.Module):
    """Token embedding, ``n_layer`` :class:`SISABlock` s and the final RMSNorm; ``forward(input_ids)`` returns the
    normalised hidden states ``(B, L, d_model)``."""

    def __init__(self, config: SISAConfig):
        super().__init__()
        self.config = config.replace()          # a checked private copy, shared by every submodule
        cfg = self.config
        self.embed = nn.Embedding(cfg.vocab_size, cfg.d_model)
        self.layers = nn.ModuleList(SISABlock(cfg, i) for i in range(cfg.n_layer))
        self.final_norm = RMSNorm(cfg.d_model, cfg.norm_eps, cfg)
        self._init_embedding_and_norm()

    @torch.no_grad()
    def _init_embedding_and_norm(self) -> None:
        self.embed.weight.normal_(0.0, self.config.init_std)
        self.final_norm.weight.fill_(1.0)

    @torch.no_grad()
    def reset_parameters(self) -> None:
        """Every parameter back to its initial distribution (embedding N(0, init_std), norm gains 1, blocks as
        :meth:`SISABlock.reset_parameters`)."""
        self._init_embedding_and_norm()
        for block in self.layers:
            block.reset_parameters()

    def forward(self, input_ids: Tensor, *, cache: "SISACache | None" = None) -> Tensor:
        x = self.embed(input_ids)
        recompute = (self.config.gradient_checkpointing and self.training and cache is None
                     and torch.is_grad_enabled())
        pending = None          # FFN output of the previous fused block, not yet added to x
        for block in self.layers:
            if DEFER_RESIDUAL and not recompute and cache is None and block._fused_norm_ok(x):
                x, pending = block._forward_hip(x, pending, defer=True)
                continue
            if pending is not None:
                x, pending = x + pending, None
            x = checkpoint(block, x, use_reentrant=False) if recompute else block(x, cache=cache)
        if pending is not None:
            x = x + pending
        return self.final_norm(x)

    def compile_common(self, **compile_kwargs: Any) -> "SISAModel":
        """Put the common, non-attention work on its fast path; returns the model, state-dict keys unchanged.

        The reference compiles the norms, the SwiGLU modules and the logits-free loss with ``torch.compile``
        (src/sisa/modeling.py:396-414). Here the norms and SwiGLU already run as fused HIP kernels on the GPU, so what
        this does is switch the logits-free loss (``forward(..., labels=..., return_logits=False)``) to the chunked
        linear cross-entropy, which on the GPU computes it in 16 bits without materialising the logits.
        ``compile_kwargs`` are accepted for signature compatibility and not used (no Inductor code is generated).
        """
        if isinstance(self, SISAForCausalLM):
            self._loss_fn = _lm_head_loss_chunked
        return self

    def set_attn_impl(self, impl: str) -> None:
        """Switch every layer to attention implementation ``impl`` (validated like ``SISAConfig.attn_impl``)."""
        checked = self.config.replace(attn_impl=impl)
        self.config.attn_impl = checked.attn_impl

    def num_parameters(self, exclude_embeddings: bool = False) -> int:
        """Parameter count, the tied LM head once; optionally without the embedding."""
        total = sum(p.numel() for p in self.parameters())
        return total - (self.embed.weight.numel() if exclude_embeddings else 0)

    def param_groups(self, lr: float, weight_decay: float = 0.1, lambda_lr: float | None = None,
                     no_decay_timescale_biases: bool = True) -> list[dict[str, Any]]:
        """Optimizer groups of src/sisa/modeling.py:366-394: ``"default"`` (everything else, ``weight_decay``),
        ``"timescale_biases"`` (the decay and forget biases, no decay; only with ``no_decay_timescale_biases``) and
        ``"lambda"`` (``lambda_raw``, no decay, learning rate ``lambda_lr`` or ``lr``). Empty groups other than the
        default one are left out."""
        settings = {"default": (lr, weight_decay), "timescale_biases": (lr, 0.0),
                    "lambda": (lr if lambda_lr is None else lambda_lr, 0.0)}
        members: dict[str, list] = {name: [] for name in settings}
        for name, p in self.named_parameters():
            if not p.requires_grad:
                continue
            if name.endswith("lambda_raw"):
                members["lambda"].append(p)
            elif no_decay_timescale_biases and name.endswith(_TIMESCALE_BIASES):
                members["timescale_biases"].append(p)
            else:
                members["default"].append(p)
        return [{"params": ps, "lr": settings[n][0], "weight_decay": settings[n][1], "name": n}
                for n, ps in members.items() if ps or n == "default"]


class SISAForCausalLM(SISAModel):
    """:class:`SISAModel` plus the tied LM head, ``logits = hidden @ embed.weight.T``.

    ``labels`` follow the Hugging Face convention: the shape of ``input_ids``, shifted inside, so the loss is the
    mean of ``CE(logits[:, t], labels[:, t+1])`` over targets other than ``-100``.
    """

    def __init__(self, config: SISAConfig):
        super().__init__(config)
        self._loss_fn = _lm_head_loss

    def forward(self, input_ids: Tensor, labels: Tensor | None = None, *, cache: "SISACache | None" = None,
                fused_ce: bool = False, return_logits: bool = True, logits_to_keep: int = 0) -> SISAOutput:
        """Loss and/or logits of ``input_ids`` ``(B, L)``.

        ``fused_ce=True`` (with labels): the loss from the HIP linear cross-entropy on the GPU, no logits returned.
        ``return_logits=False``: the loss alone. ``logits_to_keep > 0``: logits of the last that many positions only
        (without labels). ``cache``: generation state (:func:`sisa_amd.generation.generate`).
        """
        if labels is not None:
            if labels.shape != input_ids.shape:
                raise ValueError(f"labels {tuple(labels.shape)} and input_ids {tuple(input_ids.shape)} differ in "
                                 f"shape")
            if logits_to_keep:
                raise ValueError("logits_to_keep is for generation; it cannot be combined with labels")
        hidden = SISAModel.forward(self, input_ids, cache=cache)
        head = self.embed.weight
        if labels is None:
            if not return_logits:
                return SISAOutput()
            return SISAOutput(logits=F.linear(hidden[:, -logits_to_keep:] if logits_to_keep else hidden, head))
        inputs, targets = hidden[:, :-1], labels[:, 1:]          # position t predicts token t + 1
        if fused_ce:
            if not hidden.is_cuda:
                raise ValueError("fused_ce=True runs the HIP linear cross-entropy, which needs the model on a GPU")
            return SISAOutput(loss=_lm_head_loss_chunked(inputs, head, targets))
        if not return_logits:
            return SISAOutput(loss=self._loss_fn(inputs, head, targets))
        logits = F.linear(hidden, head)
        return SISAOutput(loss=_token_ce(logits[:, :-1], targets), logits=logits)

    def generate(self, input_ids: Tensor, max_new_tokens: int, temperature: float = 1.0,
                 top_k: int | None = None, eos_token_id: int | Iterable[int] | Tensor | None = None,
                 do_sample: bool = False, **kwargs: Any) -> Tensor:
        """Greedy or sampled continuation of ``input_ids``; see :func:`sisa_amd.generation.generate`."""
        from .generation import generate

        return generate(self, input_ids, max_new_tokens, temperature=temperature, top_k=top_k,
                        eos_token_id=eos_token_id, do_sample=do_sample, **kwargs)

    def save_pretrained(self, path: str, *, safe_serialization: bool = True) -> None:
        """Write ``config.json`` and the weights (``model.safetensors``, or ``pytorch_model.bin``) into ``path``."""
        from .checkpoint import save_pretrained

        save_pretrained(self, path, safe_serialization=safe_serialization)

    @classmethod
    def from_pretrained(cls, path: str, *, dtype: torch.dtype | None = None, **config_overrides: Any
                        ) -> "SISAForCausalLM":
        """A model from a directory written by :meth:`save_pretrained`."""
        from .checkpoint import from_pretrained

        return from_pretrained(path, dtype=dtype, **config_overrides)
