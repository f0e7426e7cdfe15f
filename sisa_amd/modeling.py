"""SISA language model: the attention sublayer (the caller of the hot path), pre-norm blocks of SISA attention and
SwiGLU, and the causal LM with the tied embedding as LM head.

``SISAAttention`` mirrors the reference's layer (src/sisa/modeling.py:79-255): the same parameters and
initialisation, the same unfused glue (``_prepare``: cumsums, softplus, log-sigmoid and the pair rotation in fp32),
and the same dispatch, with the Triton paths replaced by ``"hip"`` (glue + HIP attention) and ``"hip_fused"`` (one
projection GEMM + HIP prep + HIP attention). ``RMSNorm``, ``SwiGLU``, ``SISABlock``, ``SISAModel`` and
``SISAForCausalLM`` mirror src/sisa/modeling.py:26-50, 258-496: the same module tree and parameter names (so state
dicts are interchangeable), the same initialisation and the same loss conventions. On the GPU with a HIP attention
implementation, RMSNorm and the SwiGLU activation run as HIP kernels (:mod:`sisa_amd.kernels.norm`) and the LM-head
loss can use the chunked HIP linear cross-entropy (``fused_ce=True``).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import TYPE_CHECKING, Any, Iterable

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch import Tensor
from torch.utils.checkpoint import checkpoint

from .config import ATTN_IMPLS, SISAConfig
from .functional import _attend_rows, _autocast_off, _work_dtype, rotate_pairs, sisa_attention

if TYPE_CHECKING:  # pragma: no cover
    from .generation import SISACache

__all__ = ["RMSNorm", "SwiGLU", "SISAAttention", "SISABlock", "SISAModel", "SISAForCausalLM", "SISAOutput"]

IGNORE_INDEX = -100


def _use_hip_elementwise(x: Tensor, config: SISAConfig) -> bool:
    """RMSNorm / SwiGLU activation on the HIP kernels: GPU input and a HIP attention implementation requested (or
    ``auto`` with the HIP library available). A forced HIP implementation without the library raises."""
    if x.device.type != "cuda" or config.attn_impl == "torch":
        return False
    from . import backends

    ok, why = backends.hip_status(x.device)
    if not ok and config.attn_impl in ("hip", "hip_fused"):
        raise ValueError(f"attn_impl={config.attn_impl!r} is not available: {why}")
    return ok


class RMSNorm(nn.Module):
    """RMSNorm computed in float32; the output has the input's dtype (modeling.py:26-36)."""

    def __init__(self, dim: int, eps: float = 1e-6, config: SISAConfig | None = None):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps
        self._config = config

    def forward(self, x: Tensor) -> Tensor:
        d = x.shape[-1]
        if (self._config is not None and d % 8 == 0 and d <= 4096 and x.numel() > 0
                and _use_hip_elementwise(x, self._config)):
            from .kernels.norm import rms_norm_hip

            return rms_norm_hip(x, self.weight, self.eps)
        norm = torch.rsqrt(x.float().pow(2).mean(-1, keepdim=True) + self.eps)
        return ((x.float() * norm) * self.weight.float()).to(x.dtype)


class SwiGLU(nn.Module):
    """``w_down(silu(w_gate x) * w_up x)``, no biases (modeling.py:39-49)."""

    def __init__(self, d_model: int, d_ff: int, config: SISAConfig | None = None):
        super().__init__()
        self.w_gate = nn.Linear(d_model, d_ff, bias=False)
        self.w_up = nn.Linear(d_model, d_ff, bias=False)
        self.w_down = nn.Linear(d_ff, d_model, bias=False)
        self._config = config

    def forward(self, x: Tensor) -> Tensor:
        d_ff = self.w_gate.out_features
        if (self._config is not None and d_ff % 8 == 0 and x.numel() > 0 and x.shape[-1] % 8 == 0
                and _use_hip_elementwise(x, self._config)):
            # one GEMM against the gate and up weights interleaved in 8-row chunks, then the activation on the
            # chunk pairs (the same dot products as the two projections of the reference)
            from .kernels.norm import interleave_gate_up, swiglu_pairs_hip

            cd = _compute_dtype(x)
            w = interleave_gate_up(self.w_gate.weight.to(cd), self.w_up.weight.to(cd))
            return _linear(swiglu_pairs_hip(F.linear(x, w)), self.w_down.weight)
        a, b = self.w_gate(x), self.w_up(x)
        return self.w_down(F.silu(a) * b)


def _linear(x: Tensor, weight: Tensor, bias: Tensor | None = None, bias_cols: tuple[int, int] | None = None
            ) -> Tensor:
    """``F.linear`` of the HIP block path: with a 16-bit compute dtype on the GPU the weight gradient comes from the
    HIP weight-gradient kernel (fp32, split-K over the tokens) instead of the library GEMM and its cast."""
    if x.is_cuda and _compute_dtype(x) in (torch.bfloat16, torch.float16) and x.shape[-1] % 8 == 0 \
            and weight.shape[0] % 8 == 0:
        from .kernels.wgrad import linear_hip

        return linear_hip(x, weight, bias, bias_cols)
    return F.linear(x, weight, bias)


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

    def _prepare(self, x: Tensor, state: Any = None):
        """Projections and recurrences of the unfused paths: ``q, k, v, c~, b~`` in the compute dtype and ``g, F,
        Phi`` in float32 (modeling.py:171-199). With a decode ``state`` the recurrences continue from its last
        position."""
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
        if state is not None:
            g = g + state.g[..., -1:]
            phi = phi + state.phi.unsqueeze(2)
            fgate = fgate + state.fgate[..., -1:]
        c = rotate_pairs(c.float(), phi)
        b = rotate_pairs(b.float(), phi)
        cd = _compute_dtype(x)
        return q.to(cd), k.to(cd), v.to(cd), c.to(cd), b.to(cd), g, fgate, phi

    def _attend(self, q, k, v, c, b, g, fgate, impl: str) -> Tensor:
        return sisa_attention(q, k, v, c, b, g, self.lam(), fgate, impl=impl, block_q=self.config.torch_block_q)

    def _output(self, y: Tensor) -> Tensor:
        bsz, h, seq_len, dh = y.shape
        return self.W_O(y.transpose(1, 2).reshape(bsz, seq_len, h * dh))

    def _forward_fused(self, x: Tensor, z: Tensor | None = None) -> Tensor:
        """One projection GEMM + HIP prep + HIP attention (modeling.py:217-222). ``z``: the forget-gate logits when
        the caller has computed them already (the decoder block's fused norm), else ``_forget_logits(x)``."""
        from .kernels.fused_prep import concat_fused_weights, sisa_fused

        bsz, seq_len, d = x.shape
        weight, bias = concat_fused_weights(self.W_Q.weight, self.W_K.weight, self.W_V.weight, self.W_B.weight,
                                            self.W_C.weight, self.theta_proj.weight, self.alpha_proj.weight,
                                            self.alpha_proj.bias)
        if z is None:                                     # the sublayer on its own (reference dispatch)
            proj = F.linear(x, weight, bias)              # (B, L, NPAD), autocast dtype
            y = sisa_fused(proj, self._forget_logits(x), self.lam(), self.config.n_head)
            return self.W_O(y.reshape(bsz, seq_len, d))
        from .kernels.fused_prep import fused_layout

        a0 = fused_layout(self.config.n_head)["A"]      # only the alpha columns of the bias are parameters
        proj = _linear(x, weight, bias, (a0, a0 + self.config.n_head))   # the decoder block's HIP path
        y = sisa_fused(proj, z, self.lam(), self.config.n_head)
        return _linear(y.reshape(bsz, seq_len, d), self.W_O.weight)

    def _forward_cached(self, x: Tensor, cache: "SISACache", requested: str) -> Tensor:
        """Prefill (empty layer cache: regular unfused attention) or decode step (modeling.py:224-238). Decode steps
        attend to the cache with the HIP decode kernel on the GPU (``hip``/``hip_fused``/``auto`` with the library),
        else with the exact torch rows in float32."""
        state = cache.get(self.layer_idx)
        q, k, v, c, b, g, fgate, phi = self._prepare(x, state)
        if state is None:
            impl = _resolve_impl("hip" if requested == "hip_fused" else requested, x, self.config)
            y = self._attend(q, k, v, c, b, g, fgate, "hip" if impl == "hip_fused" else impl)
            cache.update(self.layer_idx, k=k, v=v, b=b, g=g, fgate=fgate, phi=phi[:, :, -1])
            return self._output(y)
        start = state.length
        state = cache.update(self.layer_idx, k=k, v=v, b=b, g=g, fgate=fgate, phi=phi[:, :, -1])
        if _use_hip_elementwise(x, self.config) and q.dtype in (torch.bfloat16, torch.float16, torch.float32):
            from .kernels.decode import sisa_decode_hip

            y = sisa_decode_hip(q, state.k, state.v, c, state.b, g, state.g, self.lam(), fgate, state.fgate, start)
            return self._output(y.to(q.dtype))
        wd = _work_dtype(q.dtype)
        y = _attend_rows(q.to(wd), state.k.to(wd), state.v.to(wd), c.to(wd), state.b.to(wd), g.to(wd),
                         state.g.to(wd), self.lam().to(wd), fgate.to(wd), state.fgate.to(wd), start)
        return self._output(y.to(q.dtype))

    def forward(self, x: Tensor, *, cache: "SISACache | None" = None, impl: str | None = None) -> Tensor:
        """Apply the sublayer to the normalised input ``x`` ``(B, L, d_model)``; returns ``(B, L, d_model)``.
        ``cache``: decode cache (:mod:`sisa_amd.generation`; an empty one is filled by this call, a filled one is
        extended). ``impl`` overrides ``config.attn_impl`` for this call."""
        requested = impl or self.config.attn_impl
        if cache is not None:
            return self._forward_cached(x, cache, requested)
        impl = _resolve_impl(requested, x, self.config)
        if impl == "hip_fused":
            return self._forward_fused(x)
        q, k, v, c, b, g, fgate, _ = self._prepare(x)
        return self._output(self._attend(q, k, v, c, b, g, fgate, impl))


class SISABlock(nn.Module):
    """``x + attn(attn_norm(x))`` followed by ``x + ffn(ffn_norm(x))`` (modeling.py:258-291). The constructor applies
    the SISA initialisation, so the block can be used on its own."""

    def __init__(self, config: SISAConfig, layer_idx: int = 0):
        super().__init__()
        self.config = config
        self.attn_norm = RMSNorm(config.d_model, config.norm_eps, config)
        self.attn = SISAAttention(config, layer_idx)
        self.ffn_norm = RMSNorm(config.d_model, config.norm_eps, config)
        self.ffn = SwiGLU(config.d_model, config.d_ff, config)
        self.fuse_norm = True          # use the fused HIP norm path where it applies (see _fused_norm_ok)
        self._reset_ffn_and_norms()

    @torch.no_grad()
    def _reset_ffn_and_norms(self) -> None:
        for lin in (self.ffn.w_gate, self.ffn.w_up, self.ffn.w_down):
            nn.init.normal_(lin.weight, std=self.config.init_std)
        nn.init.ones_(self.attn_norm.weight)
        nn.init.ones_(self.ffn_norm.weight)

    @torch.no_grad()
    def reset_parameters(self) -> None:
        """MLP weights ~ N(0, ``init_std``), norms 1, and :meth:`SISAAttention.reset_parameters`."""
        self._reset_ffn_and_norms()
        self.attn.reset_parameters()

    def _fused_norm_ok(self, x: Tensor) -> bool:
        """The HIP block path applies: GPU input, the fused HIP attention selected for it, and rows the norm
        kernels take."""
        if not self.fuse_norm or x.device.type != "cuda" or x.dim() != 3 or x.numel() == 0:
            return False
        d, h = x.shape[-1], self.config.n_head
        if d % 8 or d > 4096 or h > 64 or x.dtype not in (torch.float32, torch.bfloat16, torch.float16):
            return False
        return _resolve_impl(self.config.attn_impl, x, self.config) == "hip_fused"

    def _forward_hip(self, x: Tensor, res: Tensor | None = None, defer: bool = False):
        """The block on the HIP kernels: the attention norm and the fp32 forget-gate projection in one pass that
        also emits the normalised rows in the dtype of the projection GEMM (the reference casts them under autocast),
        the fused attention sublayer, the residual add and the FFN norm in one pass, SwiGLU.

        ``res``: the previous block's FFN output, whose residual add (``x + res``) runs in this block's attention
        norm. ``defer=True`` returns ``(h, f)`` -- the stream before the FFN residual and the FFN output -- for the
        next block to add the same way (``(h + f, None)`` when ``f`` cannot be passed on); otherwise ``h + f``."""
        from .kernels.norm import rms_norm_add_hip, rms_norm_forget_add_hip, rms_norm_forget_hip, rms_norm_hip

        cd = _compute_dtype(x)
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
        x = x + self.attn(self.attn_norm(x), cache=cache)
        return x + self.ffn(self.ffn_norm(x))


@dataclass
class SISAOutput:
    """Output of :meth:`SISAForCausalLM.forward`."""

    loss: Tensor | None = None
    logits: Tensor | None = None


def _lm_head_loss(hidden: Tensor, weight: Tensor, labels: Tensor) -> Tensor:
    """Cross-entropy of the tied LM head; ``labels`` are already aligned with ``hidden``."""
    logits = F.linear(hidden, weight)
    return F.cross_entropy(logits.reshape(-1, logits.shape[-1]).float(), labels.reshape(-1),
                           ignore_index=IGNORE_INDEX)


# Consecutive fused HIP blocks pass the FFN output on to the next block's attention norm (SISAModel.forward); False
# adds it in each block instead (same results bit for bit).
DEFER_RESIDUAL = True


class SISAModel(nn.Module):
    """Embedding, ``n_layer`` :class:`SISABlock` s and the final RMSNorm (modeling.py:308-414); ``forward(input_ids)``
    returns the final-normalised hidden states ``(B, L, d_model)``."""

    def __init__(self, config: SISAConfig):
        super().__init__()
        self.config = config.replace()          # private, validated copy shared by all submodules
        cfg = self.config
        self.embed = nn.Embedding(cfg.vocab_size, cfg.d_model)
        self.layers = nn.ModuleList([SISABlock(cfg, i) for i in range(cfg.n_layer)])
        self.final_norm = RMSNorm(cfg.d_model, cfg.norm_eps, cfg)
        self._reset_embedding_and_norm()

    @torch.no_grad()
    def _reset_embedding_and_norm(self) -> None:
        nn.init.normal_(self.embed.weight, std=self.config.init_std)
        nn.init.ones_(self.final_norm.weight)

    @torch.no_grad()
    def reset_parameters(self) -> None:
        """Re-initialise every parameter as at construction."""
        self._reset_embedding_and_norm()
        for layer in self.layers:
            layer.reset_parameters()

    def forward(self, input_ids: Tensor, *, cache: "SISACache | None" = None) -> Tensor:
        x = self.embed(input_ids)
        use_ckpt = (self.config.gradient_checkpointing and self.training and cache is None
                    and torch.is_grad_enabled())
        # Consecutive blocks on the fused HIP path pass their FFN output on instead of adding it: the next block's
        # attention norm adds it in its own pass (same arithmetic, one launch less each way per block).
        pending = None
        for layer in self.layers:
            if DEFER_RESIDUAL and not use_ckpt and cache is None and layer._fused_norm_ok(x):
                x, pending = layer._forward_hip(x, pending, defer=True)
                continue
            if pending is not None:
                x, pending = x + pending, None
            x = checkpoint(layer, x, use_reentrant=False) if use_ckpt else layer(x, cache=cache)
        if pending is not None:
            x = x + pending
        return self.final_norm(x)

    def compile_common(self) -> "SISAModel":
        """The reference compiles the RMSNorm and SwiGLU submodules with ``torch.compile`` (modeling.py:396-414), so
        that Inductor fuses their elementwise work. Here that work already runs in fused HIP kernels on the GPU
        (norm + forget projection, interleaved gate/up + SwiGLU), and this build emits no Triton, so the modules are
        left as they are: state-dict keys stay unchanged. Returns the model."""
        return self

    def set_attn_impl(self, impl: str) -> None:
        """Switch the attention implementation (``auto``/``torch``/``hip``/``hip_fused``) of every layer."""
        self.config.replace(attn_impl=impl)     # validates
        self.config.attn_impl = impl

    def num_parameters(self, exclude_embeddings: bool = False) -> int:
        """Number of parameters; the tied LM head is counted once."""
        n = sum(p.numel() for p in self.parameters())
        return n - self.embed.weight.numel() if exclude_embeddings else n

    def param_groups(self, lr: float, weight_decay: float = 0.1, lambda_lr: float | None = None,
                     no_decay_timescale_biases: bool = True) -> list[dict[str, Any]]:
        """Optimizer parameter groups (modeling.py:366-394): ``default`` (with ``weight_decay``),
        ``timescale_biases`` (``alpha_proj.bias``, ``forget_proj.bias``; no decay) and ``lambda`` (``lambda_raw``;
        no decay, at ``lambda_lr``)."""
        default, timescale, lam = [], [], []
        for name, p in self.named_parameters():
            if not p.requires_grad:
                continue
            if name.endswith("lambda_raw"):
                lam.append(p)
            elif no_decay_timescale_biases and name.endswith(("alpha_proj.bias", "forget_proj.bias")):
                timescale.append(p)
            else:
                default.append(p)
        groups = [{"params": default, "lr": lr, "weight_decay": weight_decay, "name": "default"}]
        if timescale:
            groups.append({"params": timescale, "lr": lr, "weight_decay": 0.0, "name": "timescale_biases"})
        if lam:
            groups.append({"params": lam, "lr": lr if lambda_lr is None else lambda_lr, "weight_decay": 0.0,
                           "name": "lambda"})
        return groups


class SISAForCausalLM(SISAModel):
    """:class:`SISAModel` with the tied LM head ``logits = final_norm(h) @ embed.weight.T`` (modeling.py:417-496).

    Labels follow the Hugging Face convention: ``labels`` has the shape of ``input_ids`` and the model shifts
    internally, ``loss = CE(logits[:, :-1], labels[:, 1:])`` with ``ignore_index=-100``, averaged over non-ignored
    targets.
    """

    def __init__(self, config: SISAConfig):
        super().__init__(config)
        self._loss_fn = _lm_head_loss

    def forward(self, input_ids: Tensor, labels: Tensor | None = None, *, cache: "SISACache | None" = None,
                fused_ce: bool = False, return_logits: bool = True, logits_to_keep: int = 0) -> SISAOutput:
        """``fused_ce``: compute the loss with the chunked HIP linear cross-entropy (GPU; logits are then not
        returned; no effect without ``labels``). ``return_logits=False``: the loss without keeping the logits.
        ``logits_to_keep > 0``: logits of the last positions only (not with ``labels``)."""
        if labels is not None and labels.shape != input_ids.shape:
            raise ValueError(f"labels shape {tuple(labels.shape)} must match input_ids {tuple(input_ids.shape)}")
        if labels is not None and logits_to_keep:
            raise ValueError("logits_to_keep cannot be combined with labels")
        hidden = super().forward(input_ids, cache=cache)
        weight = self.embed.weight
        loss = logits = None
        fused_ce = fused_ce and labels is not None
        if fused_ce:
            if not hidden.is_cuda:
                raise ValueError("fused_ce=True needs CUDA (GPU) tensors")
            from .kernels.linear_ce import linear_cross_entropy

            d = hidden.shape[-1]
            loss = linear_cross_entropy(hidden[:, :-1].reshape(-1, d), weight, labels[:, 1:].reshape(-1),
                                        ignore_index=IGNORE_INDEX)
        elif labels is not None and not return_logits:
            loss = self._loss_fn(hidden[:, :-1], weight, labels[:, 1:])
        if return_logits and not fused_ce:
            logits = F.linear(hidden[:, -logits_to_keep:] if logits_to_keep else hidden, weight)
            if labels is not None:
                vocab = logits.shape[-1]
                loss = F.cross_entropy(logits[:, :-1].reshape(-1, vocab).float(), labels[:, 1:].reshape(-1),
                                       ignore_index=IGNORE_INDEX)
        return SISAOutput(loss=loss, logits=logits)

    def generate(self, input_ids: Tensor, max_new_tokens: int, temperature: float = 1.0,
                 top_k: int | None = None, eos_token_id: int | Iterable[int] | Tensor | None = None,
                 do_sample: bool = False, **kwargs: Any) -> Tensor:
        """Greedy or sampled decoding with a cache; see :func:`sisa_amd.generation.generate`."""
        from .generation import generate

        return generate(self, input_ids, max_new_tokens, temperature=temperature, top_k=top_k,
                        eos_token_id=eos_token_id, do_sample=do_sample, **kwargs)

    def save_pretrained(self, path: str, *, safe_serialization: bool = True) -> None:
        """Write ``config.json`` and ``model.safetensors`` (or ``pytorch_model.bin``) to ``path``."""
        from .checkpoint import save_pretrained

        save_pretrained(self, path, safe_serialization=safe_serialization)

    @classmethod
    def from_pretrained(cls, path: str, *, dtype: torch.dtype | None = None, **config_overrides: Any
                        ) -> "SISAForCausalLM":
        """Load a directory written by :meth:`save_pretrained`."""
        from .checkpoint import from_pretrained

        return from_pretrained(path, dtype=dtype, **config_overrides)
