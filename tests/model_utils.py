"""Shared pieces of the model-level tests: a tiny kernel-compatible configuration and a model taken off the SISA
init so that every term of the score contributes."""
from __future__ import annotations

import torch

from sisa_amd import SISAConfig, SISAForCausalLM

#: Two layers of two 64-wide heads (the HIP kernels' d_head), d_state 32, vocabulary 257, torch attention.
TINY = dict(vocab_size=257, d_model=128, n_layer=2, n_head=2, d_ff=256, d_state=32, attn_impl="torch")

#: Parameters (by state-dict suffix) redrawn away from the init, and how. At init W_C = 0 switches the state term
#: off, every head shares one decay and one forget bias, lambda is one constant and the norm gains are 1.
_REDRAW = {
    "attn.W_C.weight": ("normal", 0.08),
    "attn.W_B.weight": ("normal", 0.08),
    "attn.theta_proj.weight": ("normal", 0.2),          # scaled by theta_scale
    "attn.alpha_proj.bias": ("uniform", -4.0, -1.0),
    "attn.forget_proj.bias": ("uniform", 0.0, 3.0),
    "attn.lambda_raw": ("uniform", -0.5, 1.5),
    "attn_norm.weight": ("near_one", 0.1),
    "ffn_norm.weight": ("near_one", 0.1),
}


def tiny_config(**overrides) -> SISAConfig:
    return SISAConfig(**{**TINY, **overrides})


@torch.no_grad()
def perturb_(model: SISAForCausalLM, seed: int = 0, theta_scale: float = 1.0) -> SISAForCausalLM:
    """Redraw the :data:`_REDRAW` parameters of every block in place from a generator seeded with ``seed``."""
    gen = torch.Generator().manual_seed(10_007 * seed + 3)
    for name, p in model.named_parameters():
        rule = next((r for suffix, r in _REDRAW.items() if name.endswith(suffix)), None)
        if rule is None:
            continue
        kind, *args = rule
        if kind == "uniform":
            lo, hi = args
            draw = lo + (hi - lo) * torch.rand(p.shape, generator=gen)
        else:
            draw = args[0] * torch.randn(p.shape, generator=gen)
            draw = draw * theta_scale if "theta_proj" in name else draw
            draw = draw + 1.0 if kind == "near_one" else draw
        p.copy_(draw)
    return model


def tiny_model(seed: int = 0, theta_scale: float = 1.0, **overrides) -> SISAForCausalLM:
    """A :func:`tiny_config` model (fields overridable), initialised under ``seed`` and then perturbed."""
    torch.manual_seed(seed)
    return perturb_(SISAForCausalLM(tiny_config(**overrides)), seed, theta_scale)


def token_ids(bsz: int, seq_len: int, vocab: int = TINY["vocab_size"], seed: int = 0) -> torch.Tensor:
    return torch.randint(0, vocab, (bsz, seq_len), generator=torch.Generator().manual_seed(seed))


def rel_err(x: torch.Tensor, ref: torch.Tensor) -> float:
    """Relative error in the 2-norm, computed in float64."""
    diff = torch.linalg.vector_norm(x.detach().double() - ref.detach().double())
    return float(diff / torch.linalg.vector_norm(ref.detach().double()).clamp_min(1e-300))
