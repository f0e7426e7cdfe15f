"""Helpers shared by the model-level tests: tiny kernel-compatible models moved away from the init."""
from __future__ import annotations

import torch

from sisa_amd import SISAConfig, SISAForCausalLM


def tiny_config(**overrides) -> SISAConfig:
    """Two layers of two 64-wide heads (the HIP kernels' d_head), d_state 32, vocabulary 257."""
    base = dict(vocab_size=257, d_model=128, n_layer=2, n_head=2, d_ff=256, d_state=32, attn_impl="torch")
    base.update(overrides)
    return SISAConfig(**base)


@torch.no_grad()
def perturb_(model: SISAForCausalLM, seed: int = 0, theta_scale: float = 1.0) -> SISAForCausalLM:
    """Switch on every term of the score: W_C non-zero, faster rotations, spread decay and forget biases, larger
    lambda, norm weights away from 1 (the init has W_C = 0 and identical biases)."""
    gen = torch.Generator().manual_seed(seed + 1)

    def uniform(t, lo, hi):
        return torch.rand(t.shape, generator=gen) * (hi - lo) + lo

    for layer in model.layers:
        at = layer.attn
        at.W_C.weight.copy_(0.08 * torch.randn(at.W_C.weight.shape, generator=gen))
        at.W_B.weight.copy_(0.08 * torch.randn(at.W_B.weight.shape, generator=gen))
        at.theta_proj.weight.copy_(0.2 * theta_scale * torch.randn(at.theta_proj.weight.shape, generator=gen))
        at.alpha_proj.bias.copy_(uniform(at.alpha_proj.bias, -4.0, -1.0))
        at.forget_proj.bias.copy_(uniform(at.forget_proj.bias, 0.0, 3.0))
        at.lambda_raw.copy_(uniform(at.lambda_raw, -0.5, 1.5))
        for norm in (layer.attn_norm, layer.ffn_norm):
            norm.weight.copy_(1.0 + 0.1 * torch.randn(norm.weight.shape, generator=gen))
    return model


def tiny_model(seed: int = 0, theta_scale: float = 1.0, **overrides) -> SISAForCausalLM:
    torch.manual_seed(seed)
    return perturb_(SISAForCausalLM(tiny_config(**overrides)), seed, theta_scale)


def token_ids(bsz: int, seq_len: int, vocab: int = 257, seed: int = 0) -> torch.Tensor:
    return torch.randint(0, vocab, (bsz, seq_len), generator=torch.Generator().manual_seed(seed))


def rel_err(x: torch.Tensor, ref: torch.Tensor) -> float:
    """``||x - ref|| / ||ref||`` in float64."""
    x, ref = x.detach().double(), ref.detach().double()
    return float((x - ref).norm() / ref.norm().clamp_min(1e-300))
