"""Dense float64 restatement of the SISA language model -- test infrastructure only.

Reads the parameter values of a model with the reference's parameter names (``sisa_amd.SISAForCausalLM``,
interchangeable state dicts with src/sisa/modeling.py:258-496) and recomputes logits, the loss and every parameter
gradient in float64 with plain torch ops and a dense (L x L) attention: no model code, no kernels, no float32 casts.
It restates the model formula of src/sisa/modeling.py:26-50, 162-222, 288-291, 344-354, 432-472 (the reference's own
fp64 judge does the same, tests/reference_fp64.py:37-97):

    per layer, n = RMSNorm(x):
        q, k, v = W_Q n, W_K n, W_V n;  c, b = W_C n, W_B n;  Phi = cumsum_t(theta_proj n)
        c~, b~ = pair rotation of c, b by Phi;  g = cumsum_t(-softplus(alpha_proj n));  F = cumsum_t(logsigmoid(
        forget_proj n));  lam = softplus(lambda_raw)
        s_ij = q_i.k_j / sqrt(d_head) + lam exp(g_i - g_j) (c~_i . b~_j) + (F_i - F_j)   (j <= i)
        x += W_O softmax(s) v;   x += w_down(silu(w_gate m) * w_up m),  m = RMSNorm(x)
    logits = RMSNorm_final(x) E^T;  loss = CE(logits[:, :-1], labels[:, 1:]), ignore_index -100

Pinning (tests/test_model_cpu.py): the model's own torch path (blocked float32 attention, different code) agrees to
float32 precision in loss, logits and every gradient; torch.autograd.gradcheck on a 1-layer model of width 16; a
model with lambda = 0 and zero forget gates reduces to a plain pre-norm transformer with causal softmax attention
(torch SDPA math path).
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F
from torch.utils.checkpoint import checkpoint


def _rmsnorm(x, w, eps):
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w


def _rotate(z, phi):
    """Interleaved pairs (0,1), (2,3), ... of z rotated by the angles phi (one per pair)."""
    even, odd = z[..., 0::2], z[..., 1::2]
    cs, sn = torch.cos(phi), torch.sin(phi)
    return torch.stack((even * cs - odd * sn, even * sn + odd * cs), dim=-1).flatten(-2)


def _block(x, P, pre, H, dh, ds, eps, causal):
    Bsz, L, _ = x.shape

    def lin(t, name):
        return F.linear(t, P[f"{pre}{name}.weight"], P.get(f"{pre}{name}.bias"))

    n = _rmsnorm(x, P[f"{pre}attn_norm.weight"], eps)

    def split(name, w):
        return lin(n, f"attn.{name}").reshape(Bsz, L, H, w).transpose(1, 2)

    q, k, v = split("W_Q", dh), split("W_K", dh), split("W_V", dh)
    phi = split("theta_proj", ds // 2).cumsum(2)
    ct, bt = _rotate(split("W_C", ds), phi), _rotate(split("W_B", ds), phi)
    g = (-F.softplus(lin(n, "attn.alpha_proj"))).transpose(1, 2).cumsum(2)
    fg = F.logsigmoid(lin(n, "attn.forget_proj")).transpose(1, 2).cumsum(2)
    lam = F.softplus(P[f"{pre}attn.lambda_raw"]).view(1, H, 1, 1)
    dg = (g[..., :, None] - g[..., None, :]).masked_fill(~causal, 0.0)   # future decay exponents masked before exp
    s = q @ k.transpose(-1, -2) / math.sqrt(dh) + lam * dg.exp() * (ct @ bt.transpose(-1, -2))
    s = s + (fg[..., :, None] - fg[..., None, :])
    y = s.masked_fill(~causal, float("-inf")).softmax(-1) @ v
    x = x + lin(y.transpose(1, 2).reshape(Bsz, L, H * dh), "attn.W_O")
    m = _rmsnorm(x, P[f"{pre}ffn_norm.weight"], eps)
    hidden = F.silu(F.linear(m, P[f"{pre}ffn.w_gate.weight"])) * F.linear(m, P[f"{pre}ffn.w_up.weight"])
    return x + F.linear(hidden, P[f"{pre}ffn.w_down.weight"])


def params64(model, dtype=torch.float64, requires_grad=True) -> dict:
    return {n: p.detach().to(dtype).requires_grad_(requires_grad) for n, p in model.named_parameters()}


def logits64(model, P: dict, ids: torch.Tensor) -> torch.Tensor:
    cfg = model.config
    L = ids.shape[1]
    causal = torch.ones(L, L, dtype=torch.bool, device=ids.device).tril()
    x = F.embedding(ids, P["embed.weight"])
    for i in range(cfg.n_layer):
        x = checkpoint(_block, x, P, f"layers.{i}.", cfg.n_head, cfg.d_head, cfg.d_state, cfg.norm_eps, causal,
                       use_reentrant=False)
    return _rmsnorm(x, P["final_norm.weight"], cfg.norm_eps) @ P["embed.weight"].t()


def loss_and_grads64(model, ids: torch.Tensor, labels: torch.Tensor, dtype=torch.float64):
    """-> (loss, logits, {parameter name: gradient}) in ``dtype`` with shifted (Hugging Face style) labels."""
    names = [n for n, _ in model.named_parameters()]
    P = params64(model, dtype)
    logits = logits64(model, P, ids)
    loss = F.cross_entropy(logits[:, :-1].reshape(-1, logits.shape[-1]), labels[:, 1:].reshape(-1),
                           ignore_index=-100)
    grads = torch.autograd.grad(loss, [P[n] for n in names])
    return float(loss.detach()), logits.detach(), {n: g.detach() for n, g in zip(names, grads)}
