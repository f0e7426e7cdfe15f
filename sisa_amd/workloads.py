"""Synthetic workloads of the benchmark configurations: seeded input tensors, drawn on the CPU.

Used by bench.py's GPU legs and by the tests; data generation only (no arithmetic of the path). The fused configs
(1, 'ns', 2) fill the fused projection in the column layout of src/sisa/kernels/fused_prep.py:71-96 with seeded
normal draws: q, k, v, B, C ~ N(0,1), theta ~ N(0, 0.01^2), alpha pre-activation ~ N(-5, 0.5^2) (N(-7, 1) at
config 2), forget pre-activation ~ N(4, 0.5^2).
"""
from __future__ import annotations

import torch

from .kernels.fused_prep import fused_layout


def config_inputs(cfg: int, device="cpu", dtype=None) -> dict:
    """Synthetic inputs of the benchmark configs, drawn from ``torch.Generator().manual_seed(cfg)`` on the CPU.

    cfg 0: B=1 T=256 H=4 fp32 unfused (q,k,v,B,C ~ N(0,1), theta ~ N(0,0.01^2) [B,T,H,16], a ~ N(-5,0.5^2),
           z ~ N(4,0.5^2), lambda_raw = -1, upstream gradient ~ N(0,1)).
    cfg 1: B=4 T=2048 H=8; cfg 'ns': B=4 T=4096 H=8 -- the same distributions as proj columns (bf16) and z (fp32).
    cfg 2: B=1 T=16384 H=16, a ~ N(-7,1), z ~ N(4,1).
    cfg 3: linear cross-entropy, hidden [16384, 768] ~ N(0,1), W [50277, 768] ~ N(0, 0.02^2) fp32 master,
           labels ~ U[0, 50277); hidden in ``dtype`` (default bf16).
    Returns dict(proj, z, lam_raw, dy, H) for the fused configs, dict(hidden, weight, labels) for cfg 3 and the
    unfused tensors for cfg 0."""
    if cfg == 3:
        gen = torch.Generator().manual_seed(3)
        N, D, V = 16384, 768, 50277
        hidden = torch.randn(N, D, generator=gen)
        weight = 0.02 * torch.randn(V, D, generator=gen)
        labels = torch.randint(0, V, (N,), generator=gen)
        return dict(hidden=hidden.to(dtype or torch.bfloat16).to(device), weight=weight.to(device),
                    labels=labels.to(device))
    shapes = {0: (1, 256, 4), 1: (4, 2048, 8), "ns": (4, 4096, 8), 2: (1, 16384, 16)}
    B, L, H = shapes[cfg]
    seed = {0: 0, 1: 1, "ns": 5, 2: 2}[cfg]
    a_mu, a_sd, z_sd = (-7.0, 1.0, 1.0) if cfg == 2 else (-5.0, 0.5, 0.5)
    gen = torch.Generator().manual_seed(seed)
    lam_raw = torch.full((H,), -1.0)
    if cfg == 0:
        dt = dtype or torch.float32
        q, k, v = (torch.randn(B, H, L, 64, generator=gen) for _ in range(3))
        bm, cm = (torch.randn(B, H, L, 32, generator=gen) for _ in range(2))
        theta = 0.01 * torch.randn(B, L, H, 16, generator=gen)
        a = a_mu + a_sd * torch.randn(B, L, H, generator=gen)
        z = 4.0 + z_sd * torch.randn(B, L, H, generator=gen)
        dy = torch.randn(B, H, L, 64, generator=gen)
        out = dict(q=q, k=k, v=v, b=bm, c=cm, theta=theta, a=a, z=z, lam_raw=lam_raw, dy=dy)
        return {n: t.to(device=device, dtype=dt if t.is_floating_point() else t.dtype) for n, t in out.items()}
    dt = dtype or torch.bfloat16
    off = fused_layout(H)
    P = torch.zeros(B, L, off["NPAD"])
    P[..., :off["TH"]] = torch.randn(B, L, off["TH"], generator=gen)
    P[..., off["TH"]:off["A"]] = 0.01 * torch.randn(B, L, H * 16, generator=gen)
    P[..., off["A"]:off["NTOT"]] = a_mu + a_sd * torch.randn(B, L, H, generator=gen)
    z = 4.0 + z_sd * torch.randn(B, L, H, generator=gen)
    dy = torch.randn(B, L, H * 64, generator=gen)
    return dict(proj=P.to(dt).to(device), z=z.to(device), lam_raw=lam_raw.to(device), dy=dy.to(dt).to(device), H=H)
