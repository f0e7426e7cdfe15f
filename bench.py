"""Benchmark of the SISA hot path on one MI355X: fused layer core forward + backward at the north-star shape.

One step = the work of ``sisa_fused`` forward + backward on one batch: HIP prep forward (scans, factors, rotation),
attention forward, exact-delta attention backward (dq kernel, dkv kernel, fp64 dlambda) and prep backward, at
B=4, T=4096, H=8, d_head=64, d_state=32, bf16 (BASELINE.json metric; configs[1] is the T=2048 variant of it).
Inputs are synthetic (oracle.reference.config_inputs('ns'), seeded on the CPU) and resident in HBM before timing.

Reported (one JSON line on rank 0):
  value      algorithmic attention TFLOP/s of the step: 1152 * P flop (P = B*H*T^2/2 causal pairs; fwd 320 P,
             bwd 832 P) / step time. tokens_per_s = B*T / step time.
  roofline   the attention kernels (forward + backward launches, the dominant work) against the bf16 dense MFMA
             peak: achieved = 1152 P / (their summed average duration, HIP events on the launch stream).
  roofline_prep  the prep forward against HBM peak: algorithmic bytes / its average duration.
  cpu_baseline   the reference's pure-PyTorch path (oracle restatement of src/sisa/functional.py:106-155 plus the
             modeling.py glue) on the host cores, on a bounded sample of the same workload (one batch row, all 8
             heads, T=4096, fp32 forward + backward).
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--config", default="ns", choices=["ns", "1", "2"])
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-reps", type=int, default=8)
    return p.parse_args()


def cpu_baseline(reps: int) -> dict:
    """A bounded sample of the benchmark workload on the host cores: one batch row (all heads) of the north-star
    shape (T=4096, d_h=64, d_s=32, BASELINE.json config-0 distributions) in fp32, glue + blocked attention forward +
    backward with the oracle's restatement of the reference's pure-PyTorch path."""
    import torch

    from oracle import reference as R
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    B, H, L = 1, 8, 4096
    gen = torch.Generator().manual_seed(0)
    leaves = dict(q=torch.randn(B, H, L, 64, generator=gen), k=torch.randn(B, H, L, 64, generator=gen),
                  v=torch.randn(B, H, L, 64, generator=gen), b=torch.randn(B, H, L, 32, generator=gen),
                  c=torch.randn(B, H, L, 32, generator=gen), theta=0.01 * torch.randn(B, L, H, 16, generator=gen),
                  a=-5 + 0.5 * torch.randn(B, L, H, generator=gen), z=4 + 0.5 * torch.randn(B, L, H, generator=gen),
                  lam_raw=torch.full((H,), -1.0))
    leaves = {n: t.requires_grad_(True) for n, t in leaves.items()}
    dy = torch.randn(B, H, L, 64, generator=gen)

    def step():
        c, b, g, Fg, lam = R.unfused_glue(leaves)
        o = R.attention_blocked(leaves["q"], leaves["k"], leaves["v"], c, b, g, lam, Fg, block_q=256)
        torch.autograd.grad(o, list(leaves.values()), dy)
    step()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    flop = 1152 * B * H * L * L / 2
    return {"value": round(flop / t / 1e12, 5), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"1 batch row (8 heads) of the T=4096 workload in fp32 (1/4 of one step), glue + attention "
                      f"fwd+bwd, median of {reps} runs after 1 warm-up: {t * 1e3:.0f} ms = {B * L / t:.0f} tokens/s"}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)
    import torch

    from oracle.reference import config_inputs
    from sisa_amd import backends
    from sisa_amd.kernels import attention as A
    from sisa_amd.kernels import fused_prep as FP

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    backends.set_check_mode("off")
    cfg = {"ns": "ns", "1": 1, "2": 2}[args.config]
    inp = config_inputs(cfg, device=dev)
    proj, z, dy, H = inp["proj"], inp["z"], inp["dy"], inp["H"]
    lam = torch.nn.functional.softplus(inp["lam_raw"]).float()
    B, L, NP = proj.shape
    D, S = 64, 32
    off = FP.fused_layout(H)

    def col(t, name, w=D):
        return t[..., off[name]:off[name] + H * w].view(B, L, H, w).transpose(1, 2)

    ev = lambda: torch.cuda.Event(enable_timing=True)   # noqa: E731
    marks = {k: [] for k in ("prep_fwd", "attn_fwd", "attn_bwd", "prep_bwd")}

    def step(record: bool):
        e = [ev() for _ in range(5)] if record else None
        if record:
            e[0].record()
        pf = FP._launch_prep_forward(proj, z, H)
        if record:
            e[1].record()
        q, k, v = col(proj, "Q"), col(proj, "K"), col(proj, "V")
        c, b = pf["CR"].transpose(1, 2), pf["BR"].transpose(1, 2)
        o, lse, _, _, _, o32 = A.attn_forward(q, k, v, c, b, pf["G"], lam, pf["F"], factors=(pf["ROWF"], pf["COLF"]),
                                              want32=True)
        if record:
            e[2].record()
        DP = torch.empty_like(proj)
        DCR = torch.empty((B, L, H, S), device=dev, dtype=torch.float32)
        DBR = torch.empty_like(DCR)
        do = dy.reshape(B, L, H, D).transpose(1, 2)
        _, _, _, _, _, dg, dlam, dF = A.attn_backward(q, k, v, c, b, pf["G"], pf["F"], pf["ROWF"], pf["COLF"], lam, o,
                                                      lse, do, True, dq=col(DP, "Q"), dk=col(DP, "K"), dv=col(DP, "V"),
                                                      dc=DCR.transpose(1, 2), db=DBR.transpose(1, 2), o32=o32)
        if record:
            e[3].record()
        FP._launch_prep_backward(proj, z, pf["TOT"], dg, dF, DCR, DBR, DP, H)
        if record:
            e[4].record()
            for i, k_ in enumerate(marks):
                marks[k_].append((e[i], e[i + 1]))

    for _ in range(args.warmup):
        step(False)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step(True)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_step = (t1 - t0) * 1e3 / args.steps
    phases = {k: statistics.mean(a.elapsed_time(b_) for a, b_ in v) for k, v in marks.items()}

    fl = A.flops(B, H, L)
    total_flop = fl["total"]
    value = total_flop / (ms_step * 1e-3) / 1e12
    attn_ms = phases["attn_fwd"] + phases["attn_bwd"]
    achieved = total_flop / (attn_ms * 1e-3) / 1e12
    pb = FP.prep_bytes(B, L, H)
    prep_gbs = pb["total"] / (phases["prep_fwd"] * 1e-3) / 1e9
    out = {
        "metric": "SISA attn fwd+bwd TFLOP/s & tokens/s, bf16 T=4096 1xMI355X; MFMA util %",
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded, BASELINE.json distributions)",
        "config": {"workload": "fused SISA layer core fwd+bwd (prep + attention), north star" if cfg == "ns"
                   else f"fused SISA layer core fwd+bwd, config {cfg}",
                   "B": B, "T": L, "H": H, "d_head": D, "d_state": S, "parallelism": "none (1 GPU)"},
        "tokens_per_s": round(B * L / (ms_step * 1e-3), 1),
        "mfma_util_pct": round(100 * value / PEAK_BF16_TFLOPS, 2),
        "phases_ms": {k: round(v, 4) for k, v in phases.items()},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 3), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "traffic": None,
                     "kernel": "attention fwd + bwd launches (attn_fwd, attn_bwd_dq, attn_bwd_dkv, dlam)",
                     "algorithmic": f"1152 flop per causal pair x {fl['pairs']:.4g} pairs per step"},
        "roofline_prep": {"bound": "hbm", "achieved": round(prep_gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                          "frac": round(prep_gbs / PEAK_HBM_GBS, 4),
                          "algorithmic": f"{pb['total'] / 1e6:.1f} MB per prep forward (310 B per token-head)"},
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(args.cpu_reps)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
