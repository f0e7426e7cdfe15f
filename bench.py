"""Benchmark of the SISA hot path on one MI355X: fused layer core forward + backward at the north-star shape.

One step = the work of ``sisa_fused`` forward + backward on one batch: HIP prep forward (scans, factors, rotation),
attention forward, exact-delta attention backward (dq kernel, dkv kernel, fp64 dlambda) and prep backward, at
B=4, T=4096, H=8, d_head=64, d_state=32, bf16 (BASELINE.json metric; configs[1] is the T=2048 variant of it).
Inputs are synthetic (sisa_amd.workloads.config_inputs('ns'), seeded on the CPU) and resident in HBM before timing.
The headline step is the kernels of the path (check mode "off": sisa_fused's non-finite input guard checks inputs
and is not part of the attention arithmetic). fused_layer_async times the same work as users call it -- sisa_fused
forward and backward through autograd, eager launches, in the default "async" check mode (guard included) -- and the
model step runs in the default mode too, with its "off" figure beside it.

Reported (one JSON line on rank 0):
  value      algorithmic attention TFLOP/s of the step: 1152 * P flop (P = B*H*T^2/2 causal pairs; fwd 320 P,
             bwd 832 P) / step time. tokens_per_s = B*T / step time. The timed steps are replays of a HIP graph
             holding one step's launches (every kernel runs in every replay; no host work between launches);
             eager_ms_per_step is the same step as eager launches (--eager times that instead).
  roofline   the attention kernels (forward + backward launches, the dominant work) against the bf16 dense MFMA
             peak: achieved = 1152 P / (their summed average duration, HIP events on the launch stream).
  roofline_prep  the prep forward (its two launches, queued behind a GPU spin so that host work is not timed)
             against HBM peak: algorithmic bytes / their average duration; beside it a plain device copy moving the
             same number of bytes (half read, half written), timed the same way, as the ceiling HBM offers to a
             transfer of this size (copy_same_bytes_gbs, frac_of_copy); the prep backward likewise (backward).
             phases_ms are the step's own event phases, host gaps included.
  lmce       the linear cross-entropy at config 3 (N=16384, d=768, V=50277): the gradient step on the HIP MFMA
             kernels (sisa_lmce_train; TFLOP/s of 6 N V d against the bf16 MFMA peak; the reference's arrangement with
             library GEMMs timed beside it) and the loss without gradients on the fused HIP kernel (MFMA roofline, no
             logits buffer).
  fused_layer_async  sisa_fused forward + backward through autograd in the default "async" check mode (guard
             included, eager launches): ms and TFLOP/s, beside the same calls in "off" mode.
  model_step the full decoder training step at config 4 (sisa-152m, B=8, T=2048, bf16 autocast, fused attention,
             HIP RMSNorm/SwiGLU, fused linear CE, AdamW): tokens/s in the default "async" check mode, and in "off".
  block_kernels  RMSNorm, SwiGLU activation and decode-attention kernels against HBM peak (config-4 shapes).
  projection_gemms  the library GEMMs of one config-4 layer (fwd, dx, dW of W_cat, W_O, gate/up, down) against
             the bf16 MFMA peak.
  cpu_baseline   the reference's pure-PyTorch path (oracle restatement of src/sisa/functional.py:106-155 plus the
             modeling.py glue) on the host cores, on a bounded sample of the same workload (one batch row, all 8
             heads, T=4096, fp32 forward + backward); config0: BASELINE.json config 0 itself (B=1, T=256, H=4, fp32
             fwd+bwd) on the same cores.
  config0_gpu  config 0 on the GPU through the product path (torch glue + the fp32 HIP attention kernels): a latency
             figure beside cpu_baseline.config0.
"""
from __future__ import annotations

import argparse
import contextlib
import gc
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

@contextlib.contextmanager
def _quiet_host():
    """Python's cyclic garbage collector off (after one collection) inside a timed region: a collection of the
    interpreter's heap can pause the host thread that issues the launches for tens of milliseconds (measured: one
    ~40 ms pause in the first process on a fresh box), which would be timed as GPU idle time."""
    gc.collect()
    gc.disable()
    try:
        yield
    finally:
        gc.enable()


PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0
# Profiles of this build's kernels (rocprofv3 under the commands the files name), read at run time so that the bench
# line quotes the committed measurements: HBM bytes per dispatch (FETCH_SIZE / WRITE_SIZE, each scaled by what the
# counter reads for a plain 1 GiB copy) and the counter-measured MFMA busy fraction of the attention kernels.
PROFILES = os.path.join(ROOT, "profiles")
ATTN_KERNELS = ("attn_fwd_kernelIDF16b", "attn_bwd_dq_kernelIDF16b", "attn_bwd_dkv_kernelIDF16b")
PREP_FWD_KERNELS = ("prep_sums_kernelIDF16b", "prep_fwd_kernelIDF16b")


def profiled_traffic(kernels, name: str = "hbm_traffic_ns_ce.txt") -> float | None:
    """Sum of read + written MB per dispatch (calibrated, 1 MB = 1e6 B) of the named kernels in a committed traffic
    profile (its table rows: calls FETCH_KiB WRITE_KiB read_MB written_MB kernel), in bytes; None when absent."""
    found = {}
    try:
        with open(os.path.join(PROFILES, name)) as f:
            for line in f:
                parts = line.split()
                if len(parts) < 6 or not parts[0].isdigit():
                    continue
                for k in kernels:
                    if k in parts[5] and k not in found:
                        found[k] = (float(parts[3]) + float(parts[4])) * 1e6
    except (OSError, ValueError):
        return None
    return sum(found.values()) if len(found) == len(kernels) else None


def profiled_mfma_busy(name: str = "counters_ns_ce.txt") -> dict | None:
    """Per-kernel and time-weighted MFMA busy percentages of the attention kernels from the committed counter profile
    (a table whose header row starts with ``kernel`` and names ``us`` and ``mfma_busy_pct``); None when absent."""
    rows, cols = {}, None
    try:
        with open(os.path.join(PROFILES, name)) as f:
            for line in f:
                parts = line.split()
                if parts and parts[0] == "kernel" and "mfma_busy_pct" in parts:
                    cols = (parts.index("us"), parts.index("mfma_busy_pct"))
                elif cols and len(parts) > max(cols) and parts[0] in ("attn_fwd", "attn_bwd_dq", "attn_bwd_dkv"):
                    rows[parts[0]] = (float(parts[cols[0]]), float(parts[cols[1]]))
    except (OSError, ValueError):
        return None
    if len(rows) != 3:
        return None
    t = sum(us for us, _ in rows.values())
    out = {k: v[1] for k, v in rows.items()}
    out["time_weighted"] = round(sum(us * b for us, b in rows.values()) / t, 2)
    out["source"] = f"profiles/{name} (rocprofv3 counter passes of this build, not measured in this run)"
    return out


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--config", default="ns", choices=["ns", "1", "2"])
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-reps", type=int, default=8)
    p.add_argument("--no-ce", action="store_true", help="skip the linear cross-entropy leg (config 3)")
    p.add_argument("--no-model", action="store_true", help="skip the full decoder training step leg (config 4)")
    p.add_argument("--eager", action="store_true",
                   help="time the step as eager launches instead of replays of a HIP graph of one step")
    p.add_argument("--copy-mib", type=int, default=0,
                   help="run one plain device copy of this many MiB first (calibrates HBM byte counters)")
    return p.parse_args()


def queued_seconds(launch, reps: int = 20) -> float:
    """Average seconds per call of ``launch()`` (one or more back-to-back GPU launches), the calls queued behind a GPU
    spin so that host work between them is not timed: HIP events around the reps on the launch stream."""
    import torch

    launch()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with _quiet_host():
        torch.cuda._sleep(20_000_000)      # the GPU spins while the host queues the timed launches
        e0.record()
        for _ in range(reps):
            launch()
        e1.record()
        torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps * 1e-3


def prep_kernel_rates(proj, z, H: int) -> dict:
    """The prep forward (prep_sums + prep_fwd) and backward (prep_bwd, one launch) through the C-ABI with
    prepared arguments, timed by queued_seconds, against HBM peak; beside them a plain device copy moving the same
    number of bytes (half read, half written) as the ceiling HBM offers to a transfer of that size."""
    import ctypes
    import torch
    from sisa_amd.kernels import _lib
    from sisa_amd.kernels import fused_prep as FP

    B, L, _ = proj.shape
    dev = proj.device
    lib = _lib.load()
    st = _lib.stream_of(proj)
    pf = FP.prep_forward(proj, z, H)
    fa = _lib.PrepFwdArgs(B, L, H, _lib.dtype_code(proj.dtype), proj.data_ptr(), proj.stride(0), proj.stride(1),
                          _lib.ptr(z), z.stride(0), z.stride(1), pf.cr.data_ptr(), pf.br.data_ptr(),
                          pf.g.data_ptr(), _lib.ptr(pf.f), pf.rowf.data_ptr(), pf.colf.data_ptr(),
                          pf.totals.data_ptr())
    xch = FP.exchange_workspace(proj, B, L, H)
    gen = torch.Generator().manual_seed(9)
    dg, dF = (torch.randn(B, H, L, generator=gen).to(dev) for _ in range(2))
    DCR, DBR = (torch.randn(B, L, H, 32, generator=gen).to(dev) for _ in range(2))
    DP = torch.zeros_like(proj)
    DZ = torch.empty(B, L, H, device=dev)
    ba = _lib.PrepBwdArgs(B, L, H, _lib.dtype_code(proj.dtype), proj.data_ptr(), proj.stride(0), proj.stride(1),
                          _lib.ptr(z), z.stride(0), z.stride(1), pf.totals.data_ptr(), dg.data_ptr(), dF.data_ptr(),
                          DCR.data_ptr(), DBR.data_ptr(), DP.data_ptr(), DP.stride(0), DP.stride(1), DZ.data_ptr(),
                          DZ.stride(0), DZ.stride(1), xch.data_ptr())

    def call(name, args):
        def go():
            if getattr(lib, name)(ctypes.byref(args), st) != 0:
                raise RuntimeError(f"{name}: {lib.sisa_last_error().decode()}")
        return go

    th = B * L * H
    # backward per (token, head): read C, B (2*32 * 2 B), theta (16 * 2 B), dC~, dB~ (2*32 * 4 B), dg, dF (4 B each),
    # alpha (2 B), z (4 B); write dC, dB (2*32 * 2 B), dtheta (16 * 2 B), dalpha (2 B), dz (4 B): 596 B
    sizes = {"prep_fwd": FP.prep_bytes(B, L, H)["total"], "prep_bwd": th * 596}
    out = {}
    for key, fn in (("prep_fwd", call("sisa_prep_fwd", fa)), ("prep_bwd", call("sisa_prep_bwd", ba))):
        nbytes = sizes[key]
        sec = queued_seconds(fn)
        n = nbytes // 2 // 16 * 4                      # fp32 elements of a copy moving nbytes in total
        src = torch.ones(n, device=dev)
        dst = torch.empty_like(src)
        csec = queued_seconds(lambda: dst.copy_(src))
        gbs, cgbs = nbytes / sec / 1e9, 2 * n * 4 / csec / 1e9
        out[key] = {"us": round(sec * 1e6, 2), "bytes": int(nbytes), "achieved": round(gbs, 1),
                    "frac": round(gbs / PEAK_HBM_GBS, 4), "copy_same_bytes_gbs": round(cgbs, 1),
                    "frac_of_copy": round(gbs / cgbs, 4)}
    return out


def bench_ce(steps: int, warmup: int) -> dict:
    """Linear cross-entropy at config 3 (N=16,384 tokens, d=768, V=50,277, bf16), inputs resident in HBM.

    train: the loss with both gradients as linear_cross_entropy runs it -- sisa_lmce_train over the chunk(s) of at
    most 2 GiB of stored exponentials (one chunk here): the logits GEMM storing the exponentials, the split combine,
    the scale pass, the dW + dx MFMA launch forming G in operand staging, the dx split sum. Each call queued behind a
    GPU spin (HIP events). phases_ms: the forward part (the same call without dx and dW) and the rest. Beside it the
    reference's arrangement on this GPU (library_chunk_loop_ms: hipBLASLt logits GEMM, the HIP row pass writing G over
    the logits, hipBLASLt dx and dW GEMMs; chunks of 1 GiB of logits), the design this pass replaces.
    fused_forward: the loss without gradients on the fused HIP kernel (sisa_lmce_fwd: MFMA GEMM reduced to lse and
    the label logit on the fly, no logits buffer), against the bf16 dense MFMA peak."""
    import torch

    from sisa_amd.workloads import config_inputs
    from sisa_amd.kernels import linear_ce as LC

    dev = torch.device("cuda:0")
    c = config_inputs(3, device=dev)
    x, w, lab = c["hidden"], c["weight"], c["labels"]
    N, D = x.shape
    V = w.shape[0]
    wp = LC.padded_weight(w, torch.bfloat16)
    Vp = wp.shape[0]
    rows = LC.chunk_rows(N, Vp, None, 2)
    loss_rows = torch.empty(N, device=dev)
    dx = torch.empty((N, D), device=dev)
    dw = torch.empty((Vp, D), device=dev)
    inv_n = torch.reciprocal((lab != -100).sum().to(torch.float32)).reshape(1)
    ws = LC.train_workspace({min(rows, N), N - (N - 1) // rows * rows}, Vp, D, dev)

    def train(want_grads=True):
        for s0 in range(0, N, rows):
            s1 = min(N, s0 + rows)
            LC.lmce_train_chunk(x[s0:s1], wp, lab[s0:s1], V, -100, inv_n, 1.0, loss_rows[s0:s1],
                                dx[s0:s1] if want_grads else None, dw if want_grads else None, s0 > 0, ws)

    for _ in range(warmup):
        train()
    train_s = queued_seconds(train, reps=steps)
    fwd_s = queued_seconds(lambda: train(False), reps=steps)
    fl = LC.flops(N, V, D)
    ms = train_s * 1e3

    # the reference's arrangement (library GEMMs around the HIP row pass), kept only as the comparison
    lrows = LC.chunk_rows(N, Vp, None, 2, budget=1 << 30)
    buf = torch.empty((lrows, Vp), dtype=torch.bfloat16, device=dev)

    def library_loop():
        for s0 in range(0, N, lrows):
            lg = buf[:min(N, s0 + lrows) - s0]
            xc = x[s0:s0 + lg.shape[0]]
            torch.mm(xc, wp.t(), out=lg)
            LC.lmce_rows(lg, lab[s0:s0 + lg.shape[0]], loss_rows[s0:s0 + lg.shape[0]], V, -100, inv_n, 1.0)
            torch.mm(lg, wp, out_dtype=torch.float32, out=dx[s0:s0 + lg.shape[0]])
            if s0 == 0:
                torch.mm(lg.t(), xc, out_dtype=torch.float32, out=dw)
            else:
                torch.addmm(dw, lg.t(), xc, out_dtype=torch.float32, out=dw)

    lib_s = queued_seconds(library_loop, reps=max(3, steps // 2))
    del buf

    def fused():
        LC.lmce_fused_loss_rows(x, wp, lab, V, -100)

    fused_s = queued_seconds(fused, reps=10)
    fwd_tf = fl["forward"] / fused_s / 1e12
    tr_tf = fl["total"] / train_s / 1e12
    return {"workload": "linear cross-entropy (config 3): N=16384, d=768, V=50277, bf16", "N": N, "d": D, "V": V,
            "Vp": Vp,
            "train": {"what": "loss, dx, dW: sisa_lmce_train (MFMA logits GEMM storing exponentials; one launch of "
                              "dW and dx MFMA tiles forming G in operand staging; no library GEMM)",
                      "chunk_rows": rows, "ms_per_step": round(ms, 4), "tflops": round(tr_tf, 2),
                      "tokens_per_s": round(N / train_s, 1),
                      "phases_ms": {"forward": round(fwd_s * 1e3, 4), "gradients": round((train_s - fwd_s) * 1e3, 4)},
                      "roofline": {"bound": "mfma", "achieved": round(tr_tf, 1), "peak": PEAK_BF16_TFLOPS,
                                   "unit": "TFLOP/s", "frac": round(tr_tf / PEAK_BF16_TFLOPS, 4),
                                   "algorithmic": "3 GEMMs x 2*N*V*d flop over the whole call"},
                      "library_chunk_loop_ms": round(lib_s * 1e3, 4),
                      "speedup_vs_library_loop": round(lib_s / train_s, 3)},
            "fused_forward": {"what": "loss without gradients, sisa_lmce_fwd (no logits buffer)",
                              "ms": round(fused_s * 1e3, 4), "tokens_per_s": round(N / fused_s, 1),
                              "roofline": {"bound": "mfma", "achieved": round(fwd_tf, 1), "peak": PEAK_BF16_TFLOPS,
                                           "unit": "TFLOP/s", "frac": round(fwd_tf / PEAK_BF16_TFLOPS, 4),
                                           "algorithmic": "2*N*V*d flop"}}}


def bench_fused_layer(proj, z, lam, dy, H, steps: int, mode: str, flop: float) -> dict:
    """sisa_fused forward + backward through autograd as a user calls it (eager launches, fresh outputs each call),
    in check mode ``mode`` (the default "async": the non-finite guard and its device assert included) and in "off"."""
    import torch

    from sisa_amd import backends
    from sisa_amd.kernels.fused_prep import sisa_fused

    P, Z, LM = (t.detach().clone().requires_grad_(True) for t in (proj, z, lam))

    def call():
        y = sisa_fused(P, Z, LM, H)
        torch.autograd.grad(y, (P, Z, LM), dy)

    res = {}
    for m in (mode, "off"):
        backends.set_check_mode(m)
        for _ in range(3):
            call()
        torch.cuda.synchronize()
        with _quiet_host():
            t0 = time.perf_counter()
            for _ in range(steps):
                call()
            torch.cuda.synchronize()
            res[m] = (time.perf_counter() - t0) * 1e3 / steps
    backends.set_check_mode(mode)
    return {"what": "sisa_fused forward + backward (autograd, eager launches)", "check_mode": mode,
            "ms_per_step": round(res[mode], 4), "tflops": round(flop / (res[mode] * 1e-3) / 1e12, 2),
            "ms_per_step_check_off": round(res["off"], 4)}


def bench_model(steps: int, warmup: int, brief: bool = False) -> dict:
    """Full decoder training step at config 4: sisa-152m (12 layers, d=768, H=12, d_head=64, d_state=32, SwiGLU,
    tied embedding, vocabulary 50277, README init), B=8 x T=2048 uniform random token ids, bf16 autocast; one step =
    forward with the fused HIP attention path and the chunked HIP linear cross-entropy, backward, AdamW update."""
    import torch

    from sisa_amd import SISAConfig, SISAForCausalLM

    from sisa_amd.gemm_tuning import enable_tuned_gemms

    dev = torch.device("cuda:0")
    tuned = enable_tuned_gemms()
    torch.manual_seed(4)
    cfg = SISAConfig.preset("sisa-152m", attn_impl="hip_fused")
    model = SISAForCausalLM(cfg).to(dev)
    opt = torch.optim.AdamW(model.param_groups(3e-4, weight_decay=0.1), betas=(0.9, 0.95), fused=True)
    B, T = 8, 2048
    ids = torch.randint(0, cfg.vocab_size, (B, T), generator=torch.Generator().manual_seed(4)).to(dev)

    def step():
        opt.zero_grad(set_to_none=True)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            loss = model(ids, labels=ids, fused_ce=True).loss
        loss.backward()
        opt.step()
        return loss

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    with _quiet_host():
        t0 = time.perf_counter()
        for _ in range(steps):
            loss = step()
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / steps
    if brief:
        return {"ms_per_step": round(ms, 3), "tokens_per_s": round(B * T / (ms * 1e-3), 1)}
    from sisa_amd import backends

    return {"workload": "full decoder training step (config 4): sisa-152m, B=8, T=2048, bf16 autocast, hip_fused "
                        "attention + HIP RMSNorm/SwiGLU + fused linear CE + AdamW", "B": B, "T": T,
            "check_mode": backends.get_check_mode(),
            "params": model.num_parameters(), "steps": steps, "ms_per_step": round(ms, 3),
            "tokens_per_s": round(B * T / (ms * 1e-3), 1), "loss": round(float(loss.detach()), 4), "tuned_gemms": tuned}


def bench_block_kernels(reps: int = 20) -> dict:
    """The decoder-block and decode kernels at config-4 shapes, each against the HBM roofline: RMSNorm forward and
    backward on the fp32 residual stream (16384 x 768) with the normalised rows in bf16 (the FFN norm), the same
    with the fused 12-head forget projection (the attention norm; backward: row pass, dw reduction, dW_f), the SwiGLU
    activation forward and backward (16384 x 2744 bf16), and one decode step (chunk + combine launches) of 8
    sequences x 12 heads against a 16,384-position bf16 cache. Each entry point is called through the C-ABI with
    prepared arguments, reps times back to back behind a GPU spin so that host overhead is not timed; HIP events on
    the launch stream. Algorithmic bytes: RMSNorm forward x read + y written (+ rstd), backward x, dy read + dx written
    (+ rstd, dw); SwiGLU forward a, b read + h written, backward a, b, dh read + da, db written; decode the k, v, b~
    rows and g, F of every cached position and head."""
    import ctypes

    import torch
    import torch.nn.functional as F

    from sisa_amd.kernels import _lib

    dev = torch.device("cuda:0")
    gen = torch.Generator().manual_seed(5)
    lib = _lib.load()

    def timed(name, args, anchor):
        fn, ref, st = getattr(lib, name), ctypes.byref(args), _lib.stream_of(anchor)
        if fn(ref, st) != 0:
            raise RuntimeError(f"{name}: {lib.sisa_last_error().decode()}")
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with _quiet_host():
            torch.cuda._sleep(20_000_000)      # the GPU spins while the host queues the timed launches
            e0.record()
            rcs = [fn(ref, st) for _ in range(reps)]
            e1.record()
            torch.cuda.synchronize()
        if any(rcs):
            raise RuntimeError(f"{name}: {lib.sisa_last_error().decode()}")
        return e0.elapsed_time(e1) / reps * 1e-3

    def line(nbytes, sec, **extra):
        gbs = nbytes / sec / 1e9
        return dict({"us": round(sec * 1e6, 2), "bytes": int(nbytes), "achieved": round(gbs, 1),
                     "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4)}, **extra)

    N, D, FF, HF = 16384, 768, 2744, 12
    x = torch.randn(N, D, generator=gen).to(dev)
    w = (1 + 0.1 * torch.randn(D, generator=gen)).to(dev)
    wf = (0.05 * torch.randn(HF, D, generator=gen)).to(dev)
    bfz = torch.randn(HF, generator=gen).to(dev)
    dy = torch.randn(N, D, generator=gen).to(torch.bfloat16).to(dev)
    dz = torch.randn(N, HF, generator=gen).to(dev)
    y, dx = torch.empty(N, D, device=dev, dtype=torch.bfloat16), torch.empty_like(x)
    rstd, z, dw = torch.empty(N, device=dev), torch.empty(N, HF, device=dev), torch.empty(D, device=dev)
    dwf, dbf = torch.empty(HF, D, device=dev), torch.empty(HF, device=dev)
    ws = torch.empty(_lib.workspace_bytes("sisa_norm_bwd_workspace_bytes", N, D, HF) // 4, device=dev)
    f32, bf = _lib.dtype_code(torch.float32), _lib.dtype_code(torch.bfloat16)

    def norm_args(H):
        return _lib.NormArgs(N, D, H, f32, bf, 1e-6, 0, x.data_ptr(), D, w.data_ptr(), wf.data_ptr(), bfz.data_ptr(),
                             y.data_ptr(), D, rstd.data_ptr(), z.data_ptr(), dy.data_ptr(), D, dz.data_ptr(),
                             dx.data_ptr(), D, dw.data_ptr(), dwf.data_ptr(), dbf.data_ptr(), ws.data_ptr())
    # forward: x (fp32) read, y (bf16) and rstd written, + z; backward: x, dy (bf16), rstd read, dx (fp32) written,
    # + dz read
    fwd_bytes, bwd_bytes = N * D * (4 + 2) + N * 4, N * D * (4 + 2 + 4) + N * 4 + 2 * D * 4
    t_rms_f = timed("sisa_norm_fwd", norm_args(0), x)
    t_rms_b = timed("sisa_norm_bwd", norm_args(0), x)
    t_nf_f = timed("sisa_norm_fwd", norm_args(HF), x)
    t_nf_b = timed("sisa_norm_bwd", norm_args(HF), x)
    a, b, dh = (torch.randn(N, FF, generator=gen).to(torch.bfloat16).to(dev) for _ in range(3))
    h, da, db = torch.empty_like(a), torch.empty_like(a), torch.empty_like(a)
    sf = _lib.SwigluArgs(N * FF, bf, 0, a.data_ptr(), b.data_ptr(), h.data_ptr(), None, None, None)
    sb = _lib.SwigluArgs(N * FF, bf, 0, a.data_ptr(), b.data_ptr(), None, dh.data_ptr(), da.data_ptr(), db.data_ptr())
    t_sw_f = timed("sisa_swiglu_fwd", sf, a)
    t_sw_b = timed("sisa_swiglu_bwd", sb, a)
    del a, b, dh, h, da, db
    Bd, H, T = 8, 12, 16384
    k, v = (torch.randn(Bd, H, T, 64, generator=gen).to(torch.bfloat16).to(dev) for _ in range(2))
    bb = torch.randn(Bd, H, T, 32, generator=gen).to(torch.bfloat16).to(dev)
    q = torch.randn(Bd, H, 1, 64, generator=gen).to(torch.bfloat16).to(dev)
    c = torch.randn(Bd, H, 1, 32, generator=gen).to(torch.bfloat16).to(dev)
    g = torch.cumsum(-F.softplus(torch.randn(Bd, H, T, generator=gen) - 5), -1).to(dev)
    f = torch.cumsum(F.logsigmoid(torch.randn(Bd, H, T, generator=gen) + 4), -1).to(dev)
    gq, fq = g[..., -1:].contiguous(), f[..., -1:].contiguous()
    lam = torch.full((H,), 0.31, device=dev)
    out = torch.empty(Bd, H, 1, 64, device=dev)
    dws = torch.empty(_lib.workspace_bytes("sisa_decode_workspace_bytes", Bd, H, 1, T) // 4, device=dev)
    da_ = _lib.DecodeArgs(Bd, H, 1, T, bf, T - 1, _lib.view(q), _lib.view(k), _lib.view(v), _lib.view(c),
                          _lib.view(bb), _lib.view(gq), _lib.view(g), _lib.view(fq), _lib.view(f), lam.data_ptr(), 1,
                          out.data_ptr(), dws.data_ptr())
    t_dec = timed("sisa_decode_attn", da_, q)
    return {"workload": "decoder-block and decode kernels at config-4 shapes (C-ABI calls, host overhead excluded)",
            "rmsnorm_fwd": line(fwd_bytes, t_rms_f),
            "rmsnorm_bwd": line(bwd_bytes, t_rms_b),
            "norm_forget_fwd": line(fwd_bytes + N * HF * 4, t_nf_f),
            "norm_forget_bwd": line(bwd_bytes + N * HF * 4 + 2 * HF * D * 4, t_nf_b),
            "swiglu_fwd": line(3 * N * FF * 2, t_sw_f),
            "swiglu_bwd": line(5 * N * FF * 2, t_sw_b),
            "decode_step": line(Bd * H * T * (160 * 2 + 8), t_dec, cache_positions=T, sequences=Bd, heads=H)}


def bench_projection_gemms(reps: int = 20) -> dict:
    """The projection GEMMs of the config-4 training step around the hot path (per layer: the W_cat projection with
    its bias, W_O, the interleaved gate/up projection and the down projection; forward, input-gradient and
    weight-gradient products; N = 16,384 rows) as the HIP block path runs them: forward and input gradient on the
    library GEMMs (bf16, the shipped TunableOp table), weight gradients of W_cat, W_O and down on the HIP kernel
    sisa_wgrad (fp32 output), that of gate/up on the library. Each against the dense bf16 MFMA peak: 2 M N K flop
    per call, HIP events over reps back-to-back calls."""
    import torch
    import torch.nn.functional as F

    from sisa_amd.kernels.wgrad import wgrad_hip

    dev = torch.device("cuda:0")
    gen = torch.Generator().manual_seed(6)
    M = 16384
    out = {"workload": "projection GEMMs of one sisa-152m layer at B*T = 16384 rows (bf16; library GEMMs with the "
                       "TunableOp table, HIP weight-gradient kernel for W_cat, W_O, down)"}
    total_ms, total_flop = 0.0, 0.0
    for name, n, k, bias in (("W_cat", 3280, 768, True), ("W_O", 768, 768, False), ("gate_up", 5488, 768, False),
                             ("down", 768, 2744, False)):
        x = torch.randn(M, k, generator=gen).to(torch.bfloat16).to(dev)
        w = (0.02 * torch.randn(n, k, generator=gen)).to(torch.bfloat16).to(dev)
        b = torch.zeros(n, dtype=torch.bfloat16, device=dev) if bias else None
        dy = torch.randn(M, n, generator=gen).to(torch.bfloat16).to(dev)
        fl = 2.0 * M * n * k
        row = {}
        dw_fn = (lambda: dy.t() @ x) if name == "gate_up" else (lambda: wgrad_hip(dy, x))
        for kind, fn in (("fwd", lambda: F.linear(x, w, b)), ("dx", lambda: dy @ w), ("dw", dw_fn)):
            fn()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            with _quiet_host():
                torch.cuda._sleep(20_000_000)
                e0.record()
                for _ in range(reps):
                    fn()
                e1.record()
                torch.cuda.synchronize()
            ms = e0.elapsed_time(e1) / reps
            tf = fl / (ms * 1e-3) / 1e12
            row[kind] = {"us": round(ms * 1e3, 1), "tflops": round(tf, 1), "frac": round(tf / PEAK_BF16_TFLOPS, 4)}
            total_ms += ms
            total_flop += fl
        out[name] = row
        del x, w, dy
    tf = total_flop / (total_ms * 1e-3) / 1e12
    out["layer_total"] = {"us": round(total_ms * 1e3, 1), "tflops": round(tf, 1), "frac": round(tf / PEAK_BF16_TFLOPS, 4),
                          "bound": "mfma", "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s"}
    return out


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
                      f"fwd+bwd, median of {reps} runs after 1 warm-up: {t * 1e3:.0f} ms = {B * L / t:.0f} tokens/s",
            "config0": cpu_config0(reps)}


def gpu_config0(reps: int = 20) -> dict:
    """BASELINE.json config 0 (B=1, T=256, H=4, fp32, fwd+bwd with the glue) on the GPU through the product path:
    the glue in torch (sisa_amd.functional.rotate_pairs, cumsums) and sisa_attention(impl="hip") in fp32. Median of
    ``reps`` HIP-event timed steps; each step is a handful of small launches, so this is a latency figure."""
    import torch
    import torch.nn.functional as F

    from sisa_amd.functional import rotate_pairs, sisa_attention
    dev = torch.device("cuda:0")
    B, H, L = 1, 4, 256
    gen = torch.Generator().manual_seed(0)
    leaves = dict(q=torch.randn(B, H, L, 64, generator=gen), k=torch.randn(B, H, L, 64, generator=gen),
                  v=torch.randn(B, H, L, 64, generator=gen), b=torch.randn(B, H, L, 32, generator=gen),
                  c=torch.randn(B, H, L, 32, generator=gen), theta=0.01 * torch.randn(B, L, H, 16, generator=gen),
                  a=-5 + 0.5 * torch.randn(B, L, H, generator=gen), z=4 + 0.5 * torch.randn(B, L, H, generator=gen),
                  lam_raw=torch.full((H,), -1.0))
    leaves = {n: t.to(dev).requires_grad_(True) for n, t in leaves.items()}
    dy = torch.randn(B, H, L, 64, generator=gen).to(dev)

    def step():
        phi = torch.cumsum(leaves["theta"], 1).transpose(1, 2)
        g = torch.cumsum(-F.softplus(leaves["a"]), 1).transpose(1, 2).contiguous()
        fg = torch.cumsum(F.logsigmoid(leaves["z"]), 1).transpose(1, 2).contiguous()
        o = sisa_attention(leaves["q"], leaves["k"], leaves["v"], rotate_pairs(leaves["c"], phi),
                           rotate_pairs(leaves["b"], phi), g, F.softplus(leaves["lam_raw"]), fg, impl="hip")
        torch.autograd.grad(o, list(leaves.values()), dy)
    for _ in range(3):
        step()
    torch.cuda.synchronize()
    times = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        step()
        e1.record()
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1))
    t = statistics.median(times) * 1e-3
    return {"ms": round(t * 1e3, 3), "tokens_per_s": round(B * L / t, 1),
            "shape": "B=1, T=256, H=4, d_h=64, d_s=32, fp32, fwd+bwd (glue in torch, attention on the HIP kernels)"}


def cpu_config0(reps: int) -> dict:
    """BASELINE.json config 0 as the reference defines it, on the host cores: one SISA attention op fwd+bwd in fp32 at
    B=1, T=256, H=4, d_h=64, d_s=32 (glue from theta, decay and forget logits included; upstream grad N(0,1)), with
    the oracle's restatement of the reference's pure-PyTorch path."""
    import torch

    from oracle import reference as R
    B, H, L = 1, 4, 256
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
    for _ in range(max(reps, 5)):
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    return {"ms": round(t * 1e3, 3), "tokens_per_s": round(B * L / t, 1),
            "tflops": round(1152 * B * H * L * L / 2 / t / 1e12, 6), "cores": torch.get_num_threads(),
            "shape": "B=1, T=256, H=4, d_h=64, d_s=32, fp32, fwd+bwd (glue included)"}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)
    import torch

    from sisa_amd.workloads import config_inputs
    from sisa_amd import backends
    from sisa_amd.kernels import attention as A
    from sisa_amd.kernels import fused_prep as FP

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    from sisa_amd.gemm_tuning import enable_tuned_gemms

    enable_tuned_gemms()          # library GEMM choices for the CE and model legs (the attention leg has none)
    default_mode = backends.get_check_mode()
    backends.set_check_mode("off")    # headline: the path's kernels (the guard is an input check; timed separately)
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
        pf = FP.prep_forward(proj, z, H)
        if record:
            e[1].record()
        q, k, v = col(proj, "Q"), col(proj, "K"), col(proj, "V")
        c, b = pf.state_views()
        o, lse, _, _, o32 = A.attn_forward(q, k, v, c, b, pf.g, lam, pf.f, factors=(pf.rowf, pf.colf), want32=True)
        if record:
            e[2].record()
        DP = torch.empty_like(proj)
        DCR = torch.empty((B, L, H, S), device=dev, dtype=torch.float32)
        DBR = torch.empty_like(DCR)
        do = dy.reshape(B, L, H, D).transpose(1, 2)
        _, _, _, _, _, dg, dlam, dF = A.attn_backward(q, k, v, c, b, pf.g, pf.f, pf.rowf, pf.colf, lam, o,
                                                      lse, do, True, dq=col(DP, "Q"), dk=col(DP, "K"), dv=col(DP, "V"),
                                                      dc=DCR.transpose(1, 2), db=DBR.transpose(1, 2), o32=o32)
        if record:
            e[3].record()
        FP.prep_backward(proj, z, pf.totals, dg, dF, DCR, DBR, DP, H)
        if record:
            e[4].record()
            for i, k_ in enumerate(marks):
                marks[k_].append((e[i], e[i + 1]))

    if args.copy_mib > 0:
        src = torch.ones(args.copy_mib << 18, device=dev)       # MiB of fp32
        torch.empty_like(src).copy_(src)
        torch.cuda.synchronize()
        del src
    for _ in range(args.warmup):
        step(False)
    torch.cuda.synchronize()
    # eager steps: the per-phase HIP-event breakdown (host work between launches included)
    with _quiet_host():
        t0 = time.perf_counter()
        for _ in range(args.steps):
            step(True)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
    ms_eager = (t1 - t0) * 1e3 / args.steps
    phases = {k: statistics.mean(a.elapsed_time(b_) for a, b_ in v) for k, v in marks.items()}
    ms_step, timing = ms_eager, "eager launches"
    if not args.eager:
        # the headline: the same step's launches (prep forward, attention forward, attention backward, prep
        # backward; allocations from the graph's pool) captured once into a HIP graph and replayed, so that no host
        # work sits between the launches; every kernel runs in every replay. Should capture fail, the eager time
        # stands (and the reason is reported).
        try:
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                step(False)
            torch.cuda.current_stream().wait_stream(side)
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                step(False)
            for _ in range(args.warmup):
                graph.replay()
            torch.cuda.synchronize()
            with _quiet_host():
                t0 = time.perf_counter()
                for _ in range(args.steps):
                    graph.replay()
                torch.cuda.synchronize()
                t1 = time.perf_counter()
            ms_step, timing = (t1 - t0) * 1e3 / args.steps, "replays of a HIP graph of one step"
        except RuntimeError as exc:          # capture refused by the runtime: keep the eager figure
            torch.cuda.synchronize()
            timing = f"eager launches (graph capture failed: {str(exc)[:120]})"

    fl = A.flops(B, H, L)
    total_flop = fl["total"]
    value = total_flop / (ms_step * 1e-3) / 1e12
    attn_ms = phases["attn_fwd"] + phases["attn_bwd"]
    achieved = total_flop / (attn_ms * 1e-3) / 1e12
    pb = FP.prep_bytes(B, L, H)
    prk = prep_kernel_rates(proj, z, H)
    prep_gbs = prk["prep_fwd"]["achieved"]
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
        "timing": timing,
        "eager_ms_per_step": round(ms_eager, 4),
        "algorithmic_peak_pct": round(100 * value / PEAK_BF16_TFLOPS, 2),
        "mfma_busy_pct": profiled_mfma_busy(),
        "phases_ms": {k: round(v, 4) for k, v in phases.items()},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 3), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                     "traffic": profiled_traffic(ATTN_KERNELS) if cfg == "ns" else None,
                     "traffic_source": "profiles/hbm_traffic_ns_ce.txt (rocprofv3 FETCH_SIZE / WRITE_SIZE passes of this "
                                       "build, not measured in this run)" if cfg == "ns" else None,
                     "kernel": "attention fwd + bwd launches (attn_fwd, attn_bwd_dq, attn_bwd_dkv)",
                     "algorithmic": f"1152 flop per causal pair x {fl['pairs']:.4g} pairs per step"},
        "roofline_prep": {"bound": "hbm", "achieved": round(prep_gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                          "frac": round(prep_gbs / PEAK_HBM_GBS, 4),
                          "traffic": profiled_traffic(PREP_FWD_KERNELS) if cfg == "ns" else None,
                          "algorithmic": f"{pb['total'] / 1e6:.1f} MB per prep forward (310 B per token-head)",
                          "kernels": "prep_sums + prep_fwd, queued behind a GPU spin (HIP events)",
                          "copy_same_bytes_gbs": prk["prep_fwd"]["copy_same_bytes_gbs"],
                          "frac_of_copy": prk["prep_fwd"]["frac_of_copy"],
                          "backward": prk["prep_bwd"]},
    }
    out["fused_layer_async"] = bench_fused_layer(proj, z, lam, dy, H, args.steps, default_mode, total_flop)
    backends.set_check_mode(default_mode)
    if not args.no_ce:
        out["lmce"] = bench_ce(max(3, args.steps // 2), 2)
    if not args.no_model:
        out["model_step"] = bench_model(max(3, args.steps // 4), 2)
        backends.set_check_mode("off")
        out["model_step"]["check_mode_off"] = bench_model(max(3, args.steps // 4), 2, brief=True)
        backends.set_check_mode(default_mode)
        out["block_kernels"] = bench_block_kernels()
        out["projection_gemms"] = bench_projection_gemms()
    out["config0_gpu"] = gpu_config0()
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(args.cpu_reps)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
