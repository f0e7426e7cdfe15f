"""The BASELINE configurations at their full sizes on the HIP path, against fp64.

config 1  sisa_fused forward + backward at B=4, T=2048, H=8 (prep + attention): finite, deterministic, and every
          output / gradient column group within 2e-2 (norm-wise) of the fp64 layer (oracle.fused64) evaluated one
          batch row at a time on the GPU (rows are independent; dlambda is their sum).
north star / config 2  sisa_fused forward + backward at B=4, T=4096, H=8 and at B=1, T=16384, H=16 (a ~ N(-7, 1)):
          finite, repeatable, and a subset of heads (independent of each other) within 2e-2 of the one-head fp64 layer.
config 3  linear cross-entropy forward + backward at N=16384, d=768, V=50277 under bf16 autocast, default chunking,
          a forced multi-chunk run and the grad_scale promise: loss, dL/dh and dL/dW against fp64 on the fp32 master
          inputs and on bf16-rounded inputs (oracle.lmce64), within 2 x the eager autocast formula's error + 1e-7.
config 4  one sisa-152m training step (B=8, T=2048, bf16 autocast, README init) through the fused HIP block path
          with the chunked CE, the unfused HIP path and the torch path: the loss at init within 0.05 of
          ln(50277) + d_model 0.02^2 / 2 (near-Gaussian logits of variance d_model 0.02^2),
          a repeat bitwise identical, and the reference's integration gates against the fp64 model
          (tests/test_model_cuda.py:1-8, 67-85 of tlstngud/sisa): |loss - loss64| <= max(2 d_torch, 2e-3) and per
          parameter group e <= 3 e_torch + 2e-3.
"""
from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import reference as R

pytestmark = pytest.mark.gpu
DEV = "cuda"


# ------------------------------------------------------------------------------------------------ config 1
def test_config1_fused_layer():
    from sisa_amd.kernels.fused_prep import prep_forward, sisa_fused
    from sisa_amd.workloads import config_inputs

    inp = config_inputs(1, device=DEV)
    proj, z, dy, H = inp["proj"], inp["z"], inp["dy"], inp["H"]
    lam = F.softplus(inp["lam_raw"]).float()
    B, L, _ = proj.shape
    print(f"[config1] B={B} L={L} H={H}", flush=True)
    off = R.layout(H)

    def run():
        P, Z, LM = (t.detach().clone().requires_grad_(True) for t in (proj, z, lam))
        y = sisa_fused(P, Z, LM, H)
        gP, gL, gZ = torch.autograd.grad(y, (P, LM, Z), dy)
        torch.cuda.synchronize()
        return y.detach(), gP, gL, gZ

    first, second = run(), run()
    assert all(torch.equal(a, b) for a, b in zip(first, second)), "two calls differ"
    y, dP, dl, dz = first
    assert all(bool(torch.isfinite(t).all()) for t in first)
    assert bool((dP[..., off["NTOT"]:] == 0).all()), "pad columns of d proj must be zero"
    pf = prep_forward(proj, z, H)
    glue = R.glue(proj, z, H, dtype=torch.float32)
    dl64 = torch.zeros(H, dtype=torch.float64, device=DEV)
    errs: dict[str, float] = {}
    for r in range(B):
        vals = dict(q=glue["q"][r:r + 1], k=glue["k"][r:r + 1], c=pf.cr[r:r + 1].transpose(1, 2),
                    b=pf.br[r:r + 1].transpose(1, 2), g=pf.g[r:r + 1], F=pf.f[r:r + 1])
        y64, dP64, dlr, dz64 = R.fused64(proj[r:r + 1], z[r:r + 1], lam, H, vals, dy[r:r + 1])
        dl64 += dlr.double()
        row = dict(y=R.rel(y[r:r + 1], y64), dz=R.rel(dz[r:r + 1], dz64))
        for grp, w in (("Q", 64), ("K", 64), ("V", 64), ("B", 32), ("C", 32), ("TH", 16), ("A", 1)):
            sl = slice(off[grp], off[grp] + H * w)
            row["d" + grp] = R.rel(dP[r:r + 1, :, sl], dP64[..., sl])
        for k_, v_ in row.items():
            errs[k_] = max(errs.get(k_, 0.0), v_)
        del y64, dP64, dz64
    errs["dlam"] = R.rel(dl, dl64)
    print(f"[config1] worst rel err per tensor: { {k: f'{v:.2e}' for k, v in errs.items()} }", flush=True)
    bad = {k: v for k, v in errs.items() if not v <= 2e-2}
    assert not bad, f"config 1 parity: {bad}"


# ------------------------------------------------------------------------------------------------ north star, config 2
GROUPS = (("Q", 64), ("K", 64), ("V", 64), ("B", 32), ("C", 32), ("TH", 16), ("A", 1))


def _head_columns(proj: torch.Tensor, H: int, h: int) -> torch.Tensor:
    """Head h's columns of an H-head fused projection, laid out as a one-head projection (zero padding)."""
    off, one = R.layout(H), R.layout(1)
    sub = proj.new_zeros(*proj.shape[:2], one["NPAD"])
    for key, w in GROUPS:
        sub[..., one[key]:one[key] + w] = proj[..., off[key] + h * w:off[key] + (h + 1) * w]
    return sub


@pytest.mark.parametrize("cfg,heads", [("ns", (0, 5, 7)), (2, (0, 9, 15))])
def test_fused_layer_head_subset(cfg, heads):
    """sisa_fused (prep forward, attention forward + backward, prep backward) at the north-star shape (B=4, T=4096,
    H=8) and at config 2 (B=1, T=16384, H=16, a ~ N(-7, 1), z ~ N(4, 1); 256 prep chunks). All heads run together
    and must be finite, repeatable and zero in the padding columns of d proj. Heads are independent, so a subset is
    each judged against fused64 on its own columns (a one-head problem; the fp64 (T x T) blocks of every head at once
    would not fit): y, every d proj column group, dz and dlambda within 2e-2 norm-wise. dtheta, the reverse scan of
    dPhi, is the long-sequence probe: each (query, key) pair adds its rotation term at the query and subtracts it at
    the key, and only when the dc and db operands round the same value do the two cancel."""
    from sisa_amd.kernels.fused_prep import prep_forward, sisa_fused
    from sisa_amd.workloads import config_inputs

    inp = config_inputs(cfg, device=DEV)
    proj, z, dy, H = inp["proj"], inp["z"], inp["dy"], inp["H"]
    lam = F.softplus(inp["lam_raw"]).float()
    B, L, _ = proj.shape
    off, one = R.layout(H), R.layout(1)
    print(f"[fused heads] cfg={cfg} B={B} L={L} H={H}", flush=True)

    def run():
        P, Z, LM = (t.detach().clone().requires_grad_(True) for t in (proj, z, lam))
        y = sisa_fused(P, Z, LM, H)
        gP, gL, gZ = torch.autograd.grad(y, (P, LM, Z), dy)
        torch.cuda.synchronize()
        return y.detach(), gP, gL, gZ

    first, second = run(), run()
    assert all(torch.equal(a, b) for a, b in zip(first, second)), "two calls differ"
    assert all(bool(torch.isfinite(t).all()) for t in first)
    y, dP, dl, dz = first
    assert not bool(dP[..., off["NTOT"]:].any()), "pad columns of d proj must be zero"
    pf = prep_forward(proj, z, H)
    c_all, b_all = pf.state_views()
    for h in heads:
        sub, zs = _head_columns(proj, H, h), z[..., h:h + 1].contiguous()
        qk = R.glue(sub, zs, 1, dtype=torch.float32)
        vals = dict(q=qk["q"], k=qk["k"], c=c_all[:, h:h + 1], b=b_all[:, h:h + 1], g=pf.g[:, h:h + 1],
                    F=pf.f[:, h:h + 1])
        y64, dP64, dl64, dz64 = R.fused64(sub, zs, lam[h:h + 1], 1, vals, dy[..., 64 * h:64 * (h + 1)])
        errs = {"y": R.rel(y[..., 64 * h:64 * (h + 1)], y64), "dz": R.rel(dz[..., h:h + 1], dz64),
                "dlam": R.rel(dl[h:h + 1], dl64)}
        for key, w in GROUPS:
            errs["d" + key] = R.rel(dP[..., off[key] + h * w:off[key] + (h + 1) * w], dP64[..., one[key]:one[key] + w])
        print(f"[fused heads] cfg={cfg} head {h}: { {k: f'{v:.2e}' for k, v in errs.items()} }", flush=True)
        bad = {k: v for k, v in errs.items() if not v <= 2e-2}
        assert not bad, f"cfg {cfg} head {h}: {bad}"
        del y64, dP64, dz64
        torch.cuda.empty_cache()


# ------------------------------------------------------------------------------------------------ config 3
def _ce_run(h, w, labels, seed_g, **kw):
    from sisa_amd.kernels.linear_ce import linear_cross_entropy

    hh = h.detach().clone().requires_grad_(True)
    ww = w.detach().clone().requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        loss = linear_cross_entropy(hh, ww, labels, **kw)
    (loss * seed_g).backward()
    torch.cuda.synchronize()
    return loss.detach().double(), hh.grad, ww.grad


def _ce_eager(h, w, labels, seed_g):
    hh = h.detach().clone().requires_grad_(True)
    ww = w.detach().clone().requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        loss = F.cross_entropy(F.linear(hh, ww).float(), labels)
    (loss * seed_g).backward()
    torch.cuda.synchronize()
    return loss.detach().double(), hh.grad, ww.grad


@pytest.mark.parametrize("variant", ["default", "chunks4096", "grad_scale"])
def test_config3_linear_ce_gradients(variant):
    from sisa_amd.workloads import config_inputs

    c = config_inputs(3, device=DEV, dtype=torch.float32)
    h, w, labels = c["hidden"], c["weight"], c["labels"].clone()
    labels[::97] = -100
    seed_g = 0.75
    print(f"[config3] N={h.shape[0]} d={h.shape[1]} V={w.shape[0]} variant={variant}", flush=True)
    kw = {"default": {}, "chunks4096": {"chunk_tokens": 4096}, "grad_scale": {"grad_scale": seed_g}}[variant]
    got = _ce_run(h, w, labels, seed_g, **kw)
    eager = _ce_eager(h, w, labels, seed_g)
    assert all(bool(torch.isfinite(t).all()) for t in got)
    assert bool((got[1][::97] == 0).all()), "ignored rows must get an exactly zero dL/dh"
    fails = []
    for quant in (False, True):
        ref = R.lmce64(h, w, labels, g=seed_g, quant=quant, chunk=2048)
        for i, name in enumerate(("loss", "dh", "dW")):
            e_got, e_eager = R.rel(got[i], ref[i]), R.rel(eager[i], ref[i])
            print(f"[config3] {variant} quant={quant} {name}: {e_got:.3e} (eager {e_eager:.3e})", flush=True)
            if not e_got <= 2.0 * e_eager + 1e-7:
                fails.append(f"{name} (quant={quant}): {e_got:.3e} > 2 x eager {e_eager:.3e} + 1e-7")
        del ref
    assert not fails, "; ".join(fails)


# ------------------------------------------------------------------------------------------------ config 4
_GROUPS = {"qkvo": ("W_Q", "W_K", "W_V", "W_O"), "bc": ("W_B", "W_C"), "alpha": ("alpha_proj",),
           "theta": ("theta_proj",), "lambda": ("lambda_raw",), "forget": ("forget_proj",), "norms": ("norm",),
           "ffn": ("ffn.",), "embed": ("embed",)}


def _grouped(grads):
    return {grp: torch.cat([g.flatten().double() for n, g in sorted(grads.items()) if any(k in n for k in keys)])
            for grp, keys in _GROUPS.items()}


def _rel(x, ref):
    x, ref = x.double(), ref.double()
    return float((x - ref).norm() / ref.norm().clamp_min(1e-300))


def test_config4_training_step():
    from oracle import model64 as M64
    from sisa_amd import SISAConfig, SISAForCausalLM

    torch.manual_seed(4)
    cfg = SISAConfig.preset("sisa-152m", attn_impl="hip_fused")
    model = SISAForCausalLM(cfg).to(DEV)
    B, T = 8, 2048
    ids = torch.randint(0, cfg.vocab_size, (B, T), generator=torch.Generator().manual_seed(4)).to(DEV)
    print(f"[config4] sisa-152m B={B} T={T}", flush=True)

    def step(impl, fused_ce):
        model.set_attn_impl(impl)
        model.zero_grad(set_to_none=True)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            loss = model(ids, labels=ids, fused_ce=fused_ce).loss
        loss.backward()
        torch.cuda.synchronize()
        return loss.item(), {n: p.grad.detach().clone() for n, p in model.named_parameters()}

    fused = step("hip_fused", True)
    again = step("hip_fused", True)
    assert fused[0] == again[0] and all(torch.equal(fused[1][n], again[1][n]) for n in fused[1]), "not deterministic"
    # at init the final-norm rows have rms 1 and the tied embedding std 0.02, so the logits are close to
    # N(0, s^2) with s^2 = d_model * 0.02^2 and the expected loss is ln V + s^2 / 2 (10.979 here)
    expect = math.log(cfg.vocab_size) + 0.5 * cfg.d_model * cfg.init_std ** 2
    assert math.isfinite(fused[0]) and abs(fused[0] - expect) < 0.05, (fused[0], expect)
    for n, g in fused[1].items():
        assert g.dtype == torch.float32 and bool(torch.isfinite(g).all()), n
    del again
    unfused = step("hip", True)
    torch_path = step("torch", False)
    loss64, _, grads64 = M64.loss_and_grads64(model, ids, ids)
    ref_g, tor_g = _grouped(grads64), _grouped(torch_path[1])
    d_torch = abs(torch_path[0] - loss64)
    report = {"loss64": loss64, "torch": torch_path[0]}
    fails = []
    for name, (loss, grads) in (("hip_fused", fused), ("hip", unfused)):
        report[name] = loss
        if not abs(loss - loss64) <= max(2.0 * d_torch, 2e-3):
            fails.append(f"{name} loss {loss:.6f} vs fp64 {loss64:.6f} (torch {torch_path[0]:.6f})")
        got_g = _grouped(grads)
        for grp in _GROUPS:
            e, e_t = _rel(got_g[grp], ref_g[grp]), _rel(tor_g[grp], ref_g[grp])
            report[f"{name}.{grp}"] = (round(e, 5), round(e_t, 5))
            if not e <= 3.0 * e_t + 2e-3:
                fails.append(f"{name} {grp}: {e:.3e} > 3 x torch {e_t:.3e} + 2e-3")
    print(f"[config4] {report}", flush=True)
    assert not fails, "; ".join(fails)
