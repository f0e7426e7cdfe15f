"""GPU parity tests of the fused layer core: HIP prep (scans, factors, rotation) + HIP attention, forward and backward.

Follows the reference's fused-prep judge (tests/test_fused_prep.py:366-491 of tlstngud/sisa):
  prep       g, F and the rotated C/B against fp64, no worse than the unfused torch glue (g/F: 2x + 1e-7; c/b: 1.02x
             the torch bf16 path + 1e-7); g non-increasing across chunk boundaries; rowf/colf bitwise equal to the
             attention's own factor kernel on the same g.
  grads      d proj per column group, dz and dlambda against an fp64 reference with the candidate's forward values
             passed straight through: norm-wise relative error <= 2e-2 (the build's contract) and no worse than torch
             glue + HIP attention (1.05x + 1e-6; 1.5x + 1e-5 for the fp32 scalar chains dz, dlambda). Padding columns
             of d proj are exactly zero.
  props      determinism, inputs unchanged, causality.
"""
from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from oracle import reference as R

pytestmark = pytest.mark.gpu
DEV = "cuda"


def FP():
    from sisa_amd.kernels import fused_prep
    return fused_prep


def torch_glue(proj, z, H):
    """The unfused fp32 torch glue on the GPU (src/sisa/modeling.py:185-197)."""
    return R.glue(proj, z, H, dtype=torch.float32)


@pytest.mark.parametrize("B,L,H,seed,hasf,kw", [
    (2, 2048, 8, 1, True, {}), (1, 300, 12, 2, True, {}), (1, 1, 8, 3, True, {}), (1, 129, 8, 4, False, {}),
    (1, 2048, 8, 6, True, dict(alpha_mu=-8.0, alpha_sd=0.5)), (1, 1000, 16, 7, True, {}), (1, 65, 5, 8, True, {}),
    (1, 8300, 6, 9, True, {}), (1, 16384, 16, 10, True, dict(alpha_mu=-7.0, alpha_sd=1.0))])
def test_prep_accuracy(B, L, H, seed, hasf, kw):
    from sisa_amd.kernels import attention as A
    proj, z, off = R.make_proj(B, L, H, seed, device=DEV, **kw)
    z = z if hasf else None
    P = FP().prep_forward(proj, z, H)
    T = torch_glue(proj, z, H)
    X = R.glue(proj, z, H)
    bad = []
    if L > 1:
        inc = float((P.g[..., 1:] - P.g[..., :-1]).max())
        if inc > 0:
            bad.append(f"g not monotone (+{inc:.3e})")
    eg, egt = R.rel(P.g, X["g"]), R.rel(T["g"], X["g"])
    if eg > 2 * egt + 1e-7:
        bad.append(f"g error {eg:.2e} > 2x torch {egt:.2e}")
    if hasf:
        ef, eft = R.rel(P.f, X["F"]), R.rel(T["F"], X["F"])
        if ef > 2 * eft + 1e-7:
            bad.append(f"F error {ef:.2e} > 2x torch {eft:.2e}")
    for n, key in (("c", "cr"), ("b", "br")):
        e_k = R.rel(getattr(P, key).transpose(1, 2), X[n])
        e_t = R.rel(T[n].to(torch.bfloat16), X[n])
        if e_k > 1.02 * e_t + 1e-7:
            bad.append(f"{n} error {e_k:.2e} above the torch bf16 path {e_t:.2e}")
    rowf, colf, _ = A.compute_factors(P.g)
    if not (torch.equal(rowf, P.rowf) and torch.equal(colf, P.colf)):
        bad.append("rowf/colf != factor kernel on the same g")
    assert not bad, "; ".join(bad)


def run_fused(proj, z, lam, H, dy):
    Pp = proj.detach().clone().requires_grad_(True)
    Zp = None if z is None else z.detach().clone().requires_grad_(True)
    Lp = lam.detach().clone().requires_grad_(True)
    y = FP().sisa_fused(Pp, Zp, Lp, H)
    gr = torch.autograd.grad(y, [Pp, Lp] + ([Zp] if Zp is not None else []), dy)
    return y.detach(), gr[0], gr[1], (gr[2] if Zp is not None else None)


def run_glue_hip(proj, z, lam, H, dy):
    from sisa_amd.kernels.attention import sisa_attention_hip
    B, L, _ = proj.shape
    Pp = proj.detach().clone().requires_grad_(True)
    Zp = None if z is None else z.detach().clone().requires_grad_(True)
    Lp = lam.detach().clone().requires_grad_(True)
    T = R.glue(Pp, Zp, H, dtype=torch.float32)
    off = R.layout(H)

    def cols(nm):   # q, k, v stay strided bf16 views of proj (the unfused layer's W_Q x etc.)
        return Pp[..., off[nm]:off[nm] + H * 64].view(B, L, H, 64).transpose(1, 2)
    o = sisa_attention_hip(cols("Q"), cols("K"), cols("V"), T["c"].to(torch.bfloat16), T["b"].to(torch.bfloat16),
                           T["g"].contiguous(), Lp, None if T["F"] is None else T["F"].contiguous())
    y = o.transpose(1, 2).reshape(B, L, H * 64)
    gr = torch.autograd.grad(y, [Pp, Lp] + ([Zp] if Zp is not None else []), dy)
    return y.detach(), gr[0], gr[1], (gr[2] if Zp is not None else None)


@pytest.mark.parametrize("B,L,H,seed,hasf", [(1, 300, 4, 11, True), (1, 1024, 8, 12, True), (1, 129, 4, 13, False),
                                              (1, 1, 4, 14, True), (2, 700, 4, 15, True), (1, 4200, 4, 16, True)])
def test_fused_gradients_vs_fp64(B, L, H, seed, hasf):
    print(f"[fused] B={B} L={L} H={H} seed={seed} hasf={hasf}", flush=True)
    proj, z, off = R.make_proj(B, L, H, seed, device=DEV)
    z = z if hasf else None
    lam = torch.tensor([0.31, 3.0, 1e-7, 0.8, 0.31, 0.3, 0.29, 0.31][:H], device=DEV)
    dy = torch.randn(B, L, H * 64, generator=torch.Generator().manual_seed(seed + 100)).to(DEV).to(torch.bfloat16)
    pf = FP().prep_forward(proj, z, H)
    glue32 = R.glue(proj, z, H, dtype=torch.float32)
    vals = {"fused": dict(q=glue32["q"], k=glue32["k"], c=pf.state_views()[0], b=pf.state_views()[1],
                          g=pf.g, F=pf.f),
            "glue": dict(q=glue32["q"], k=glue32["k"], c=glue32["c"].to(torch.bfloat16),
                         b=glue32["b"].to(torch.bfloat16), g=glue32["g"], F=glue32["F"])}
    res = {}
    for name, runner in (("fused", run_fused), ("glue", run_glue_hip)):
        y64, dP64, dl64, dz64 = R.fused64(proj, z, lam, H, vals[name], dy)
        y, dP, dl, dz = runner(proj, z, lam, H, dy)
        r = dict(y=R.rel(y, y64), dlam=R.rel(dl, dl64))
        for grp, (a, w) in dict(Q=("Q", H * 64), K=("K", H * 64), V=("V", H * 64), B=("B", H * 32),
                                C=("C", H * 32), TH=("TH", H * 16), A=("A", H)).items():
            r["d" + grp] = R.rel(dP[..., off[a]:off[a] + w], dP64[..., off[a]:off[a] + w])
        if dz is not None:
            r["dz"] = R.rel(dz, dz64)
        if name == "fused":
            assert bool(torch.isfinite(dP).all()) and (dz is None or bool(torch.isfinite(dz).all()))
            if off["NPAD"] > off["NTOT"]:
                assert bool((dP[..., off["NTOT"]:] == 0).all()), "padding columns of d proj must be zero"
        res[name] = r
    bad = []
    for kk, vv in res["fused"].items():
        if vv > 2e-2:
            bad.append(f"{kk}: fused rel err {vv:.3e} > 2e-2")
        fac, fl = (1.5, 1e-5) if kk in ("dz", "dlam") else (1.05, 1e-6)
        if vv > fac * res["glue"][kk] + fl:
            bad.append(f"{kk}: fused {vv:.3e} > glue {res['glue'][kk]:.3e}")
    assert not bad, "; ".join(bad) + f"\nfused {res['fused']}\nglue  {res['glue']}"


@pytest.mark.parametrize("L,t_cut", [(1000, 437), (2048, 1)])
def test_fused_determinism_and_causality(L, t_cut):
    H = 8
    proj, z, off = R.make_proj(2, L, H, 21, device=DEV)
    lam = torch.tensor([0.31, 3.0, 1e-7, 0.8, 0.31, 0.3, 0.29, 0.31], device=DEV)
    dy = torch.randn(2, L, H * 64, generator=torch.Generator().manual_seed(5)).to(DEV).to(torch.bfloat16)

    def run(P_, Z_, dy_):
        Pp = P_.detach().clone().requires_grad_(True)
        Zp = Z_.detach().clone().requires_grad_(True)
        Lp = lam.detach().clone().requires_grad_(True)
        snap = (Pp.detach().clone(), Zp.detach().clone())
        y = FP().sisa_fused(Pp, Zp, Lp, H)
        gP, gZ, gL = torch.autograd.grad(y, (Pp, Zp, Lp), dy_)
        same_in = torch.equal(Pp.detach(), snap[0]) and torch.equal(Zp.detach(), snap[1])
        return y.detach(), gP, gZ, gL, same_in
    a = run(proj, z, dy)
    b = run(proj, z, dy)
    assert all(torch.equal(x, y_) for x, y_ in zip(a[:4], b[:4])), "not deterministic"
    assert a[4] and b[4], "inputs were modified"
    P2 = proj.clone()
    z2 = z.clone()
    gen = torch.Generator().manual_seed(77)
    P2[:, t_cut:] = (torch.randn(P2[:, t_cut:].shape, generator=gen) * 0.5).to(DEV).to(P2.dtype)
    z2[:, t_cut:] = torch.randn(z2[:, t_cut:].shape, generator=gen).to(DEV)
    dyc = dy.clone()
    dyc[:, t_cut:] = 0
    c1 = run(proj, z, dyc)
    c2 = run(P2, z2, dyc)
    assert torch.equal(c1[0][:, :t_cut], c2[0][:, :t_cut]), "output prefix depends on the future"
    assert torch.equal(c1[1][:, :t_cut], c2[1][:, :t_cut]) and torch.equal(c1[2][:, :t_cut], c2[2][:, :t_cut])
    assert torch.equal(c1[3], c2[3]), "dlam depends on the future"
    assert bool((c1[1][:, t_cut:] == 0).all() and (c1[2][:, t_cut:] == 0).all()
                and (c2[1][:, t_cut:] == 0).all() and (c2[2][:, t_cut:] == 0).all())


def test_fused_input_validation():
    H, L = 4, 70
    proj, z, off = R.make_proj(1, L, H, 3, device=DEV)
    lam = torch.full((H,), 0.3, device=DEV)
    f = FP().sisa_fused
    with pytest.raises(ValueError):
        f(proj[..., :-16], z, lam, H)
    with pytest.raises(TypeError):
        f(proj.float(), z, lam, H)
    with pytest.raises(TypeError):
        f(proj, z.double(), lam, H)
    with pytest.raises(ValueError):
        f(proj, z, lam[:2], H)
    y = f(proj, None, lam, H)
    assert y.shape == (1, L, H * 64) and y.dtype == torch.bfloat16 and bool(torch.isfinite(y.float()).all())
    y16 = f(proj.to(torch.float16), z, lam, H)
    assert y16.dtype == torch.float16 and bool(torch.isfinite(y16.float()).all())


def test_nan_guard_sync_mode():
    from sisa_amd import backends
    H, L = 4, 70
    proj, z, off = R.make_proj(1, L, H, 3, device=DEV)
    lam = torch.full((H,), 0.3, device=DEV)
    old = backends.get_check_mode()
    backends.set_check_mode("sync")
    try:
        zn = z.clone()
        zn[0, 5, 1] = float("nan")
        with pytest.raises(FloatingPointError):
            FP().sisa_fused(proj, zn, lam, H)
        pn = proj.clone()
        pn[0, 7, off["A"] + 2] = float("inf")
        with pytest.raises(FloatingPointError):
            FP().sisa_fused(pn, z, lam, H)
        pt = proj.clone()                  # theta: the rotation angles of C and B
        pt[0, 40, off["TH"] + 5] = float("-inf")
        with pytest.raises(FloatingPointError):
            FP().sisa_fused(pt, z, lam, H)
        ln = lam.clone()
        ln[1] = float("nan")
        with pytest.raises(FloatingPointError):
            FP().sisa_fused(proj, z, ln, H)
        FP().sisa_fused(proj, z, lam, H)   # finite inputs pass the same check
    finally:
        backends.set_check_mode(old)


def test_finite_sum_flag():
    """The fused non-finite check (one launch, fixed-order fp32 sum): 1 for finite data, 0 when a NaN or an inf sits
    anywhere in either operand, and for sizes that are not multiples of the 16-byte vector; the flag is read back
    here, never asserted on the device."""
    fp = FP()
    gen = torch.Generator().manual_seed(3)
    for na, nb in ((196608, 55296), (1003, 7), (4, 0), (0, 33)):
        a = torch.randn(na, generator=gen).to(DEV)
        b = torch.randn(nb, generator=gen).to(DEV)
        assert bool(fp.finite_sum_flag(a, b).item())
        for bad in (float("nan"), float("inf"), float("-inf")):
            for t in (a, b):
                if t.numel() == 0:
                    continue
                i = int(torch.randint(0, t.numel(), (1,), generator=gen))
                keep = t[i].item()
                t[i] = bad
                assert not bool(fp.finite_sum_flag(a, b).item()), (na, nb, bad)
                t[i] = keep
