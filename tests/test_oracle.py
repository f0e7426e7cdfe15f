"""Pins the CPU oracle (oracle/reference.py) before it is trusted as the checker of the HIP kernels.

Each check is independent of the function it pins: pure-Python scalar evaluations written by
tests/golden/make_golden.py (math module only), finite differences, textbook special cases computed with other torch
routines, closed forms and a second derivation. The planted-mistake test shows that a dropped term, a wrong sign, a
transposed decay or a wrong scale fails the golden comparison. CPU only, fp64, seconds.
"""
from __future__ import annotations

import json
import math
import os

import pytest
import torch
import torch.nn.functional as F

from oracle import reference as R

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
D64 = torch.float64


def _load(name):
    with open(os.path.join(GOLD, name)) as f:
        return json.load(f)


def _t(x):
    return torch.tensor(x, dtype=D64)


def _attn_golden():
    G = _load("attn_tiny.json")
    X = G["inputs"]
    ins = {n: _t(X[n])[None] for n in ("q", "k", "v", "c", "b", "g", "F")}
    ins["lam"] = _t(X["lam"])
    ins["do"] = _t(G["do"])[None]
    return G, ins


def _rand_ins(B=1, H=2, L=9, D=8, S=4, seed=0, lam=(0.7, 2.0), fscale=1.0):
    gen = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=gen, dtype=D64)   # noqa: E731
    g = torch.cumsum(-F.softplus(r(B, H, L) - 1.0), -1)
    Fg = torch.cumsum(F.logsigmoid(r(B, H, L) + 1.0), -1) * fscale
    return dict(q=r(B, H, L, D), k=r(B, H, L, D), v=r(B, H, L, D), c=0.8 * r(B, H, L, S), b=0.8 * r(B, H, L, S),
                g=g, F=Fg, lam=torch.tensor(lam[:H], dtype=D64), do=r(B, H, L, D))


def _dense(ins, **over):
    a = dict(ins)
    a.update(over)
    return R.dense_attention(a["q"], a["k"], a["v"], a["c"], a["b"], a["g"], a["lam"], a["F"])


# ------------------------------------------------------------------------------------------------ attention
def test_golden_attention_forward():
    G, ins = _attn_golden()
    o = _dense(ins)[0]
    assert torch.allclose(o, _t(G["o"]), rtol=0, atol=1e-12)


def test_golden_attention_grads():
    G, ins = _attn_golden()
    T = R.truth64(ins)
    for n, gn in zip(R.IN_NAMES, R.GRAD_NAMES):
        ref = _t(G["grads"][n])
        got = T[gn][0] if n != "lam" else T[gn]
        assert torch.allclose(got, ref, rtol=0, atol=2e-7), (n, (got - ref).abs().max().item())


def test_golden_detects_planted_mistakes():
    """Plausible formula mistakes, planted on the CPU as equivalent input changes, all miss the golden output."""
    G, ins = _attn_golden()
    ref = _t(G["o"])
    mistakes = {
        "forget-gate sign (F_j - F_t)": dict(F=-ins["F"]),
        "decay transposed (g_j - g_t)": dict(g=-ins["g"]),
        "decay term dropped": dict(lam=torch.zeros_like(ins["lam"])),
        "scale 1/d instead of 1/sqrt(d)": dict(q=ins["q"] / math.sqrt(ins["q"].shape[-1])),
        "c and b swapped": dict(c=ins["b"], b=ins["c"]),
        "q and k swapped": dict(q=ins["k"], k=ins["q"]),
    }
    for what, over in mistakes.items():
        assert (_dense(ins, **over)[0] - ref).abs().max().item() > 1e-4, what


def test_gradcheck_dense():
    ins = _rand_ins(L=5, D=4, S=2, seed=3)
    args = [ins[n].clone().requires_grad_(True) for n in ("q", "k", "v", "c", "b", "g", "lam", "F")]
    assert torch.autograd.gradcheck(lambda *a: R.dense_attention(*a), args, eps=1e-6, atol=1e-6)


def test_special_cases():
    ins = _rand_ins(H=2, L=11, D=64, S=32, seed=4)
    # lam = 0 and F = 0: causal softmax attention (SDPA math path, fp64)
    sd = F.scaled_dot_product_attention(ins["q"], ins["k"], ins["v"], is_causal=True)
    o = _dense(ins, lam=torch.zeros(2, dtype=D64), F=None)
    assert torch.allclose(o, sd, atol=1e-12)
    # lam = 0: forgetting attention softmax(q k / sqrt(d) + F_t - F_j)
    L = ins["q"].shape[2]
    s = ins["q"] @ ins["k"].transpose(-1, -2) / 8.0 + ins["F"][..., :, None] - ins["F"][..., None, :]
    s = s.masked_fill(~torch.ones(L, L, dtype=torch.bool).tril(), -math.inf)
    assert torch.allclose(_dense(ins, lam=torch.zeros(2, dtype=D64)), torch.softmax(s, -1) @ ins["v"], atol=1e-12)
    # c = 0: independent of lam
    c0 = torch.zeros_like(ins["c"])
    assert torch.equal(_dense(ins, c=c0), _dense(ins, c=c0, lam=ins["lam"] * 5 + 1))
    # L = 1: o = v
    one = {n: (t[:, :, :1] if t.dim() >= 3 else t) for n, t in ins.items()}
    assert torch.allclose(_dense(one), one["v"], atol=1e-15)
    # a constant shift of g or F changes nothing
    o0 = _dense(ins)
    assert torch.allclose(_dense(ins, g=ins["g"] - 37.0), o0, atol=1e-12)
    assert torch.allclose(_dense(ins, F=ins["F"] + 300.0), o0, atol=1e-10)


def test_analytic_grads_vs_autograd():
    ins = _rand_ins(B=2, H=2, L=13, D=8, S=4, seed=5)
    T = R.truth64(ins)
    for bb in range(2):
        for h in range(2):
            A = R.analytic_grads64(*(ins[n][bb, h] for n in ("q", "k", "v", "c", "b", "g")), ins["lam"][h],
                                   ins["F"][bb, h], ins["do"][bb, h])
            for gn in ("o", "dq", "dk", "dv", "dc", "db", "dg", "dF"):
                assert torch.allclose(A[gn], T[gn][bb, h], atol=1e-11), gn
    # dlam summed over (b, h) per head
    for h in range(2):
        tot = sum(R.analytic_grads64(*(ins[n][bb, h] for n in ("q", "k", "v", "c", "b", "g")), ins["lam"][h],
                                     ins["F"][bb, h], ins["do"][bb, h])["dlam"] for bb in range(2))
        assert abs(tot.item() - T["dlam"][h].item()) < 1e-10


def _head(ins, bb, h):
    return [ins[n][bb, h].double().cpu() for n in ("q", "k", "v", "c", "b", "g")] + [
        ins["lam"][h].double(), None if ins["F"] is None else ins["F"][bb, h].double().cpu(),
        ins["do"][bb, h].double().cpu()]


def _worst_vs(A, M, names=("o", "dq", "dk", "dv", "dc", "db", "dg", "dF", "dlam")):
    worst = 0.0
    for n in names:
        a, m = A[n].reshape(-1), M[n].reshape(-1)
        worst = max(worst, ((a - m).norm() / m.norm()).item())
    return worst


@pytest.mark.parametrize("forget", [-3.0, -20.0, -40.0, -60.0])
def test_analytic_grads_vs_mpmath_strong_forgetting(forget):
    """The delta-free analytic gradients against a 60-digit evaluation of the direct formula (dS = P (dP - T),
    diagonal included) at L = 10, where P_tt rounds to 1 in fp64 beyond about -30 nats per token: <= 1e-12."""
    ins = R.diag_inputs(1, 1, 10, seed=7, forget=[forget], lam=0.9)
    args = _head(ins, 0, 0)
    A = R.analytic_grads64(*args)
    M = R.direct_grads_mp(*args)
    assert _worst_vs(A, M) <= 1e-12


def test_mpmath_check_detects_a_dropped_diagonal():
    """Planted mistake: dq without its diagonal term dS_tt k_t / 8 fails the mpmath check that the oracle passes."""
    ins = R.diag_inputs(1, 1, 10, seed=7, forget=[-3.0], lam=0.9)
    args = _head(ins, 0, 0)
    q, k, v, c, b, g, lam, Fg, do = args
    M = R.direct_grads_mp(*args)
    A = R.analytic_grads64(*args)
    i = torch.arange(q.shape[0])
    dec = torch.exp((g[:, None] - g[None, :]).clamp(max=0))
    s = (q @ k.T) / 8 + lam * dec * (c @ b.T) + (Fg[:, None] - Fg[None, :])
    P = torch.softmax(s.masked_fill(i[:, None] < i[None, :], -math.inf), -1)
    dP = do @ v.T
    dS_tt = torch.diagonal(P) * (torch.diagonal(dP) - (P * dP).sum(1))
    planted = dict(A, dq=A["dq"] - dS_tt[:, None] * k / 8)
    assert _worst_vs(A, M, ("dq",)) <= 1e-12
    assert _worst_vs(planted, M, ("dq",)) > 1e-6


def test_analytic_grads_vs_autograd_mild_forgetting():
    """The delta-free analytic gradients against fp64 autograd at mild forgetting, L = 512, lam including 0:
    <= 1e-10 (the reference's refcheck, tests/test_attention_diag.py:383-388)."""
    ins = R.diag_inputs(1, 4, 512, seed=8, forget=[-0.05, -1.0, -3.0, -6.0], lam=[0.31, 3.0, 0.0, 0.8],
                        dt=torch.float64)
    T = R.truth64(ins)
    worst = 0.0
    for h in range(4):
        A = R.analytic_grads64(*_head(ins, 0, h))
        for n in ("o", "dq", "dk", "dv", "dc", "db", "dg", "dF"):
            worst = max(worst, R.rel(A[n], T[n][0, h]))
        worst = max(worst, abs(A["dlam"].item() - T["dlam"][h].item()) / abs(T["dlam"][h].item()))
        for n, src in (("dloga", "dg"), ("dlogf", "dF")):
            worst = max(worst, R.rel(R.revcumsum(A[src]), R.revcumsum(T[src][0, h])))
    assert worst <= 1e-10


def test_diag_inputs_layouts():
    """The model layout holds the same values as the head-major one, as (B,L,H,.) memory."""
    a = R.diag_inputs(2, 3, 17, seed=3, forget=[-20.0, -3.0, -1.0])
    b = R.diag_inputs(2, 3, 17, seed=3, forget=[-20.0, -3.0, -1.0], layout="blhd")
    for n in ("q", "k", "v", "c", "b", "do"):
        assert torch.equal(a[n], b[n])
        assert b[n].transpose(1, 2).is_contiguous() and not b[n].is_contiguous()
    assert bool((a["F"].diff(dim=-1) <= 0).all()) and bool((a["g"].diff(dim=-1) <= 0).all())


@pytest.mark.parametrize("block_q", [1, 7, 64])
def test_blocked_vs_dense(block_q):
    ins = _rand_ins(H=2, L=70, D=16, S=8, seed=6)
    ob = R.attention_blocked(ins["q"], ins["k"], ins["v"], ins["c"], ins["b"], ins["g"], ins["lam"], ins["F"],
                             block_q=block_q)
    assert torch.allclose(ob, _dense(ins), atol=1e-12)


@pytest.mark.parametrize("M", [1, 3, 70])
def test_decode_rows_are_the_last_rows_of_dense(M):
    """The decode-step oracle equals the last M rows of the full attention, and changes when a cached key does."""
    ins = _rand_ins(H=2, L=70, D=16, S=8, seed=7)
    q, k, v, c, b, g, lam, Fg = (ins[n] for n in ("q", "k", "v", "c", "b", "g", "lam", "F"))
    rows = R.decode_rows(q[:, :, -M:], k, v, c[:, :, -M:], b, g, lam, Fg, 70 - M)
    assert torch.allclose(rows, _dense(ins)[:, :, -M:], atol=1e-12)
    k2 = k.clone()
    k2[:, :, -2] += 1.0
    assert not torch.allclose(R.decode_rows(q[:, :, -M:], k2, v, c[:, :, -M:], b, g, lam, Fg, 70 - M), rows)


def test_fa_emulation_modes():
    ins = _rand_ins(H=2, L=20, D=64, S=32, seed=7)
    T = R.truth64(ins)
    E = R.fa_emulation(ins, "exact64")
    for gn in ("o", "dq", "dk", "dv", "dc", "db", "dg", "dF", "dlam"):
        assert torch.allclose(E[gn].double(), T[gn], atol=1e-10), gn
    ins32 = {n: (t.float() if t is not None else None) for n, t in ins.items()}
    fa, ideal = R.fa_emulation(ins32, "fa"), R.fa_emulation(ins32, "ideal")
    for gn in fa:
        assert torch.equal(fa[gn], ideal[gn]), gn
    # bf16 'fa' differs from the truth by about the bf16 rounding of its operands, not more
    insb = {n: (t.to(torch.bfloat16) if (t is not None and n in "qkvcb" or n == "do") else t) for n, t in ins.items()}
    Tb, fab = R.truth64(insb), R.fa_emulation(insb, "fa")
    assert 1e-5 < R.rel(fab["o"], Tb["o"]) < 2e-2


def test_factors_closed_form():
    gen = torch.Generator().manual_seed(8)
    g = torch.cumsum(-F.softplus(torch.randn(2, 3, 200, generator=gen, dtype=D64)), -1)
    T = 64
    rowf, colf = R.factors(g, T)
    idx = torch.arange(200)
    start = (idx // T) * T
    end = torch.clamp(start + T - 1, max=199)
    for i in (70, 130, 199):
        for j in (0, 63, 64, 100):
            if j // T >= i // T:
                continue
            mid = torch.exp(g[..., start[i]] - g[..., end[j]])
            assert torch.allclose(rowf[..., i] * mid * colf[..., j], torch.exp(g[..., i] - g[..., j]), rtol=1e-12)
    assert (rowf <= 1).all() and (colf <= 1).all() and (rowf > 0).all()


# ------------------------------------------------------------------------------------------------ glue / layout
def test_golden_glue():
    G = _load("glue_tiny.json")
    X = G["inputs"]
    L, H = len(X["a"]), len(X["a"][0])
    c = _t(X["c"]).permute(1, 0, 2)[None]                  # (1, H, L, S)
    inp = dict(theta=_t(X["theta"])[None], a=_t(X["a"])[None], z=_t(X["z"])[None], c=c, b=c,
               lam_raw=torch.zeros(H, dtype=D64))
    cr, br, g, Fg, lam = R.unfused_glue(inp)
    assert torch.allclose(g[0], _t(G["g"]), atol=1e-13)
    assert torch.allclose(Fg[0], _t(G["F"]), atol=1e-13)
    assert torch.allclose(cr[0], _t(G["c_rot"]), atol=1e-13)
    rowf, colf = R.factors(g, X["T"])
    assert torch.allclose(rowf[0], _t(G["rowf"]), atol=1e-14)
    assert torch.allclose(colf[0], _t(G["colf"]), atol=1e-14)
    assert (g[0, :, 1:] <= g[0, :, :-1]).all()              # g is non-increasing


def test_rotate_pairs_is_complex_multiplication():
    gen = torch.Generator().manual_seed(9)
    z = torch.randn(2, 3, 5, 8, generator=gen, dtype=D64)
    phi = torch.randn(2, 3, 5, 4, generator=gen, dtype=D64)
    zc = torch.view_as_complex(z.reshape(2, 3, 5, 4, 2).contiguous())
    ref = torch.view_as_real(zc * torch.exp(1j * phi)).reshape(2, 3, 5, 8)
    assert torch.allclose(R.rotate_pairs(z, phi), ref, atol=1e-14)


def test_layout():
    for H, npad in ((8, 2192), (12, 3280), (16, 4368)):
        off = R.layout(H)
        assert off["NTOT"] == 273 * H and off["NPAD"] == npad
        assert [off[k] for k in ("Q", "K", "V", "B", "C", "TH", "A")] == [0, 64 * H, 128 * H, 192 * H, 224 * H,
                                                                          256 * H, 272 * H]


def test_glue_of_fused_projection_matches_unfused():
    B, L, H = 1, 9, 2
    proj, z, off = R.make_proj(B, L, H, seed=1, dt=D64)
    z = z.double()
    G = R.glue(proj, z, H)

    def cols(nm, w):
        return proj[..., off[nm]:off[nm] + H * w].view(B, L, H, w)
    inp = dict(theta=cols("TH", 16), a=proj[..., off["A"]:off["A"] + H], z=z,
               c=cols("C", 32).transpose(1, 2), b=cols("B", 32).transpose(1, 2), lam_raw=torch.zeros(H, dtype=D64))
    cr, br, g, Fg, _ = R.unfused_glue(inp)
    for a, b_ in ((G["c"], cr), (G["b"], br), (G["g"], g), (G["F"], Fg)):
        assert torch.allclose(a, b_, atol=1e-13)
    assert torch.equal(G["q"], cols("Q", 64).transpose(1, 2))


def test_fused64_matches_composition():
    B, L, H = 1, 8, 2
    proj, z, off = R.make_proj(B, L, H, seed=2, dt=D64)
    z = z.double()
    lam = torch.tensor([0.4, 1.3], dtype=D64)
    dy = torch.randn(B, L, H * 64, generator=torch.Generator().manual_seed(3), dtype=D64)
    G = R.glue(proj, z, H)
    y, dproj, dlam, dz = R.fused64(proj, z, lam, H, G, dy)
    P = proj.clone().requires_grad_(True)
    Z = z.clone().requires_grad_(True)
    LAM = lam.clone().requires_grad_(True)
    G2 = R.glue(P, Z, H)
    o = R.dense_attention(G2["q"], G2["k"], G2["v"], G2["c"], G2["b"], G2["g"], LAM, G2["F"])
    y2 = o.transpose(1, 2).reshape(B, L, H * 64)
    gr = torch.autograd.grad(y2, [P, LAM, Z], dy)
    assert torch.allclose(y, y2.detach(), atol=1e-13)
    for a, b_ in zip((dproj, dlam, dz), gr):
        assert torch.allclose(a, b_, atol=1e-11)
    assert (dproj[..., off["NTOT"]:] == 0).all()


def test_config_inputs():
    c0 = R.config_inputs(0)
    assert c0["q"].shape == (1, 4, 256, 64) and c0["theta"].shape == (1, 256, 4, 16) and c0["q"].dtype == torch.float32
    assert abs(c0["a"].mean().item() + 5.0) < 0.05 and abs(c0["z"].mean().item() - 4.0) < 0.05
    c1 = R.config_inputs(1)
    assert c1["proj"].shape == (4, 2048, 2192) and c1["proj"].dtype == torch.bfloat16 and c1["z"].shape == (4, 2048, 8)
    assert (c1["proj"][..., 2184:] == 0).all()


# ------------------------------------------------------------------------------------------------ linear CE
def test_golden_lmce():
    G = _load("lmce_tiny.json")
    X = G["inputs"]
    x, W = _t(X["x"]), _t(X["W"])
    lab = torch.tensor(X["labels"])
    loss, dx, dW = R.lmce64(x, W, lab, 1.0, ignore_index=X["ignore_index"])
    assert abs(loss.item() - G["loss"]) < 1e-13
    assert torch.allclose(dx, _t(G["dx"]), atol=1e-14) and torch.allclose(dW, _t(G["dW"]), atol=1e-14)
    assert (dx[2] == 0).all()


def test_lmce64_vs_cross_entropy():
    gen = torch.Generator().manual_seed(10)
    N, D, V = 300, 16, 1001
    h = torch.randn(3, N // 3, D, generator=gen, dtype=D64)
    w = torch.randn(V, D, generator=gen, dtype=D64) * 0.5
    lab = torch.randint(0, V, (3, N // 3), generator=gen)
    lab[0, :7] = -100
    g = 0.3
    loss, dx, dW = R.lmce64(h, w, lab, g, chunk=64)
    hh, ww = h.clone().requires_grad_(True), w.clone().requires_grad_(True)
    ref = F.cross_entropy(F.linear(hh, ww).reshape(-1, V), lab.reshape(-1), ignore_index=-100)
    (ref * g).backward()
    assert abs(loss.item() - ref.item()) < 1e-12
    assert torch.allclose(dx, hh.grad, atol=1e-14) and torch.allclose(dW, ww.grad, atol=1e-14)
    assert (dx[0, :7] == 0).all()


def test_lmce_rows64():
    gen = torch.Generator().manual_seed(12)
    T, V, Vp = 40, 997, 1024
    x = 3.0 * torch.randn(T, Vp, generator=gen, dtype=D64)
    lab = torch.randint(0, V, (T,), generator=gen)
    lab[3] = -100
    inv_n = 1.0 / 39.0
    lse, loss, G = R.lmce_rows64(x, lab, V, inv_n=inv_n, gscale=0.5)
    ce = F.cross_entropy(x[:, :V], lab, reduction="none", ignore_index=-100)
    assert torch.allclose(loss, ce, atol=1e-12) and loss[3] == 0
    assert torch.allclose(lse, torch.logsumexp(x[:, :V], 1), atol=1e-13)
    xr = x[:, :V].clone().requires_grad_(True)
    (F.cross_entropy(xr, lab, reduction="sum", ignore_index=-100) * inv_n * 0.5).backward()
    assert torch.allclose(G[:, :V], xr.grad, atol=1e-15) and (G[:, V:] == 0).all() and (G[3] == 0).all()
    # composed with the two GEMMs it is lmce64
    h = torch.randn(T, 8, generator=gen, dtype=D64)
    w = torch.cat([torch.randn(V, 8, generator=gen, dtype=D64), torch.zeros(Vp - V, 8, dtype=D64)])
    _, loss_r, G2 = R.lmce_rows64(h @ w.T, lab, V, inv_n=inv_n)
    l64, dx64, dW64 = R.lmce64(h, w[:V], lab)
    assert abs(loss_r.sum().item() * inv_n - l64.item()) < 1e-12
    assert torch.allclose(G2 @ w, dx64, atol=1e-14) and torch.allclose((G2.T @ h)[:V], dW64, atol=1e-14)
    # a label outside [0, V) gives a NaN loss row
    lab2 = lab.clone()
    lab2[5] = V + 3
    assert math.isnan(R.lmce_rows64(x, lab2, V)[1][5].item())
