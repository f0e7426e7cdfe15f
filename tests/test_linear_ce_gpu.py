"""GPU tests of the chunked linear cross-entropy (HIP row kernel + hipBLASLt GEMMs) against fp64.

Follows the reference's tests/test_linear_ce.py of tlstngud/sisa. For each case the loss, dL/dh and dL/dW (backward
seeded with g) are computed with
  ref64    fp64 math on the fp32 master inputs                                   -- "the math"
  ref64q   fp64 math on bf16-rounded inputs (h, W rounded as autocast does)     -- isolates the op's own rounding
  eager    F.cross_entropy(F.linear(h, w).float(), y) under autocast
  lmce     linear_cross_entropy under autocast (default chunks, odd chunks, one chunk, grad_scale promise)
and compared as rel-L2 = ||a - ref|| / ||ref||. Rule (the reference's, test_linear_ce.py:106-121):
err(lmce) <= 2 x err(eager) + 1e-7 against both references, for every tensor.
The row kernel alone is checked against the fp64 row pass of the oracle on stored logits: lse and loss rows to fp32
accuracy, G within one unit in the last place of the compute dtype, pad columns and ignored rows exactly zero.
"""
from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import reference as R

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _lce():
    from sisa_amd.kernels.linear_ce import linear_cross_entropy
    return linear_cross_entropy


def _eager(h, w, labels, ignore_index=-100):
    logits = F.linear(h, w)
    return F.cross_entropy(logits.view(-1, logits.size(-1)).float(), labels.reshape(-1), ignore_index=ignore_index)


def run_path(fn, h, w, labels, g, need=(True, True), autocast=torch.bfloat16, **kw):
    hh = h.detach().clone().requires_grad_(need[0])
    ww = w.detach().clone().requires_grad_(need[1])
    if autocast is not None:
        with torch.autocast("cuda", dtype=autocast):
            loss = fn(hh, ww, labels, **kw)
    else:
        loss = fn(hh, ww, labels, **kw)
    (loss * g).backward()
    torch.cuda.synchronize()
    return loss.detach().float(), (hh.grad if need[0] else None), (ww.grad if need[1] else None)


def compare(res, refs, tol=2.0, floor=1e-7):
    fails = []
    for p, t in res.items():
        if p == "eager":
            continue
        for i, nm in enumerate(("loss", "dh", "dw")):
            if t[i] is None:
                continue
            for r, ref in refs.items():
                e_new, e_ref = R.rel(t[i], ref[i]), R.rel(res["eager"][i], ref[i])
                if not (e_new <= tol * e_ref + floor):
                    fails.append(f"{p} {nm} vs {r}: {e_new:.3e} > {tol} x eager {e_ref:.3e}")
    return fails


def make_case(D, N, V, seed, sharp=3.0):
    """Final-norm-like hidden states and labels drawn from the model's own softmax (peaked targets), generated on
    the CPU from a seeded generator."""
    gen = torch.Generator().manual_seed(seed)
    B = max(1, N // 1024)
    L = N // B
    h = torch.randn(B, L, D, generator=gen)
    h = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + 1e-6)
    h = h * (1.0 + 0.8 * torch.rand(D, generator=gen))
    w = torch.randn(V, D, generator=gen) * (sharp / math.sqrt(D))
    xf = h.reshape(-1, D)
    lab = torch.empty(B * L, dtype=torch.int64)
    for s in range(0, B * L, 512):
        p = torch.softmax(xf[s:s + 512] @ w.t(), -1)
        lab[s:s + 512] = torch.multinomial(p, 1, generator=gen)[:, 0]
    return h.to(DEV), w.to(DEV), lab.view(B, L).to(DEV)


def ref64(h, w, lab, g, quant, ignore_index=-100):
    return R.lmce64(h, w, lab, g, quant=quant, ignore_index=ignore_index)


# ------------------------------------------------------------------------------------------------ row kernel
def _rows_case(T, V, Vp, stride, dtype, seed):
    gen = torch.Generator().manual_seed(seed)
    buf = torch.full((T, stride), 7.0)                       # garbage beyond Vp must stay untouched
    buf[:, :Vp] = 3.0 * torch.randn(T, Vp, generator=gen)
    lab = torch.randint(0, V, (T,), generator=gen)
    lab[1] = -100
    if T > 3:
        lab[3] = V - 1
        lab[2] = 0
    return buf.to(dtype).to(DEV), lab.to(DEV)


def _ulp(x: torch.Tensor, dt: torch.dtype) -> torch.Tensor:
    mant = {torch.bfloat16: 7, torch.float16: 10}[dt]
    tiny = {torch.bfloat16: 2.0 ** -133, torch.float16: 2.0 ** -24}[dt]
    e = torch.floor(torch.log2(x.abs().clamp_min(1e-300)))
    return torch.maximum(torch.exp2(e - mant), torch.full_like(x, tiny))


@pytest.mark.parametrize("V,Vp,stride,dtype", [
    (1003, 1024, 1024, torch.bfloat16),      # 4 vectors per thread, ragged vocabulary
    (20011, 20096, 20104, torch.bfloat16),   # 8 vectors per thread, row stride > Vp
    (50277, 50304, 50304, torch.bfloat16),   # the GPT-NeoX vocabulary: 16 vectors per thread
    (50277, 50304, 50304, torch.float16),
    (70001, 70016, 70016, torch.bfloat16),   # streamed twice
    (8, 8, 8, torch.bfloat16),               # a single vector
])
def test_rows_kernel_vs_oracle(V, Vp, stride, dtype):
    from sisa_amd.kernels.linear_ce import lmce_rows
    T = 37
    buf, lab = _rows_case(T, V, Vp, stride, dtype, seed=V)
    lg = buf[:, :Vp]
    x0 = lg.detach().cpu().clone()
    inv_n, gscale = 1.0 / 29.0, 0.5
    lse_ref, loss_ref, G_ref = R.lmce_rows64(x0, lab.cpu(), V, inv_n=inv_n, gscale=gscale)
    loss = torch.empty(T, device=DEV)
    lse = torch.empty(T, device=DEV)
    # loss only: logits untouched
    lmce_rows(lg, lab, loss, V, -100, None, 1.0, lse)
    torch.cuda.synchronize()
    assert torch.equal(lg.cpu(), x0)
    tol = 4e-6 * lse_ref.abs().clamp_min(1.0)
    assert ((lse.cpu().double() - lse_ref).abs() <= tol).all()
    assert ((loss.cpu().double() - loss_ref).abs() <= tol).all()
    assert loss[1].item() == 0.0
    # with G
    inv = torch.tensor([inv_n], device=DEV, dtype=torch.float32)
    loss2 = torch.empty(T, device=DEV)
    lmce_rows(lg, lab, loss2, V, -100, inv, gscale)
    torch.cuda.synchronize()
    assert torch.equal(loss2, loss)
    G = lg.cpu().double()
    assert torch.equal(buf[:, Vp:].cpu(), torch.full((T, stride - Vp), 7.0, dtype=dtype))
    assert (G[:, V:] == 0).all() and (G[1] == 0).all()
    # fp32 scale of the reference value: inv_n is an fp32 scalar on the device
    G_ref = G_ref * (float(torch.tensor(inv_n, dtype=torch.float32)) / inv_n)
    # one unit in the last place of the stored value, plus the fp32 error of the exponent argument
    # (|x - lse| * log2(e) rounded to fp32: about 4e-6 relative on exp, i.e. on the softmax part of G)
    bound = _ulp(G_ref, dtype) + 4e-6 * inv_n * gscale
    err = (G - G_ref).abs()
    assert (err <= bound).all(), float((err / bound).max())


def test_rows_kernel_nan_and_labels():
    from sisa_amd.kernels.linear_ce import lmce_rows
    T, V, Vp = 6, 5000, 5120
    buf, lab = _rows_case(T, V, Vp, Vp, torch.bfloat16, seed=1)
    buf[0, 17] = float("nan")
    buf[2, V - 1] = float("inf")
    lab[4] = V + 3                                      # outside the vocabulary (a pad column)
    lab[5] = -7                                         # negative and not ignore_index
    loss = torch.empty(T, device=DEV)
    inv = torch.tensor([0.25], device=DEV)
    lmce_rows(buf, lab, loss, V, -100, inv, 1.0)
    torch.cuda.synchronize()
    lc = loss.cpu()
    assert math.isnan(lc[0]) and torch.isnan(buf[0].float()).all()
    assert not math.isfinite(lc[2])
    assert math.isnan(lc[4]) and math.isnan(lc[5])
    assert lc[1] == 0.0 and math.isfinite(lc[3])
    assert (buf[4, V:].float() == 0).all()              # no onehot in the pad columns


def test_rows_kernel_validation():
    from sisa_amd.kernels import _lib
    from sisa_amd.kernels.linear_ce import lmce_rows
    buf = torch.zeros(4, 64, device=DEV, dtype=torch.bfloat16)
    lab = torch.zeros(4, dtype=torch.int64, device=DEV)
    loss = torch.empty(4, device=DEV)
    with pytest.raises(RuntimeError, match="multiple of 8"):
        lmce_rows(buf[:, :60], lab, loss, 60, -100)
    with pytest.raises(RuntimeError, match="V <= Vp"):
        lmce_rows(buf, lab, loss, 65, -100)
    with pytest.raises(RuntimeError, match="dtype"):
        lmce_rows(buf.float(), lab, loss, 64, -100)
    with pytest.raises(ValueError):
        lmce_rows(buf, lab.int(), loss, 64, -100)
    args = _lib.LmceRowsArgs(4, 64, 64, 64, _lib.BF16, 1, buf.data_ptr(), lab.data_ptr(), -100, None, 1.0,
                             loss.data_ptr(), None)
    with pytest.raises(RuntimeError, match="inv_n"):
        _lib.call("sisa_lmce_rows", args, buf)


# ------------------------------------------------------------------------------------------------ full op
_SHAPES = [("D512_V50277", 512, 2048, 50277, 1 / 16), ("D768_Vodd", 768, 1024, 1003, 1 / 32),
           pytest.param(("D1024_V50277_N4096", 1024, 4096, 50277, 1 / 64), marks=pytest.mark.slow)]


@pytest.mark.parametrize("case", _SHAPES, ids=lambda c: c[0])
def test_accuracy_vs_fp64(case):
    _, D, N, V, g = case
    lce = _lce()
    h, w, lab = make_case(D, N, V, seed=D + V)
    refs = {"ref64": ref64(h, w, lab, g, False), "ref64q": ref64(h, w, lab, g, True)}
    res = {"eager": run_path(_eager, h, w, lab, g), "lmce": run_path(lce, h, w, lab, g),
           "lmce_c300": run_path(lce, h, w, lab, g, chunk_tokens=300),
           "lmce_full": run_path(lce, h, w, lab, g, chunk_tokens=N),
           "lmce_gs": run_path(lce, h, w, lab, g, grad_scale=g)}
    fails = compare(res, refs)
    assert not fails, "\n".join(fails)
    assert abs(res["lmce"][0].item() - res["eager"][0].item()) < 1e-3


def test_semantics():
    lce = _lce()
    D, N, V = 512, 1024, 4099
    h, w, lab = make_case(D, N, V, seed=7)
    lab_i = lab.clone()
    gm = torch.Generator().manual_seed(3)
    lab_i[(torch.rand(lab.shape, generator=gm) < 0.05).to(DEV)] = -100
    refs = {"ref64": ref64(h, w, lab_i, 1 / 16, False), "ref64q": ref64(h, w, lab_i, 1 / 16, True)}
    res = {"eager": run_path(_eager, h, w, lab_i, 1 / 16), "lmce": run_path(lce, h, w, lab_i, 1 / 16),
           "lmce_c100": run_path(lce, h, w, lab_i, 1 / 16, chunk_tokens=100)}
    assert not compare(res, refs)
    assert res["lmce"][1].reshape(-1, D)[lab_i.reshape(-1) == -100].abs().max().item() == 0.0
    # a non-power-of-two seed
    gg = 0.3
    refs = {"ref64": ref64(h, w, lab, gg, False), "ref64q": ref64(h, w, lab, gg, True)}
    res = {"eager": run_path(_eager, h, w, lab, gg), "lmce": run_path(lce, h, w, lab, gg),
           "lmce_gs": run_path(lce, h, w, lab, gg, grad_scale=gg)}
    assert not compare(res, refs)
    # gradients for h only / W only: bit-identical to the run with both
    both = run_path(lce, h, w, lab, 1 / 16)
    for need in ((True, False), (False, True)):
        r1 = run_path(lce, h, w, lab, 1 / 16, need=need)
        assert torch.equal(r1[0], both[0])
        for x, y, n in zip(r1[1:], both[1:], need):
            assert (x is None) == (not n) and (x is None or torch.equal(x, y))
    # no_grad forward == grad forward loss
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        l0 = lce(h, w, lab)
    assert torch.equal(l0.float(), both[0]) and not l0.requires_grad
    # bf16 tensors without autocast
    hb, wb = h.to(torch.bfloat16), w.to(torch.bfloat16)
    refs = {"ref64": ref64(hb.float(), wb.float(), lab, 1 / 16, False)}
    res = {"eager": run_path(_eager, hb, wb, lab, 1 / 16, autocast=None),
           "lmce": run_path(lce, hb, wb, lab, 1 / 16, autocast=None)}
    assert not compare(res, refs)
    assert res["lmce"][1].dtype == torch.bfloat16 and res["lmce"][2].dtype == torch.bfloat16
    # fp16 autocast
    refs = {"ref64": ref64(h, w, lab, 1 / 16, False)}
    res = {"eager": run_path(_eager, h, w, lab, 1 / 16, autocast=torch.float16),
           "lmce": run_path(lce, h, w, lab, 1 / 16, autocast=torch.float16)}
    assert not compare(res, refs)
    # 2-D input == 3-D input, and deterministic
    r3 = run_path(lce, h, w, lab, 1 / 16)
    r2 = run_path(lce, h.reshape(-1, D), w, lab.reshape(-1), 1 / 16)
    assert torch.equal(r3[0], r2[0]) and torch.equal(r3[1].reshape(-1, D), r2[1]) and torch.equal(r3[2], r2[2])
    r3b = run_path(lce, h, w, lab, 1 / 16)
    assert all(torch.equal(a, b) for a, b in zip(r3, r3b))


def test_all_ignored_and_empty():
    lce = _lce()
    h, w, lab = make_case(256, 128, 1000, seed=11)
    lab_all = torch.full_like(lab, -100)
    loss, dh, dw = run_path(lce, h, w, lab_all, 1.0)
    eager = run_path(_eager, h, w, lab_all, 1.0)
    assert math.isnan(loss.item()) and math.isnan(eager[0].item())
    # an empty batch: NaN loss like the eager formula, zero weight gradient
    he = h.reshape(-1, 256)[:0]
    le = lab.reshape(-1)[:0]
    loss, dh, dw = run_path(lce, he, w, le, 1.0)
    assert math.isnan(loss.item()) and dh.shape == he.shape


def test_nan_inf_propagation():
    lce = _lce()
    D, N, V = 256, 512, 20011
    h, w, lab = make_case(D, N, V, seed=9)
    hn = h.clone()
    hn[0, 5, 3] = float("nan")
    rl = run_path(lce, hn, w, lab, 1 / 16)
    assert bool(torch.isnan(rl[0])) and bool(torch.isnan(rl[2]).any()) and bool(torch.isnan(rl[1][0, 5]).any())
    for col in (5, 2 * 8192 + 17, V - 1):
        wn = w.clone()
        wn[col, 7] = float("nan")
        rp = run_path(_eager, h, wn, lab, 1 / 16)
        rl = run_path(lce, h, wn, lab, 1 / 16)
        assert bool(torch.isnan(rl[0])) and bool(torch.isnan(rp[0])), col
    hi = h.clone()
    hi[0, 9, :] = float("inf")
    rl = run_path(lce, hi, w, lab, 1 / 16)
    assert not bool(torch.isfinite(rl[0]))


def test_validation_errors():
    lce = _lce()
    h = torch.randn(4, 8, 64, device=DEV, dtype=torch.bfloat16)
    w = torch.randn(100, 32, device=DEV)
    y = torch.zeros(4, 8, dtype=torch.int64, device=DEV)
    with pytest.raises(ValueError, match="weight"):
        lce(h, w, y)
    with pytest.raises(ValueError, match="labels"):
        lce(h, torch.randn(100, 64, device=DEV), y[:, :7])


def test_north_star_shape_properties():
    """The CE benchmark shape (16,384 tokens, d 768, V 50,277): loss within eager's rounding, ignored rows zero."""
    lce = _lce()
    c = R.config_inputs(3, device=DEV, dtype=torch.float32)
    h, w, lab = c["hidden"], c["weight"], c["labels"].clone()
    lab[::97] = -100
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        l_hip = lce(h, w, lab)
        l_eag = _eager(h, w, lab)
    torch.cuda.synchronize()
    assert abs(l_hip.item() - l_eag.item()) <= 1e-4 * abs(l_eag.item())
    assert abs(l_hip.item() - math.log(50277)) < 0.5     # near-uniform logits at init scale (std 0.55)
