"""GPU tests of the linear cross-entropy: the HIP row pass, the fused no-gradient forward and the gradient path.

Truths: oracle.lmce64 (fp64 math on the fp32 master inputs, and on the inputs rounded to the compute dtype as
autocast rounds them) and oracle.lmce_rows64 (the fp64 row pass on stored logits).

  * row pass (sisa_lmce_rows): lse and loss rows to fp32 accuracy; G within one unit in the last place of the
    compute dtype; pad columns and ignored rows exactly zero; NaN / inf / out-of-range labels as the reference.
  * fused forward (sisa_lmce_fwd, used when no gradient is wanted): loss rows and lse against the fp64 row pass of the
    fp64 logits of the rounded inputs, themselves rounded once to the compute dtype as the reference's logits are,
    |err| <= 2e-5 max(1, |lse|) plus what one-unit flips of logits within 3e-5 of a rounding midpoint can move (the
    kernel's fp32 accumulation order differs from fp64's); no logits buffer (the peak device memory of the call stays
    below the logits' size); labels, padding and NaN as above.
  * gradient path: loss, dL/dh and dL/dW against both fp64 truths, each no worse than 2 x the error of the eager
    autocast formula F.cross_entropy(F.linear(h, W).float(), y) + 1e-7 -- the acceptance rule of the reference's
    tests/test_linear_ce.py:106-121 (restated); chunking, grad_scale, dtypes, ignored rows, determinism.
"""
from __future__ import annotations

import math
from typing import NamedTuple

import pytest
import torch
import torch.nn.functional as F

from oracle import reference as R

pytestmark = pytest.mark.gpu
DEV = "cuda"


def lce_fn():
    from sisa_amd.kernels.linear_ce import linear_cross_entropy
    return linear_cross_entropy


def eager_fn(h, w, labels, ignore_index=-100):
    z = F.linear(h, w)
    return F.cross_entropy(z.reshape(-1, z.shape[-1]).float(), labels.reshape(-1), ignore_index=ignore_index)


def lm_head_case(N: int, D: int, V: int, seed: int, temp: float = 2.5, batch: int = 1):
    """Unit-rms hidden rows, a weight whose logits have standard deviation ``temp``, and labels that are the argmax
    of the fp32 logits with probability 1/2 (else uniform; uniform only for the largest cases) -- a loss neither near 0
    nor near ln V. Drawn on the CPU."""
    gen = torch.Generator().manual_seed(seed)
    h = torch.randn(N, D, generator=gen)
    h = h / h.pow(2).mean(1, keepdim=True).sqrt()
    w = torch.randn(V, D, generator=gen) * (temp / math.sqrt(D))
    rand = torch.randint(0, V, (N,), generator=gen)
    if N and N * V * D <= 6e10:   # the CPU argmax stays within seconds
        top = torch.cat([(h[r:r + 256] @ w.t()).argmax(1) for r in range(0, N, 256)])
    else:
        top = rand
    lab = torch.where(torch.rand(N, generator=gen) < 0.5, top, rand).to(torch.int64)
    return h.reshape(batch, N // batch, D).to(DEV), w.to(DEV), lab.reshape(batch, N // batch).to(DEV)


class Run(NamedTuple):
    loss: torch.Tensor
    dh: torch.Tensor | None
    dw: torch.Tensor | None


def train_pass(fn, h, w, labels, seed, *, autocast=torch.bfloat16, want=(True, True), **kw) -> Run:
    hh = h.detach().clone().requires_grad_(want[0])
    ww = w.detach().clone().requires_grad_(want[1])
    with torch.autocast("cuda", dtype=autocast or torch.bfloat16, enabled=autocast is not None):
        loss = fn(hh, ww, labels, **kw)
    (loss * seed).backward()
    torch.cuda.synchronize()
    return Run(loss.detach().float(), hh.grad, ww.grad)


def truths(h, w, labels, seed, ignore_index=-100, only_exact=False) -> dict:
    t = {"fp64": Run(*R.lmce64(h, w, labels, seed, quant=False, ignore_index=ignore_index))}
    if not only_exact:
        t["fp64_rounded_inputs"] = Run(*R.lmce64(h, w, labels, seed, quant=True, ignore_index=ignore_index))
    return t


def within_eager(runs: dict, eager: Run, refs: dict, slack: float = 1e-7) -> list:
    """Every tensor of every run within 2 x the eager formula's error (+ slack) against every truth."""
    bad = []
    for name, run in runs.items():
        for field in Run._fields:
            got = getattr(run, field)
            if got is None:
                continue
            for tname, truth in refs.items():
                e_run = R.rel(got, getattr(truth, field))
                e_eager = R.rel(getattr(eager, field), getattr(truth, field))
                if not e_run <= 2.0 * e_eager + slack:
                    bad.append(f"{name}.{field} vs {tname}: {e_run:.3e} > 2 x eager {e_eager:.3e}")
    return bad


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


# ------------------------------------------------------------------------------------------------ fused forward
def _fused_truth(x16: torch.Tensor, wpad: torch.Tensor, labels: torch.Tensor, V: int, ignore_index=-100,
                 tau: float = 3e-5):
    """fp64 lse and loss rows of the rounded inputs, from the fp64 logits rounded once to the compute dtype (the
    logits the reference's row kernel reads), in row chunks; and per row the rounding-flip allowance. The kernel rounds
    its fp32 accumulations, whose summation order differs from fp64's by about 1e-6: a logit lying within ``tau`` of a
    rounding midpoint may come out one unit away. The allowance is what such flips can move: sum p_v ulp_v over those
    logits for lse, plus the label logit's unit when the label logit is one of them (for the loss row)."""
    lses, losses, slack_lse, slack_row = [], [], [], []
    for r0 in range(0, x16.shape[0], 2048):
        z = x16[r0:r0 + 2048].double() @ wpad.double().t()
        zr = z.to(x16.dtype).double()
        lab = labels[r0:r0 + 2048]
        lse, loss, _ = R.lmce_rows64(zr, lab, V, ignore_index=ignore_index)
        u = R.ulp(z, x16.dtype)
        near = (0.5 * u - (z - zr).abs()) <= tau
        p = torch.softmax(zr[:, :V], 1)
        sl = (p * u[:, :V] * near[:, :V]).sum(1)
        idx = lab.clamp(0, z.shape[1] - 1).unsqueeze(1)
        lab_flip = (near.gather(1, idx) * u.gather(1, idx)).squeeze(1)
        lses.append(lse)
        losses.append(loss)
        slack_lse.append(sl)
        slack_row.append(sl + lab_flip)
    return torch.cat(lses), torch.cat(losses), torch.cat(slack_lse), torch.cat(slack_row)


def _fused_call(h, w, labels, dtype=torch.bfloat16, ignore_index=-100):
    from sisa_amd.kernels import linear_ce as LC
    x = h.reshape(-1, h.shape[-1]).to(dtype).contiguous()
    wpad = LC.padded_weight(w, dtype)
    lab = labels.reshape(-1).to(torch.int64).contiguous()
    lse = torch.empty(x.shape[0], device=DEV)
    rows = LC.lmce_fused_loss_rows(x, wpad, lab, w.shape[0], ignore_index, lse)
    torch.cuda.synchronize()
    return x, wpad, lab, lse, rows


@pytest.mark.parametrize("N,D,V,dtype", [(16384, 768, 50277, torch.bfloat16), (300, 512, 1003, torch.bfloat16),
                                         (1, 64, 65, torch.bfloat16), (129, 1024, 4099, torch.float16),
                                         (2000, 128, 256, torch.bfloat16), (77, 192, 50277, torch.float16)])
def test_fused_forward_vs_fp64(N, D, V, dtype):
    print(f"[fused] N={N} D={D} V={V} {dtype}", flush=True)
    h, w, lab = lm_head_case(N, D, V, seed=N + D + V)
    lab = lab.clone()
    lab.view(-1)[::13] = -100
    x, wpad, lab1, lse, rows = _fused_call(h, w, lab, dtype)
    lse_ref, loss_ref, flip_lse, flip_row = _fused_truth(x, wpad, lab1, V)
    tol = 2e-5 * lse_ref.abs().clamp_min(1.0) + flip_lse
    assert ((lse.double() - lse_ref).abs() <= tol).all(), float(((lse.double() - lse_ref).abs() / tol).max())
    tol_rows = 2e-5 * lse_ref.abs().clamp_min(1.0) + flip_row
    assert ((rows.double() - loss_ref).abs() <= tol_rows).all(), \
        float(((rows.double() - loss_ref).abs() / tol_rows).max())
    assert (rows[lab1 == -100] == 0).all()
    again = _fused_call(h, w, lab, dtype)
    assert torch.equal(again[4], rows) and torch.equal(again[3], lse)


def test_fused_forward_labels_and_nan():
    N, D, V = 40, 256, 5000
    h, w, lab = lm_head_case(N, D, V, seed=5)
    lab = lab.clone().view(-1)
    lab[3], lab[4], lab[5], lab[6] = V + 1, -7, 0, V - 1     # outside, negative (not ignored), both ends
    h = h.clone().view(-1, D)
    h[9, 11] = float("nan")
    w = w.clone()
    w[7, 3] = float("inf")                                   # one infinite weight: rows with h[:, 3] != 0 see +-inf
    _, _, lab1, lse, rows = _fused_call(h, w, lab)
    rc = rows.cpu()
    assert math.isnan(rc[3]) and math.isnan(rc[4]) and math.isnan(rc[9])
    assert not bool(torch.isfinite(lse).all())
    w2 = w.clone()
    w2[7, 3] = 0.0
    _, _, _, lse2, rows2 = _fused_call(h, w2, lab)
    fin = [r for r in range(N) if r not in (3, 4, 9)]
    assert bool(torch.isfinite(rows2[fin]).all()) and math.isfinite(rows2[5]) and math.isfinite(rows2[6])


def test_fused_forward_has_no_logits_buffer():
    """Config 3 without gradients: the call's peak device memory stays far below one logits chunk (1.65 GB)."""
    from sisa_amd.workloads import config_inputs
    lce = lce_fn()
    c = config_inputs(3, device=DEV)
    h, w, lab = c["hidden"], c["weight"], c["labels"]
    with torch.no_grad():
        lce(h, w.to(torch.bfloat16), lab)                      # warm-up (library handles, caches)
        torch.cuda.synchronize()
        base = torch.cuda.memory_allocated()
        torch.cuda.reset_peak_memory_stats()
        loss = lce(h, w.to(torch.bfloat16), lab)
        torch.cuda.synchronize()
    extra = torch.cuda.max_memory_allocated() - base
    logits_bytes = h.shape[0] * 50304 * 2
    assert extra < logits_bytes // 8, (extra, logits_bytes)
    assert math.isfinite(loss.item())


def test_fused_and_gradient_paths_agree():
    lce = lce_fn()
    h, w, lab = lm_head_case(1024, 512, 4099, seed=3)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        fused = lce(h, w, lab)
    grad = train_pass(lce, h, w, lab, 1.0).loss
    exact = truths(h, w, lab, 1.0, only_exact=True)["fp64"].loss
    # one logits GEMM and one reduction serve both paths: the same loss, bit for bit
    assert torch.equal(fused, grad)
    assert abs(fused.item() - exact.item()) < 1e-3 * abs(exact.item())


# ------------------------------------------------------------------------------------------------ gradient path
# the last case: a ragged row count, a hidden size that is not a multiple of 64 (zero columns added) and a vocabulary
# that is not a multiple of 128 (zero rows added)
@pytest.mark.parametrize("N,D,V,seed", [(2048, 512, 50277, 1 / 16), (1024, 768, 1003, 1 / 32),
                                        (4096, 1024, 50277, 1 / 64), (74, 200, 1000, 1 / 8)])
def test_gradients_vs_fp64(N, D, V, seed):
    print(f"[train] N={N} D={D} V={V}", flush=True)
    lce = lce_fn()
    h, w, lab = lm_head_case(N, D, V, seed=N + V, batch=2)
    refs = truths(h, w, lab, seed)
    eager = train_pass(eager_fn, h, w, lab, seed)
    runs = {"default": train_pass(lce, h, w, lab, seed),
            "chunks_of_300": train_pass(lce, h, w, lab, seed, chunk_tokens=300),
            "one_chunk": train_pass(lce, h, w, lab, seed, chunk_tokens=N),
            "grad_scale": train_pass(lce, h, w, lab, seed, grad_scale=seed)}
    bad = within_eager(runs, eager, refs)
    assert not bad, "\n".join(bad)


def test_gradient_path_semantics():
    lce = lce_fn()
    D, N, V = 512, 1024, 4099
    h, w, lab = lm_head_case(N, D, V, seed=7, batch=2)
    ign = lab.clone()
    ign.view(-1)[::17] = -100
    base = train_pass(lce, h, w, ign, 1 / 16)
    assert base.dh.reshape(-1, D)[ign.reshape(-1) == -100].abs().max().item() == 0.0
    assert not within_eager({"ignored": base}, train_pass(eager_fn, h, w, ign, 1 / 16), truths(h, w, ign, 1 / 16))
    # a seed that is not a power of two, with and without the promise
    refs = truths(h, w, lab, 0.3)
    eager = train_pass(eager_fn, h, w, lab, 0.3)
    assert not within_eager({"plain": train_pass(lce, h, w, lab, 0.3),
                             "promised": train_pass(lce, h, w, lab, 0.3, grad_scale=0.3)}, eager, refs)
    # one gradient only: bitwise the run with both
    both = train_pass(lce, h, w, lab, 1 / 16)
    only_h = train_pass(lce, h, w, lab, 1 / 16, want=(True, False))
    only_w = train_pass(lce, h, w, lab, 1 / 16, want=(False, True))
    assert only_h.dw is None and only_w.dh is None
    assert torch.equal(only_h.dh, both.dh) and torch.equal(only_w.dw, both.dw) and torch.equal(only_h.loss, both.loss)
    # 16-bit tensors without autocast keep their dtype
    hb, wb = h.to(torch.bfloat16), w.to(torch.bfloat16)
    r16 = train_pass(lce, hb, wb, lab, 1 / 16, autocast=None)
    e16 = train_pass(eager_fn, hb, wb, lab, 1 / 16, autocast=None)
    assert r16.dh.dtype == torch.bfloat16 and r16.dw.dtype == torch.bfloat16
    assert not within_eager({"bf16": r16}, e16, {"fp64": Run(*R.lmce64(hb.float(), wb.float(), lab, 1 / 16))})
    # fp16 autocast
    assert not within_eager({"fp16": train_pass(lce, h, w, lab, 1 / 16, autocast=torch.float16)},
                            train_pass(eager_fn, h, w, lab, 1 / 16, autocast=torch.float16),
                            truths(h, w, lab, 1 / 16, only_exact=True))
    # flat rows == batched rows; repeat bitwise
    flat = train_pass(lce, h.reshape(-1, D), w, lab.reshape(-1), 1 / 16)
    assert torch.equal(flat.loss, both.loss) and torch.equal(flat.dh, both.dh.reshape(-1, D))
    assert torch.equal(flat.dw, both.dw)
    again = train_pass(lce, h, w, lab, 1 / 16)
    assert all(torch.equal(a, b) for a, b in zip(again, both))


def test_all_ignored_and_empty():
    lce = lce_fn()
    h, w, lab = lm_head_case(128, 256, 1000, seed=11)
    none = torch.full_like(lab, -100)
    run = train_pass(lce, h, w, none, 1.0)
    assert math.isnan(run.loss.item()) and math.isnan(train_pass(eager_fn, h, w, none, 1.0).loss.item())
    he, le = h.reshape(-1, 256)[:0], lab.reshape(-1)[:0]
    run = train_pass(lce, he, w, le, 1.0)
    assert math.isnan(run.loss.item()) and run.dh.shape == he.shape and bool((run.dw == 0).all())
    with torch.no_grad():
        assert math.isnan(lce(he.to(torch.bfloat16), w.to(torch.bfloat16), le).item())


def test_nan_and_inf_reach_the_loss():
    lce = lce_fn()
    D, N, V = 256, 512, 20011
    h, w, lab = lm_head_case(N, D, V, seed=9)
    hn = h.clone()
    hn.view(-1, D)[5, 3] = float("nan")
    run = train_pass(lce, hn, w, lab, 1 / 16)
    assert math.isnan(run.loss.item()) and bool(torch.isnan(run.dw).any())
    for col in (5, 16401, V - 1):
        wn = w.clone()
        wn[col, 7] = float("nan")
        assert math.isnan(train_pass(lce, h, wn, lab, 1 / 16).loss.item()), col
        with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
            assert math.isnan(lce(h, wn, lab).item()), col
    hi = h.clone()
    hi.view(-1, D)[9, :] = float("inf")
    assert not math.isfinite(train_pass(lce, hi, w, lab, 1 / 16).loss.item())


def test_shape_errors():
    lce = lce_fn()
    h = torch.randn(4, 8, 64, device=DEV, dtype=torch.bfloat16)
    y = torch.zeros(4, 8, dtype=torch.int64, device=DEV)
    with pytest.raises(ValueError, match="weight"):
        lce(h, torch.randn(100, 32, device=DEV), y)
    with pytest.raises(ValueError, match="labels"):
        lce(h, torch.randn(100, 64, device=DEV), y[:, :7])
