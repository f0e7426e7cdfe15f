"""Strong-forgetting and diagonal judge of the HIP attention backward (the reference's test_attention_diag.py gates).

Why: on heads that forget strongly (forget increments of -14 nats per token and below) P_tt -> 1 and the diagonal
dS_tt = P_tt (dP_tt - Delta_t) is a tiny true value computed as the difference of two O(|dP|) numbers; below about
-30 nats per token P_tt is 1.0 even in fp64, so fp64 autograd carries that noise too. The exact-delta backward
(self-normalised fp32 o'', delta-free dS_tt) exists for this regime, and this file judges it there.

Truth: oracle.analytic_grads64, the delta-free fp64 formula, pinned on the CPU against a 60-digit mpmath evaluation
of the direct formula at -3 .. -60 nats per token and against fp64 autograd at mild forgetting (tests/test_oracle.py).

Gates, per head and tensor, rel = ||X - REF|| / ||REF|| (reference tests/test_attention_diag.py:17-27, 320-352):
  * o, dq, dk, dv, dc, db: rel <= 3 ideal + 1e-6 (fp32 inputs: + 5e-6), ideal = rel of REF rounded to the output
    dtype, or rel <= 0.5 x the FlashAttention-standard mode of the same kernels (exact=False);
  * dg, dF, d log(decay) = revcumsum(dg), d log(forget) = revcumsum(dF): <= 3e-5;
    dlambda: <= max(3e-5, 1e-6 cond), cond = sum over rows |row part| / |dlambda|;
    where an fp32 dense emulation without intermediate rounding is given (the sharp heads), also <= 3 x its error;
  * comparison: the scalar gradients of the exact mode <= 1.5 x those of the FA-standard mode + 1e-5;
  * truths below the fp32 normal range (||REF|| < 1e-30) are judged by |X - REF| <= 1e-30 sqrt(n).
"""
from __future__ import annotations

import math

import pytest
import torch

from oracle import reference as R

pytestmark = pytest.mark.gpu
DEV = "cuda"
VECS = ("o", "dq", "dk", "dv", "dc", "db")
SCALARS = ("dg", "dF", "dloga", "dlogf", "dlam")
DTYPES = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}
SWEEP = [-1.0, -5.0, -10.0, -14.0, -17.0, -20.0, -25.0, -30.0, -40.0, -60.0]


def with_logs(d: dict) -> dict:
    d["dloga"] = R.revcumsum(d["dg"])
    d["dlogf"] = R.revcumsum(d["dF"]) if d.get("dF") is not None else None
    return d


def truth(ins: dict) -> dict:
    """Delta-free fp64 gradients, one (b, h) at a time on the GPU."""
    B, H, L, _ = ins["q"].shape
    acc = {n: [[None] * H for _ in range(B)] for n in ("o", "dq", "dk", "dv", "dc", "db", "dg", "dF")}
    dlam = torch.zeros(H, dtype=torch.float64, device=DEV)
    cond_num = torch.zeros(H, dtype=torch.float64, device=DEV)
    for bb in range(B):
        for h in range(H):
            r = R.analytic_grads64(*[ins[n][bb, h].double() for n in ("q", "k", "v", "c", "b", "g")],
                                   ins["lam"][h].double(), None if ins["F"] is None else ins["F"][bb, h].double(),
                                   ins["do"][bb, h].double())
            for n in acc:
                acc[n][bb][h] = r[n]
            dlam[h] += r["dlam"]
            cond_num[h] += r["dlam_abs"]
    out = {n: (None if acc[n][0][0] is None else torch.stack([torch.stack(row) for row in acc[n]])) for n in acc}
    out["dlam"] = dlam
    out["dlam_abs"] = cond_num
    return with_logs(out)


def run(ins: dict, exact: bool) -> dict:
    from sisa_amd.kernels import attention as A

    leaves = {n: ins[n].detach().clone().requires_grad_(True) for n in ("q", "k", "v", "c", "b", "g", "lam")}
    Fx = ins["F"].detach().clone().requires_grad_(True) if ins["F"] is not None else None
    args = [leaves[n] for n in ("q", "k", "v", "c", "b", "g", "lam")] + [Fx]
    if exact:
        o = A.sisa_attention_hip(*args)
    else:
        o = A._SISAAttentionFn.apply(*A.kernel_operands(*args), False)
    o.backward(ins["do"])
    torch.cuda.synchronize()
    d = {"o": o.detach(), "dlam": leaves["lam"].grad, "dF": None if Fx is None else Fx.grad}
    d.update({"d" + n: leaves[n].grad for n in ("q", "k", "v", "c", "b", "g")})
    return with_logs(d)


def head_slice(x: torch.Tensor, name: str, h: int) -> torch.Tensor:
    return x[h:h + 1] if name == "dlam" else x[:, h]


def rel_err(x: torch.Tensor | None, ref: torch.Tensor | None) -> float | None:
    if x is None or ref is None:
        return None
    x, ref = x.double(), ref.double()
    if not bool(torch.isfinite(x).all()):
        return math.inf
    n = ref.norm().item()
    e = (x - ref).norm().item()
    return e / (1e-30 * math.sqrt(ref.numel())) if n < 1e-30 else e / n


def judge(tag: str, ins: dict, dt: torch.dtype, compare: bool = True, floor32: dict | None = None) -> list[str]:
    ref = truth(ins)
    got = run(ins, exact=True)
    fa = run(ins, exact=False)
    H = ins["q"].shape[1]
    fails = []
    for h in range(H):
        bad = []
        for n in VECS:
            r = head_slice(ref[n], n, h)
            e = rel_err(head_slice(got[n], n, h), r)
            e_fa = rel_err(head_slice(fa[n], n, h), r)
            odt = ins["c"].dtype if n in ("dc", "db") else dt
            ideal = rel_err(r.to(odt), r)
            tol = 3 * ideal + (5e-6 if dt == torch.float32 else 1e-6)
            if not (e <= tol or e <= 0.5 * e_fa):
                bad.append(f"{n} {e:.2e} > {tol:.2e} (ideal {ideal:.1e}) and > 0.5 FA ({e_fa:.1e})")
        cond = (ref["dlam_abs"][h] / ref["dlam"][h].abs().clamp_min(1e-300)).item()
        for n in SCALARS:
            if ref.get(n) is None:
                continue
            r = head_slice(ref[n], n, h)
            e = rel_err(head_slice(got[n], n, h), r)
            tol = max(3e-5, 1e-6 * cond) if n == "dlam" else 3e-5
            if floor32 is not None and floor32.get(n) is not None:
                tol = max(tol, 3 * rel_err(head_slice(floor32[n], n, h), r))
            if not e <= tol:
                bad.append(f"{n} {e:.2e} > {tol:.1e}" + (f" (cond {cond:.0f})" if n == "dlam" else ""))
            if compare:
                e_fa = rel_err(head_slice(fa[n], n, h), r)
                if not e <= 1.5 * e_fa + 1e-5:
                    bad.append(f"{n} {e:.2e} > 1.5 FA ({e_fa:.2e}) + 1e-5")
        if bad:
            fails.append(f"{tag} head {h}: " + "; ".join(bad))
    return fails


def check(tag, ins, dt, compare=True, emulate=False):
    print(f"[diag] {tag} B,H,L={tuple(ins['q'].shape[:3])} {dt}", flush=True)
    floor32 = with_logs(R.fa_emulation(ins, "ideal")) if emulate else None
    fails = judge(tag, ins, dt, compare, floor32)
    torch.cuda.empty_cache()
    assert not fails, "\n".join(fails)


@pytest.mark.parametrize("dtn", ["bf16", "fp16", "fp32"])
def test_forgetting_sweep(dtn):
    """One mean forget increment per head from -1 to -60 nats per token (+- 2 N(0,1)), L = 1024, lam = 0.31."""
    dt = DTYPES[dtn]
    ins = R.diag_inputs(1, len(SWEEP), 1024, seed=5, dt=dt, forget=SWEEP, lam=0.31, device=DEV)
    check(f"sweep_{dtn}", ins, dt)


def test_forgetting_sweep_lams_model_layout():
    ins = R.diag_inputs(1, 4, 2048, seed=9, forget=[-14.0, -20.0, -25.0, -20.0], lam=[0.31, 3.0, 0.0, 0.8],
                        layout="blhd", device=DEV)
    check("sweep_lams_blhd_L2048", ins, torch.bfloat16)


def test_local_qk_diagonal():
    """No forget term; the diagonal dominated by q.k (k = 6 q)."""
    ins = R.diag_inputs(1, 2, 1024, seed=11, forget=None, lam=[0.31, 0.0], k_of_q=6.0, device=DEV)
    check("local_qk", ins, torch.bfloat16)


def test_local_cb_diagonal_fast_decay():
    """No forget term; the diagonal dominated by the side term (b = 8 c, fast decay, lam = 3)."""
    ins = R.diag_inputs(1, 2, 1024, seed=12, forget=None, lam=[3.0, 1.0], b_of_c=8.0, decay="fast", device=DEV)
    check("local_cb_fast", ins, torch.bfloat16)


def test_local_forget_large_lambda_fast_decay():
    ins = R.diag_inputs(1, 3, 1024, seed=13, forget=[-20.0, -10.0, -30.0], lam=[3.0, 3.0, 3.0], decay="fast",
                        device=DEV)
    check("local_forget_lam3_fast", ins, torch.bfloat16)


@pytest.mark.parametrize("L", [1, 2, 63, 64, 65, 129, 4096])
def test_edge_lengths(L):
    """-20 and -3 nats per token, B = 2, model layout; L <= 2 has no off-diagonal mass to compare against."""
    ins = R.diag_inputs(2, 2, L, seed=20 + L, forget=[-20.0, -3.0], lam=[0.31, 3.0], layout="blhd", device=DEV)
    check(f"edge_L{L}", ins, torch.bfloat16, compare=L > 2)


@pytest.mark.parametrize("sharp", [1.0, 1.5, 2.0, 2.5, 3.0])
def test_sharp_previous_token(sharp):
    """One dominant off-diagonal entry (previous-token head: k_j = s q_{j+1}, median P_max 0.81 .. 0.999999): the
    precision of delta decides the vector gradients. The fp32 emulation gives the scalar-chain floor."""
    ins = R.diag_inputs(1, 2, 1024, seed=41, forget=[-0.05, -0.05], lam=[0.31, 3.0], device=DEV)
    q = ins["q"].float()
    k = torch.empty_like(q)
    k[:, :, :-1] = sharp * q[:, :, 1:]
    k[:, :, -1] = q[:, :, -1]
    ins["k"] = k.to(torch.bfloat16).contiguous()
    check(f"sharp_prev_s{sharp:g}", ins, torch.bfloat16, emulate=True)
