"""HIP-graph capture of the fused SISA layer step (the bench's timed step): prep forward, attention forward, exact-delta
attention backward and prep backward captured once, replayed several times with eager work and synchronisations
between the replays; every replay must reproduce the eager results bit for bit (the kernels are deterministic and
allocate nothing themselves; the graph's allocations come from its private pool)."""
from __future__ import annotations

import pytest
import torch

from oracle import reference as R

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _step(proj, z, lam, dy, H):
    from sisa_amd.kernels import attention as A
    from sisa_amd.kernels import fused_prep as FP
    B, L, _ = proj.shape
    off = FP.fused_layout(H)

    def col(t, name, w=64):
        return t[..., off[name]:off[name] + H * w].view(B, L, H, w).transpose(1, 2)

    pf = FP.prep_forward(proj, z, H)
    q, k, v = col(proj, "Q"), col(proj, "K"), col(proj, "V")
    c, b = pf.state_views()
    o, lse, _, _, o32 = A.attn_forward(q, k, v, c, b, pf.g, lam, pf.f, factors=(pf.rowf, pf.colf), want32=True)
    DP = torch.empty_like(proj)
    DCR = torch.empty((B, L, H, 32), device=proj.device, dtype=torch.float32)
    DBR = torch.empty_like(DCR)
    do = dy.reshape(B, L, H, 64).transpose(1, 2)
    _, _, _, _, _, dg, dlam, dF = A.attn_backward(q, k, v, c, b, pf.g, pf.f, pf.rowf, pf.colf, lam, o,
                                                  lse, do, True, dq=col(DP, "Q"), dk=col(DP, "K"), dv=col(DP, "V"),
                                                  dc=DCR.transpose(1, 2), db=DBR.transpose(1, 2), o32=o32)
    DZ = FP.prep_backward(proj, z, pf.totals, dg, dF, DCR, DBR, DP, H)
    return o, DP, dlam, DZ


@pytest.mark.parametrize("B,L,H", [(1, 1000, 4), (4, 2048, 8)])   # (4, 2048, 8): config 1
def test_layer_step_graph_replays(B, L, H):
    from sisa_amd import backends
    print(f"[graph] B={B} L={L} H={H}", flush=True)
    prev = backends.get_check_mode()
    backends.set_check_mode("off")
    try:
        proj, z, _ = R.make_proj(B, L, H, seed=31, device=DEV)
        proj2, z2, _ = R.make_proj(B, L, H, seed=32, device=DEV)
        lam = torch.tensor([0.31, 3.0, 1e-7, 0.8, 0.31, 0.3, 0.29, 0.31][:H], device=DEV)
        dy = torch.randn(B, L, H * 64, generator=torch.Generator().manual_seed(33)).to(DEV).to(torch.bfloat16)
        eager = [t.clone() for t in _step(proj, z, lam, dy, H)]
        cur = torch.cuda.current_stream()
        side = torch.cuda.Stream()
        side.wait_stream(cur)
        with torch.cuda.stream(side):
            _step(proj, z, lam, dy, H)
        cur.wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            outs = _step(proj, z, lam, dy, H)
        for rep in range(3):
            _step(proj2, z2, lam, dy, H)        # eager work between the replays
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            names = ("o", "dproj", "dlam", "dz")
            bad = [n for n, a, e in zip(names, outs, eager) if not torch.equal(a, e)]
            assert not bad, f"replay {rep}: {bad} differ from the eager step"
    finally:
        backends.set_check_mode(prev)


def _block_step(x, res, w, wf, bf, a_b, dy, dz, dh):
    """The decoder block's HIP kernels with their backward: the attention norm with the fp32 forget projection (the
    matrix-core forward and backward at these shapes, with the weight-gradient reductions), the same behind the
    residual add, the plain residual add + FFN norm, and the SwiGLU activation on interleaved gate/up chunks."""
    from sisa_amd.kernels.norm import rms_norm_add_hip, rms_norm_forget_add_hip, rms_norm_forget_hip, swiglu_pairs_hip
    y, z = rms_norm_forget_hip(x, w, 1e-6, wf, bf, torch.bfloat16)
    gx, gw, gwf, gbf = torch.autograd.grad((y, z), (x, w, wf, bf), (dy, dz))
    h1, y1, z1 = rms_norm_forget_add_hip(x, res, w, 1e-6, wf, bf, torch.bfloat16)
    gx1, gres1, gw1, gwf1 = torch.autograd.grad((h1, y1, z1), (x, res, w, wf), (dh, dy, dz))
    h, m = rms_norm_add_hip(x, res, w, 1e-6, torch.bfloat16)
    gx2, gres, gw2 = torch.autograd.grad((h, m), (x, res, w), (dh, dy))
    act = swiglu_pairs_hip(a_b)
    (gab,) = torch.autograd.grad(act, (a_b,), dy[:, :act.shape[1]].contiguous())
    return (y, z, gx, gw, gwf, gbf, h1, y1, z1, gx1, gres1, gw1, gwf1, h, m, gx2, gres, gw2, act, gab)


# torch.autograd.grad accumulates into no leaf here; the leaves' accumulation nodes merely outlive the eager calls
@pytest.mark.filterwarnings("ignore:The AccumulateGrad node's stream does not match")
def test_block_kernels_graph_replays():
    """The decoder-block kernels captured once and replayed with eager work between the replays: every replay
    reproduces the eager results bit for bit."""
    print("[graph] decoder block N=1000 D=768 H=12", flush=True)
    gen = torch.Generator().manual_seed(41)
    N, D, H, FF = 1000, 768, 12, 384

    def inputs(seed):
        g = torch.Generator().manual_seed(seed)
        x = (2 * torch.randn(N, D, generator=g)).to(DEV).requires_grad_(True)
        res = torch.randn(N, D, generator=g).to(DEV).to(torch.bfloat16).requires_grad_(True)
        a_b = torch.randn(N, 2 * FF, generator=g).to(DEV).to(torch.bfloat16).requires_grad_(True)
        return x, res, a_b

    w = (1 + 0.1 * torch.randn(D, generator=gen)).to(DEV).requires_grad_(True)
    wf = (0.05 * torch.randn(H, D, generator=gen)).to(DEV).requires_grad_(True)
    bf = torch.randn(H, generator=gen).to(DEV).requires_grad_(True)
    dy = torch.randn(N, D, generator=gen).to(DEV).to(torch.bfloat16)
    dz = torch.randn(N, H, generator=gen).to(DEV)
    dh = torch.randn(N, D, generator=gen).to(DEV)
    x, res, a_b = inputs(1)
    x2, res2, a_b2 = inputs(2)
    eager = [t.detach().clone() for t in _block_step(x, res, w, wf, bf, a_b, dy, dz, dh)]
    cur = torch.cuda.current_stream()
    side = torch.cuda.Stream()
    side.wait_stream(cur)
    with torch.cuda.stream(side):
        _block_step(x, res, w, wf, bf, a_b, dy, dz, dh)
    cur.wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = _block_step(x, res, w, wf, bf, a_b, dy, dz, dh)
    for rep in range(3):
        _block_step(x2, res2, w, wf, bf, a_b2, dy, dz, dh)       # eager work between the replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        bad = [i for i, (a, e) in enumerate(zip(outs, eager)) if not torch.equal(a, e)]
        assert not bad, f"replay {rep}: outputs {bad} differ from the eager step"
