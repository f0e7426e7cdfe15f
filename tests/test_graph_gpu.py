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
