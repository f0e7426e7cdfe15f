"""The allocation-free attention backward (sisa_attn_bwd_noalloc) against sisa_attn_bwd through the C ABI.

The no-alloc entry point keeps the backward's row buffers in the library's static device scratch and must give
bitwise the results of the entry point with a caller workspace, on consecutive calls whose scratch still holds the
previous call's contents (the second call smaller than the first). Sizes past the scratch limit and a non-null
workspace are rejected on the host before anything is launched.
"""
from __future__ import annotations

import ctypes

import pytest
import torch

from oracle import reference as R

pytestmark = pytest.mark.gpu
DEV = "cuda"
NOALLOC_MAX_BHL = 1 << 20        # SISA_NOALLOC_MAX_BHL of include/sisa_hip.h


def _backward(entry: str, ins: dict, exact: bool = True) -> list[torch.Tensor]:
    from sisa_amd.kernels import _lib
    from sisa_amd.kernels import attention as A

    q, k, v, c, b, g, lam, Fg = A.kernel_operands(*[ins[n] for n in R.IN_NAMES])
    o, lse, rowf, colf, o32 = A.attn_forward(q, k, v, c, b, g, lam, Fg, want32=exact)
    B, H, L, _ = q.shape
    do = ins["do"]
    dq, dk, dv, dc, db = (torch.full_like(x, float("nan")) for x in (q, k, v, c, b))
    dg = torch.full((B, H, L), float("nan"), device=DEV)
    dF = torch.full_like(dg, float("nan")) if Fg is not None else None
    dlam = torch.full((H,), float("nan"), device=DEV)
    ws = None
    if entry == "sisa_attn_bwd":
        ws = torch.empty(_lib.workspace_bytes("sisa_attn_bwd_workspace_bytes", B, H, L) // 4, device=DEV)
    args = _lib.AttnBwdArgs(B, H, L, _lib.dtype_code(q.dtype), _lib.dtype_code(dc.dtype), _lib.view(q), _lib.view(k),
                            _lib.view(v), _lib.view(c), _lib.view(b), _lib.view(g), _lib.view(Fg), lam.data_ptr(),
                            lam.stride(0), rowf.data_ptr(), colf.data_ptr(), _lib.view(o),
                            o32.data_ptr() if (exact and o32 is not None and o32 is not o) else None, lse.data_ptr(),
                            _lib.view(do), _lib.view(dq), _lib.view(dk), _lib.view(dv), _lib.view(dc), _lib.view(db),
                            dg.data_ptr(), _lib.ptr(dF), dlam.data_ptr(), _lib.ptr(ws), 1 if exact else 0)
    _lib.call(entry, args, q)
    torch.cuda.synchronize()
    return [t for t in (dq, dk, dv, dc, db, dg, dF, dlam) if t is not None]


# the last case fills the scratch to its last element: B*H*L = SISA_NOALLOC_MAX_BHL at L = 1, where the fp64 dlambda
# group sums (one per (batch, head, 16 rows)) are largest
@pytest.mark.parametrize("shapes", [((2, 8, 1500, 11), (1, 3, 200, 12)), ((1, 12, 4096, 13), (3, 2, 65, 14)),
                                    ((4096, 256, 1, 16), (1024, 64, 15, 17))])
def test_noalloc_matches_workspace_entry(shapes):
    from sisa_amd.kernels import _lib

    _lib.load()
    for B, H, L, seed in shapes:        # the second call is smaller: the scratch holds the first call's rows
        print(f"[noalloc] B={B} H={H} L={L} seed={seed}", flush=True)
        assert B * H * L <= NOALLOC_MAX_BHL
        heads = [R.MIX12[h % 12] for h in range(H)]     # the judge's head mix, repeated past 12 heads
        ins = R.make_attention_inputs(dict(B=B, H=H, L=L, dtype="bf16", seed=seed, heads=heads), DEV)
        got = _backward("sisa_attn_bwd_noalloc", ins)
        ref = _backward("sisa_attn_bwd", ins)
        names = ("dq", "dk", "dv", "dc", "db", "dg", "dF", "dlam")
        bad = [n for n, x, y in zip(names, got, ref) if not torch.equal(x, y)]
        assert not bad, f"B={B} H={H} L={L}: {bad} differ from sisa_attn_bwd"
        assert all(bool(torch.isfinite(x).all()) for x in got)


def test_noalloc_fa_mode_matches():
    ins = R.make_attention_inputs(dict(B=1, H=4, L=333, dtype="fp16", seed=15), DEV)
    got = _backward("sisa_attn_bwd_noalloc", ins, exact=False)
    ref = _backward("sisa_attn_bwd", ins, exact=False)
    assert all(torch.equal(x, y) for x, y in zip(got, ref))


def test_noalloc_rejections_on_the_host():
    from sisa_amd.kernels import _lib

    lib = _lib.load()
    args = _lib.AttnBwdArgs()
    args.B, args.H, args.L = 1, 1, NOALLOC_MAX_BHL + 1
    assert lib.sisa_attn_bwd_noalloc(ctypes.byref(args), None) == 1
    assert "SISA_NOALLOC_MAX_BHL" in lib.sisa_last_error().decode()
    args.L = 64
    args.workspace = 16
    assert lib.sisa_attn_bwd_noalloc(ctypes.byref(args), None) == 1
    assert "workspace must be NULL" in lib.sisa_last_error().decode()
