"""GPU tests of the weight-gradient GEMM (sisa_wgrad) and the linear layer built on it, against float64 products of
the same 16-bit operands (the kernel accumulates exact bf16/fp16 products in fp32)."""
from __future__ import annotations

import pytest
import torch

from model_utils import rel_err

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("M,N,K,dtype,nsplit", [(16384, 768, 768, torch.bfloat16, None),
                                                (16384, 3280, 768, torch.bfloat16, None),
                                                (1000, 200, 72, torch.bfloat16, None),
                                                (1000, 200, 72, torch.bfloat16, 3),
                                                (64, 16, 8, torch.float16, 1),
                                                (4097, 768, 2744, torch.bfloat16, None),
                                                (333, 5488, 768, torch.float16, 2)])
def test_wgrad_kernel(M, N, K, dtype, nsplit):
    from sisa_amd.kernels.wgrad import wgrad_hip
    gen = torch.Generator().manual_seed(M + N + K)
    dy = torch.randn(M, N, generator=gen).to(dtype).to(DEV)
    x = torch.randn(M, K, generator=gen).to(dtype).to(DEV)
    got = wgrad_hip(dy, x, nsplit=nsplit)
    ref = dy.double().t() @ x.double()
    assert got.dtype == torch.float32 and got.shape == (N, K)
    assert rel_err(got, ref) < 2e-6
    assert torch.equal(wgrad_hip(dy, x, nsplit=nsplit), got)                  # deterministic


def test_wgrad_strided_rows():
    """Row-strided views (a column slice of a wider matrix) read only their own columns."""
    from sisa_amd.kernels.wgrad import wgrad_hip
    gen = torch.Generator().manual_seed(3)
    big = torch.randn(700, 400, generator=gen).to(torch.bfloat16).to(DEV)
    dy, x = big[:, 8:208], big[:, 240:312]
    got = wgrad_hip(dy, x)
    assert rel_err(got, dy.double().t() @ x.double()) < 2e-6


def test_linear_hip_matches_autograd():
    from sisa_amd.kernels.wgrad import linear_hip
    gen = torch.Generator().manual_seed(4)
    x = torch.randn(4, 300, 256, generator=gen).to(DEV).requires_grad_(True)
    w = (0.05 * torch.randn(384, 256, generator=gen)).to(DEV).requires_grad_(True)
    b = torch.randn(384, generator=gen).to(DEV).requires_grad_(True)
    dy = torch.randn(4, 300, 384, generator=gen).to(DEV)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = linear_hip(x, w, b)
    assert y.dtype == torch.bfloat16
    dx, dw, db = torch.autograd.grad(y, (x, w, b), dy)
    x16, w16 = x.detach().bfloat16().double(), w.detach().bfloat16().double()
    dy16 = dy.bfloat16().double()
    assert dx.dtype == torch.float32 and dw.dtype == torch.float32 and db.dtype == torch.float32
    assert rel_err(dw, dy16.reshape(-1, 384).t() @ x16.reshape(-1, 256)) < 2e-6
    assert rel_err(dx, dy16 @ w16) < 1e-2 and rel_err(db, dy16.sum((0, 1))) < 1e-6
    assert rel_err(y, x16 @ w16.t() + b.detach().bfloat16().double()) < 1e-2


def test_linear_hip_bias_columns():
    """With bias_cols only those bias entries get a gradient (the rest is constant padding); they match the full
    bias gradient."""
    from sisa_amd.kernels.wgrad import linear_hip
    gen = torch.Generator().manual_seed(5)
    x = torch.randn(2, 200, 128, generator=gen).to(DEV).bfloat16()
    w = (0.05 * torch.randn(256, 128, generator=gen)).to(DEV).requires_grad_(True)
    b = torch.randn(256, generator=gen).to(DEV).requires_grad_(True)
    dy = torch.randn(2, 200, 256, generator=gen).to(DEV)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        full = torch.autograd.grad(linear_hip(x, w, b), (b,), dy)[0]
        part = torch.autograd.grad(linear_hip(x, w, b, (40, 52)), (b,), dy)[0]
    assert torch.equal(part[40:52], full[40:52]) and not part[:40].any() and not part[52:].any()


def test_wgrad_row_ranges(monkeypatch):
    """Operands past the one-launch limit are reduced in row ranges and summed in range order: with the limit
    lowered to a few hundred rows the result matches one launch to fp32 summation order, and fp64 to 2e-6."""
    from sisa_amd.kernels import wgrad as W
    gen = torch.Generator().manual_seed(6)
    M, N, K = 1000, 320, 192
    dy = torch.randn(M, N, generator=gen).to(DEV).bfloat16()
    x = torch.randn(M, K, generator=gen).to(DEV).bfloat16()
    whole = W.wgrad_hip(dy, x)
    monkeypatch.setattr(W, "OPERAND_LIMIT", 256 * N * 2 + 1)     # 256 rows of dy per launch
    assert len(W.row_pieces(M, N, K)) == 4
    pieces = W.wgrad_hip(dy, x)
    ref = dy.double().t() @ x.double()
    assert rel_err(pieces, ref) < 2e-6 and rel_err(pieces, whole) < 2e-6
