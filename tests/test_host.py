"""CPU tests of the boundary and the host side: the C-ABI library loads and exports every function that
include/sisa_hip.h declares, the ctypes mirrors have the C layout (checked against gcc's offsetof), argument checks of
the entry points return errors without touching a GPU, and the Python API that mirrors the reference (backends,
functional, modeling, linear CE, fused layout) behaves as the reference's on the CPU. No kernel runs here.
"""
from __future__ import annotations

import ctypes
import math
import os
import re
import subprocess
import sys

import pytest
import torch

from oracle import reference as R

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "sisa_hip.h")


@pytest.fixture(scope="session")
def lib():
    from sisa_amd.kernels import _lib
    if not os.path.exists(_lib.LIB_PATH):
        from sisa_amd import build
        build.build()
    return _lib.load()


def _header_functions():
    src = open(HEADER).read()
    return set(re.findall(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\*?\s*(sisa_\w+)\s*\(", src, re.M))


# ------------------------------------------------------------------------------------------------ C ABI
def test_library_exports_every_header_function(lib):
    from sisa_amd.kernels import _lib
    declared = _header_functions()
    assert len(declared) == 30
    assert declared == set(_lib.SIGNATURES), declared ^ set(_lib.SIGNATURES)
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True, check=True)
    exported = set(re.findall(r"\bT (sisa_\w+)$", out.stdout, re.M))
    assert declared <= exported, declared - exported
    assert lib.sisa_abi_version() == _lib.ABI_VERSION


def test_struct_layout_matches_c(tmp_path):
    """Every ctypes Structure mirrors its C struct: same size and field offsets (gcc on the real header)."""
    from sisa_amd.kernels import _lib
    pairs = {"View": "sisa_view", "FactorsArgs": "sisa_factors_args", "AttnFwdArgs": "sisa_attn_fwd_args",
             "AttnBwdArgs": "sisa_attn_bwd_args", "PrepFwdArgs": "sisa_prep_fwd_args",
             "PrepBwdArgs": "sisa_prep_bwd_args", "LmceRowsArgs": "sisa_lmce_rows_args",
             "RmsNormArgs": "sisa_rmsnorm_args", "NormArgs": "sisa_norm_args", "SwigluArgs": "sisa_swiglu_args",
             "DecodeArgs": "sisa_decode_args", "WgradArgs": "sisa_wgrad_args", "LmceFwdArgs": "sisa_lmce_fwd_args",
             "Round16Args": "sisa_round16_args", "LmceTrainArgs": "sisa_lmce_train_args"}
    lines = ["#include <stdio.h>", "#include <stddef.h>", '#include "sisa_hip.h"', "int main(void) {"]
    expect = []
    for py, c in pairs.items():
        cls = getattr(_lib, py)
        lines.append(f'printf("%zu\\n", sizeof({c}));')
        expect.append(ctypes.sizeof(cls))
        for name, _ in cls._fields_:
            lines.append(f'printf("%zu\\n", offsetof({c}, {name}));')
            expect.append(getattr(cls, name).offset)
    lines += ["return 0;", "}"]
    (tmp_path / "layout.c").write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", "-I", os.path.join(ROOT, "include"), str(tmp_path / "layout.c"), "-o",
                    str(exe)], check=True)
    got = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    assert got == expect


def test_entry_points_reject_bad_arguments_without_a_gpu(lib):
    from sisa_amd.kernels import _lib
    # null argument structs
    for name in ("sisa_attn_fwd", "sisa_attn_bwd", "sisa_prep_fwd", "sisa_prep_bwd", "sisa_lmce_rows",
                 "sisa_factors", "sisa_rmsnorm_fwd", "sisa_rmsnorm_bwd", "sisa_norm_fwd", "sisa_norm_bwd",
                 "sisa_swiglu_fwd", "sisa_swiglu_bwd", "sisa_decode_attn", "sisa_wgrad"):
        rc = getattr(lib, name)(None, None)
        assert rc != 0, name
        assert lib.sisa_last_error().decode().startswith(name), name
    # unsupported head size / dtype / misaligned views are refused before any launch
    a = _lib.AttnFwdArgs()
    a.B, a.H, a.L, a.dtype = 1, 1, 64, 7
    assert lib.sisa_attn_fwd(ctypes.byref(a), None) != 0
    assert "dtype" in lib.sisa_last_error().decode()
    r = _lib.LmceRowsArgs(4, 65, 64, 64, _lib.BF16, 0, 16, 16, -100, None, 1.0, 16, None)
    assert lib.sisa_lmce_rows(ctypes.byref(r), None) != 0 and "V <= Vp" in lib.sisa_last_error().decode()
    r = _lib.LmceRowsArgs(4, 60, 64, 64, _lib.BF16, 0, 8, 16, -100, None, 1.0, 16, None)
    assert lib.sisa_lmce_rows(ctypes.byref(r), None) != 0 and "aligned" in lib.sisa_last_error().decode()
    r = _lib.LmceRowsArgs(0, 60, 64, 64, _lib.BF16, 0, None, None, -100, None, 1.0, None, None)
    assert lib.sisa_lmce_rows(ctypes.byref(r), None) == 0              # zero rows: nothing to do


def test_decoder_block_entry_points_reject_bad_arguments(lib):
    from sisa_amd.kernels import _lib
    r = _lib.RmsNormArgs(4, 100, _lib.BF16, 1e-6, 16, 104, 16, 16, 104, None, None, 0, None, 0, None, None)
    assert lib.sisa_rmsnorm_fwd(ctypes.byref(r), None) != 0 and "multiple of 8" in lib.sisa_last_error().decode()
    r = _lib.RmsNormArgs(4, 8192, _lib.BF16, 1e-6, 16, 8192, 16, 16, 8192, None, None, 0, None, 0, None, None)
    assert lib.sisa_rmsnorm_fwd(ctypes.byref(r), None) != 0 and "4096" in lib.sisa_last_error().decode()
    r = _lib.RmsNormArgs(0, 64, _lib.BF16, 1e-6, 16, 64, 16, 16, 64, None, None, 0, None, 0, None, None)
    assert lib.sisa_rmsnorm_fwd(ctypes.byref(r), None) == 0               # zero rows: nothing to do
    # fused norm + projection: width, dtype pair and the projection operands are checked before any launch
    def norm(N=4, D=64, H=12, xd=_lib.F32, yd=_lib.BF16, wf=16, bf=16, z=16):
        return _lib.NormArgs(N, D, H, xd, yd, 1e-6, 0, 16, D, 16, wf, bf, 16, D, 16, z)
    for args, msg in ((norm(H=65), "[0, 64]"), (norm(xd=_lib.BF16, yd=_lib.F32), "dtype pair"),
                      (norm(wf=None), "needs wf"), (norm(z=None), "needs z"), (norm(D=4100), "multiple of 8")):
        assert lib.sisa_norm_fwd(ctypes.byref(args), None) != 0 and msg in lib.sisa_last_error().decode(), msg
    assert lib.sisa_norm_fwd(ctypes.byref(norm(N=0)), None) == 0
    bwd = norm()
    assert lib.sisa_norm_bwd(ctypes.byref(bwd), None) != 0 and "workspace" in lib.sisa_last_error().decode()
    s = _lib.SwigluArgs(12, _lib.BF16, 0, 16, 16, 16, None, None, None)
    assert lib.sisa_swiglu_fwd(ctypes.byref(s), None) != 0 and "multiple of 8" in lib.sisa_last_error().decode()
    s = _lib.SwigluArgs(16, _lib.BF16, 0, 16, 16, None, None, None, None)
    assert lib.sisa_swiglu_fwd(ctypes.byref(s), None) != 0 and "h must be given" in lib.sisa_last_error().decode()
    s = _lib.SwigluArgs(16, _lib.BF16, 2, 16, 16, 16, None, None, None)
    assert lib.sisa_swiglu_fwd(ctypes.byref(s), None) != 0 and "pairs" in lib.sisa_last_error().decode()
    s = _lib.SwigluArgs(0, _lib.BF16, 0, 16, 16, 16, None, None, None)
    assert lib.sisa_swiglu_fwd(ctypes.byref(s), None) == 0


def test_workspace_sizes(lib):
    B, H, L = 2, 3, 1000
    # five fp32 (B,H,L) row buffers and the fp64 dlambda sums of 16-row groups (B*H*L even: no alignment pad)
    assert lib.sisa_attn_bwd_workspace_bytes(B, H, L) == 5 * 4 * B * H * L + 8 * B * H * -(-L // 16)
    # prep backward exchange: a 256-byte header, then per (batch row, group of 4 heads, 64-row chunk) 72 fp64 totals
    # of two 8-byte words each
    words = B * -(-H // 4) * -(-L // 64) * 72
    assert lib.sisa_prep_bwd_workspace_bytes(B, L, H) == 256 + 16 * words
    assert lib.sisa_prep_bwd_workspace_bytes(0, L, H) == 0
    assert lib.sisa_rmsnorm_bwd_workspace_bytes(16384, 768) >= (16384 // 8 + 64) * 768 * 4
    assert lib.sisa_norm_bwd_workspace_bytes(16384, 768, 12) >= (16384 // 8 + 64 + 64 * 16) * 768 * 4


def test_missing_library_fails_loudly(monkeypatch):
    from sisa_amd.kernels import _lib
    monkeypatch.setattr(_lib, "_LIB", None)
    monkeypatch.setattr(_lib, "LIB_PATH", "/nonexistent/libsisa_hip.so")
    with pytest.raises(RuntimeError, match="not built"):
        _lib.load()


# ------------------------------------------------------------------------------------------------ backends
def test_backend_selection_on_cpu():
    from sisa_amd import SISAConfig, backends
    x = torch.zeros(1, 4, 512)
    cfg = SISAConfig.preset("sisa-50m")
    assert backends.select_impl("auto", x, cfg) == "torch"
    assert backends.select_impl("torch", x, cfg) == "torch"
    for forced in ("hip", "hip_fused"):
        with pytest.raises(ValueError, match="not available"):
            backends.select_impl(forced, x, cfg)
    with pytest.raises(ValueError):
        backends.select_impl("triton", x, cfg)
    ok, why = backends.hip_status()
    assert why and (ok is False or torch.cuda.is_available())
    assert not backends.fused_eligible(x)
    assert "check mode" in backends.describe()
    assert backends.attention_config(None, torch.bfloat16)["mfma"].endswith("bf16")


def test_check_mode():
    from sisa_amd import backends
    old = backends.get_check_mode()
    try:
        for m in ("sync", "off", "async"):
            backends.set_check_mode(m)
            assert backends.get_check_mode() == m
        with pytest.raises(ValueError):
            backends.set_check_mode("loud")
    finally:
        backends.set_check_mode(old)


# ------------------------------------------------------------------------------------------------ torch paths
@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("with_f", [True, False])
def test_sisa_attention_torch_matches_oracle(dtype, with_f):
    from sisa_amd.functional import sisa_attention
    ins = R.make_attention_inputs(dict(B=2, H=4, L=77, dtype="fp32", seed=3))
    args = [ins[n].to(dtype) for n in ("q", "k", "v", "c", "b")]
    Fg = ins["F"] if with_f else None
    o = sisa_attention(*args, ins["g"], ins["lam"], Fg, impl="torch", block_q=32)
    ref = R.dense_attention(*(a.double() for a in args), ins["g"].double(), ins["lam"].double(),
                            None if Fg is None else Fg.double())
    assert o.dtype == dtype
    assert R.rel(o, ref) < (1e-12 if dtype == torch.float64 else 1e-5)
    with pytest.raises(ValueError, match="not available"):
        sisa_attention(*args, ins["g"], ins["lam"], Fg, impl="hip")
    with pytest.raises(ValueError):
        sisa_attention(*args, ins["g"], ins["lam"], Fg, impl="hip_fused")


def test_sisa_attention_torch_gradients():
    from sisa_amd.functional import sisa_attention_torch
    ins = R.make_attention_inputs(dict(B=1, H=4, L=40, dtype="fp32", seed=4))
    X = {n: ins[n].double().requires_grad_(True) for n in R.IN_NAMES}
    o = sisa_attention_torch(*(X[n] for n in R.IN_NAMES), block_q=16)
    gs = torch.autograd.grad(o, [X[n] for n in R.IN_NAMES], ins["do"].double())
    T = R.truth64({**{n: ins[n] for n in R.IN_NAMES}, "do": ins["do"]})
    for gn, gv in zip(R.GRAD_NAMES, gs):
        assert R.rel(gv, T[gn]) < 1e-10, gn


def test_sisa_attention_layer_torch_path():
    from sisa_amd import SISAAttention, SISAConfig
    torch.manual_seed(0)
    cfg = SISAConfig(d_model=128, n_layer=1, n_head=2, d_ff=256, attn_impl="auto", zero_init_c=False)
    layer = SISAAttention(cfg).double()
    x = torch.randn(2, 33, 128, dtype=torch.float64)
    y = layer(x)
    # composition through the oracle: projections, glue (modeling.py:171-199) and dense attention
    h, dh, s = 2, 64, cfg.d_state
    heads = lambda t, w: t.view(2, 33, h, w).transpose(1, 2)   # noqa: E731
    q, k, v = heads(layer.W_Q(x), dh), heads(layer.W_K(x), dh), heads(layer.W_V(x), dh)
    inp = dict(theta=layer.theta_proj(x).view(2, 33, h, s // 2), a=layer.alpha_proj(x),
               z=layer._forget_logits(x).double(), c=heads(layer.W_C(x), s), b=heads(layer.W_B(x), s),
               lam_raw=layer.lambda_raw.double())
    cr, br, g, Fg, lam = R.unfused_glue(inp)
    o = R.dense_attention(q, k, v, cr, br, g, lam, Fg)
    ref = layer.W_O(o.transpose(1, 2).reshape(2, 33, 128))
    assert R.rel(y, ref) < 1e-6          # forget logits are computed in fp32 (modeling.py:164-169)
    with pytest.raises(ValueError, match="GPU"):
        layer(x, impl="hip")
    # lambda_raw stays fp32 under a low-precision cast
    lb = SISAAttention(cfg).to(torch.bfloat16)
    assert lb.lambda_raw.dtype == torch.float32 and lb.W_Q.weight.dtype == torch.bfloat16


def test_config_presets():
    from sisa_amd import SISAConfig
    c = SISAConfig.preset("sisa-152m")
    assert (c.d_model, c.n_head, c.d_head, c.d_state) == (768, 12, 64, 32)
    with pytest.raises(ValueError):
        SISAConfig.preset("nope")
    with pytest.raises(ValueError):
        SISAConfig(d_model=128, n_layer=1, n_head=2, d_ff=256, attn_impl="triton")
    assert SISAConfig.from_dict(c.to_dict()) == c


# ------------------------------------------------------------------------------------------------ fused layout
def test_fused_layout_and_weights():
    from sisa_amd.kernels.fused_prep import concat_fused_weights, fused_layout
    for H in (8, 12, 16):
        off = fused_layout(H)
        ref = R.layout(H)
        assert {k: off[k] for k in ref} == ref
    H, d = 2, 96
    mk = lambda r: torch.randn(r, d)                      # noqa: E731
    W, b = concat_fused_weights(mk(128), mk(128), mk(128), mk(64), mk(64), mk(32), mk(2), torch.tensor([1.0, 2.0]))
    off = fused_layout(H)
    assert W.shape == (off["NPAD"], d) and b.shape == (off["NPAD"],)
    assert (W[off["NTOT"]:] == 0).all() and b[off["A"]:off["A"] + 2].tolist() == [1.0, 2.0]
    assert (b[:off["A"]] == 0).all() and (b[off["NTOT"]:] == 0).all()
    with pytest.raises(ValueError):
        fused_layout(8, d_head=128)


# ------------------------------------------------------------------------------------------------ linear CE
def test_linear_ce_cpu_falls_back_to_eager():
    from sisa_amd.kernels.linear_ce import linear_cross_entropy, reference_linear_cross_entropy
    torch.manual_seed(0)
    h = torch.randn(2, 5, 16, requires_grad=True)
    w = torch.randn(37, 16, requires_grad=True)
    y = torch.randint(0, 37, (2, 5))
    y[0, 1] = -100
    a = linear_cross_entropy(h, w, y)
    b = reference_linear_cross_entropy(h, w, y)
    assert torch.equal(a, b)
    a.backward()
    assert h.grad is not None and w.grad is not None


def test_linear_ce_chunk_policy_and_padding():
    from sisa_amd.kernels import linear_ce as LC
    # 16,384 tokens x 50,304 bf16 columns = 1.65 GB of exponentials: one chunk under the 2 GiB budget
    n = LC.chunk_rows(16384, 50304, None, 2)
    assert n == 16384 and n * 50304 * 2 <= LC.PROBS_BUDGET
    n = LC.chunk_rows(100000, 50304, None, 2)
    assert n % 128 == 0 and n * 50304 * 2 <= LC.PROBS_BUDGET + 128 * 50304 * 2 and -(-100000 // n) == 5
    assert LC.chunk_rows(1000, 50304, 300, 2) == 300 and LC.chunk_rows(10, 50304, 300, 2) == 10
    assert LC.chunk_rows(0, 50304, None, 2) == 1
    w = torch.randn(1003, 8)
    wp = LC.padded_weight(w, torch.bfloat16)
    assert wp.shape == (1024, 8) and (wp[1003:] == 0).all() and torch.equal(wp[:1003], w.to(torch.bfloat16))
    assert LC.padded_weight(torch.randn(256, 8), torch.float16).shape == (256, 8)
    wq = LC.padded_weight(w, torch.bfloat16, 64)                  # hidden size padded with zero columns
    assert wq.shape == (1024, 64) and not wq[:, 8:].any() and torch.equal(wq[:1003, :8], w.to(torch.bfloat16))
    assert LC.flops(16384, 50277, 768)["total"] == pytest.approx(3.80e12, rel=1e-2)


def test_compute_dtype_follows_autocast():
    """The compute dtype every HIP path keys on: the input's dtype, or autocast's when autocast is on."""
    from sisa_amd import backends
    assert backends.compute_dtype(torch.randn(2, 2)) == torch.float32
    with torch.autocast("cpu", dtype=torch.bfloat16):
        assert backends.compute_dtype(torch.randn(2, 2)) == torch.bfloat16


# ------------------------------------------------------------------------------------------------ entry points
def test_bench_refuses_more_than_one_gpu():
    pr = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                        text=True, timeout=60)
    assert pr.returncode == 2 and "one GPU" in pr.stderr


def test_build_flags_name_existing_sources():
    """Every per-source compiler addition of the build names a HIP source that exists (a renamed or split source would
    otherwise silently lose its scheduler choice), and the HIP sources all carry the packed-fp32 exclusion."""
    from sisa_amd import build
    sources = {os.path.basename(p) for p in build.glob.glob(os.path.join(build.CSRC, "*.hip"))}
    assert set(build.EXTRA_FLAGS) <= sources, set(build.EXTRA_FLAGS) - sources
    assert "-packed-fp32-ops" in build.HIPFLAGS


def test_graft_entry_points_exist():
    sys.path.insert(0, ROOT)
    import __graft_entry__ as ge
    assert callable(ge.build) and callable(ge.smoke)


def test_hip_attention_refuses_cpu_tensors():
    from sisa_amd.kernels.attention import sisa_attention_hip
    ins = R.make_attention_inputs(dict(B=1, H=4, L=64, dtype="bf16", seed=1))
    with pytest.raises((ValueError, RuntimeError)):
        sisa_attention_hip(*(ins[n] for n in R.IN_NAMES))
    assert math.isfinite(float(ins["q"].float().sum()))


def test_wgrad_row_pieces():
    """The weight-gradient launches keep each operand's row range below 2 GiB (32-bit buffer offsets)."""
    from sisa_amd.kernels.wgrad import OPERAND_LIMIT, row_pieces
    assert row_pieces(16384, 3280, 768) == [(0, 16384)]
    M, lda = 400_000, 3280                      # 2.6 GB of dy: beyond one launch
    pieces = row_pieces(M, lda, 768)
    assert len(pieces) == 2 and pieces[0][0] == 0 and pieces[-1][1] == M
    assert all(a1 == b0 for (_, a1), (b0, _) in zip(pieces, pieces[1:]))
    assert all((r1 - r0) * lda * 2 < OPERAND_LIMIT and (r1 - r0) % 64 == 0 for r0, r1 in pieces[:-1])
    assert (pieces[-1][1] - pieces[-1][0]) * lda * 2 < OPERAND_LIMIT
    assert row_pieces(0, 8, 8) == []
