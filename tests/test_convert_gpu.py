"""The library's 16-bit operand rounding (pack8 / cvt, csrc/common.h) against torch's conversions, bit for bit.

The reference specifies its pair helper as identical to tensor.to(torch.bfloat16) and its widening as the bf16 ->
fp32 shift (src/sisa/kernels/attention.py:156-173). sisa_round16 runs the kernels' own conversions over a buffer;
every finite or infinite input must give exactly torch's bits in bf16 and fp16, and the widened values exactly
y.float(). Inputs: exact round-to-nearest-even ties (even and odd neighbours), fp32 subnormals (those that keep a
bf16 subnormal and those that round to zero), ±0, ±inf, values beyond the 16-bit maxima, and 2^20 random 32-bit
patterns (every exponent, NaNs included). A NaN input must give a NaN (its payload is not specified here).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _patterns() -> np.ndarray:
    rng = np.random.default_rng(20251202)
    special = [0x00000000, 0x80000000, 0x7F800000, 0xFF800000, 0x7F7FFFFF, 0xFF7FFFFF,   # ±0, ±inf, ±FLT_MAX
               0x7F7F7FFF, 0x7F7F8000, 0x7F7F8001, 0x477FEFFF, 0x477FF000, 0x477FF001,   # near the bf16 / fp16 maxima
               0x7FC00000, 0x7F800001, 0xFFFFFFFF, 0x7FBFFFFF,                           # NaNs (quiet, signalling)
               0x00000001, 0x00008000, 0x00008001, 0x00018000, 0x007FFFFF, 0x807F8000,   # fp32 subnormals
               0x00800000, 0x33800000, 0x33000000, 0x387FC000, 0x38800000]               # fp16 subnormal range edge
    ties = []
    for hi in rng.integers(0, 1 << 16, 4096, dtype=np.uint64):
        ties.append((int(hi) << 16) | 0x8000)           # exactly halfway between two bf16 neighbours
    for hi in rng.integers(0, 1 << 19, 4096, dtype=np.uint64):
        ties.append((int(hi) << 13) | 0x1000)           # exactly halfway between two fp16 neighbours (normal range)
    rand = rng.integers(0, 1 << 32, 1 << 20, dtype=np.uint64)
    scaled = (rng.standard_normal(1 << 16) * np.float64(10.0) ** rng.integers(-45, 39, 1 << 16)).astype(np.float32)
    bits = np.concatenate([np.array(special + ties, dtype=np.uint64), rand, scaled.view(np.uint32).astype(np.uint64)])
    return bits.astype(np.uint32)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("tail", [0, 5])
def test_round16_matches_torch_bitwise(dtype, tail):
    from sisa_amd.kernels import _lib

    bits = _patterns()
    bits = bits[:len(bits) - (len(bits) % 8) + tail] if tail else bits[:len(bits) - len(bits) % 8]
    x = torch.from_numpy(bits.view(np.float32).copy()).to(DEV)
    y = torch.empty(x.numel(), dtype=dtype, device=DEV)
    back = torch.empty(x.numel(), dtype=torch.float32, device=DEV)
    print(f"[round16] dtype={dtype} n={x.numel()}", flush=True)
    args = _lib.Round16Args(x.numel(), _lib.dtype_code(dtype), x.data_ptr(), y.data_ptr(), back.data_ptr())
    _lib.call("sisa_round16", args, x)
    torch.cuda.synchronize()
    want = x.to(dtype)
    nan_in = torch.isnan(x)
    got_bits, want_bits = y.view(torch.int16), want.view(torch.int16)
    wrong = (got_bits != want_bits) & ~nan_in
    if bool(wrong.any()):
        i = int(wrong.nonzero()[0])
        raise AssertionError(f"{int(wrong.sum())} values differ; first: x bits {int(bits[i]):#010x} -> "
                             f"{int(got_bits[i]) & 0xFFFF:#06x}, torch {int(want_bits[i]) & 0xFFFF:#06x}")
    assert bool(torch.isnan(y[nan_in]).all()), "a NaN input did not give a NaN"
    widened = y.float()
    assert torch.equal(back.view(torch.int32)[~nan_in], widened.view(torch.int32)[~nan_in])
    assert bool(torch.isnan(back[nan_in]).all())
    same_nan = bool((got_bits[nan_in] == want_bits[nan_in]).all())
    print(f"[round16] NaN bits equal to torch's as well: {same_nan}", flush=True)


def test_round16_rejects_bad_arguments():
    from sisa_amd.kernels import _lib

    x = torch.zeros(16, device=DEV)
    y = torch.zeros(16, dtype=torch.bfloat16, device=DEV)
    for args in (_lib.Round16Args(16, _lib.F32, x.data_ptr(), y.data_ptr(), None),
                 _lib.Round16Args(16, _lib.BF16, x.data_ptr() + 4, y.data_ptr(), None),
                 _lib.Round16Args(-1, _lib.BF16, x.data_ptr(), y.data_ptr(), None)):
        with pytest.raises(RuntimeError, match="sisa_round16"):
            _lib.call("sisa_round16", args, x)
