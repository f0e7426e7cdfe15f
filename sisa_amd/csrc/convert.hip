// The 16-bit rounding and widening every kernel of this library uses for its MFMA operands, over a flat buffer: a
// thread rounds 8 consecutive fp32 values with pack8 (one v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32 per pair,
// round-to-nearest-even) and widens the 8 results back to fp32 with the conversion the kernels' loads use.
//
// Reference: `_bf16x2` / `_bf16x2_f32` (src/sisa/kernels/attention.py:156-173), specified there as identical to
// tensor.to(torch.bfloat16) and to the bf16 -> fp32 shift. This entry point exists so that the helpers can be checked
// bit for bit against torch's conversions; the kernels inline them.
#include "common.h"
#include "host.h"

namespace {

template <class T>
__global__ __launch_bounds__(256) void round16_kernel(sisa_round16_args a) {
    const int64_t i0 = 8 * ((int64_t)blockIdx.x * 256 + threadIdx.x);
    if (i0 >= a.n) return;
    T* y = (T*)a.y;
    if (i0 + 8 <= a.n) {
        const f32x8 v = load_f32x8<float>(a.x + i0);
        const frag8<T> r = pack8<T>(f32x4{v[0], v[1], v[2], v[3]}, f32x4{v[4], v[5], v[6], v[7]});
        *reinterpret_cast<frag8<T>*>(y + i0) = r;
        if (a.back) store_f32x8<float>(a.back + i0, load_f32x8<T>(y + i0));
    } else {   // the ragged tail: the scalar form of the same conversion
        for (int64_t i = i0; i < a.n; ++i) {
            y[i] = cvt<T>(a.x[i]);
            if (a.back) a.back[i] = (float)y[i];
        }
    }
}

}  // namespace

extern "C" int sisa_round16(const sisa_round16_args* a, void* stream) {
    SISA_REQUIRE(a != nullptr, "sisa_round16: null args");
    if (a->n == 0) return SISA_OK;
    SISA_REQUIRE(a->n > 0 && a->x && a->y && sisa::aligned16(a->x) && sisa::aligned16(a->y) &&
                     (a->back == nullptr || sisa::aligned16(a->back)),
                 "sisa_round16: n >= 0 and 16-byte aligned x, y (and back when given)");
    SISA_REQUIRE(a->dtype == SISA_BF16 || a->dtype == SISA_F16, "sisa_round16: dtype %d (bf16 or fp16)", a->dtype);
    const unsigned grid = (unsigned)sisa::cdiv(sisa::cdiv(a->n, 8), 256);
    hipStream_t st = (hipStream_t)stream;
    if (a->dtype == SISA_BF16) round16_kernel<__bf16><<<grid, 256, 0, st>>>(*a);
    else round16_kernel<_Float16><<<grid, 256, 0, st>>>(*a);
    return sisa::launch_status("sisa_round16");
}
