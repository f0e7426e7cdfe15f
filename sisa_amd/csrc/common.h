// Device-side building blocks shared by the SISA kernels (gfx950 / CDNA4, wave64).
//
// MFMA fragments. All matrix products use the 16x16 output block of v_mfma_f32_16x16x32_{bf16,f16}
// (fp32 inputs: eight v_mfma_f32_16x16x4_f32). The output (C) layout of every 16x16 MFMA is
//     lane l holds C[row = 4*(l/16) + i][col = l%16], i = 0..3.
// An operand fragment is 8 elements per lane: A fragments hold row l%16, B fragments column l%16, and the 8
// elements of lane group grp = l/16 are the K-slots (grp, 0..7). The physical K index of a slot never matters as
// long as A and B use the same slot->k map; two maps are used:
//   feature-contracted products (k = feature):  slot (grp, j) -> k = 32*step + 8*grp + j   (16 contiguous bytes)
//   sequence-contracted products (k = position): slot (grp, j) -> pos = (2*step + j/4)*16 + 4*grp + j%4
// The second map lets the C blocks of a previous product be used directly as the B fragment of the next one
// (block 2*step gives slots j<4, block 2*step+1 gives slots j>=4): no register shuffles, no LDS round trip.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define SISA_DEV __device__ __forceinline__

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

static constexpr float LOG2E = 1.4426950408889634f;
static constexpr int LDS_PAD = 16;  // elements of padding per LDS tile row

template <class T> struct Vec;
template <> struct Vec<__bf16> { typedef bf16x8 x8; typedef bf16x4 x4; typedef bf16x2 x2; };
template <> struct Vec<_Float16> { typedef f16x8 x8; typedef f16x4 x4; typedef f16x2 x2; };
template <> struct Vec<float> { typedef f32x8 x8; typedef f32x4 x4; typedef f32x2 x2; };

template <class T> using frag8 = typename Vec<T>::x8;
template <class T> using vec4 = typename Vec<T>::x4;

// 16x16 block += A(16 x 32 K-slots) * B(32 K-slots x 16)
SISA_DEV f32x4 mma(bf16x8 a, bf16x8 b, f32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0); }
SISA_DEV f32x4 mma(f16x8 a, f16x8 b, f32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }
SISA_DEV f32x4 mma(f32x8 a, f32x8 b, f32x4 c) {
#pragma unroll
    for (int j = 0; j < 8; ++j) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j], b[j], c, 0, 0, 0);
    return c;
}

// Round-to-nearest-even conversion (v_cvt_pk_bf16_f32 on gfx950; identical to torch's .to(bfloat16)).
template <class T> SISA_DEV T cvt(float x) { return (T)x; }

// Packs 8 fp32 values into an operand fragment, rounding each once to T.
template <class T> SISA_DEV frag8<T> pack8(f32x4 lo, f32x4 hi) {
    f32x8 v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    return __builtin_convertvector(v, frag8<T>);
}

// Sum of the 8 (rounded) fragment values in fp32 (exact conversions, fixed order).
template <class T> SISA_DEV float frag_sum(const frag8<T>& f) {
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) s += (float)f[j];
    return s;
}

// exp2 of an exponent clamped to <= 0 with NaN propagation (the reference's minimum(x, 0, propagate_nan=ALL)).
SISA_DEV float exp2_le0(float x) { return __builtin_amdgcn_exp2f(x > 0.f ? 0.f : x); }
SISA_DEV float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// NaN-propagating max.
SISA_DEV float nmax(float a, float b) { return (a != a || b != b) ? __builtin_nanf("") : fmaxf(a, b); }

SISA_DEV f32x4 lds4f(const float* p) { return *reinterpret_cast<const f32x4*>(p); }

// Cross-lane butterfly over the four lane groups (lanes l, l^16, l^32, l^48) with the gfx950 permlane swaps:
// every lane of a group gets the same result (the pairwise combination order is identical in all four lanes).
SISA_DEV float xswap32_max(float x) {
    const unsigned u = __float_as_uint(x);
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
SISA_DEV float group_max(float x) {
    x = xswap32_max(x);
    const unsigned u = __float_as_uint(x);
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
SISA_DEV float group_sum(float x) {
    unsigned u = __float_as_uint(x);
    auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    x = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    u = __float_as_uint(x);
    r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// Value of lane (l % 16) (lane group 0) broadcast to the four lanes of its group.
SISA_DEV float group_bcast0(float x, int lane) {
    const unsigned u = __float_as_uint(x);
    const unsigned v = (unsigned)__builtin_amdgcn_ds_bpermute((lane & 15) << 2, (int)u);
    return __uint_as_float(v);
}

// 16-byte / 8-byte loads of 8 or 4 consecutive elements.
template <class T> SISA_DEV frag8<T> load8(const T* p) { return *reinterpret_cast<const frag8<T>*>(p); }
template <class T> SISA_DEV vec4<T> load4(const T* p) { return *reinterpret_cast<const vec4<T>*>(p); }
template <class T> SISA_DEV void store4(T* p, vec4<T> v) { *reinterpret_cast<vec4<T>*>(p) = v; }

template <class T> SISA_DEV frag8<T> join(vec4<T> lo, vec4<T> hi) {
    frag8<T> r;
    r[0] = lo[0]; r[1] = lo[1]; r[2] = lo[2]; r[3] = lo[3];
    r[4] = hi[0]; r[5] = hi[1]; r[6] = hi[2]; r[7] = hi[3];
    return r;
}

template <class T> SISA_DEV frag8<T> zero8() {
    frag8<T> r;
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = (T)0.f;
    return r;
}

SISA_DEV f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

template <class T> SISA_DEV vec4<T> to_vec4(f32x4 x) { return __builtin_convertvector(x, vec4<T>); }

// Cooperative staging of a (64 x C) tile of a sequence-major tensor (rows = positions, C in {32, 64} contiguous
// features) into a row-major LDS tile X[r][f] (row stride C + LDS_PAD), in two phases so that the global loads of the
// next tile are in flight while the current one is being used: load() issues 16-byte (8-element) vector loads into
// registers, store() writes them to LDS. Rows >= nvalid are zero. Consecutive threads read consecutive 16-byte
// pieces of a row (coalesced).
template <class T, int C, int NTH>
struct TileStage {
    static constexpr int NVEC = 64 * C / 8;
    static constexpr int PER = (NVEC + NTH - 1) / NTH;
    frag8<T> v[PER];

    SISA_DEV void load(const T* __restrict__ src, int64_t srow, int nvalid, int tid) {
#pragma unroll
        for (int p = 0; p < PER; ++p) {
            const int idx = tid + p * NTH;
            const int row = idx / (C / 8), c8 = idx % (C / 8);
            if (idx < NVEC && row < nvalid) v[p] = load8<T>(src + (int64_t)row * srow + c8 * 8);
            else v[p] = zero8<T>();
        }
    }
    SISA_DEV void store(T* __restrict__ X, int tid) const {
#pragma unroll
        for (int p = 0; p < PER; ++p) {
            const int idx = tid + p * NTH;
            const int row = idx / (C / 8), c8 = idx % (C / 8);
            if (idx < NVEC) *reinterpret_cast<frag8<T>*>(X + row * (C + LDS_PAD) + c8 * 8) = v[p];
        }
    }
};

// Buffer-resource staging of the same (64 x C) tiles: one resource per (batch, head) view covering rows 0..L-1, a
// per-lane byte offset that does not change from tile to tile, and the tile's row offset as a wave-uniform scalar.
// Rows at or beyond L fall outside the resource and read as zero (no per-row bounds test, no 64-bit address
// arithmetic per tile). The view's extent must be below 2^31 bytes (checked by the host).
typedef int i32x4 __attribute__((ext_vector_type(4)));
SISA_DEV __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
template <class T>
SISA_DEV frag8<T> buf_load8(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    if constexpr (sizeof(T) == 2) {
        return __builtin_bit_cast(frag8<T>, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
    } else {
        const f32x4 lo = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
        const f32x4 hi = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff + 16, soff, 0));
        return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    }
}

template <class T, int C, int NTH>
struct BufStage {
    static constexpr int NVEC = 64 * C / 8;
    static constexpr int PER = (NVEC + NTH - 1) / NTH;
    frag8<T> v[PER];
    int voff[PER];

    SISA_DEV void init(int64_t srow, int tid) {
#pragma unroll
        for (int p = 0; p < PER; ++p) {
            const int idx = tid + p * NTH;
            voff[p] = (int)(((idx / (C / 8)) * srow + (idx % (C / 8)) * 8) * (int64_t)sizeof(T));
        }
    }
    // rows [row0, row0 + 64) of the view; soff = row0 * srow * sizeof(T)
    SISA_DEV void load(__amdgpu_buffer_rsrc_t r, int soff, int tid) {
#pragma unroll
        for (int p = 0; p < PER; ++p)
            v[p] = (tid + p * NTH < NVEC) ? buf_load8<T>(r, voff[p], soff) : zero8<T>();
    }
    SISA_DEV void store(T* __restrict__ X, int tid) const {
#pragma unroll
        for (int p = 0; p < PER; ++p) {
            const int idx = tid + p * NTH;
            const int row = idx / (C / 8), c8 = idx % (C / 8);
            if (idx < NVEC) *reinterpret_cast<frag8<T>*>(X + row * (C + LDS_PAD) + c8 * 8) = v[p];
        }
    }
};

// Operand fragment of a row-major LDS tile X: row (position) r0 + lane%16, features 32*step + 8*grp + 0..7
// (feature-contracted products: A/B operand whose row is a position).
template <class T, int C>
SISA_DEV frag8<T> frag_rows(const T* X, int r0, int step, int lane) {
    return load8<T>(X + (r0 + (lane & 15)) * (C + LDS_PAD) + 32 * step + 8 * (lane >> 4));
}

// Operand fragment of the transpose of a row-major LDS tile X (rows = positions): row (feature) f0 + lane%16,
// K = the positions of the sequence map for `step` (positions 32*step .. 32*step+31 of the tile).
// 16-bit types use the gfx950 LDS transpose read ds_read_b64_tr_b16: within each block of 16 lanes, destination
// lane d receives, as element j, element d%4 of the 8 bytes addressed by source lane 4j + d/4. Source lane
// s = 4j + q of lane group grp therefore addresses position 16*blk + 4*grp + j, features f0 + 4q .. f0 + 4q + 3, and
// destination lane d gets feature f0 + d at positions 16*blk + 4*grp + 0..3 -- slots j (blk = 2*step) and j + 4
// (blk = 2*step + 1) of the sequence map.
typedef short s16x4 __attribute__((ext_vector_type(4)));
template <class T>
SISA_DEV vec4<T> lds_tr4(const T* p) {
    const s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)p);
    return __builtin_bit_cast(vec4<T>, r);
}

template <class T, int C>
SISA_DEV frag8<T> frag_tr(const T* X, int f0, int step, int lane) {
    const int s = lane & 15, grp = lane >> 4;
    const T* p0 = X + ((2 * step) * 16 + 4 * grp + (s >> 2)) * (C + LDS_PAD) + f0 + 4 * (s & 3);
    return join<T>(lds_tr4<T>(p0), lds_tr4<T>(p0 + 16 * (C + LDS_PAD)));
}

// fp32 tiles: plain element gathers (the fp32 path exists for correctness, not speed).
template <>
SISA_DEV frag8<float> frag_tr<float, 64>(const float* X, int f0, int step, int lane) {
    const int m = lane & 15, grp = lane >> 4;
    frag8<float> r;
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = X[((2 * step + j / 4) * 16 + 4 * grp + j % 4) * (64 + LDS_PAD) + f0 + m];
    return r;
}
template <>
SISA_DEV frag8<float> frag_tr<float, 32>(const float* X, int f0, int step, int lane) {
    const int m = lane & 15, grp = lane >> 4;
    frag8<float> r;
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = X[((2 * step + j / 4) * 16 + 4 * grp + j % 4) * (32 + LDS_PAD) + f0 + m];
    return r;
}

// The A fragment of a 16-row block whose row 0 is all ones and rows 1..15 are zero: MFMA with it sums the B
// operand over K into row 0 of the output block.
template <class T>
SISA_DEV frag8<T> ones_row_frag(int lane) {
    frag8<T> r;
    const float v = (lane & 15) == 0 ? 1.f : 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = (T)v;
    return r;
}
