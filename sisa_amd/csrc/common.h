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
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

static constexpr float LOG2E = 1.4426950408889634f;

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

// 16-byte / 8-byte loads of 8 or 4 consecutive elements.
template <class T> SISA_DEV frag8<T> load8(const T* p) { return *reinterpret_cast<const frag8<T>*>(p); }
template <class T> SISA_DEV vec4<T> load4(const T* p) { return *reinterpret_cast<const vec4<T>*>(p); }
template <class T> SISA_DEV void store4(T* p, vec4<T> v) { *reinterpret_cast<vec4<T>*>(p) = v; }

// 8 consecutive elements of any type as fp32 (two 16-byte loads for fp32, one for 16-bit types), and back.
template <class T> SISA_DEV f32x8 load_f32x8(const T* p) {
    if constexpr (sizeof(T) == 4) {
        const f32x4 lo = *reinterpret_cast<const f32x4*>(p), hi = *reinterpret_cast<const f32x4*>(p + 4);
        return f32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    } else {
        return __builtin_convertvector(load8<T>(p), f32x8);
    }
}
template <class T> SISA_DEV void store_f32x8(T* p, const f32x8& v) {
    if constexpr (sizeof(T) == 4) {
        *reinterpret_cast<f32x4*>(p) = f32x4{v[0], v[1], v[2], v[3]};
        *reinterpret_cast<f32x4*>(p + 4) = f32x4{v[4], v[5], v[6], v[7]};
    } else {
        *reinterpret_cast<frag8<T>*>(p) = __builtin_convertvector(v, frag8<T>);
    }
}

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

// ------------------------------------------------------------------------------------------------ LDS tiles
// A tile is 64 rows (sequence positions) x C features stored densely row-major in LDS, in 16-byte chunks. For 16-bit
// types the chunks of a row are XOR-swizzled so that both fragment reads below are free of bank conflicts:
//   C = 64 (8 chunks per row): physical chunk = chunk ^ (row % 8);
//   C = 32 (4 chunks per row): physical chunk = chunk ^ 2 * ((row / 4) % 2);
//   C >= 128 (16+ chunks per row, transpose reads only): physical chunk = chunk ^ 2 * (row % 4) ^ 8 * b(row), with
//   b(row) = bit 2 of row xor bit 3 of row.
// (8 consecutive rows of one chunk column, and the 4-row x 32-byte footprint of a transpose read, then fall on
// distinct banks. For C >= 128 every row starts on the same bank: the 2 (row % 4) term separates the 4 rows of one
// lane group's transpose read, and b(row) moves the other lane group of each pair serviced together by 128 bytes:
// it differs between rows r and r + 4 (lane groups 0/1 and 2/3 of the sequence map, r % 8 < 4) and between rows r
// and r + 8 (those of the feature map, r % 16 < 8).) fp32 tiles (the accuracy path) are not swizzled.
template <class T, int C>
SISA_DEV int swz(int row) {
    if constexpr (sizeof(T) != 2) return 0;
    else if constexpr (C == 64) return row & 7;
    else if constexpr (C >= 128) return ((row & 3) << 1) ^ ((((row >> 2) ^ (row >> 3)) & 1) << 3);
    else return ((row >> 2) & 1) << 1;
}
// element offset of (row, 16-byte chunk) in a tile
template <class T, int C>
SISA_DEV int toff(int row, int chunk) {
    return row * C + (16 / (int)sizeof(T)) * (chunk ^ swz<T, C>(row));
}

// Buffer resource over one (batch, head) view: rows 0..L-1 of `bytes` total extent; rows at or beyond L read as zero.
// The extent must be below 2^31 bytes (checked by the host).
typedef int i32x4 __attribute__((ext_vector_type(4)));
SISA_DEV __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// Staging of a tile straight from global memory into LDS (buffer loads with the LDS destination, no registers):
// wave instruction k of a tile fills tile bytes [1024 k, 1024 k + 1024), lane i the 16-byte chunk 64 k + i, so a
// tile of CPR chunks per row takes CPR instructions, spread over the NW waves of the workgroup. The per-lane global
// offsets do not change from tile to tile; the tile's first row enters as a scalar offset. The loads complete
// asynchronously: a workgroup barrier after them (the compiler waits for the loads before it) publishes the tile.
template <class T, int C, int NW>
struct DmaStage {
    static constexpr int CPR = C * (int)sizeof(T) / 16;   // chunks per row = wave instructions per tile
    static constexpr int PER = (CPR + NW - 1) / NW;
    int voff[PER];

    SISA_DEV void init(int64_t srow, int w, int lane) {
#pragma unroll
        for (int p = 0; p < PER; ++p) {
            const int ci = 64 * (w + NW * p) + lane;
            const int row = ci / CPR, phys = ci % CPR;
            voff[p] = (int)(row * srow * (int64_t)sizeof(T) + 16 * (phys ^ swz<T, C>(row)));
        }
    }
};

// Issue the staging of rows [row0, row0 + 64) of a view (base pointer, extent in bytes) into tile X
// (soff = row0 * srow * sizeof(T)). The buffer resource is formed here: the resource type is device-only, and kernel
// code that the host compilation pass also analyses must not pass it around. KERNEL gives each kernel its own
// specialization: the host pass of this compiler rejects a second kernel's use of a specialization already used by
// another kernel (and silently drops that kernel's launch stub when the call is a member function).
template <int KERNEL, class T, int C, int NW>
SISA_DEV void dma_issue(const DmaStage<T, C, NW>& st, const void* base, int64_t bytes, int soff, T* X, int w) {
    const __amdgpu_buffer_rsrc_t r = make_rsrc(base, bytes);
#pragma unroll
    for (int p = 0; p < DmaStage<T, C, NW>::PER; ++p) {
        const int k = w + NW * p;
        // (always true when the waves split the instructions evenly: no per-instruction branch then)
        if (DmaStage<T, C, NW>::CPR % NW == 0 || k < DmaStage<T, C, NW>::CPR)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                r, (__attribute__((address_space(3))) void*)(X + k * (1024 / (int)sizeof(T))), 16, st.voff[p], soff, 0,
                0);
    }
}

// Operand fragment of a tile X: row (position) r0 + lane%16, features 32*step + 8*grp + 0..7 (feature-contracted
// products: A/B operand whose row is a position).
template <class T, int C>
SISA_DEV frag8<T> frag_rows(const T* X, int r0, int step, int lane) {
    const int row = r0 + (lane & 15);
    if constexpr (sizeof(T) == 2) {
        return load8<T>(X + toff<T, C>(row, 4 * step + (lane >> 4)));
    } else {
        const int c0 = (32 * step + 8 * (lane >> 4)) / 4;
        return join<T>(load4<T>(X + toff<T, C>(row, c0)), load4<T>(X + toff<T, C>(row, c0 + 1)));
    }
}

// Operand fragment of the transpose of a tile X (rows = positions): row (feature) f0 + lane%16, K = the positions of
// the sequence map for `step` (positions 32*step .. 32*step+31 of the tile).
// 16-bit types use the gfx950 LDS transpose read ds_read_b64_tr_b16: within each block of 16 lanes, destination
// lane d receives, as element j, element d%4 of the 8 bytes addressed by source lane 4j + d/4. Source lane
// s = 4j + q of lane group grp therefore addresses position 16*blk + 4*grp + j, features f0 + 4q .. f0 + 4q + 3, and
// destination lane d gets feature f0 + d at positions 16*blk + 4*grp + 0..3 -- slots j (blk = 2*step) and j + 4
// (blk = 2*step + 1) of the sequence map. The swizzle of a row equals that of the row 16 below it.
typedef short s16x4 __attribute__((ext_vector_type(4)));
template <class T>
SISA_DEV vec4<T> lds_tr4(const T* __restrict__ p) {
    const s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)p);
    return __builtin_bit_cast(vec4<T>, r);
}

template <class T, int C>
SISA_DEV frag8<T> frag_tr(const T* X, int f0, int step, int lane) {
    const int s = lane & 15, grp = lane >> 4;
    const int row = 32 * step + 4 * grp + (s >> 2);
    const int f = f0 + 4 * (s & 3);
    const T* p0 = X + toff<T, C>(row, f >> 3) + (f & 4);
    return join<T>(lds_tr4<T>(p0), lds_tr4<T>(p0 + 16 * C));
}

// The same transpose read with the feature map instead of the sequence map: row (feature) f0 + lane%16, K = tile
// rows 32*step + 8*grp + 0..7 (source lane s of lane group grp addresses row 32*step + 8*grp + s/4, then 4 rows
// further for slots 4..7). Pairs with frag_rows of a tile whose rows are the other operand's rows and whose columns
// are the same K (16-bit types, C >= 128).
template <class T, int C>
SISA_DEV frag8<T> frag_trf(const T* X, int f0, int step, int lane) {
    static_assert(sizeof(T) == 2 && C >= 128, "frag_trf: 16-bit tiles of at least 128 columns");
    const int s = lane & 15, grp = lane >> 4;
    const int row = 32 * step + 8 * grp + (s >> 2);
    const int f = f0 + 4 * (s & 3);
    return join<T>(lds_tr4<T>(X + toff<T, C>(row, f >> 3) + (f & 4)), lds_tr4<T>(X + toff<T, C>(row + 4, f >> 3) + (f & 4)));
}

// fp32 tiles: plain element gathers (the fp32 path exists for accuracy, not speed).
template <>
SISA_DEV frag8<float> frag_tr<float, 64>(const float* X, int f0, int step, int lane) {
    const int m = lane & 15, grp = lane >> 4;
    frag8<float> r;
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = X[((2 * step + j / 4) * 16 + 4 * grp + j % 4) * 64 + f0 + m];
    return r;
}
template <>
SISA_DEV frag8<float> frag_tr<float, 32>(const float* X, int f0, int step, int lane) {
    const int m = lane & 15, grp = lane >> 4;
    frag8<float> r;
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = X[((2 * step + j / 4) * 16 + 4 * grp + j % 4) * 32 + f0 + m];
    return r;
}

// The A fragment of a 16-row block of ones: MFMA with it sums the B operand over K into every row of the output
// block, so each lane holds the column sums of its columns.
template <class T>
SISA_DEV frag8<T> ones_frag() {
    frag8<T> r;
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = (T)1.f;
    return r;
}
