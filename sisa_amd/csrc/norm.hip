// Elementwise parts of the SISA decoder block for gfx950: RMSNorm (forward, backward with a deterministic weight
// gradient) and the SwiGLU activation silu(a) * b (forward, backward). All arithmetic in fp32, one rounding to the
// output dtype.
//
// Reference: src/sisa/modeling.py:26-50 (RMSNorm computed in float32 with the output in the input dtype; SwiGLU as
// w_down(silu(w_gate x) * w_up x)). The reference runs these as torch elementwise kernels; here each is one pass:
// RMSNorm reads a row once and writes it once (the backward reads x and dy once and writes dx once, plus per-block
// column partials of dw), the activation reads a and b once and writes h (backward: da and db) once.
//
// Work decomposition: RMSNorm gives each wave whole rows (16-byte vectors, the row in registers between the
// reduction and the write); the weight gradient is reduced in three fixed-order levels (per wave over RMS_RPW rows,
// per column over DW_SPLIT ranges of those partials, then over the ranges), so the result is bitwise reproducible.
// The activation is a flat grid-stride loop over 8-element vectors.
#include "common.h"
#include "host.h"

namespace {

constexpr int RMS_WAVES = 4;                 // rows in flight per workgroup (one per wave)
constexpr int RMS_MAXV = 8;                  // 8-element vectors per lane: rows of up to 64*8*8 = 4096
constexpr int RMS_RPW = 8;                   // backward: rows per wave, i.e. rows per dw partial row
constexpr int DW_SPLIT = 64;                 // backward: second-level dw partials per column

SISA_DEV float wave_sum(float x) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
    return x;
}

// ------------------------------------------------------------------------------------------------ RMSNorm
// y = (x * rsqrt(mean(x^2) + eps)) * w, rstd saved for the backward.
// NVL = 8-element vectors per lane (the row length rounded up to 512 elements per vector slot).
template <class T, int NVL>
__global__ __launch_bounds__(64 * RMS_WAVES) void rmsnorm_fwd_kernel(sisa_rmsnorm_args a) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * RMS_WAVES + (threadIdx.x >> 6);
    if (row >= a.N) return;
    const int nv = a.D / 8;
    const T* x = (const T*)a.x + row * a.sx;
    f32x8 v[NVL];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < NVL; ++i) {
        const int c = lane + 64 * i;
        if (c < nv) {
            v[i] = load_f32x8<T>(x + 8 * c);
#pragma unroll
            for (int j = 0; j < 8; ++j) ss = fmaf(v[i][j], v[i][j], ss);
        }
    }
    const float rstd = 1.f / sqrtf(wave_sum(ss) / (float)a.D + a.eps);
    T* y = (T*)a.y + row * a.sy;
#pragma unroll
    for (int i = 0; i < NVL; ++i) {
        const int c = lane + 64 * i;
        if (c < nv) {
            const f32x8 w = load_f32x8<float>(a.w + 8 * c);
            f32x8 o;
#pragma unroll
            for (int j = 0; j < 8; ++j) o[j] = (v[i][j] * rstd) * w[j];
            store_f32x8<T>(y + 8 * c, o);
        }
    }
    if (lane == 0 && a.rstd) a.rstd[row] = rstd;
}

// dx = rstd * (dy*w - n * mean(dy*w*n)), n = x*rstd. Each wave owns RMS_RPW consecutive rows and writes their dw
// contribution sum(dy*n) as one partial row: partial row p covers rows [RMS_RPW p, RMS_RPW (p+1)).
template <class T, int NVL>
__global__ __launch_bounds__(64 * RMS_WAVES) void rmsnorm_bwd_kernel(sisa_rmsnorm_args a) {
    const int lane = threadIdx.x & 63;
    const int64_t p = (int64_t)blockIdx.x * RMS_WAVES + (threadIdx.x >> 6);   // partial row = wave
    const int64_t r0 = p * RMS_RPW;
    if (r0 >= a.N) return;
    const int nv = a.D / 8;
    f32x8 w[NVL], dwacc[NVL];
#pragma unroll
    for (int i = 0; i < NVL; ++i) {
        const int c = lane + 64 * i;
        if (c < nv) w[i] = load_f32x8<float>(a.w + 8 * c);
#pragma unroll
        for (int j = 0; j < 8; ++j) dwacc[i][j] = 0.f;
    }
    for (int r = 0; r < RMS_RPW && r0 + r < a.N; ++r) {
        const int64_t row = r0 + r;
        const T* x = (const T*)a.x + row * a.sx;
        const T* dy = (const T*)a.dy + row * a.sdy;
        const float rstd = a.rstd[row];
        f32x8 n[NVL], gw[NVL];
        float dot = 0.f;
#pragma unroll
        for (int i = 0; i < NVL; ++i) {
            const int c = lane + 64 * i;
            if (c < nv) {
                const f32x8 xv = load_f32x8<T>(x + 8 * c), g = load_f32x8<T>(dy + 8 * c);
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    n[i][j] = xv[j] * rstd;
                    gw[i][j] = g[j] * w[i][j];
                    dot = fmaf(gw[i][j], n[i][j], dot);
                    dwacc[i][j] = fmaf(g[j], n[i][j], dwacc[i][j]);
                }
            }
        }
        const float mdot = wave_sum(dot) / (float)a.D;
        T* dx = (T*)a.dx + row * a.sdx;
#pragma unroll
        for (int i = 0; i < NVL; ++i) {
            const int c = lane + 64 * i;
            if (c < nv) {
                f32x8 o;
#pragma unroll
                for (int j = 0; j < 8; ++j) o[j] = rstd * (gw[i][j] - n[i][j] * mdot);
                store_f32x8<T>(dx + 8 * c, o);
            }
        }
    }
    float* dwp = a.dw_partial + p * a.D;
#pragma unroll
    for (int i = 0; i < NVL; ++i) {
        const int c = lane + 64 * i;
        if (c < nv) store_f32x8<float>(dwp + 8 * c, dwacc[i]);
    }
}

// s + p[0] + p[stride] + ... + p[(n-1) stride], added in that order; the loads go out 8 at a time ahead of their adds
// (a load-add chain would wait for every load in turn).
SISA_DEV float ordered_sum(const float* __restrict__ p, int64_t stride, int64_t n, float s) {
    int64_t k = 0;
    for (; k + 8 <= n; k += 8) {
        float t[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) t[e] = __builtin_nontemporal_load(p + (k + e) * stride);
#pragma unroll
        for (int e = 0; e < 8; ++e) s += t[e];
    }
    for (; k < n; ++k) s += p[k * stride];
    return s;
}

// Level 2: column block blockIdx.x (256 columns), split blockIdx.y sums partial rows [k0, k1) in order.
__global__ __launch_bounds__(256) void rmsnorm_dw2_kernel(const float* __restrict__ part, float* __restrict__ part2,
                                                         int64_t np, int D) {
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c >= D) return;
    const int64_t per = (np + DW_SPLIT - 1) / DW_SPLIT;
    const int64_t k0 = blockIdx.y * per, k1 = k0 + per < np ? k0 + per : np;
    part2[(int64_t)blockIdx.y * D + c] = k1 > k0 ? ordered_sum(part + k0 * D + c, D, k1 - k0, 0.f) : 0.f;
}

// Level 3: dw[c] = sum over the DW_SPLIT level-2 partials in order.
__global__ __launch_bounds__(256) void rmsnorm_dw3_kernel(const float* __restrict__ part2, float* __restrict__ dw,
                                                         int D) {
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c >= D) return;
    dw[c] = ordered_sum(part2 + c, D, DW_SPLIT, 0.f);
}

// ------------------------------------------------------------------------------------------------ SwiGLU
SISA_DEV float sigmoidf_(float a) { return 1.f / (1.f + expf(-a)); }

// h = silu(a) * b
template <class T>
__global__ __launch_bounds__(256) void swiglu_fwd_kernel(sisa_swiglu_args a) {
    const int64_t nv = a.n / 8;
    for (int64_t v = (int64_t)blockIdx.x * 256 + threadIdx.x; v < nv; v += (int64_t)gridDim.x * 256) {
        const f32x8 x = load_f32x8<T>((const T*)a.a + 8 * v), y = load_f32x8<T>((const T*)a.b + 8 * v);
        f32x8 h;
#pragma unroll
        for (int j = 0; j < 8; ++j) h[j] = (x[j] * sigmoidf_(x[j])) * y[j];
        store_f32x8<T>((T*)a.h + 8 * v, h);
    }
}

// da = dh * b * silu'(a), db = dh * silu(a); silu'(a) = s * (1 + a * (1 - s)), s = sigmoid(a)
template <class T>
__global__ __launch_bounds__(256) void swiglu_bwd_kernel(sisa_swiglu_args a) {
    const int64_t nv = a.n / 8;
    for (int64_t v = (int64_t)blockIdx.x * 256 + threadIdx.x; v < nv; v += (int64_t)gridDim.x * 256) {
        const f32x8 x = load_f32x8<T>((const T*)a.a + 8 * v), y = load_f32x8<T>((const T*)a.b + 8 * v);
        const f32x8 g = load_f32x8<T>((const T*)a.dh + 8 * v);
        f32x8 da, db;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float s = sigmoidf_(x[j]);
            db[j] = g[j] * (x[j] * s);
            da[j] = (g[j] * y[j]) * (s * (1.f + x[j] * (1.f - s)));
        }
        store_f32x8<T>((T*)a.da + 8 * v, da);
        store_f32x8<T>((T*)a.db + 8 * v, db);
    }
}

template <class T, int NVL>
int launch_rmsnorm_nvl(const sisa_rmsnorm_args* a, int bwd, hipStream_t st) {
    if (!bwd) {
        rmsnorm_fwd_kernel<T, NVL><<<(unsigned)sisa::cdiv(a->N, RMS_WAVES), 64 * RMS_WAVES, 0, st>>>(*a);
        return sisa::launch_status("sisa_rmsnorm_fwd");
    }
    const int64_t np = sisa::cdiv(a->N, RMS_RPW);
    if (np > 0) {
        rmsnorm_bwd_kernel<T, NVL><<<(unsigned)sisa::cdiv(np, RMS_WAVES), 64 * RMS_WAVES, 0, st>>>(*a);
        const int rc = sisa::launch_status("sisa_rmsnorm_bwd");
        if (rc) return rc;
    }
    float* part2 = a->dw_partial + np * a->D;
    rmsnorm_dw2_kernel<<<dim3((unsigned)sisa::cdiv(a->D, 256), DW_SPLIT), 256, 0, st>>>(a->dw_partial, part2, np,
                                                                                         a->D);
    int rc = sisa::launch_status("sisa_rmsnorm_bwd (dw)");
    if (rc) return rc;
    rmsnorm_dw3_kernel<<<(unsigned)sisa::cdiv(a->D, 256), 256, 0, st>>>(part2, a->dw, a->D);
    return sisa::launch_status("sisa_rmsnorm_bwd (dw)");
}

template <class T>
int launch_rmsnorm(const sisa_rmsnorm_args* a, int bwd, hipStream_t st) {
    const int nvl = (int)sisa::cdiv(a->D / 8, 64);
    if (nvl <= 1) return launch_rmsnorm_nvl<T, 1>(a, bwd, st);
    if (nvl <= 2) return launch_rmsnorm_nvl<T, 2>(a, bwd, st);
    if (nvl <= 4) return launch_rmsnorm_nvl<T, 4>(a, bwd, st);
    if (nvl <= 8) return launch_rmsnorm_nvl<T, 8>(a, bwd, st);
    return launch_rmsnorm_nvl<T, RMS_MAXV>(a, bwd, st);
}

template <class T>
int launch_swiglu(const sisa_swiglu_args* a, int bwd, hipStream_t st) {
    const int64_t nv = a->n / 8;
    const unsigned grid = (unsigned)(sisa::cdiv(nv, 256) < 8192 ? sisa::cdiv(nv, 256) : 8192);
    if (bwd) swiglu_bwd_kernel<T><<<grid, 256, 0, st>>>(*a);
    else swiglu_fwd_kernel<T><<<grid, 256, 0, st>>>(*a);
    return sisa::launch_status(bwd ? "sisa_swiglu_bwd" : "sisa_swiglu_fwd");
}

int check_rms(const sisa_rmsnorm_args* a, int bwd, const char* fn) {
    SISA_REQUIRE(a != nullptr, "%s: null args", fn);
    SISA_REQUIRE(a->N >= 0 && a->D >= 8 && a->D % 8 == 0 && a->D <= 64 * RMS_MAXV * 8,
                 "%s: row length D=%d must be a multiple of 8 in [8, %d]", fn, a->D, 64 * RMS_MAXV * 8);
    SISA_REQUIRE(a->dtype == SISA_BF16 || a->dtype == SISA_F16 || a->dtype == SISA_F32, "%s: dtype %d", fn, a->dtype);
    SISA_REQUIRE(a->x && a->w && sisa::aligned16(a->x) && sisa::aligned16(a->w) && a->sx % 8 == 0 && a->sx >= a->D,
                 "%s: x/w must be 16-byte aligned with a row stride >= D that is a multiple of 8", fn);
    if (!bwd) {
        SISA_REQUIRE(a->y && sisa::aligned16(a->y) && a->sy % 8 == 0 && a->sy >= a->D, "%s: bad y", fn);
    } else {
        SISA_REQUIRE(a->dy && a->dx && a->rstd && a->dw && a->dw_partial && sisa::aligned16(a->dy) &&
                         sisa::aligned16(a->dx) && sisa::aligned16(a->dw_partial) && a->sdy % 8 == 0 &&
                         a->sdx % 8 == 0 && a->sdy >= a->D && a->sdx >= a->D,
                     "%s: dy/dx/rstd/dw/dw_partial must be given, 16-byte aligned, row strides >= D and multiples of 8",
                     fn);
    }
    return SISA_OK;
}

}  // namespace

extern "C" int64_t sisa_rmsnorm_bwd_workspace_bytes(int64_t N, int32_t D) {
    return (sisa::cdiv(N, RMS_RPW) + DW_SPLIT) * (int64_t)D * (int64_t)sizeof(float);
}

extern "C" int sisa_rmsnorm_fwd(const sisa_rmsnorm_args* a, void* stream) {
    const int rc = check_rms(a, 0, "sisa_rmsnorm_fwd");
    if (rc) return rc;
    if (a->N == 0) return SISA_OK;
    hipStream_t st = (hipStream_t)stream;
    switch (a->dtype) {
        case SISA_BF16: return launch_rmsnorm<__bf16>(a, 0, st);
        case SISA_F16: return launch_rmsnorm<_Float16>(a, 0, st);
        default: return launch_rmsnorm<float>(a, 0, st);
    }
}

extern "C" int sisa_rmsnorm_bwd(const sisa_rmsnorm_args* a, void* stream) {
    const int rc = check_rms(a, 1, "sisa_rmsnorm_bwd");
    if (rc) return rc;
    hipStream_t st = (hipStream_t)stream;
    switch (a->dtype) {
        case SISA_BF16: return launch_rmsnorm<__bf16>(a, 1, st);
        case SISA_F16: return launch_rmsnorm<_Float16>(a, 1, st);
        default: return launch_rmsnorm<float>(a, 1, st);
    }
}

static int swiglu_entry(const sisa_swiglu_args* a, int bwd, void* stream) {
    const char* fn = bwd ? "sisa_swiglu_bwd" : "sisa_swiglu_fwd";
    SISA_REQUIRE(a != nullptr, "%s: null args", fn);
    SISA_REQUIRE(a->n >= 0 && a->n % 8 == 0, "%s: element count %lld must be a multiple of 8", fn, (long long)a->n);
    SISA_REQUIRE(a->dtype == SISA_BF16 || a->dtype == SISA_F16 || a->dtype == SISA_F32, "%s: dtype %d", fn, a->dtype);
    SISA_REQUIRE(a->a && a->b && sisa::aligned16(a->a) && sisa::aligned16(a->b), "%s: a/b must be 16-byte aligned",
                 fn);
    if (bwd)
        SISA_REQUIRE(a->dh && a->da && a->db && sisa::aligned16(a->dh) && sisa::aligned16(a->da) &&
                         sisa::aligned16(a->db),
                     "%s: dh/da/db must be given and 16-byte aligned", fn);
    else
        SISA_REQUIRE(a->h && sisa::aligned16(a->h), "%s: h must be given and 16-byte aligned", fn);
    if (a->n == 0) return SISA_OK;
    hipStream_t st = (hipStream_t)stream;
    switch (a->dtype) {
        case SISA_BF16: return launch_swiglu<__bf16>(a, bwd, st);
        case SISA_F16: return launch_swiglu<_Float16>(a, bwd, st);
        default: return launch_swiglu<float>(a, bwd, st);
    }
}

extern "C" int sisa_swiglu_fwd(const sisa_swiglu_args* a, void* stream) { return swiglu_entry(a, 0, stream); }
extern "C" int sisa_swiglu_bwd(const sisa_swiglu_args* a, void* stream) { return swiglu_entry(a, 1, stream); }
