// Row pass of the chunked linear cross-entropy (log-sum-exp, loss row, G written over the logits).
//
// Reference: `_lmce_row_kernel` (src/sisa/kernels/linear_ce.py:60-96), one program per token row that reads the row
// twice (online max / sum-exp, then G). Here one 512-thread workgroup owns a row; for rows of up to 65,536 columns the
// row is loaded once into registers (16-byte loads, 8 columns each, column-interleaved across threads so that every
// load instruction of the workgroup covers 8 KB of contiguous memory), reduced with a row max and one exp per column,
// and G is written from the registers: one HBM read and one write per element, the minimum for an in-place pass.
// Longer rows stream twice with a per-thread online max / sum-exp.
#include "common.h"
#include "host.h"

namespace {

constexpr int RT = 512;          // threads per row
constexpr int RW = RT / 64;      // waves per row
constexpr int COLS = RT * 8;     // columns covered by one 16-byte load of every thread

SISA_DEV float wave_max(float x) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x = nmax(x, __shfl_xor(x, o));
    return x;
}

SISA_DEV float wave_sum(float x) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
    return x;
}

// Row-wide reductions through LDS; `red` is reused, so each call ends with a barrier.
SISA_DEV float row_max(float x, float* red, int tid) {
    x = wave_max(x);
    if ((tid & 63) == 0) red[tid >> 6] = x;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int i = 1; i < RW; ++i) r = nmax(r, red[i]);
    __syncthreads();
    return r;
}

SISA_DEV float row_sum(float x, float* red, int tid) {
    x = wave_sum(x);
    if ((tid & 63) == 0) red[tid >> 6] = x;
    __syncthreads();
    float r = 0.f;
#pragma unroll
    for (int i = 0; i < RW; ++i) r += red[i];
    __syncthreads();
    return r;
}

// Keeps a loaded vector in its packed 16-bit form: without it the compiler holds the fp32 conversions of the whole
// row from one pass to the next (eight registers per vector instead of four).
template <class T>
SISA_DEV void keep_packed(frag8<T>& v) { asm volatile("" : "+v"(v)); }

// element j of an 8-column vector with nreal of its columns inside the real vocabulary; -inf beyond it
template <class T>
SISA_DEV float col_value(const frag8<T>& v, int j, int nreal) {
    return j < nreal ? (float)v[j] : -__builtin_inff();
}

// columns of the vector at col that lie inside the real vocabulary, in [0, 8]
SISA_DEV int real_cols(int col, int V) { return min(max(V - col, 0), 8); }

// Vectors wholly inside the real vocabulary (every one but the last of a row) take the branch-free forms below; the
// masked forms differ only in the columns they exclude, so both give the same value for a full vector.

// running maximum over a vector (fmaxf: a NaN logit still makes the row NaN, through its exponential in the sum)
template <class T>
SISA_DEV float vec_max(const frag8<T>& v, int col, int V, float m) {
    if (col + 8 <= V) {
#pragma unroll
        for (int j = 0; j < 8; ++j) m = fmaxf(m, (float)v[j]);
    } else {
        const int nreal = real_cols(col, V);
#pragma unroll
        for (int j = 0; j < 8; ++j) m = fmaxf(m, col_value<T>(v, j, nreal));
    }
    return m;
}

// running sum of exp(x - M) over a vector, in column order
template <class T>
SISA_DEV float vec_sumexp(const frag8<T>& v, int col, int V, float m2, float s) {
    if (col + 8 <= V) {
#pragma unroll
        for (int j = 0; j < 8; ++j) s += fast_exp2((float)v[j] * LOG2E - m2);
    } else {
        const int nreal = real_cols(col, V);
#pragma unroll
        for (int j = 0; j < 8; ++j) s += fast_exp2(col_value<T>(v, j, nreal) * LOG2E - m2);
    }
    return s;
}

template <class T>
SISA_DEV void store_grad(T* p, int col, const frag8<T>& v, int V, int hot, float lse2, float scale) {
    f32x4 lo, hi;
    if (col + 8 <= V && (unsigned)(hot - col) >= 8u) {   // no masked column, not the label's vector
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float g = fast_exp2((float)v[j] * LOG2E - lse2) * scale;
            if (j < 4) lo[j] = g; else hi[j - 4] = g;
        }
    } else {
        const int nreal = real_cols(col, V), jh = hot - col;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float e = fast_exp2(col_value<T>(v, j, nreal) * LOG2E - lse2);
            const float g = (e - (j == jh ? 1.f : 0.f)) * scale;
            if (j < 4) lo[j] = g; else hi[j - 4] = g;
        }
    }
    *reinterpret_cast<frag8<T>*>(p + col) = pack8<T>(lo, hi);
}

// NV > 0: the row is held in NV 16-byte vectors per thread (Vp <= NV * COLS). NV == 0: the row is streamed twice.
template <class T, int NV>
__global__ __launch_bounds__(RT) void lmce_rows_kernel(sisa_lmce_rows_args a) {
    __shared__ float red[RW];
    const int tid = threadIdx.x;
    const int64_t row = blockIdx.x;
    T* p = (T*)a.logits + row * a.stride;
    const int V = (int)a.V, Vp = (int)a.Vp;       // column counts fit in int (checked on the host)
    const int64_t lab = a.labels[row];
    const bool valid = lab != a.ignore_index;
    const bool inrange = lab >= 0 && lab < V;
    // the label's logit is read before the first barrier, so before any G store of this row
    const float tgt = (tid == 0 && valid && inrange) ? (float)p[lab] : 0.f;

    float M, S;
    frag8<T> x[NV > 0 ? NV : 1];
    if constexpr (NV > 0) {
        float m = -__builtin_inff();
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            const int col = v * COLS + 8 * tid;
            x[v] = col < Vp ? *reinterpret_cast<const frag8<T>*>(p + col) : zero8<T>();
        }
#pragma unroll
        for (int v = 0; v < NV; ++v) m = vec_max<T>(x[v], v * COLS + 8 * tid, V, m);
        M = row_max(m, red, tid);
#pragma unroll
        for (int v = 0; v < NV; ++v) keep_packed<T>(x[v]);
        const float m2 = M * LOG2E;
        float s = 0.f;
#pragma unroll
        for (int v = 0; v < NV; ++v) s = vec_sumexp<T>(x[v], v * COLS + 8 * tid, V, m2, s);
        S = row_sum(s, red, tid);
#pragma unroll
        for (int v = 0; v < NV; ++v) keep_packed<T>(x[v]);
    } else {
        // per-thread online max / sum-exp, one rescale per 8-column vector
        float m = -__builtin_inff(), s = 0.f;
        for (int col = 8 * tid; col < Vp; col += COLS) {
            const frag8<T> xv = *reinterpret_cast<const frag8<T>*>(p + col);
            const int nreal = real_cols(col, V);
            float lm = -__builtin_inff();
#pragma unroll
            for (int j = 0; j < 8; ++j) lm = nmax(lm, col_value<T>(xv, j, nreal));
            const float mn = nmax(m, lm);
            if (mn == -__builtin_inff()) continue;           // only masked columns so far: (m, s) stays (-inf, 0)
            float add = 0.f;
#pragma unroll
            for (int j = 0; j < 8; ++j) add += fast_exp2((col_value<T>(xv, j, nreal) - mn) * LOG2E);
            s = s * fast_exp2((m - mn) * LOG2E) + add;
            m = mn;
        }
        M = row_max(m, red, tid);
        S = row_sum(m == -__builtin_inff() ? 0.f : s * fast_exp2((m - M) * LOG2E), red, tid);
    }
    const float lse = M + __logf(S);
    if (tid == 0) {
        a.loss_rows[row] = valid ? (inrange ? lse - tgt : __builtin_nanf("")) : 0.f;
        if (a.lse) a.lse[row] = lse;
    }
    if (!a.compute_grad) return;
    const float scale = valid ? *a.inv_n * a.gscale : 0.f;
    const int hot = valid ? (inrange ? (int)lab : -8) : 0;     // ignored rows: column 0 (scaled by 0)
    const float lse2 = lse * LOG2E;
    if constexpr (NV > 0) {
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            const int col = v * COLS + 8 * tid;
            if (col < Vp) store_grad<T>(p, col, x[v], V, hot, lse2, scale);
        }
    } else {
        for (int col = 8 * tid; col < Vp; col += COLS)
            store_grad<T>(p, col, *reinterpret_cast<const frag8<T>*>(p + col), V, hot, lse2, scale);
    }
}

template <class T>
void launch_rows(const sisa_lmce_rows_args& a, hipStream_t st) {
    const int64_t need = (a.Vp + COLS - 1) / COLS;
    const dim3 grid((unsigned)a.T);
    if (need <= 4) lmce_rows_kernel<T, 4><<<grid, RT, 0, st>>>(a);
    else if (need <= 8) lmce_rows_kernel<T, 8><<<grid, RT, 0, st>>>(a);
    else if (need <= 16) lmce_rows_kernel<T, 16><<<grid, RT, 0, st>>>(a);
    else lmce_rows_kernel<T, 0><<<grid, RT, 0, st>>>(a);
}

}  // namespace

extern "C" int sisa_lmce_rows(const sisa_lmce_rows_args* a, void* stream) {
    SISA_REQUIRE(a != nullptr, "sisa_lmce_rows: null args");
    SISA_REQUIRE(a->dtype == SISA_BF16 || a->dtype == SISA_F16, "sisa_lmce_rows: dtype must be bf16 or fp16");
    SISA_REQUIRE(a->T >= 0 && a->T <= INT32_MAX, "sisa_lmce_rows: T = %lld out of range", (long long)a->T);
    if (a->T == 0) return SISA_OK;
    SISA_REQUIRE(a->V >= 1 && a->Vp >= a->V && a->Vp % 8 == 0 && a->Vp <= (1 << 30),
                 "sisa_lmce_rows: need 1 <= V <= Vp <= 2^30 and Vp a multiple of 8 (V=%lld Vp=%lld)", (long long)a->V,
                 (long long)a->Vp);
    SISA_REQUIRE(a->stride >= a->Vp && a->stride % 8 == 0,
                 "sisa_lmce_rows: row stride %lld must be >= Vp and a multiple of 8", (long long)a->stride);
    SISA_REQUIRE(a->logits && sisa::aligned16(a->logits), "sisa_lmce_rows: logits must be non-null and 16-byte aligned");
    SISA_REQUIRE(a->labels && a->loss_rows, "sisa_lmce_rows: labels and loss_rows are required");
    SISA_REQUIRE(!a->compute_grad || a->inv_n, "sisa_lmce_rows: inv_n is required when compute_grad is set");
    hipStream_t st = (hipStream_t)stream;
    if (a->dtype == SISA_BF16) launch_rows<__bf16>(*a, st);
    else launch_rows<_Float16>(*a, st);
    return sisa::launch_status("sisa_lmce_rows");
}
