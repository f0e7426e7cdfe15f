// Elementwise parts of the SISA decoder block for gfx950: RMSNorm with an optional fused projection of the normalised
// rows (the attention sublayer's forget-gate logits), its backward with deterministic weight gradients, and the SwiGLU
// activation silu(a) * b (forward, backward). All arithmetic in fp32.
//
// Reference: src/sisa/modeling.py:26-50 (RMSNorm computed in float32 with the output in the input dtype; SwiGLU as
// w_down(silu(w_gate x) * w_up x)) and modeling.py:166-169, 217-220 (the fused attention path projects the normalised
// input twice: the concatenated W_cat GEMM in the autocast dtype and the forget-gate logits z = n W_f^T + b_f in
// float32 with autocast off). The reference runs the norm, the autocast cast of n, the fp32 forget GEMM and, in the
// backward, their adjoints and the gradient sum as separate torch kernels; here
//   forward:  y = round_y(n), n = round_x((x * rstd) * w), z = n . W_f^T + b_f          one pass over x
//   backward: dn = dy + dz W_f (rounded as the reference's autograd sums it), dx, dw     one pass over x, dy
//             dW_f = dz^T n, db_f = sum dz  (fp32 MFMA over x, rstd)                   one more read of x
// with y in the dtype the consumer GEMM takes (the autocast dtype), so no separate cast pass exists.
//
// Work decomposition: a wave holds RB = 64 / HP rows (HP = the projection width padded to 16, 32 or 64) with NVL =
// HP / 8 eight-element vectors per lane (lane l holds elements 8 c .. 8 c + 7, c = l + 64 i), so RB * NVL = 8 and
// the row length is at most 512 NVL. For up to 16 outputs and rows of at most 768 (a multiple of 64) the projection
// and its adjoint run on the matrix cores: the workgroup's sixteen rows of n (of dz W_f) pass through LDS and each
// wave forms a quarter of the columns with v_mfma_f32_16x16x4_f32 (norm_fwd_mfma_kernel, norm_bwd_mfma_kernel).
// Otherwise a lane's RB * HP projection partial sums are reduced over the 64 lanes with a halving exchange (63
// shuffles): lane l ends with the total of row l / HP, output l % HP. Weight gradients are reduced in fixed order
// through caller-provided partials, the independent reductions of the backward sharing launches: bitwise
// reproducible, no atomics.
#include "common.h"
#include "host.h"

namespace {

constexpr int NORM_WAVES = 4;                // waves per workgroup
constexpr int NORM_RPW = 8;                  // backward: rows per wave = rows per dw partial row
constexpr int DW_SPLIT = 64;                 // backward: second-level dw partials per column
constexpr int WF_ROWS = 128;                 // backward: rows per dW_f partial (workgroup)
constexpr int WF_UNROLL = 16;                // backward: dW_f row steps (of 4 rows) whose loads go out together
constexpr int WF_TPW = 3;                    // backward: 16-column dW_f tiles per wave

template <class T> SISA_DEV float rnd(float x) { return (float)cvt<T>(x); }

SISA_DEV float wave_sum(float x) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
    return x;
}

// v[0..63] summed over the wave's 64 lanes by halving exchanges (step M: lanes with bit M set keep the upper half);
// afterwards v[0] of lane l holds the total of element l.
template <int M> SISA_DEV void reduce_scatter64(float (&v)[64], int lane) {
    const bool up = (lane & M) != 0;
#pragma unroll
    for (int k = 0; k < M; ++k) {
        const float send = up ? v[k] : v[k + M];
        const float keep = up ? v[k + M] : v[k];
        v[k] = keep + __shfl_xor(send, M);
    }
    if constexpr (M > 1) reduce_scatter64<M / 2>(v, lane);
}

// The projection weight W_f (H x D fp32) as the kernels read it: staged in LDS when HP = 16 (then H * D <= 16 *
// 1024 floats), else read through the caches.
template <int HP> struct WfSrc {
    static constexpr bool LDS = HP == 16;
    static constexpr int LDS_FLOATS = LDS ? 16 * 1024 : 1;
};

template <int HP>
SISA_DEV const float* stage_wf(const sisa_norm_args& a, float* lds) {
    if constexpr (WfSrc<HP>::LDS) {
        // all loads first (at most 16 per thread), then the LDS writes: one memory round trip
        constexpr int PER = WfSrc<HP>::LDS_FLOATS / 4 / (64 * NORM_WAVES);
        const int n4 = a.H * a.D / 4;
        f32x4 t[PER];
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const int k = threadIdx.x + 64 * NORM_WAVES * j;
            if (k < n4) t[j] = reinterpret_cast<const f32x4*>(a.wf)[k];
        }
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const int k = threadIdx.x + 64 * NORM_WAVES * j;
            if (k < n4) reinterpret_cast<f32x4*>(lds)[k] = t[j];
        }
        __syncthreads();
        return lds;
    } else {
        return a.wf;
    }
}

// ------------------------------------------------------------------------------------------------ RMSNorm forward
template <class TX, class TY, int HP>
__global__ __launch_bounds__(64 * NORM_WAVES) void norm_fwd_kernel(sisa_norm_args a) {
    constexpr int RB = 64 / HP, NVL = HP / 8;
    __shared__ float wlds[WfSrc<HP>::LDS_FLOATS];
    const int lane = threadIdx.x & 63;
    const int64_t r0 = ((int64_t)blockIdx.x * NORM_WAVES + (threadIdx.x >> 6)) * RB;
    const int nv = a.D / 8;
    // the rows are loaded first, so that their latency overlaps the staging of W_f
    f32x8 n[RB][NVL];
#pragma unroll
    for (int r = 0; r < RB; ++r) {
        const int64_t row = r0 + r;
#pragma unroll
        for (int i = 0; i < NVL; ++i) {
            const int c = lane + 64 * i;
            if (row < a.N && c < nv) {
                n[r][i] = load_f32x8<TX>((const TX*)a.x + row * a.sx + 8 * c);
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) n[r][i][e] = 0.f;
            }
        }
    }
    if (a.res) {   // h = x + res, rounded to x's dtype as the residual add, normalised in place of x
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            const int64_t row = r0 + r;
#pragma unroll
            for (int i = 0; i < NVL; ++i) {
                const int c = lane + 64 * i;
                if (row < a.N && c < nv) {
                    const f32x8 rv = load_f32x8<TY>((const TY*)a.res + row * a.sres + 8 * c);
#pragma unroll
                    for (int e = 0; e < 8; ++e) n[r][i][e] = rnd<TX>(n[r][i][e] + rv[e]);
                    store_f32x8<TX>((TX*)a.h + row * a.sh + 8 * c, n[r][i]);
                }
            }
        }
    }
    const float* wf = a.H > 0 ? stage_wf<HP>(a, wlds) : nullptr;
    if (r0 >= a.N) return;
    float rstd[RB];
#pragma unroll
    for (int r = 0; r < RB; ++r) {
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < NVL; ++i)
#pragma unroll
            for (int e = 0; e < 8; ++e) ss = fmaf(n[r][i][e], n[r][i][e], ss);
        rstd[r] = 1.f / sqrtf(wave_sum(ss) / (float)a.D + a.eps);
    }
#pragma unroll
    for (int i = 0; i < NVL; ++i) {
        const int c = lane + 64 * i;
        if (c < nv) {
            const f32x8 w = load_f32x8<float>(a.w + 8 * c);
#pragma unroll
            for (int r = 0; r < RB; ++r) {
#pragma unroll
                for (int e = 0; e < 8; ++e) n[r][i][e] = rnd<TX>((n[r][i][e] * rstd[r]) * w[e]);
                if (r0 + r < a.N) store_f32x8<TY>((TY*)a.y + (r0 + r) * a.sy + 8 * c, n[r][i]);
            }
        }
    }
    if (a.rstd && lane < RB && r0 + lane < a.N) {
        float rs = rstd[0];
#pragma unroll
        for (int r = 1; r < RB; ++r)
            if (lane == r) rs = rstd[r];
        a.rstd[r0 + lane] = rs;
    }
    if (a.H == 0) return;
    // z[row][h] = n[row] . W_f[h] + b_f[h]: per-lane partial sums of all RB * HP outputs, then one reduce-scatter
    float v[64];
#pragma unroll
    for (int k = 0; k < 64; ++k) v[k] = 0.f;
#pragma unroll
    for (int h = 0; h < HP; ++h) {
        if (h < a.H) {
#pragma unroll
            for (int i = 0; i < NVL; ++i) {
                const int c = lane + 64 * i;
                if (c < nv) {
                    const f32x8 wv = load_f32x8<float>(wf + h * a.D + 8 * c);
#pragma unroll
                    for (int r = 0; r < RB; ++r)
#pragma unroll
                        for (int e = 0; e < 8; ++e) v[r * HP + h] = fmaf(n[r][i][e], wv[e], v[r * HP + h]);
                }
            }
        }
    }
    reduce_scatter64<32>(v, lane);
    const float t = v[0];
    const int64_t row = r0 + lane / HP;
    const int h = lane % HP;
    if (row < a.N && h < a.H) a.z[row * a.H + h] = t + a.bf[h];
}

// Forward with the projection on the matrix cores, for 0 < H <= 16 and D a multiple of 64 up to MFMA_DMAX: the
// normalisation as above (four rows per wave, sixteen per workgroup), then the workgroup's sixteen rows of n go to LDS
// and wave w forms the 16 x 16 partial z tile of columns [w D/4, (w+1) D/4) with v_mfma_f32_16x16x4_f32 (A = n: lane l
// holds row l % 16 and reads four consecutive columns with one 16-byte LDS read, one per MFMA of the step; B = W_f:
// the same four columns of row l % 16 of W_f), and the four partial tiles are summed in wave order (in the LDS
// space of n once every wave is done with it).
constexpr int MFMA_DMAX = 768;                  // W_f operand of at most 12 steps in registers
constexpr int NL_PAD = 4;                       // row padding of the staged n: conflict-free 16-byte reads
inline int64_t norm_mfma_lds_bytes(int D) { return (int64_t)16 * (D + NL_PAD) * (int64_t)sizeof(float); }
template <class TX, class TY>
__global__ __launch_bounds__(64 * NORM_WAVES) void norm_fwd_mfma_kernel(sisa_norm_args a) {
    constexpr int RB = 4, NVL = 2;
    extern __shared__ __attribute__((aligned(16))) float dyn_lds[];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int D = a.D, ld = D + NL_PAD, nv = D / 8;
    float* nl = dyn_lds;                                   // [16][ld]: n of the workgroup's rows
    f32x4* red = reinterpret_cast<f32x4*>(dyn_lds);        // then [NORM_WAVES][64]: the partial tiles
    const int64_t g0 = (int64_t)blockIdx.x * 16;
    const int64_t r0 = g0 + w * RB;
    f32x8 n[RB][NVL];
#pragma unroll
    for (int r = 0; r < RB; ++r) {
        const int64_t row = r0 + r;
#pragma unroll
        for (int i = 0; i < NVL; ++i) {
            const int c = lane + 64 * i;
            if (row < a.N && c < nv) {
                n[r][i] = load_f32x8<TX>((const TX*)a.x + row * a.sx + 8 * c);
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) n[r][i][e] = 0.f;
            }
        }
    }
    // W_f operand of the wave's columns: step q, lane l -> W_f[l % 16][w D/4 + 16 q + 4 (l / 16) .. + 3]
    const int hq = lane & 15, kg = lane >> 4;
    const int nq = D / 64;                                 // 16-column steps per wave
    const int cw = w * (D / 4) + 4 * kg;
    f32x4 wb[MFMA_DMAX / 64];
#pragma unroll
    for (int q = 0; q < MFMA_DMAX / 64; ++q)
        wb[q] = (q < nq && hq < a.H) ? *reinterpret_cast<const f32x4*>(a.wf + (int64_t)hq * D + cw + 16 * q)
                                     : f32x4{0.f, 0.f, 0.f, 0.f};
    if (a.res) {   // h = x + res, rounded to x's dtype as the residual add, normalised in place of x
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            const int64_t row = r0 + r;
#pragma unroll
            for (int i = 0; i < NVL; ++i) {
                const int c = lane + 64 * i;
                if (row < a.N && c < nv) {
                    const f32x8 rv = load_f32x8<TY>((const TY*)a.res + row * a.sres + 8 * c);
#pragma unroll
                    for (int e = 0; e < 8; ++e) n[r][i][e] = rnd<TX>(n[r][i][e] + rv[e]);
                    store_f32x8<TX>((TX*)a.h + row * a.sh + 8 * c, n[r][i]);
                }
            }
        }
    }
    float rstd[RB];
#pragma unroll
    for (int r = 0; r < RB; ++r) {
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < NVL; ++i)
#pragma unroll
            for (int e = 0; e < 8; ++e) ss = fmaf(n[r][i][e], n[r][i][e], ss);
        rstd[r] = 1.f / sqrtf(wave_sum(ss) / (float)D + a.eps);
    }
#pragma unroll
    for (int i = 0; i < NVL; ++i) {
        const int c = lane + 64 * i;
        if (c < nv) {
            const f32x8 wv = load_f32x8<float>(a.w + 8 * c);
#pragma unroll
            for (int r = 0; r < RB; ++r) {
#pragma unroll
                for (int e = 0; e < 8; ++e) n[r][i][e] = rnd<TX>((n[r][i][e] * rstd[r]) * wv[e]);
                if (r0 + r < a.N) store_f32x8<TY>((TY*)a.y + (r0 + r) * a.sy + 8 * c, n[r][i]);
                float* dst = nl + (w * RB + r) * ld + 8 * c;
                *reinterpret_cast<f32x4*>(dst) = f32x4{n[r][i][0], n[r][i][1], n[r][i][2], n[r][i][3]};
                *reinterpret_cast<f32x4*>(dst + 4) = f32x4{n[r][i][4], n[r][i][5], n[r][i][6], n[r][i][7]};
            }
        }
    }
    if (a.rstd && lane < RB && r0 + lane < a.N) {
        float rs = rstd[0];
#pragma unroll
        for (int r = 1; r < RB; ++r)
            if (lane == r) rs = rstd[r];
        a.rstd[r0 + lane] = rs;
    }
    __syncthreads();
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    const float* arow = nl + hq * ld + cw;
#pragma unroll
    for (int q = 0; q < MFMA_DMAX / 64; ++q) {
        if (q < nq) {
            const f32x4 av = *reinterpret_cast<const f32x4*>(arow + 16 * q);
#pragma unroll
            for (int t = 0; t < 4; ++t) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[t], wb[q][t], acc, 0, 0, 0);
        }
    }
    __syncthreads();   // every wave is done reading n
    red[w * 64 + lane] = acc;
    __syncthreads();
    if (w != 0) return;
    // lane l holds rows 4 (l / 16) + v of the tile for output h = l % 16
    f32x4 z = red[lane];
#pragma unroll
    for (int k = 1; k < NORM_WAVES; ++k) z += red[k * 64 + lane];
    if (hq < a.H) {
        const float bh = a.bf[hq];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int64_t row = g0 + 4 * kg + v;
            if (row < a.N) a.z[row * a.H + hq] = z[v] + bh;
        }
    }
}

// ------------------------------------------------------------------------------------------------ RMSNorm backward
// dn = dy + dz W_f (the projection term summed first, then added to dy, as autograd sums the two adjoints; for a
// 16-bit x both roundings to x's dtype are kept: dn = round_x(dy + round_x(dz W_f))), du = dn * w, u = x * rstd,
// dx = rstd * (du - u * mean(du * u)), dw += dn * u. Each wave owns NORM_RPW consecutive rows (RB at a time) and
// writes their dw contribution as one partial row.
template <class TX, class TY, int HP>
__global__ __launch_bounds__(64 * NORM_WAVES) void norm_bwd_kernel(sisa_norm_args a, float* __restrict__ dw_part) {
    constexpr int RB = 64 / HP, NVL = HP / 8;
    constexpr bool WREG = NVL <= 2;                    // norm weight held in registers
    __shared__ float wlds[WfSrc<HP>::LDS_FLOATS];
    const int lane = threadIdx.x & 63;
    const int64_t p = (int64_t)blockIdx.x * NORM_WAVES + (threadIdx.x >> 6);   // partial row = wave
    const int nv = a.D / 8;
    f32x8 u[RB][NVL];
    auto load_rows = [&](int64_t r0) {
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            const int64_t row = r0 + r;
#pragma unroll
            for (int i = 0; i < NVL; ++i) {
                const int c = lane + 64 * i;
                if (row < a.N && c < nv) {
                    u[r][i] = load_f32x8<TX>((const TX*)a.x + row * a.sx + 8 * c);
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e) u[r][i][e] = 0.f;
                }
            }
        }
    };
    load_rows(p * NORM_RPW);                           // in flight while W_f is staged
    const float* wf = a.H > 0 ? stage_wf<HP>(a, wlds) : nullptr;
    if (p * NORM_RPW >= a.N) return;
    f32x8 wreg[WREG ? NVL : 1], dwacc[NVL];
#pragma unroll
    for (int i = 0; i < NVL; ++i) {
        const int c = lane + 64 * i;
        if constexpr (WREG) {
            if (c < nv) wreg[i] = load_f32x8<float>(a.w + 8 * c);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) dwacc[i][e] = 0.f;
    }
#pragma unroll 1
    for (int it = 0; it < NORM_RPW / RB; ++it) {
        const int64_t r0 = p * NORM_RPW + it * RB;
        if (r0 >= a.N) break;
        if (it > 0) load_rows(r0);
        f32x8 dn[RB][NVL];
        float rstd[RB];
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            rstd[r] = r0 + r < a.N ? a.rstd[r0 + r] : 0.f;
#pragma unroll
            for (int i = 0; i < NVL; ++i)
#pragma unroll
                for (int e = 0; e < 8; ++e) dn[r][i][e] = 0.f;
        }
        if (a.H > 0) {
            // lane l loads dz of (row r0 + l / HP, output l % HP); readlane broadcasts each value
            const int64_t zr = r0 + lane / HP;
            const int zh = lane % HP;
            const float dzl = (zr < a.N && zh < a.H) ? a.dz[zr * a.H + zh] : 0.f;
#pragma unroll 4
            for (int h = 0; h < a.H; ++h) {
#pragma unroll
                for (int i = 0; i < NVL; ++i) {
                    const int c = lane + 64 * i;
                    if (c < nv) {
                        const f32x8 wv = load_f32x8<float>(wf + h * a.D + 8 * c);
#pragma unroll
                        for (int r = 0; r < RB; ++r) {
                            const float dzv =
                                __int_as_float(__builtin_amdgcn_readlane(__float_as_int(dzl), r * HP + h));
#pragma unroll
                            for (int e = 0; e < 8; ++e) dn[r][i][e] = fmaf(dzv, wv[e], dn[r][i][e]);
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            const int64_t row = r0 + r;
            float dot = 0.f;
#pragma unroll
            for (int i = 0; i < NVL; ++i) {
                const int c = lane + 64 * i;
                if (row < a.N && c < nv) {
                    const f32x8 g = load_f32x8<TY>((const TY*)a.dy + row * a.sdy + 8 * c);
                    const f32x8 w = WREG ? wreg[WREG ? i : 0] : load_f32x8<float>(a.w + 8 * c);
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const float d = sizeof(TX) == 4 ? g[e] + dn[r][i][e] : rnd<TX>(g[e] + rnd<TX>(dn[r][i][e]));
                        u[r][i][e] *= rstd[r];
                        dwacc[i][e] = fmaf(d, u[r][i][e], dwacc[i][e]);
                        dn[r][i][e] = d * w[e];                       // du
                        dot = fmaf(dn[r][i][e], u[r][i][e], dot);
                    }
                }
            }
            const float mdot = wave_sum(dot) / (float)a.D;
            if (row < a.N) {
#pragma unroll
                for (int i = 0; i < NVL; ++i) {
                    const int c = lane + 64 * i;
                    if (c < nv) {
                        f32x8 o;
#pragma unroll
                        for (int e = 0; e < 8; ++e) o[e] = rstd[r] * (dn[r][i][e] - u[r][i][e] * mdot);
                        if (a.dh) {   // plus the residual stream's gradient of h, summed in x's dtype
                            const f32x8 hv = load_f32x8<TX>((const TX*)a.dh + row * a.sdh + 8 * c);
#pragma unroll
                            for (int e = 0; e < 8; ++e) o[e] = rnd<TX>(o[e]) + hv[e];
                        }
                        store_f32x8<TX>((TX*)a.dx + row * a.sdx + 8 * c, o);
                    }
                }
            }
        }
    }
    float* dwp = dw_part + p * a.D;
#pragma unroll
    for (int i = 0; i < NVL; ++i) {
        const int c = lane + 64 * i;
        if (c < nv) store_f32x8<float>(dwp + 8 * c, dwacc[i]);
    }
}

// Backward with the projection's adjoint on the matrix cores (the shapes of norm_fwd_mfma_kernel): per step of four
// rows per wave the workgroup's sixteen rows of dz W_f are formed as (W_f^T dz^T) tiles, wave w the columns [w D/4,
// (w+1) D/4), with v_mfma_f32_16x16x4_f32 (A = W_f^T: lane l holds column l % 16 of the tile for the four outputs
// 4 s + l / 16 of K-step s; B = dz^T of tile row l % 16), so that a lane ends with four consecutive columns of one row,
// stored to LDS as one 16-byte write; the row pass then reads its rows' products from there. Every wave takes part
// in both steps (its rows past the end contribute zeros), so the barriers see the whole workgroup.
template <class TX, class TY>
__global__ __launch_bounds__(64 * NORM_WAVES) void norm_bwd_mfma_kernel(sisa_norm_args a, float* __restrict__ dw_part) {
    constexpr int RB = 4, NVL = 2;
    extern __shared__ __attribute__((aligned(16))) float dyn_lds[];   // [16][D + NL_PAD]: dz W_f of the step's rows
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int D = a.D, ld = D + NL_PAD, nv = D / 8;
    const int64_t pw0 = (int64_t)blockIdx.x * NORM_WAVES;
    const int64_t p = pw0 + w;                         // partial row = wave
    f32x8 u[RB][NVL];
    auto load_rows = [&](int64_t r0) {
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            const int64_t row = r0 + r;
#pragma unroll
            for (int i = 0; i < NVL; ++i) {
                const int c = lane + 64 * i;
                if (row < a.N && c < nv) {
                    u[r][i] = load_f32x8<TX>((const TX*)a.x + row * a.sx + 8 * c);
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e) u[r][i][e] = 0.f;
                }
            }
        }
    };
    load_rows(p * NORM_RPW);
    // W_f^T operand: step q, K-step s, lane l -> W_f[4 s + l / 16][w D/4 + 16 q + l % 16]
    const int jq = lane & 15, kg = lane >> 4;
    const int nq = D / 64;
    const int cw = w * (D / 4) + jq;
    f32x4 wa[MFMA_DMAX / 64];
#pragma unroll
    for (int q = 0; q < MFMA_DMAX / 64; ++q)
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2) {
            const int h = 4 * s2 + kg;
            wa[q][s2] = (q < nq && h < a.H) ? a.wf[(int64_t)h * D + cw + 16 * q] : 0.f;
        }
    f32x8 wreg[NVL], dwacc[NVL];
#pragma unroll
    for (int i = 0; i < NVL; ++i) {
        const int c = lane + 64 * i;
        if (c < nv) wreg[i] = load_f32x8<float>(a.w + 8 * c);
#pragma unroll
        for (int e = 0; e < 8; ++e) dwacc[i][e] = 0.f;
    }
#pragma unroll 1
    for (int it = 0; it < NORM_RPW / RB; ++it) {
        const int64_t r0 = p * NORM_RPW + it * RB;
        if (it > 0) load_rows(r0);
        float rstd[RB];
#pragma unroll
        for (int r = 0; r < RB; ++r) rstd[r] = r0 + r < a.N ? a.rstd[r0 + r] : 0.f;
        // dz^T operand of tile row jq: row (pw0 + jq / 4) * NORM_RPW + it * RB + jq % 4, outputs 4 s + kg
        const int64_t zrow = (pw0 + (jq >> 2)) * NORM_RPW + it * RB + (jq & 3);
        float dzb[4];
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2) {
            const int h = 4 * s2 + kg;
            dzb[s2] = (zrow < a.N && h < a.H) ? a.dz[zrow * a.H + h] : 0.f;
        }
        if (it > 0) __syncthreads();                   // every wave is done reading the previous products
#pragma unroll
        for (int q = 0; q < MFMA_DMAX / 64; ++q) {
            if (q < nq) {
                f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int s2 = 0; s2 < 4; ++s2) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(wa[q][s2], dzb[s2], acc, 0, 0, 0);
                // lane l: columns w D/4 + 16 q + 4 (l / 16) .. + 3 of tile row l % 16
                *reinterpret_cast<f32x4*>(dyn_lds + jq * ld + w * (D / 4) + 16 * q + 4 * kg) = acc;
            }
        }
        __syncthreads();
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            const int64_t row = r0 + r;
            const float* pr = dyn_lds + (w * RB + r) * ld;
            float dot = 0.f;
            f32x8 dn[NVL];
#pragma unroll
            for (int i = 0; i < NVL; ++i) {
                const int c = lane + 64 * i;
                if (row < a.N && c < nv) {
                    const f32x8 g = load_f32x8<TY>((const TY*)a.dy + row * a.sdy + 8 * c);
                    const f32x4 plo = *reinterpret_cast<const f32x4*>(pr + 8 * c);
                    const f32x4 phi = *reinterpret_cast<const f32x4*>(pr + 8 * c + 4);
                    const f32x8 pj = {plo[0], plo[1], plo[2], plo[3], phi[0], phi[1], phi[2], phi[3]};
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const float d = sizeof(TX) == 4 ? g[e] + pj[e] : rnd<TX>(g[e] + rnd<TX>(pj[e]));
                        u[r][i][e] *= rstd[r];
                        dwacc[i][e] = fmaf(d, u[r][i][e], dwacc[i][e]);
                        dn[i][e] = d * wreg[i][e];                     // du
                        dot = fmaf(dn[i][e], u[r][i][e], dot);
                    }
                }
            }
            const float mdot = wave_sum(dot) / (float)D;
            if (row < a.N) {
#pragma unroll
                for (int i = 0; i < NVL; ++i) {
                    const int c = lane + 64 * i;
                    if (c < nv) {
                        f32x8 o;
#pragma unroll
                        for (int e = 0; e < 8; ++e) o[e] = rstd[r] * (dn[i][e] - u[r][i][e] * mdot);
                        if (a.dh) {   // plus the residual stream's gradient of h, summed in x's dtype
                            const f32x8 hv = load_f32x8<TX>((const TX*)a.dh + row * a.sdh + 8 * c);
#pragma unroll
                            for (int e = 0; e < 8; ++e) o[e] = rnd<TX>(o[e]) + hv[e];
                        }
                        store_f32x8<TX>((TX*)a.dx + row * a.sdx + 8 * c, o);
                    }
                }
            }
        }
    }
    if (p * NORM_RPW >= a.N) return;
    float* dwp = dw_part + p * D;
#pragma unroll
    for (int i = 0; i < NVL; ++i) {
        const int c = lane + 64 * i;
        if (c < nv) store_f32x8<float>(dwp + 8 * c, dwacc[i]);
    }
}

// dW_f partials: workgroup (column block bx, row block by, output block bz of 16) computes
// P[h][f] = sum over its WF_ROWS rows of dz[row][h] * n[row][f] with v_mfma_f32_16x16x4_f32 (A = dz^T, 16 outputs x
// 4 rows; B = n, 4 rows x 16 columns; n recomputed as round_x((x * rstd) * w)); wave w owns WF_TPW column tiles.
// The workgroup of column block 0 also writes the row block's sum of dz.
template <class TX>
SISA_DEV void forget_dw_block(const sisa_norm_args& a, float* __restrict__ part, float* __restrict__ dbpart, int bx,
                              int by, int bz) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int kr = lane >> 4, col = lane & 15;
    const int hp = 16 * ((a.H + 15) / 16);
    const int h = 16 * bz + col;                       // A operand: output index of this lane
    const int64_t rb0 = (int64_t)by * WF_ROWS;
    const int f0 = (bx * NORM_WAVES + w) * 16 * WF_TPW;
    float wv[WF_TPW];
#pragma unroll
    for (int t = 0; t < WF_TPW; ++t) {
        const int f = f0 + 16 * t + col;
        wv[t] = f < a.D ? a.w[f] : 0.f;
    }
    f32x4 acc[WF_TPW];
#pragma unroll
    for (int t = 0; t < WF_TPW; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    float dbs = 0.f;
#pragma unroll 1
    for (int rs0 = 0; rs0 < WF_ROWS; rs0 += 4 * WF_UNROLL) {
        // all loads of WF_UNROLL steps first (dz, rstd and WF_TPW x values per step), then the MFMAs
        float dzv[WF_UNROLL], rsv[WF_UNROLL], xv[WF_UNROLL][WF_TPW];
#pragma unroll
        for (int k = 0; k < WF_UNROLL; ++k) {
            const int64_t row = rb0 + rs0 + 4 * k + kr;
            const bool rok = row < a.N;
            dzv[k] = (rok && h < a.H) ? a.dz[row * a.H + h] : 0.f;
            rsv[k] = rok ? a.rstd[row] : 0.f;
#pragma unroll
            for (int t = 0; t < WF_TPW; ++t) {
                const int f = f0 + 16 * t + col;
                xv[k][t] = (rok && f < a.D) ? (float)((const TX*)a.x)[row * a.sx + f] : 0.f;
            }
        }
#pragma unroll
        for (int k = 0; k < WF_UNROLL; ++k) {
            dbs += dzv[k];
#pragma unroll
            for (int t = 0; t < WF_TPW; ++t)
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(dzv[k], rnd<TX>((xv[k][t] * rsv[k]) * wv[t]), acc[t],
                                                              0, 0, 0);
        }
    }
    // D layout: lane l, register i -> output 4 (l / 16) + i of this block, column f0 + 16 t + l % 16
    float* P = part + (int64_t)by * hp * a.D;
#pragma unroll
    for (int t = 0; t < WF_TPW; ++t) {
        const int f = f0 + 16 * t + col;
        if (f < a.D)
#pragma unroll
            for (int i = 0; i < 4; ++i) P[(int64_t)(16 * bz + 4 * kr + i) * a.D + f] = acc[t][i];
    }
    if (bx == 0 && w == 0) {
        dbs += __shfl_xor(dbs, 16);
        dbs += __shfl_xor(dbs, 32);
        if (kr == 0) dbpart[(int64_t)by * hp + h] = dbs;
    }
}

// s + p[0] + p[stride] + ... + p[(n-1) stride], added in that order; the loads go out BATCH at a time ahead of their
// adds (a load-add chain would wait for every load in turn).
template <int BATCH = 16>
SISA_DEV float ordered_sum(const float* __restrict__ p, int64_t stride, int64_t n, float s) {
    int64_t k = 0;
    for (; k + BATCH <= n; k += BATCH) {
        float t[BATCH];
#pragma unroll
        for (int e = 0; e < BATCH; ++e) t[e] = __builtin_nontemporal_load(p + (k + e) * stride);
#pragma unroll
        for (int e = 0; e < BATCH; ++e) s += t[e];
    }
    for (; k < n; ++k) s += p[k * stride];
    return s;
}

// Column sums of a (rows, cols) fp32 matrix in row order, split over DW_SPLIT row ranges: level 2 writes
// part2[split][col], level 3 sums the splits.
SISA_DEV void colsum2_block(const float* __restrict__ part, float* __restrict__ part2, int64_t rows, int cols, int bx,
                            int by) {
    const int c = bx * 256 + threadIdx.x;
    if (c >= cols) return;
    const int64_t per = (rows + DW_SPLIT - 1) / DW_SPLIT;
    const int64_t k0 = by * per, k1 = k0 + per < rows ? k0 + per : rows;
    part2[(int64_t)by * cols + c] = k1 > k0 ? ordered_sum<32>(part + k0 * cols + c, cols, k1 - k0, 0.f) : 0.f;
}

SISA_DEV void colsum3_block(const float* __restrict__ part2, float* __restrict__ out, int cols, int bx) {
    const int c = bx * 256 + threadIdx.x;
    if (c >= cols) return;
    out[c] = ordered_sum<64>(part2 + c, cols, DW_SPLIT, 0.f);
}

// dW_f[h][f] (and db_f[h]) = sum over the row-block partials in order.
SISA_DEV void forget_dw_final_block(const sisa_norm_args& a, const float* __restrict__ part,
                                    const float* __restrict__ dbpart, int nrb, int bx) {
    const int64_t idx = (int64_t)bx * 256 + threadIdx.x;
    const int hp = 16 * ((a.H + 15) / 16);
    if (idx < (int64_t)a.H * a.D) {
        const int h = (int)(idx / a.D), f = (int)(idx % a.D);
        a.dwf[idx] = ordered_sum<64>(part + (int64_t)h * a.D + f, (int64_t)hp * a.D, nrb, 0.f);
    }
    if (bx == 0 && threadIdx.x < a.H) a.dbf[threadIdx.x] = ordered_sum<64>(dbpart + threadIdx.x, hp, nrb, 0.f);
}

// Workspace of the backward: per-wave dw partial rows, their DW_SPLIT second-level sums, the dW_f and db_f partials
// of the row blocks.
struct NormWs {
    float *dw_part, *dw_part2, *wf_part, *db_part;
};

// The reductions after the row pass run as two launches whose workgroups take different jobs (all are independent
// within a launch): the second has the dW_f partial workgroups (nf of them; grid nfx x nfy x nfz, numbered x
// fastest) and the level-2 dw column sums (DW_SPLIT x ceil(D / 256) workgroups); the third the level-3 dw sums and
// the dW_f / db_f totals.
template <class TX>
__global__ __launch_bounds__(256) void norm_dw_stage2_kernel(sisa_norm_args a, NormWs ws, int64_t np, int nfx, int nfy,
                                                            int nfz) {
    const int64_t nf = (int64_t)nfx * nfy * nfz;
    const int64_t b = blockIdx.x;
    if (b < nf) {
        forget_dw_block<TX>(a, ws.wf_part, ws.db_part, (int)(b % nfx), (int)((b / nfx) % nfy), (int)(b / ((int64_t)nfx * nfy)));
        return;
    }
    const int cb = (int)(b - nf), nc = (a.D + 255) / 256;
    colsum2_block(ws.dw_part, ws.dw_part2, np, a.D, cb % nc, cb / nc);
}

__global__ __launch_bounds__(256) void norm_dw_final_kernel(sisa_norm_args a, NormWs ws, int nrb) {
    const int nc = (a.D + 255) / 256;
    if ((int)blockIdx.x < nc) {
        colsum3_block(ws.dw_part2, a.dw, a.D, blockIdx.x);
        return;
    }
    forget_dw_final_block(a, ws.wf_part, ws.db_part, nrb, (int)blockIdx.x - nc);
}

// ------------------------------------------------------------------------------------------------ host side
int norm_hp(const sisa_norm_args* a) {
    const int nvl = (int)sisa::cdiv(a->D / 8, 64);
    int hp = 16;
    while (hp < a->H || hp < 8 * nvl) hp *= 2;
    return hp;
}

int64_t norm_nrb(int64_t N) { return sisa::cdiv(N, WF_ROWS); }

NormWs norm_ws(const sisa_norm_args* a) {
    NormWs w;
    const int64_t np = sisa::cdiv(a->N, NORM_RPW);
    const int hp = 16 * (int)sisa::cdiv(a->H, 16);
    w.dw_part = a->workspace;
    w.dw_part2 = w.dw_part + np * a->D;
    w.wf_part = w.dw_part2 + (int64_t)DW_SPLIT * a->D;
    w.db_part = w.wf_part + norm_nrb(a->N) * hp * a->D;
    return w;
}

int64_t norm_ws_floats(int64_t N, int32_t D, int32_t H) {
    const int64_t np = sisa::cdiv(N, NORM_RPW);
    const int64_t hp = H > 0 ? 16 * sisa::cdiv(H, 16) : 0;
    return np * D + (int64_t)DW_SPLIT * D + (H > 0 ? norm_nrb(N) * hp * (D + 1) : 0);
}

template <class TX, class TY, int HP>
int launch_norm_hp(const sisa_norm_args* a, int bwd, hipStream_t st) {
    constexpr int RB = 64 / HP;
    if (!bwd) {
        if (HP == 16 && a->H > 0 && a->D % 64 == 0 && a->D <= MFMA_DMAX) {
            norm_fwd_mfma_kernel<TX, TY><<<(unsigned)sisa::cdiv(a->N, 16), 64 * NORM_WAVES,
                                           (size_t)norm_mfma_lds_bytes(a->D), st>>>(*a);
            return sisa::launch_status("sisa_norm_fwd");
        }
        const int64_t waves = sisa::cdiv(a->N, RB);
        norm_fwd_kernel<TX, TY, HP><<<(unsigned)sisa::cdiv(waves, NORM_WAVES), 64 * NORM_WAVES, 0, st>>>(*a);
        return sisa::launch_status("sisa_norm_fwd");
    }
    const NormWs ws = norm_ws(a);
    const int64_t np = sisa::cdiv(a->N, NORM_RPW);
    if (HP == 16 && a->H > 0 && a->D % 64 == 0 && a->D <= MFMA_DMAX)
        norm_bwd_mfma_kernel<TX, TY><<<(unsigned)sisa::cdiv(np, NORM_WAVES), 64 * NORM_WAVES,
                                       (size_t)norm_mfma_lds_bytes(a->D), st>>>(*a, ws.dw_part);
    else
        norm_bwd_kernel<TX, TY, HP><<<(unsigned)sisa::cdiv(np, NORM_WAVES), 64 * NORM_WAVES, 0, st>>>(*a, ws.dw_part);
    int rc = sisa::launch_status("sisa_norm_bwd");
    if (rc) return rc;
    const int nrb = (int)norm_nrb(a->N);
    const int nfx = a->H > 0 ? (int)sisa::cdiv(a->D, 16 * WF_TPW * NORM_WAVES) : 0, nfz = (int)sisa::cdiv(a->H, 16);
    const int64_t nf = (int64_t)nfx * nrb * nfz, nc = sisa::cdiv(a->D, 256);
    norm_dw_stage2_kernel<TX><<<(unsigned)(nf + nc * DW_SPLIT), 256, 0, st>>>(*a, ws, np, nfx, nrb, nfz);
    rc = sisa::launch_status("sisa_norm_bwd (dw, dW_f partials)");
    if (rc) return rc;
    const int64_t nfin = a->H > 0 ? sisa::cdiv((int64_t)a->H * a->D, 256) : 0;
    norm_dw_final_kernel<<<(unsigned)(nc + nfin), 256, 0, st>>>(*a, ws, nrb);
    return sisa::launch_status("sisa_norm_bwd (dw, dW_f totals)");
}

template <class TX, class TY>
int launch_norm(const sisa_norm_args* a, int bwd, hipStream_t st) {
    switch (norm_hp(a)) {
        case 16: return launch_norm_hp<TX, TY, 16>(a, bwd, st);
        case 32: return launch_norm_hp<TX, TY, 32>(a, bwd, st);
        default: return launch_norm_hp<TX, TY, 64>(a, bwd, st);
    }
}

int dispatch_norm(const sisa_norm_args* a, int bwd, hipStream_t st) {
    const int x = a->xdtype, y = a->ydtype;
    if (x == SISA_F32 && y == SISA_F32) return launch_norm<float, float>(a, bwd, st);
    if (x == SISA_F32 && y == SISA_BF16) return launch_norm<float, __bf16>(a, bwd, st);
    if (x == SISA_F32 && y == SISA_F16) return launch_norm<float, _Float16>(a, bwd, st);
    if (x == SISA_BF16 && y == SISA_BF16) return launch_norm<__bf16, __bf16>(a, bwd, st);
    return launch_norm<_Float16, _Float16>(a, bwd, st);
}

bool rows_ok(const void* p, int64_t stride, int32_t D, int dtype) {
    return p && sisa::aligned16(p) && stride >= D && (stride * sisa::elem_size(dtype)) % 16 == 0;
}

int check_norm(const sisa_norm_args* a, int bwd, const char* fn) {
    SISA_REQUIRE(a != nullptr, "%s: null args", fn);
    SISA_REQUIRE(a->N >= 0 && a->D >= 8 && a->D % 8 == 0 && a->D <= 4096,
                 "%s: row length D=%d must be a multiple of 8 in [8, 4096]", fn, a->D);
    SISA_REQUIRE(a->H >= 0 && a->H <= 64, "%s: projection width H=%d must be in [0, 64]", fn, a->H);
    const int x = a->xdtype, y = a->ydtype;
    SISA_REQUIRE((x == SISA_F32 && (y == SISA_F32 || y == SISA_BF16 || y == SISA_F16)) ||
                     ((x == SISA_BF16 || x == SISA_F16) && y == x),
                 "%s: dtype pair x=%d y=%d not supported (fp32 x with any output, or a 16-bit x with the same output)",
                 fn, x, y);
    SISA_REQUIRE(rows_ok(a->x, a->sx, a->D, x) && a->w && sisa::aligned16(a->w),
                 "%s: x/w must be 16-byte aligned with a row stride >= D whose byte size is a multiple of 16", fn);
    SISA_REQUIRE(a->H == 0 || (a->wf && sisa::aligned16(a->wf) && a->bf),
                 "%s: a projection (H > 0) needs wf (16-byte aligned) and bf", fn);
    if (!bwd) {
        SISA_REQUIRE(rows_ok(a->y, a->sy, a->D, y), "%s: bad y (16-byte aligned rows, stride >= D)", fn);
        SISA_REQUIRE(a->H == 0 || a->z, "%s: a projection (H > 0) needs z", fn);
        SISA_REQUIRE(a->res == nullptr || (rows_ok(a->res, a->sres, a->D, y) && rows_ok(a->h, a->sh, a->D, x)),
                     "%s: a residual needs res (ydtype) and h (xdtype) with 16-byte aligned rows, stride >= D", fn);
    } else {
        SISA_REQUIRE(a->dh == nullptr || rows_ok(a->dh, a->sdh, a->D, x),
                     "%s: dh must have 16-byte aligned rows (xdtype, stride >= D)", fn);
        SISA_REQUIRE(rows_ok(a->dy, a->sdy, a->D, y) && rows_ok(a->dx, a->sdx, a->D, x) && a->rstd && a->dw &&
                         a->workspace && sisa::aligned16(a->workspace),
                     "%s: dy/dx (16-byte aligned rows), rstd, dw and a 16-byte aligned workspace must be given", fn);
        SISA_REQUIRE(a->H == 0 || (a->dz && a->dwf && a->dbf), "%s: a projection (H > 0) needs dz, dwf and dbf", fn);
    }
    return SISA_OK;
}

}  // namespace

extern "C" int64_t sisa_norm_bwd_workspace_bytes(int64_t N, int32_t D, int32_t H) {
    return norm_ws_floats(N, D, H) * (int64_t)sizeof(float);
}

extern "C" int sisa_norm_fwd(const sisa_norm_args* a, void* stream) {
    const int rc = check_norm(a, 0, "sisa_norm_fwd");
    if (rc) return rc;
    if (a->N == 0) return SISA_OK;
    return dispatch_norm(a, 0, (hipStream_t)stream);
}

extern "C" int sisa_norm_bwd(const sisa_norm_args* a, void* stream) {
    const int rc = check_norm(a, 1, "sisa_norm_bwd");
    if (rc) return rc;
    return dispatch_norm(a, 1, (hipStream_t)stream);
}

// The plain RMSNorm entry points: the H = 0, same-dtype case of the above.
static sisa_norm_args from_rms(const sisa_rmsnorm_args* r) {
    sisa_norm_args a = {};
    a.N = r->N;
    a.D = r->D;
    a.H = 0;
    a.xdtype = a.ydtype = r->dtype;
    a.eps = r->eps;
    a.x = r->x;
    a.sx = r->sx;
    a.w = r->w;
    a.y = r->y;
    a.sy = r->sy;
    a.rstd = r->rstd;
    a.dy = r->dy;
    a.sdy = r->sdy;
    a.dx = r->dx;
    a.sdx = r->sdx;
    a.dw = r->dw;
    a.workspace = r->dw_partial;
    return a;
}

extern "C" int64_t sisa_rmsnorm_bwd_workspace_bytes(int64_t N, int32_t D) {
    return sisa_norm_bwd_workspace_bytes(N, D, 0);
}

extern "C" int sisa_rmsnorm_fwd(const sisa_rmsnorm_args* r, void* stream) {
    SISA_REQUIRE(r != nullptr, "sisa_rmsnorm_fwd: null args");
    const sisa_norm_args a = from_rms(r);
    const int rc = check_norm(&a, 0, "sisa_rmsnorm_fwd");
    if (rc) return rc;
    if (a.N == 0) return SISA_OK;
    return dispatch_norm(&a, 0, (hipStream_t)stream);
}

extern "C" int sisa_rmsnorm_bwd(const sisa_rmsnorm_args* r, void* stream) {
    SISA_REQUIRE(r != nullptr, "sisa_rmsnorm_bwd: null args");
    const sisa_norm_args a = from_rms(r);
    const int rc = check_norm(&a, 1, "sisa_rmsnorm_bwd");
    if (rc) return rc;
    return dispatch_norm(&a, 1, (hipStream_t)stream);
}

namespace {

// ------------------------------------------------------------------------------------------------ SwiGLU
// sigmoid(a) = 1 / (1 + exp(-a)). For 16-bit data (results rounded to 8 or 11 bits) from the hardware base-2
// exponential and reciprocal, 1 / (1 + 2^(-a log2 e)), a few fp32 ulp; for fp32 data with the library expf and an
// IEEE division. Both give 0 for a -> -inf, 1 for a -> +inf and propagate NaN.
template <class T>
SISA_DEV float sigmoidf_(float a) {
    if constexpr (sizeof(T) == 2) return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-a * LOG2E));
    else return 1.f / (1.f + expf(-a));
}

// h = silu(a) * b. PAIRS: a and b come interleaved in 8-element chunks from one array (a_8k..a_8k+7, b_8k..b_8k+7),
// the layout of a GEMM against the gate and up weights interleaved in 8-row chunks.
template <class T, bool PAIRS>
__global__ __launch_bounds__(256) void swiglu_fwd_kernel(sisa_swiglu_args a) {
    const int64_t nv = a.n / 8;
    for (int64_t v = (int64_t)blockIdx.x * 256 + threadIdx.x; v < nv; v += (int64_t)gridDim.x * 256) {
        const T* pa = (const T*)a.a + (PAIRS ? 16 * v : 8 * v);
        const T* pb = PAIRS ? pa + 8 : (const T*)a.b + 8 * v;
        const f32x8 x = load_f32x8<T>(pa), y = load_f32x8<T>(pb);
        f32x8 h;
#pragma unroll
        for (int j = 0; j < 8; ++j) h[j] = (x[j] * sigmoidf_<T>(x[j])) * y[j];
        store_f32x8<T>((T*)a.h + 8 * v, h);
    }
}

// da = dh * b * silu'(a), db = dh * silu(a); silu'(a) = s * (1 + a * (1 - s)), s = sigmoid(a). PAIRS: da receives
// the interleaved (da, db) chunks.
template <class T, bool PAIRS>
__global__ __launch_bounds__(256) void swiglu_bwd_kernel(sisa_swiglu_args a) {
    const int64_t nv = a.n / 8;
    for (int64_t v = (int64_t)blockIdx.x * 256 + threadIdx.x; v < nv; v += (int64_t)gridDim.x * 256) {
        const T* pa = (const T*)a.a + (PAIRS ? 16 * v : 8 * v);
        const T* pb = PAIRS ? pa + 8 : (const T*)a.b + 8 * v;
        const f32x8 x = load_f32x8<T>(pa), y = load_f32x8<T>(pb);
        const f32x8 g = load_f32x8<T>((const T*)a.dh + 8 * v);
        f32x8 da, db;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float s = sigmoidf_<T>(x[j]);
            db[j] = g[j] * (x[j] * s);
            da[j] = (g[j] * y[j]) * (s * (1.f + x[j] * (1.f - s)));
        }
        T* qa = (T*)a.da + (PAIRS ? 16 * v : 8 * v);
        store_f32x8<T>(qa, da);
        store_f32x8<T>(PAIRS ? qa + 8 : (T*)a.db + 8 * v, db);
    }
}

template <class T>
int launch_swiglu(const sisa_swiglu_args* a, int bwd, hipStream_t st) {
    const int64_t nv = a->n / 8;
    const unsigned grid = (unsigned)(sisa::cdiv(nv, 256) < 8192 ? sisa::cdiv(nv, 256) : 8192);
    if (a->pairs) {
        if (bwd) swiglu_bwd_kernel<T, true><<<grid, 256, 0, st>>>(*a);
        else swiglu_fwd_kernel<T, true><<<grid, 256, 0, st>>>(*a);
    } else {
        if (bwd) swiglu_bwd_kernel<T, false><<<grid, 256, 0, st>>>(*a);
        else swiglu_fwd_kernel<T, false><<<grid, 256, 0, st>>>(*a);
    }
    return sisa::launch_status(bwd ? "sisa_swiglu_bwd" : "sisa_swiglu_fwd");
}

}  // namespace

static int swiglu_entry(const sisa_swiglu_args* a, int bwd, void* stream) {
    const char* fn = bwd ? "sisa_swiglu_bwd" : "sisa_swiglu_fwd";
    SISA_REQUIRE(a != nullptr, "%s: null args", fn);
    SISA_REQUIRE(a->n >= 0 && a->n % 8 == 0, "%s: element count %lld must be a multiple of 8", fn, (long long)a->n);
    SISA_REQUIRE(a->dtype == SISA_BF16 || a->dtype == SISA_F16 || a->dtype == SISA_F32, "%s: dtype %d", fn, a->dtype);
    SISA_REQUIRE(a->pairs == 0 || a->pairs == 1, "%s: pairs must be 0 or 1", fn);
    SISA_REQUIRE(a->a && sisa::aligned16(a->a) && (a->pairs || (a->b && sisa::aligned16(a->b))),
                 "%s: a/b must be 16-byte aligned", fn);
    if (bwd)
        SISA_REQUIRE(a->dh && a->da && sisa::aligned16(a->dh) && sisa::aligned16(a->da) &&
                         (a->pairs || (a->db && sisa::aligned16(a->db))),
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
