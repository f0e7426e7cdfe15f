// Fused SISA preparation for gfx950: the prefix scans over the sequence and the pair rotations of C and B, forward
// and backward, reading the projection output `proj` (B, L, NPAD) in place.
//
//   g = cumsum(-softplus(alpha)),  F = cumsum(logsigmoid(z)),  Phi = cumsum(theta)          (fp32)
//   C~ = R(Phi) C,  B~ = R(Phi) B   (interleaved pairs (0,1),(2,3),... rotated by Phi[pair])  (fp32, one RNE rounding)
//   rowf/colf = the 64-row decay factors of the attention kernels (bitwise equal to sisa_factors on the same g)
//
// Reference: src/sisa/kernels/fused_prep.py (Triton): layout :71-96, element formulas :188-213 (torch's formulas,
// softplus threshold 20), _prep_sums :247-274, _prep_fwd :277-352, _prep_bsums :385-411, _prep_bwd :414-494.
//
// Scan scheme (deterministic reduce-then-scan over 64-row chunks): pass 1 writes per-chunk totals TOT; pass 2 adds
// the totals of the preceding chunks in sequence order to a sequential in-chunk scan. The chunk total is produced by
// the same sequential loop as the last in-chunk value, so carry_{c+1} = carry_c + TOT_c equals the last g of chunk c
// bit for bit and g is non-increasing across chunk boundaries. The backward runs the same scheme in reverse with
// fp64 accumulators.
//
// Decomposition: one workgroup per (64-row chunk, batch row, group of HG heads); 256 threads. The chunk's theta,
// alpha and z slab is staged in LDS with coalesced loads; the rotation reads/writes the C and B columns of the head
// group (contiguous in a proj row) directly.
#include "common.h"
#include "host.h"

namespace {

constexpr int DH = 64, DS = 32, S2 = 16, CH = 64, HG = 4, NCOMP = 2 + S2;

struct Layout {
    int Q, K, V, B, C, TH, A, NTOT, NPAD;
};

__host__ __device__ inline Layout layout_of(int H) {
    Layout o;
    o.Q = 0;
    o.K = H * DH;
    o.V = 2 * H * DH;
    o.B = 3 * H * DH;
    o.C = 3 * H * DH + H * DS;
    o.TH = 3 * H * DH + 2 * H * DS;
    o.A = o.TH + H * S2;
    o.NTOT = o.A + H;
    o.NPAD = (o.NTOT + 15) / 16 * 16;
    return o;
}

// torch's formulas (fused_prep.py:188-213)
SISA_DEV float neg_softplus(float a) { return -(a > 20.f ? a : log1pf(expf(a))); }
SISA_DEV float softplus_grad(float a) {
    const float e = expf(a);
    return a > 20.f ? 1.f : e / (e + 1.f);
}
SISA_DEV float logsigmoid(float z) {
    const float mn = (z != z) ? z : (z < 0.f ? z : 0.f);   // NaN-propagating min(z, 0)
    return mn - log1pf(expf(-fabsf(z)));
}
SISA_DEV float logsigmoid_grad(float z) {
    const float e = expf(-fabsf(z));
    const float r = e / (1.f + e);
    return z < 0.f ? 1.f - r : r;
}

template <class T>
struct PrepLds {
    float th[CH][HG * S2];   // theta, later Phi (forward) or dPhi (backward)
    float al[CH][HG];        // alpha
    float zz[CH][HG];        // z
    float g[HG][CH];         // scan results of components 0 / 1
    float f[HG][CH];
};

// Stage theta / alpha / z of rows [r0, r0+64) for heads [h0, h0+hn) (zero beyond L or without z).
template <class T>
SISA_DEV void stage_slab(PrepLds<T>& sm, const T* P, int64_t s_pl, const float* Z, int64_t s_zl, int r0, int L,
                         int h0, int hn, const Layout& off, int tid) {
    for (int idx = tid; idx < CH * HG * S2; idx += 256) {
        const int r = idx / (HG * S2), cc = idx % (HG * S2);
        const int row = r0 + r;
        float v = 0.f;
        if (row < L && cc < hn * S2) v = (float)P[(int64_t)row * s_pl + off.TH + h0 * S2 + cc];
        sm.th[r][cc] = v;
    }
    for (int idx = tid; idx < CH * HG; idx += 256) {
        const int r = idx / HG, hl = idx % HG;
        const int row = r0 + r;
        const bool ok = row < L && hl < hn;
        sm.al[r][hl] = ok ? (float)P[(int64_t)row * s_pl + off.A + h0 + hl] : 0.f;
        sm.zz[r][hl] = (ok && Z) ? Z[(int64_t)row * s_zl + h0 + hl] : 0.f;
    }
}

// Element value of component `comp` at chunk row r (0 for rows >= L).
template <class T>
SISA_DEV float elem(const PrepLds<T>& sm, int comp, int hl, int r, bool valid) {
    if (!valid) return 0.f;
    if (comp == 0) return neg_softplus(sm.al[r][hl]);
    if (comp == 1) return logsigmoid(sm.zz[r][hl]);
    return sm.th[r][hl * S2 + comp - 2];
}

// Pass 1: TOT[bh][c][comp] = sequential in-chunk sum.
template <class T>
__global__ __launch_bounds__(256) void prep_sums_kernel(sisa_prep_fwd_args a) {
    __shared__ PrepLds<T> sm;
    const int c = blockIdx.x, b = blockIdx.y, h0 = blockIdx.z * HG;
    const int H = a.H, L = a.L, NCH = gridDim.x;
    const int hn = (H - h0 < HG) ? H - h0 : HG;
    const Layout off = layout_of(H);
    const int tid = threadIdx.x;
    const T* P = (const T*)a.proj + (int64_t)b * a.s_pb;
    const float* Z = a.z ? a.z + (int64_t)b * a.s_zb : nullptr;
    stage_slab<T>(sm, P, a.s_pl, Z, a.s_zl, c * CH, L, h0, hn, off, tid);
    __syncthreads();
    if (tid < HG * NCOMP) {
        const int hl = tid / NCOMP, comp = tid % NCOMP;
        if (hl < hn) {
            float incl = 0.f;
            for (int r = 0; r < CH; ++r) incl += elem<T>(sm, comp, hl, r, c * CH + r < L && (comp != 1 || a.z));
            a.tot[((int64_t)(b * H + h0 + hl) * NCH + c) * NCOMP + comp] = incl;
        }
    }
}

// Pass 2: scans, factors, rotation.
template <class T>
__global__ __launch_bounds__(256) void prep_fwd_kernel(sisa_prep_fwd_args a) {
    __shared__ PrepLds<T> sm;
    const int c = blockIdx.x, b = blockIdx.y, h0 = blockIdx.z * HG;
    const int H = a.H, L = a.L, NCH = gridDim.x;
    const int hn = (H - h0 < HG) ? H - h0 : HG;
    const Layout off = layout_of(H);
    const int tid = threadIdx.x;
    const T* P = (const T*)a.proj + (int64_t)b * a.s_pb;
    const float* Z = a.z ? a.z + (int64_t)b * a.s_zb : nullptr;
    stage_slab<T>(sm, P, a.s_pl, Z, a.s_zl, c * CH, L, h0, hn, off, tid);
    __syncthreads();
    // one thread per (head, component); a theta column is read and overwritten with Phi by its own thread only
    if (tid < HG * NCOMP && tid / NCOMP < hn) {
        const int hl = tid / NCOMP, comp = tid % NCOMP;
        const float* tb = a.tot + (int64_t)(b * H + h0 + hl) * NCH * NCOMP + comp;
        float carry = 0.f;
        for (int cc = 0; cc < c; ++cc) carry += tb[(int64_t)cc * NCOMP];
        float incl = 0.f;
        for (int r = 0; r < CH; ++r) {
            incl += elem<T>(sm, comp, hl, r, c * CH + r < L && (comp != 1 || a.z));
            const float v = carry + incl;
            if (comp == 0) sm.g[hl][r] = v;
            else if (comp == 1) sm.f[hl][r] = v;
            else sm.th[r][hl * S2 + comp - 2] = v;
        }
    }
    __syncthreads();
    // g, F, rowf, colf: (B,H,L) rows, coalesced along L
    for (int idx = tid; idx < hn * CH; idx += 256) {
        const int hh = idx / CH, r = idx % CH;
        const int row = c * CH + r;
        if (row >= L) continue;
        const int64_t o = ((int64_t)(b * H + h0 + hh)) * L + row;
        const float g = sm.g[hh][r];
        a.g[o] = g;
        a.rowf[o] = exp2_le0((g - sm.g[hh][0]) * LOG2E);
        a.colf[o] = exp2_le0((sm.g[hh][CH - 1] - g) * LOG2E);   // rows >= L add 0: the last valid g
        if (a.z) a.f[o] = sm.f[hh][r];
    }
    // rotation of C and B by Phi (fp32, one rounding to T)
    T* CR = (T*)a.cr;
    T* BR = (T*)a.br;
    for (int idx = tid; idx < CH * hn * S2; idx += 256) {
        const int r = idx / (hn * S2), rem = idx % (hn * S2);
        const int hh = rem / S2, pr = rem % S2;
        const int row = c * CH + r;
        if (row >= L) continue;
        float sn, cs;
        sincosf(sm.th[r][hh * S2 + pr], &sn, &cs);
        const T* prow = P + (int64_t)row * a.s_pl;
        const int h = h0 + hh;
        const typename Vec<T>::x2 cv = *reinterpret_cast<const typename Vec<T>::x2*>(prow + off.C + h * DS + 2 * pr);
        const typename Vec<T>::x2 bv = *reinterpret_cast<const typename Vec<T>::x2*>(prow + off.B + h * DS + 2 * pr);
        const int64_t o = (((int64_t)b * L + row) * H + h) * DS + 2 * pr;
        {
            const float ze = (float)cv[0], zo = (float)cv[1];
            f32x2 out = {ze * cs - zo * sn, ze * sn + zo * cs};
            *reinterpret_cast<typename Vec<T>::x2*>(CR + o) = __builtin_convertvector(out, typename Vec<T>::x2);
        }
        {
            const float ze = (float)bv[0], zo = (float)bv[1];
            f32x2 out = {ze * cs - zo * sn, ze * sn + zo * cs};
            *reinterpret_cast<typename Vec<T>::x2*>(BR + o) = __builtin_convertvector(out, typename Vec<T>::x2);
        }
    }
}

// ------------------------------------------------------------------------------------------------ backward
struct BwdLds {
    float th[CH][HG * S2];   // theta -> Phi -> dPhi
    float al[CH][HG];
    float zz[CH][HG];
    float dg[HG][CH];
    float df[HG][CH];
};

// Recompute Phi for the chunk (identical code to the forward scan) into sm.th, then replace it with
// dPhi = sum over {C, B} of (dout_odd * out_even - dout_even * out_odd), optionally writing the inverse-rotated
// gradients dC, dB into dproj.
template <class T, bool WRITE>
SISA_DEV void phi_and_dphi(BwdLds& sm, const sisa_prep_bwd_args& a, const T* P, int b, int c, int h0, int hn,
                           int NCH, const Layout& off, int tid) {
    const int H = a.H, L = a.L;
    if (tid < hn * S2) {
        const int hl = tid / S2, pr = tid % S2;
        const float* tb = a.tot + (int64_t)(b * H + h0 + hl) * NCH * NCOMP + 2 + pr;
        float carry = 0.f;
        for (int cc = 0; cc < c; ++cc) carry += tb[(int64_t)cc * NCOMP];
        float incl = 0.f;
        for (int r = 0; r < CH; ++r) {
            incl += (c * CH + r < L) ? sm.th[r][hl * S2 + pr] : 0.f;
            sm.th[r][hl * S2 + pr] = carry + incl;
        }
    }
    __syncthreads();
    T* DP = (T*)a.dproj + (int64_t)b * a.s_db;
    for (int idx = tid; idx < CH * hn * S2; idx += 256) {
        const int r = idx / (hn * S2), rem = idx % (hn * S2);
        const int hh = rem / S2, p2 = rem % S2;
        const int row = c * CH + r;
        float dphi = 0.f;
        if (row < L) {
            float sn, cs;
            sincosf(sm.th[r][hh * S2 + p2], &sn, &cs);
            const T* prow = P + (int64_t)row * a.s_pl;
            const int h = h0 + hh;
            const int64_t o = (((int64_t)b * L + row) * H + h) * DS + 2 * p2;
            const f32x2 dcv = *reinterpret_cast<const f32x2*>(a.dcr + o);
            const f32x2 dbv = *reinterpret_cast<const f32x2*>(a.dbr + o);
            const typename Vec<T>::x2 cv =
                *reinterpret_cast<const typename Vec<T>::x2*>(prow + off.C + h * DS + 2 * p2);
            const typename Vec<T>::x2 bv =
                *reinterpret_cast<const typename Vec<T>::x2*>(prow + off.B + h * DS + 2 * p2);
            float d1, d2;
            {
                const float ze = (float)cv[0], zo = (float)cv[1];
                const float oe = ze * cs - zo * sn, oo = ze * sn + zo * cs;
                d1 = dcv[1] * oe - dcv[0] * oo;
                if (WRITE) {
                    f32x2 dz = {dcv[0] * cs + dcv[1] * sn, dcv[1] * cs - dcv[0] * sn};
                    *reinterpret_cast<typename Vec<T>::x2*>(DP + (int64_t)row * a.s_dl + off.C + h * DS + 2 * p2) =
                        __builtin_convertvector(dz, typename Vec<T>::x2);
                }
            }
            {
                const float ze = (float)bv[0], zo = (float)bv[1];
                const float oe = ze * cs - zo * sn, oo = ze * sn + zo * cs;
                d2 = dbv[1] * oe - dbv[0] * oo;
                if (WRITE) {
                    f32x2 dz = {dbv[0] * cs + dbv[1] * sn, dbv[1] * cs - dbv[0] * sn};
                    *reinterpret_cast<typename Vec<T>::x2*>(DP + (int64_t)row * a.s_dl + off.B + h * DS + 2 * p2) =
                        __builtin_convertvector(dz, typename Vec<T>::x2);
                }
            }
            dphi = d1 + d2;
        }
        sm.th[r][hh * S2 + p2] = dphi;   // each element is read and replaced by its own thread
    }
}

template <class T>
SISA_DEV void stage_bwd(BwdLds& sm, const sisa_prep_bwd_args& a, const T* P, int b, int c, int h0, int hn,
                        const Layout& off, int tid) {
    const int H = a.H, L = a.L;
    const float* Z = a.z ? a.z + (int64_t)b * a.s_zb : nullptr;
    for (int idx = tid; idx < CH * HG * S2; idx += 256) {
        const int r = idx / (HG * S2), cc = idx % (HG * S2);
        const int row = c * CH + r;
        float v = 0.f;
        if (row < L && cc < hn * S2) v = (float)P[(int64_t)row * a.s_pl + off.TH + h0 * S2 + cc];
        sm.th[r][cc] = v;
    }
    for (int idx = tid; idx < CH * HG; idx += 256) {
        const int r = idx / HG, hl = idx % HG;
        const int row = c * CH + r;
        const bool ok = row < L && hl < hn;
        sm.al[r][hl] = ok ? (float)P[(int64_t)row * a.s_pl + off.A + h0 + hl] : 0.f;
        sm.zz[r][hl] = (ok && Z) ? Z[(int64_t)row * a.s_zl + h0 + hl] : 0.f;
    }
    for (int idx = tid; idx < HG * CH; idx += 256) {
        const int hl = idx / CH, r = idx % CH;
        const int row = c * CH + r;
        const bool ok = row < L && hl < hn;
        const int64_t o = (int64_t)(b * H + h0 + hl) * L + row;
        sm.dg[hl][r] = ok ? a.dg[o] : 0.f;
        sm.df[hl][r] = (ok && a.df) ? a.df[o] : 0.f;
    }
}

// Backward pass 1: fp64 chunk totals BT[bh][c] = (sum dg, sum dF, sum dPhi[16]).
template <class T>
__global__ __launch_bounds__(256) void prep_bsums_kernel(sisa_prep_bwd_args a) {
    __shared__ BwdLds sm;
    const int c = blockIdx.x, b = blockIdx.y, h0 = blockIdx.z * HG;
    const int H = a.H, NCH = gridDim.x;
    const int hn = (H - h0 < HG) ? H - h0 : HG;
    const Layout off = layout_of(H);
    const int tid = threadIdx.x;
    const T* P = (const T*)a.proj + (int64_t)b * a.s_pb;
    stage_bwd<T>(sm, a, P, b, c, h0, hn, off, tid);
    __syncthreads();
    phi_and_dphi<T, false>(sm, a, P, b, c, h0, hn, NCH, off, tid);
    __syncthreads();
    double* BT = (double*)a.workspace;
    if (tid < hn * NCOMP) {
        const int hl = tid / NCOMP, comp = tid % NCOMP;
        double s = 0.0;
        for (int r = 0; r < CH; ++r) {
            const float v = comp == 0 ? sm.dg[hl][r] : (comp == 1 ? sm.df[hl][r] : sm.th[r][hl * S2 + comp - 2]);
            s += (double)v;
        }
        BT[((int64_t)(b * H + h0 + hl) * NCH + c) * NCOMP + comp] = s;
    }
}

// Backward pass 2: reverse scans (fp64 carries of the following chunks + sequential in-chunk reverse sums).
template <class T>
__global__ __launch_bounds__(256) void prep_bwd_kernel(sisa_prep_bwd_args a) {
    __shared__ BwdLds sm;
    __shared__ float outv[CH][HG * NCOMP];
    const int c = blockIdx.x, b = blockIdx.y, h0 = blockIdx.z * HG;
    const int H = a.H, L = a.L, NCH = gridDim.x;
    const int hn = (H - h0 < HG) ? H - h0 : HG;
    const Layout off = layout_of(H);
    const int tid = threadIdx.x;
    const T* P = (const T*)a.proj + (int64_t)b * a.s_pb;
    stage_bwd<T>(sm, a, P, b, c, h0, hn, off, tid);
    __syncthreads();
    phi_and_dphi<T, true>(sm, a, P, b, c, h0, hn, NCH, off, tid);
    __syncthreads();
    const double* BT = (const double*)a.workspace;
    if (tid < hn * NCOMP) {
        const int hl = tid / NCOMP, comp = tid % NCOMP;
        const double* tb = BT + (int64_t)(b * H + h0 + hl) * NCH * NCOMP + comp;
        double sa = 0.0;
        for (int cc = c + 1; cc < NCH; ++cc) sa += tb[(int64_t)cc * NCOMP];
        double rev = 0.0;
        for (int r = CH - 1; r >= 0; --r) {
            const float v = comp == 0 ? sm.dg[hl][r] : (comp == 1 ? sm.df[hl][r] : sm.th[r][hl * S2 + comp - 2]);
            rev += (double)v;
            const float tot = (float)(sa + rev);
            float out;
            if (comp == 0) out = -tot * softplus_grad(sm.al[r][hl]);
            else if (comp == 1) out = tot * logsigmoid_grad(sm.zz[r][hl]);
            else out = tot;
            outv[r][hl * NCOMP + comp] = out;
        }
    }
    __syncthreads();
    T* DP = (T*)a.dproj + (int64_t)b * a.s_db;
    // d theta: contiguous HG*16 columns per row
    for (int idx = tid; idx < CH * hn * S2; idx += 256) {
        const int r = idx / (hn * S2), rem = idx % (hn * S2);
        const int hh = rem / S2, pr = rem % S2;
        const int row = c * CH + r;
        if (row >= L) continue;
        DP[(int64_t)row * a.s_dl + off.TH + (h0 + hh) * S2 + pr] = cvt<T>(outv[r][hh * NCOMP + 2 + pr]);
    }
    for (int idx = tid; idx < CH * hn; idx += 256) {
        const int r = idx / hn, hh = idx % hn;
        const int row = c * CH + r;
        if (row >= L) continue;
        DP[(int64_t)row * a.s_dl + off.A + h0 + hh] = cvt<T>(outv[r][hh * NCOMP + 0]);
        if (a.dz) a.dz[(int64_t)b * a.s_dzb + (int64_t)row * a.s_dzl + h0 + hh] = outv[r][hh * NCOMP + 1];
    }
    // zero padding columns (they multiply the zero rows of W_cat; keeps NaN out of dX)
    if (blockIdx.z == 0 && off.NPAD > off.NTOT) {
        const int npad = off.NPAD - off.NTOT;
        for (int idx = tid; idx < CH * npad; idx += 256) {
            const int r = idx / npad, j = idx % npad;
            const int row = c * CH + r;
            if (row >= L) continue;
            DP[(int64_t)row * a.s_dl + off.NTOT + j] = cvt<T>(0.f);
        }
    }
}

template <class T>
int launch_prep_fwd(const sisa_prep_fwd_args* a, hipStream_t st) {
    dim3 grid((unsigned)sisa::cdiv(a->L, CH), (unsigned)a->B, (unsigned)sisa::cdiv(a->H, HG));
    prep_sums_kernel<T><<<grid, 256, 0, st>>>(*a);
    int rc = sisa::launch_status("sisa_prep_fwd (sums)");
    if (rc) return rc;
    prep_fwd_kernel<T><<<grid, 256, 0, st>>>(*a);
    return sisa::launch_status("sisa_prep_fwd");
}

template <class T>
int launch_prep_bwd(const sisa_prep_bwd_args* a, hipStream_t st) {
    dim3 grid((unsigned)sisa::cdiv(a->L, CH), (unsigned)a->B, (unsigned)sisa::cdiv(a->H, HG));
    prep_bsums_kernel<T><<<grid, 256, 0, st>>>(*a);
    int rc = sisa::launch_status("sisa_prep_bwd (sums)");
    if (rc) return rc;
    prep_bwd_kernel<T><<<grid, 256, 0, st>>>(*a);
    return sisa::launch_status("sisa_prep_bwd");
}

}  // namespace

extern "C" int sisa_prep_fwd(const sisa_prep_fwd_args* a, void* stream) {
    SISA_REQUIRE(a != nullptr, "sisa_prep_fwd: null args");
    SISA_REQUIRE(a->B >= 1 && a->L >= 1 && a->H >= 1, "sisa_prep_fwd: bad shape B=%d L=%d H=%d", a->B, a->L, a->H);
    SISA_REQUIRE(a->dtype == SISA_BF16 || a->dtype == SISA_F16, "sisa_prep_fwd: proj dtype must be bf16/fp16");
    SISA_REQUIRE(a->proj && a->cr && a->br && a->g && a->rowf && a->colf && a->tot, "sisa_prep_fwd: null pointer");
    SISA_REQUIRE(a->z == nullptr || a->f != nullptr, "sisa_prep_fwd: f is required with z");
    SISA_REQUIRE(a->s_pl >= layout_of(a->H).NPAD && (a->s_pl % 2) == 0, "sisa_prep_fwd: proj row stride %lld",
                 (long long)a->s_pl);
    hipStream_t st = (hipStream_t)stream;
    return a->dtype == SISA_BF16 ? launch_prep_fwd<__bf16>(a, st) : launch_prep_fwd<_Float16>(a, st);
}

extern "C" int64_t sisa_prep_bwd_workspace_bytes(int32_t B, int32_t L, int32_t H) {
    return (int64_t)B * H * sisa::cdiv(L, CH) * NCOMP * (int64_t)sizeof(double);
}

extern "C" int sisa_prep_bwd(const sisa_prep_bwd_args* a, void* stream) {
    SISA_REQUIRE(a != nullptr, "sisa_prep_bwd: null args");
    SISA_REQUIRE(a->B >= 1 && a->L >= 1 && a->H >= 1, "sisa_prep_bwd: bad shape B=%d L=%d H=%d", a->B, a->L, a->H);
    SISA_REQUIRE(a->dtype == SISA_BF16 || a->dtype == SISA_F16, "sisa_prep_bwd: proj dtype must be bf16/fp16");
    SISA_REQUIRE(a->proj && a->tot && a->dg && a->dcr && a->dbr && a->dproj && a->workspace,
                 "sisa_prep_bwd: null pointer");
    SISA_REQUIRE((a->z == nullptr) == (a->df == nullptr) && (a->z == nullptr) == (a->dz == nullptr),
                 "sisa_prep_bwd: z, df and dz must all be given or all be null");
    SISA_REQUIRE(a->s_pl >= layout_of(a->H).NPAD && a->s_dl >= layout_of(a->H).NPAD, "sisa_prep_bwd: row strides");
    hipStream_t st = (hipStream_t)stream;
    return a->dtype == SISA_BF16 ? launch_prep_bwd<__bf16>(a, st) : launch_prep_bwd<_Float16>(a, st);
}
