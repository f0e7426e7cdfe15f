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
// Decomposition: one 256-thread workgroup per (64-row chunk, batch row, group of HG = 4 heads). Every global access is
// issued up front as 16-byte vectors (theta 8 vectors per row; C, B, dC~, dB~ 16 per row), element functions are
// evaluated by all threads before the 72 scan lanes (head, component) run their sequential 64-row scans out of LDS,
// and the totals of the preceding (following) chunks are staged through LDS with one parallel load before each lane
// folds them in chunk order. The backward's first pass also applies the inverse rotation and keeps dPhi rows in the
// workspace, so its second pass reads only dg, dF, dPhi, alpha and z.
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

constexpr int NT = 512;              // threads per workgroup
constexpr int NU = 1024 / NT;        // C/B vectors (units) per thread
constexpr int HC = HG * NCOMP;       // (head, component) scan lanes of a workgroup

// sin and cos of x: one fp32 reduction to revolutions in [-1/2, 1/2] and the hardware sine/cosine (input in
// revolutions). The reduction error, |x| * 2^-24 radians, is about one unit in the last place of x itself; the
// outputs are rounded to bf16/fp16 afterwards.
SISA_DEV void sincos_rev(float x, float* s, float* c) {
    const float r = x * 0.159154943091895336f;
    const float f = r - __builtin_rintf(r);
    *s = __builtin_amdgcn_sinf(f);
    *c = __builtin_amdgcn_cosf(f);
}

// Column slabs of one 64-row chunk and HG heads: 16-byte vectors of 8 elements.
//   theta: 8 vectors per row (head hl = part/2, pairs 8*(part%2)..+7)
//   C, B : 16 vectors per row (head hl = part/4, elements 8*(part%4)..+7, i.e. pairs 4*(part%4)..+3)
struct Unit {
    int row, hl, q;
};
SISA_DEV Unit cb_unit(int v) { return Unit{v >> 4, (v >> 2) & 3, v & 3}; }

template <class T>
SISA_DEV frag8<T> load8_if(const T* p, bool ok) { return ok ? load8<T>(p) : zero8<T>(); }

// Scan lanes: x[hl*NCOMP + comp][r] holds the element values of chunk row r (0 beyond L), then the inclusive scan plus
// the carry of the preceding chunks. Rows padded to 65 floats: the 72 scanning lanes read one row each without bank
// conflicts.
struct ScanLds {
    float x[HC][CH + 1];
};

// Staging loads of one thread: theta vector `tid` of the chunk (row tid>>3, head (tid>>1)&3, pairs 8*(tid&1)..+7)
// and, for tid < 256, alpha and z of (row tid>>2, head tid&3). Split from the LDS stores so that a kernel issues
// every global load it needs before the first wait.
static_assert(NT == CH * HG * 2, "one theta vector per thread");
template <class T>
struct StageVals {
    frag8<T> th;
    float al, zv;
};
template <class T, bool AZ = true>
SISA_DEV StageVals<T> stage_load(const T* P, int64_t s_pl, const float* Z, int64_t s_zl, int nrows, int hn,
                                 const Layout& off, int h0, int tid) {
    StageVals<T> s;
    {
        const int row = tid >> 3, hl = (tid >> 1) & 3, half = tid & 1;
        s.th = load8_if<T>(P + (int64_t)row * s_pl + off.TH + (h0 + hl) * S2 + 8 * half, row < nrows && hl < hn);
    }
    s.al = 0.f;
    s.zv = 0.f;
    if (AZ && tid < CH * HG) {
        const int row = tid >> 2, hl = tid & 3;
        const bool ok = row < nrows && hl < hn;
        if (ok) s.al = (float)P[(int64_t)row * s_pl + off.A + h0 + hl];
        if (ok && Z) s.zv = Z[(int64_t)row * s_zl + h0 + hl];
    }
    return s;
}
// theta into components 2..17; with AZ, the element functions of alpha and z into components 0 and 1.
template <class T, bool AZ>
SISA_DEV void stage_store(ScanLds& sm, const StageVals<T>& s, int nrows, int hn, bool has_z, int tid) {
    {
        const int row = tid >> 3, hl = (tid >> 1) & 3, half = tid & 1;
#pragma unroll
        for (int j = 0; j < 8; ++j) sm.x[hl * NCOMP + 2 + 8 * half + j][row] = (float)s.th[j];
    }
    if (AZ && tid < CH * HG) {
        const int row = tid >> 2, hl = tid & 3;
        const bool ok = row < nrows && hl < hn;
        sm.x[hl * NCOMP + 0][row] = ok ? neg_softplus(s.al) : 0.f;
        sm.x[hl * NCOMP + 1][row] = (ok && has_z) ? logsigmoid(s.zv) : 0.f;
    }
}

// Carries of the scans: the left fold, in chunk order, of the chunk totals of a range of chunks [c0, c1) (the
// preceding chunks for the forward scans, fp32; the following chunks for the reverse scans, fp64). The totals of up
// to TB chunks are staged through LDS by all threads (coalesced loads of at most TPT values per thread, issued with
// the kernel's other loads); after a barrier each scan lane folds its column sequentially, so that in the forward
// carry_{c+1} = carry_c + TOT_c bit for bit. Longer ranges take further batches.
constexpr int TB = 64;                         // chunks per staged batch
constexpr int TPT = (HG * TB * NCOMP) / NT;    // totals loaded per thread and batch
static_assert(TPT * NT == HG * TB * NCOMP, "staged totals split evenly over the threads");
template <class Acc>
struct TotLds {
    Acc t[HG][TB * NCOMP];
};
// Loads of the totals of chunks [c0, c1) (at most TB of them) of the workgroup's heads; zero past the range.
template <class Acc>
SISA_DEV void tot_load(Acc (&v)[TPT], const Acc* tot, int bh0, int hn, int NCH, int c0, int c1, int tid) {
    const int n = (c1 - c0) * NCOMP;
#pragma unroll
    for (int q = 0; q < TPT; ++q) {
        const int e = tid + NT * q;
        const int hl = e / (TB * NCOMP), idx = e - hl * (TB * NCOMP);
        v[q] = (hl < hn && idx < n) ? tot[((int64_t)(bh0 + hl) * NCH + c0) * NCOMP + idx] : (Acc)0;
    }
}
template <class Acc>
SISA_DEV void tot_store(TotLds<Acc>& tl, const Acc (&v)[TPT], int tid) {
#pragma unroll
    for (int q = 0; q < TPT; ++q) (&tl.t[0][0])[tid + NT * q] = v[q];
}
// Sequential fold of `n` <= TB staged chunks into acc for scan lane (hl, comp). The LDS reads of a batch of FB
// chunks are all issued before the first add; chunks past n (still inside the staged array) add zero.
template <class Acc>
SISA_DEV Acc tot_fold(const TotLds<Acc>& tl, int hl, int comp, int n, Acc acc) {
    constexpr int FB = 16;
    static_assert(TB % FB == 0, "whole batches");
    const Acc* col = tl.t[hl] + comp;
    for (int k0 = 0; k0 < n; k0 += FB) {
        Acc buf[FB];
#pragma unroll
        for (int k = 0; k < FB; ++k) buf[k] = col[(k0 + k) * NCOMP];
#pragma unroll
        for (int k = 0; k < FB; ++k) acc += (k0 + k < n) ? buf[k] : (Acc)0;
    }
    return acc;
}
// The carry of scan lane tid (when `lane`) over chunks [c0, c1). The caller has loaded the first batch into v with
// tot_load(v, ..., c0, min(c1, c0 + TB)), stored it (tot_store) and passed a barrier. Further batches are loaded and
// folded here; every thread of the workgroup calls this (it has barriers when c1 - c0 > TB).
template <class Acc>
SISA_DEV Acc carry_of(TotLds<Acc>& tl, Acc (&v)[TPT], const Acc* tot, int bh0, int hn, int NCH, int c0, int c1,
                      bool lane, int tid) {
    const int hl = tid / NCOMP, comp = tid % NCOMP;
    Acc acc = lane ? tot_fold(tl, hl, comp, (c1 - c0 < TB) ? c1 - c0 : TB, (Acc)0) : (Acc)0;
    for (int cb = c0 + TB; cb < c1; cb += TB) {
        const int ce = (c1 - cb < TB) ? c1 : cb + TB;
        tot_load(v, tot, bh0, hn, NCH, cb, ce, tid);
        __syncthreads();   // every lane is done with the previous batch
        tot_store(tl, v, tid);
        __syncthreads();
        if (lane) acc = tot_fold(tl, hl, comp, ce - cb, acc);
    }
    return acc;
}

// In-chunk inclusive scan of one lane with the carry added: x[r] = carry + sum_{i <= r} x[i] (sequential order).
SISA_DEV void scan_lane(float* x, float carry) {
    float v[CH];
#pragma unroll
    for (int r = 0; r < CH; ++r) v[r] = x[r];
    float incl = 0.f;
#pragma unroll
    for (int r = 0; r < CH; ++r) {
        incl += v[r];
        x[r] = carry + incl;
    }
}

// ------------------------------------------------------------------------------------------------ forward
// Pass 1: TOT[bh][c][comp] = sequential sum of the chunk's element values (the same loop as the pass-2 scan, so the
// total equals the chunk's last inclusive value bit for bit).
template <class T>
__global__ __launch_bounds__(NT) void prep_sums_kernel(sisa_prep_fwd_args a) {
    __shared__ ScanLds sm;
    const int c = blockIdx.x, b = blockIdx.y, h0 = blockIdx.z * HG;
    const int H = a.H, L = a.L, NCH = gridDim.x;
    const int hn = (H - h0 < HG) ? H - h0 : HG;
    const int nrows = (L - c * CH < CH) ? L - c * CH : CH;
    const Layout off = layout_of(H);
    const int tid = threadIdx.x;
    const T* P = (const T*)a.proj + (int64_t)b * a.s_pb + (int64_t)c * CH * a.s_pl;
    const float* Z = a.z ? a.z + (int64_t)b * a.s_zb + (int64_t)c * CH * a.s_zl : nullptr;
    stage_store<T, true>(sm, stage_load<T>(P, a.s_pl, Z, a.s_zl, nrows, hn, off, h0, tid), nrows, hn, Z != nullptr,
                         tid);
    __syncthreads();
    if (tid < HC && tid / NCOMP < hn) {
        float incl = 0.f;
#pragma unroll 16
        for (int r = 0; r < CH; ++r) incl += sm.x[tid][r];
        a.tot[((int64_t)(b * H + h0 + tid / NCOMP) * NCH + c) * NCOMP + tid % NCOMP] = incl;
    }
}

// Pass 2: scans (carry of the preceding chunks + in-chunk inclusive scan), g/F/rowf/colf, rotation of C and B.
template <class T>
__global__ __launch_bounds__(NT) void prep_fwd_kernel(sisa_prep_fwd_args a) {
    __shared__ ScanLds sm;
    __shared__ TotLds<float> tl;
    const int c = blockIdx.x, b = blockIdx.y, h0 = blockIdx.z * HG;
    const int H = a.H, L = a.L, NCH = gridDim.x;
    const int hn = (H - h0 < HG) ? H - h0 : HG;
    const int nrows = (L - c * CH < CH) ? L - c * CH : CH;
    const Layout off = layout_of(H);
    const int tid = threadIdx.x;
    const T* P = (const T*)a.proj + (int64_t)b * a.s_pb + (int64_t)c * CH * a.s_pl;
    const float* Z = a.z ? a.z + (int64_t)b * a.s_zb + (int64_t)c * CH * a.s_zl : nullptr;
    // Every global load is issued before the first wait, in the order of use: the staged scan inputs, the totals of
    // the preceding chunks, then the C and B vectors this thread rotates.
    const StageVals<T> sv = stage_load<T>(P, a.s_pl, Z, a.s_zl, nrows, hn, off, h0, tid);
    const bool lane = tid < HC && tid / NCOMP < hn;
    float tv[TPT];
    tot_load(tv, a.tot, b * H + h0, hn, NCH, 0, c < TB ? c : TB, tid);
    frag8<T> cv[NU], bv[NU];
#pragma unroll
    for (int i = 0; i < NU; ++i) {
        const Unit u = cb_unit(tid + NT * i);
        const bool ok = u.row < nrows && u.hl < hn;
        const T* prow = P + (int64_t)u.row * a.s_pl + (h0 + u.hl) * DS + 8 * u.q;
        cv[i] = load8_if<T>(prow + off.C, ok);
        bv[i] = load8_if<T>(prow + off.B, ok);
    }
    stage_store<T, true>(sm, sv, nrows, hn, Z != nullptr, tid);
    tot_store(tl, tv, tid);
    __syncthreads();
    const float carry = carry_of(tl, tv, a.tot, b * H + h0, hn, NCH, 0, c, lane, tid);
    if (lane) scan_lane(sm.x[tid], carry);
    __syncthreads();
    // g, F, rowf, colf: (B,H,L) rows, one (head, row) per thread, coalesced along L
    {
        const int hh = tid >> 6, r = tid & 63;
        if (hh < hn && r < nrows) {   // hh >= HG for the upper half of the workgroup
            const int64_t o = ((int64_t)(b * H + h0 + hh)) * L + c * CH + r;
            const float* gx = sm.x[hh * NCOMP];
            const float g = gx[r];
            a.g[o] = g;
            a.rowf[o] = exp2_le0((g - gx[0]) * LOG2E);
            a.colf[o] = exp2_le0((gx[CH - 1] - g) * LOG2E);   // rows >= L added 0: the last valid g
            if (a.z) a.f[o] = sm.x[hh * NCOMP + 1][r];
        }
    }
    // rotation of C and B by Phi (fp32, one rounding to T); 4 pairs per vector
    T* CR = (T*)a.cr;
    T* BR = (T*)a.br;
#pragma unroll
    for (int i = 0; i < NU; ++i) {
        const Unit u = cb_unit(tid + NT * i);
        if (u.row >= nrows || u.hl >= hn) continue;
        f32x4 clo, chi, blo, bhi;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            float sn, cs;
            sincos_rev(sm.x[u.hl * NCOMP + 2 + 4 * u.q + p][u.row], &sn, &cs);
            const float ce = (float)cv[i][2 * p], co = (float)cv[i][2 * p + 1];
            const float be = (float)bv[i][2 * p], bo = (float)bv[i][2 * p + 1];
            const float c0 = ce * cs - co * sn, c1 = ce * sn + co * cs;
            const float b0 = be * cs - bo * sn, b1 = be * sn + bo * cs;
            if (p < 2) {
                clo[2 * p] = c0; clo[2 * p + 1] = c1; blo[2 * p] = b0; blo[2 * p + 1] = b1;
            } else {
                chi[2 * p - 4] = c0; chi[2 * p - 3] = c1; bhi[2 * p - 4] = b0; bhi[2 * p - 3] = b1;
            }
        }
        const int64_t o = (((int64_t)b * L + c * CH + u.row) * H + h0 + u.hl) * DS + 8 * u.q;
        *reinterpret_cast<frag8<T>*>(CR + o) = pack8<T>(clo, chi);
        *reinterpret_cast<frag8<T>*>(BR + o) = pack8<T>(blo, bhi);
    }
}

// ------------------------------------------------------------------------------------------------ backward
// Workspace: fp64 chunk totals BT (B*H, NCH, 18), then dPhi rows (B, L, H, 16) fp32 written by pass 1.
__host__ __device__ inline int64_t bt_bytes(int B, int L, int H) {
    return ((int64_t)B * H * ((L + CH - 1) / CH) * NCOMP * (int64_t)sizeof(double) + 255) / 256 * 256;
}

// Pass 1: recompute Phi (the forward scan of theta), then per (row, head, 4 pairs): dPhi = sum over {C, B} of
// dout_odd * out_even - dout_even * out_odd, the inverse rotation dC = R(-Phi) dC~, dB = R(-Phi) dB~ into dproj, dPhi
// rows into the workspace, and the fp64 chunk totals of (dg, dF, dPhi[16]).
template <class T>
__global__ __launch_bounds__(NT) void prep_bsums_kernel(sisa_prep_bwd_args a) {
    __shared__ ScanLds sm;
    __shared__ TotLds<float> tl;
    const int c = blockIdx.x, b = blockIdx.y, h0 = blockIdx.z * HG;
    const int H = a.H, L = a.L, NCH = gridDim.x;
    const int hn = (H - h0 < HG) ? H - h0 : HG;
    const int nrows = (L - c * CH < CH) ? L - c * CH : CH;
    const Layout off = layout_of(H);
    const int tid = threadIdx.x;
    const T* P = (const T*)a.proj + (int64_t)b * a.s_pb + (int64_t)c * CH * a.s_pl;
    // Every global load is issued before the first wait, in the order of use: theta, dg and dF, the forward totals
    // of the preceding chunks, then the C, B, dC~ and dB~ vectors of this thread.
    const StageVals<T> sv = stage_load<T, false>(P, a.s_pl, nullptr, 0, nrows, hn, off, h0, tid);
    float dgv = 0.f, dfv = 0.f;   // dg and dF of (head tid>>6, row tid&63)
    if (tid < CH * HG) {
        const int hh = tid >> 6, r = tid & 63;
        const bool ok = hh < hn && r < nrows;
        const int64_t o = (int64_t)(b * H + h0 + hh) * L + c * CH + r;
        if (ok) dgv = a.dg[o];
        if (ok && a.df) dfv = a.df[o];
    }
    const bool lane = tid < HC && tid / NCOMP < hn && tid % NCOMP >= 2;   // Phi lanes (components 2..17)
    float tv[TPT];
    tot_load(tv, a.tot, b * H + h0, hn, NCH, 0, c < TB ? c : TB, tid);
    frag8<T> cv[NU], bv[NU];
    f32x4 dc[NU][2], db[NU][2];
#pragma unroll
    for (int i = 0; i < NU; ++i) {
        const Unit u = cb_unit(tid + NT * i);
        const bool ok = u.row < nrows && u.hl < hn;
        const T* prow = P + (int64_t)u.row * a.s_pl + (h0 + u.hl) * DS + 8 * u.q;
        cv[i] = load8_if<T>(prow + off.C, ok);
        bv[i] = load8_if<T>(prow + off.B, ok);
        const int64_t o = (((int64_t)b * L + c * CH + u.row) * H + h0 + u.hl) * DS + 8 * u.q;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            dc[i][k] = ok ? *reinterpret_cast<const f32x4*>(a.dcr + o + 4 * k) : zero4();
            db[i][k] = ok ? *reinterpret_cast<const f32x4*>(a.dbr + o + 4 * k) : zero4();
        }
    }
    stage_store<T, false>(sm, sv, nrows, hn, false, tid);
    if (tid < CH * HG) {
        const int hh = tid >> 6, r = tid & 63;
        sm.x[(hh & 3) * NCOMP + 0][r] = dgv;
        sm.x[(hh & 3) * NCOMP + 1][r] = dfv;
    }
    tot_store(tl, tv, tid);
    __syncthreads();
    const float carry = carry_of(tl, tv, a.tot, b * H + h0, hn, NCH, 0, c, lane, tid);
    if (lane) scan_lane(sm.x[tid], carry);   // Phi: the forward scan of theta
    __syncthreads();
    T* DP = (T*)a.dproj + (int64_t)b * a.s_db + (int64_t)c * CH * a.s_dl;
    float* DPHI = (float*)((char*)a.workspace + bt_bytes(a.B, L, H));
    float dphi[NU][4];
#pragma unroll
    for (int i = 0; i < NU; ++i) {
        const Unit u = cb_unit(tid + NT * i);
        const bool ok = u.row < nrows && u.hl < hn;
        f32x4 xlo, xhi, ylo, yhi;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            float sn, cs;
            sincos_rev(ok ? sm.x[u.hl * NCOMP + 2 + 4 * u.q + p][u.row] : 0.f, &sn, &cs);
            const float dc0 = dc[i][p >> 1][2 * (p & 1)], dc1 = dc[i][p >> 1][2 * (p & 1) + 1];
            const float db0 = db[i][p >> 1][2 * (p & 1)], db1 = db[i][p >> 1][2 * (p & 1) + 1];
            const float ce = (float)cv[i][2 * p], co = (float)cv[i][2 * p + 1];
            const float be = (float)bv[i][2 * p], bo = (float)bv[i][2 * p + 1];
            const float coe = ce * cs - co * sn, coo = ce * sn + co * cs;
            const float boe = be * cs - bo * sn, boo = be * sn + bo * cs;
            const float d1 = dc1 * coe - dc0 * coo;
            const float d2 = db1 * boe - db0 * boo;
            dphi[i][p] = ok ? d1 + d2 : 0.f;
            const float x0 = dc0 * cs + dc1 * sn, x1 = dc1 * cs - dc0 * sn;
            const float y0 = db0 * cs + db1 * sn, y1 = db1 * cs - db0 * sn;
            if (p < 2) {
                xlo[2 * p] = x0; xlo[2 * p + 1] = x1; ylo[2 * p] = y0; ylo[2 * p + 1] = y1;
            } else {
                xhi[2 * p - 4] = x0; xhi[2 * p - 3] = x1; yhi[2 * p - 4] = y0; yhi[2 * p - 3] = y1;
            }
        }
        if (ok) {
            T* drow = DP + (int64_t)u.row * a.s_dl + (h0 + u.hl) * DS + 8 * u.q;
            *reinterpret_cast<frag8<T>*>(drow + off.C) = pack8<T>(xlo, xhi);
            *reinterpret_cast<frag8<T>*>(drow + off.B) = pack8<T>(ylo, yhi);
            const int64_t o = (((int64_t)b * L + c * CH + u.row) * H + h0 + u.hl) * S2 + 4 * u.q;
            *reinterpret_cast<f32x4*>(DPHI + o) = f32x4{dphi[i][0], dphi[i][1], dphi[i][2], dphi[i][3]};
        }
    }
    __syncthreads();   // every Phi read is done before the lanes are overwritten with dPhi
#pragma unroll
    for (int i = 0; i < NU; ++i) {
        const Unit u = cb_unit(tid + NT * i);
#pragma unroll
        for (int p = 0; p < 4; ++p) sm.x[u.hl * NCOMP + 2 + 4 * u.q + p][u.row] = dphi[i][p];
    }
    __syncthreads();
    double* BT = (double*)a.workspace;
    if (tid < HC && tid / NCOMP < hn) {
        double s = 0.0;
#pragma unroll 16
        for (int r = 0; r < CH; ++r) s += (double)sm.x[tid][r];
        BT[((int64_t)(b * H + h0 + tid / NCOMP) * NCH + c) * NCOMP + tid % NCOMP] = s;
    }
}

// Pass 2: reverse scans (fp64 carry of the following chunks + in-chunk reverse sums) into d alpha, dz, d theta; pad
// columns set to zero. d alpha = -suffix * softplus'(alpha) and dz = suffix * logsigmoid'(z) are formed by the
// threads that loaded alpha and z, when they write them.
template <class T>
__global__ __launch_bounds__(NT) void prep_bwd_kernel(sisa_prep_bwd_args a) {
    __shared__ ScanLds sm;
    __shared__ TotLds<double> tl;
    const int c = blockIdx.x, b = blockIdx.y, h0 = blockIdx.z * HG;
    const int H = a.H, L = a.L, NCH = gridDim.x;
    const int hn = (H - h0 < HG) ? H - h0 : HG;
    const int nrows = (L - c * CH < CH) ? L - c * CH : CH;
    const Layout off = layout_of(H);
    const int tid = threadIdx.x;
    const T* P = (const T*)a.proj + (int64_t)b * a.s_pb + (int64_t)c * CH * a.s_pl;
    const float* DPHI = (const float*)((const char*)a.workspace + bt_bytes(a.B, L, H));
    const double* BT = (const double*)a.workspace;
    // Every global load is issued before the first wait: dPhi rows (written by pass 1; one (row, head, 4 pairs)
    // vector per thread and iteration), dg and dF, alpha and z, and the fp64 totals of the following chunks.
    f32x4 dph[NU];
#pragma unroll
    for (int i = 0; i < NU; ++i) {
        const Unit u = cb_unit(tid + NT * i);
        const bool ok = u.row < nrows && u.hl < hn;
        const int64_t o = (((int64_t)b * L + c * CH + u.row) * H + h0 + u.hl) * S2 + 4 * u.q;
        dph[i] = ok ? *reinterpret_cast<const f32x4*>(DPHI + o) : zero4();
    }
    float dgv = 0.f, dfv = 0.f, al = 0.f, zv = 0.f;
    if (tid < CH * HG) {
        const int hh = tid >> 6, r = tid & 63;   // dg, dF of (head hh, row r): coalesced along L
        if (hh < hn && r < nrows) {
            const int64_t o = (int64_t)(b * H + h0 + hh) * L + c * CH + r;
            dgv = a.dg[o];
            if (a.df) dfv = a.df[o];
        }
        const int row = tid >> 2, hl = tid & 3;   // alpha, z of (row, head hl): contiguous in the row
        if (row < nrows && hl < hn) {
            al = (float)P[(int64_t)row * a.s_pl + off.A + h0 + hl];
            if (a.z) zv = a.z[(int64_t)b * a.s_zb + (int64_t)(c * CH + row) * a.s_zl + h0 + hl];
        }
    }
    // fp64 totals of the following chunks (carries of the reverse scans)
    const int c0 = c + 1;
    double tv[TPT];
    tot_load(tv, BT, b * H + h0, hn, NCH, c0, (NCH - c0 < TB) ? NCH : c0 + TB, tid);
#pragma unroll
    for (int i = 0; i < NU; ++i) {
        const Unit u = cb_unit(tid + NT * i);
#pragma unroll
        for (int p = 0; p < 4; ++p) sm.x[u.hl * NCOMP + 2 + 4 * u.q + p][u.row] = dph[i][p];
    }
    if (tid < CH * HG) {
        const int hh = tid >> 6, r = tid & 63;
        sm.x[hh * NCOMP + 0][r] = dgv;
        sm.x[hh * NCOMP + 1][r] = dfv;
    }
    tot_store(tl, tv, tid);
    const bool lane = tid < HC && tid / NCOMP < hn;
    __syncthreads();
    const double sa = carry_of(tl, tv, BT, b * H + h0, hn, NCH, c0, NCH, lane, tid);
    if (lane) {
        float* x = sm.x[tid];
        float v[CH];
#pragma unroll
        for (int r = 0; r < CH; ++r) v[r] = x[r];
        double rev = 0.0;
#pragma unroll
        for (int r = CH - 1; r >= 0; --r) {
            rev += (double)v[r];
            x[r] = (float)(sa + rev);   // the suffix sum; d alpha and dz take their element derivative below
        }
    }
    __syncthreads();
    T* DP = (T*)a.dproj + (int64_t)b * a.s_db + (int64_t)c * CH * a.s_dl;
    // d theta: 8 columns per vector
#pragma unroll
    for (int i = 0; i < 512 / NT; ++i) {
        const int v = tid + NT * i;
        const int row = v >> 3, hl = (v >> 1) & 3, half = v & 1;
        if (row >= nrows || hl >= hn) continue;
        f32x4 lo, hi;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            lo[j] = sm.x[hl * NCOMP + 2 + 8 * half + j][row];
            hi[j] = sm.x[hl * NCOMP + 6 + 8 * half + j][row];
        }
        *reinterpret_cast<frag8<T>*>(DP + (int64_t)row * a.s_dl + off.TH + (h0 + hl) * S2 + 8 * half) =
            pack8<T>(lo, hi);
    }
    if (tid < CH * HG) {
        const int row = tid >> 2, hl = tid & 3;
        if (row < nrows && hl < hn) {
            DP[(int64_t)row * a.s_dl + off.A + h0 + hl] = cvt<T>(-sm.x[hl * NCOMP + 0][row] * softplus_grad(al));
            if (a.dz)
                a.dz[(int64_t)b * a.s_dzb + (int64_t)(c * CH + row) * a.s_dzl + h0 + hl] =
                    sm.x[hl * NCOMP + 1][row] * logsigmoid_grad(zv);
        }
    }
    // zero padding columns (they multiply the zero rows of W_cat; keeps NaN out of dX)
    if (blockIdx.z == 0 && off.NPAD > off.NTOT) {
        const int npad = off.NPAD - off.NTOT;
        for (int idx = tid; idx < CH * npad; idx += NT) {
            const int r = idx / npad, j = idx % npad;
            if (r < nrows) DP[(int64_t)r * a.s_dl + off.NTOT + j] = cvt<T>(0.f);
        }
    }
}

// ------------------------------------------------------------------------------------------------ non-finite guard
// ok = (sum(a) + sum(b) is finite) as one byte: the input check of the fused path (fused_prep.py:502-523: a NaN or
// inf anywhere in lse, where every score input meets, or in the block totals makes the sum non-finite) in one
// launch of one workgroup. fp32 sums in a fixed order (per-thread strided partials over 16-byte vectors, then a
// fixed tree), so the result does not depend on scheduling.
constexpr int GT = 1024;
SISA_DEV float strided_sum(const float* p, int64_t n, int tid) {
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    const int64_t nv = n / 4;
    const f32x4* pv = reinterpret_cast<const f32x4*>(p);
    int64_t i = tid;
    for (; i + 3 * GT < nv; i += 4 * GT) {   // four vectors in flight per thread
        const f32x4 v0 = pv[i], v1 = pv[i + GT], v2 = pv[i + 2 * GT], v3 = pv[i + 3 * GT];
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] += (v0[e] + v1[e]) + (v2[e] + v3[e]);
    }
    for (; i < nv; i += GT) {
        const f32x4 v = pv[i];
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] += v[e];
    }
    for (int64_t j = 4 * nv + tid; j < n; j += GT) acc[0] += p[j];
    return (acc[0] + acc[1]) + (acc[2] + acc[3]);
}

__global__ __launch_bounds__(GT) void finite_sum_kernel(const float* a, int64_t na, const float* b, int64_t nb,
                                                        uint8_t* ok) {
    __shared__ float red[GT / 64];
    const int tid = threadIdx.x;
    float s = strided_sum(a, na, tid) + strided_sum(b, nb, tid);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
    if ((tid & 63) == 0) red[tid >> 6] = s;
    __syncthreads();
    if (tid == 0) {
        float t = 0.f;
#pragma unroll
        for (int w = 0; w < GT / 64; ++w) t += red[w];
        ok[0] = (t - t == 0.f) ? 1 : 0;   // x - x is 0 for finite x, NaN for NaN and +-inf
    }
}

template <class T>
int launch_prep_fwd(const sisa_prep_fwd_args* a, hipStream_t st) {
    dim3 grid((unsigned)sisa::cdiv(a->L, CH), (unsigned)a->B, (unsigned)sisa::cdiv(a->H, HG));
    prep_sums_kernel<T><<<grid, NT, 0, st>>>(*a);
    int rc = sisa::launch_status("sisa_prep_fwd (sums)");
    if (rc) return rc;
    prep_fwd_kernel<T><<<grid, NT, 0, st>>>(*a);
    return sisa::launch_status("sisa_prep_fwd");
}

template <class T>
int launch_prep_bwd(const sisa_prep_bwd_args* a, hipStream_t st) {
    dim3 grid((unsigned)sisa::cdiv(a->L, CH), (unsigned)a->B, (unsigned)sisa::cdiv(a->H, HG));
    prep_bsums_kernel<T><<<grid, NT, 0, st>>>(*a);
    int rc = sisa::launch_status("sisa_prep_bwd (sums)");
    if (rc) return rc;
    prep_bwd_kernel<T><<<grid, NT, 0, st>>>(*a);
    return sisa::launch_status("sisa_prep_bwd");
}

}  // namespace

extern "C" int sisa_prep_fwd(const sisa_prep_fwd_args* a, void* stream) {
    SISA_REQUIRE(a != nullptr, "sisa_prep_fwd: null args");
    SISA_REQUIRE(a->B >= 1 && a->L >= 1 && a->H >= 1, "sisa_prep_fwd: bad shape B=%d L=%d H=%d", a->B, a->L, a->H);
    SISA_REQUIRE(a->dtype == SISA_BF16 || a->dtype == SISA_F16, "sisa_prep_fwd: proj dtype must be bf16/fp16");
    SISA_REQUIRE(a->proj && a->cr && a->br && a->g && a->rowf && a->colf && a->tot, "sisa_prep_fwd: null pointer");
    SISA_REQUIRE(a->z == nullptr || a->f != nullptr, "sisa_prep_fwd: f is required with z");
    SISA_REQUIRE(a->s_pl >= layout_of(a->H).NPAD && a->s_pl % 8 == 0 && a->s_pb % 8 == 0 && sisa::aligned16(a->proj),
                 "sisa_prep_fwd: proj must be 16-byte aligned with row and batch strides that are multiples of 8 "
                 "(row stride %lld)", (long long)a->s_pl);
    SISA_REQUIRE(sisa::aligned16(a->cr) && sisa::aligned16(a->br), "sisa_prep_fwd: cr/br must be 16-byte aligned");
    hipStream_t st = (hipStream_t)stream;
    return a->dtype == SISA_BF16 ? launch_prep_fwd<__bf16>(a, st) : launch_prep_fwd<_Float16>(a, st);
}

extern "C" int sisa_finite_sum(const float* a, int64_t na, const float* b, int64_t nb, uint8_t* ok, void* stream) {
    SISA_REQUIRE(ok != nullptr && na >= 0 && nb >= 0 && (na == 0 || a) && (nb == 0 || b),
                 "sisa_finite_sum: bad arguments (na=%lld nb=%lld)", (long long)na, (long long)nb);
    SISA_REQUIRE((na == 0 || sisa::aligned16(a)) && (nb == 0 || sisa::aligned16(b)),
                 "sisa_finite_sum: a and b must be 16-byte aligned");
    finite_sum_kernel<<<1, GT, 0, (hipStream_t)stream>>>(a, na, b, nb, ok);
    return sisa::launch_status("sisa_finite_sum");
}

extern "C" int64_t sisa_prep_bwd_workspace_bytes(int32_t B, int32_t L, int32_t H) {
    return bt_bytes(B, L, H) + (int64_t)B * L * H * S2 * (int64_t)sizeof(float);
}

extern "C" int sisa_prep_bwd(const sisa_prep_bwd_args* a, void* stream) {
    SISA_REQUIRE(a != nullptr, "sisa_prep_bwd: null args");
    SISA_REQUIRE(a->B >= 1 && a->L >= 1 && a->H >= 1, "sisa_prep_bwd: bad shape B=%d L=%d H=%d", a->B, a->L, a->H);
    SISA_REQUIRE(a->dtype == SISA_BF16 || a->dtype == SISA_F16, "sisa_prep_bwd: proj dtype must be bf16/fp16");
    SISA_REQUIRE(a->proj && a->tot && a->dg && a->dcr && a->dbr && a->dproj && a->workspace,
                 "sisa_prep_bwd: null pointer");
    SISA_REQUIRE((a->z == nullptr) == (a->df == nullptr) && (a->z == nullptr) == (a->dz == nullptr),
                 "sisa_prep_bwd: z, df and dz must all be given or all be null");
    SISA_REQUIRE(a->s_pl >= layout_of(a->H).NPAD && a->s_dl >= layout_of(a->H).NPAD && a->s_pl % 8 == 0 &&
                     a->s_pb % 8 == 0 && a->s_dl % 8 == 0 && a->s_db % 8 == 0,
                 "sisa_prep_bwd: row strides must be >= NPAD and, like the batch strides, multiples of 8");
    SISA_REQUIRE(sisa::aligned16(a->proj) && sisa::aligned16(a->dproj) && sisa::aligned16(a->dcr) &&
                     sisa::aligned16(a->dbr) && sisa::aligned16(a->workspace),
                 "sisa_prep_bwd: proj, dproj, dcr, dbr and workspace must be 16-byte aligned");
    hipStream_t st = (hipStream_t)stream;
    return a->dtype == SISA_BF16 ? launch_prep_bwd<__bf16>(a, st) : launch_prep_bwd<_Float16>(a, st);
}
