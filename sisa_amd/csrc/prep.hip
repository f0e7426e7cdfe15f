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
// Scan scheme (deterministic reduce-then-scan over 64-row chunks): chunk totals first, then the left fold of the
// preceding chunks' totals (the carry) added to a two-level in-chunk scan: four 16-row sub-chunks scanned in row order
// by separate threads, then each value offset by the fold of the preceding sub-chunk totals. The chunk total is formed
// by the same code, so carry_{c+1} = carry_c + TOT_c equals the last value of chunk c bit for bit, and for
// non-positive inputs (g, F) every level of the nesting carry + (P_s + v_r) is non-increasing: g never increases,
// inside a chunk or across a boundary. The backward runs the same scheme in reverse with fp64 accumulators.
//
// Decomposition: one 512-thread workgroup per (64-row chunk, batch row, group of HG = 4 heads); 288 scan tasks (head,
// component, sub-chunk) run out of LDS while 72 other threads fold the carry from totals staged through LDS.
//   forward   two launches: prep_sums writes the chunk totals TOT; prep_fwd loads the totals and the scan inputs
//             (cached by prep_sums) first and has waves 0..3 move C and B straight into LDS, so the carry fold and
//             the scans run while C and B are in flight (LDS-only barriers until the rotation).
//   backward  one launch, prep_bwd: Phi recomputed from theta and TOT, dPhi and the inverse rotation, the fp64 chunk
//             totals of (dg, dF, dPhi) handed to the other workgroups of the launch through the workspace (the total
//             exchange below), the reverse scans. No dPhi rows leave the chip.
#include <stdlib.h>

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

// Scan columns: x[hl*NCOMP + comp][r] holds the element values of chunk row r (0 beyond L), then the inclusive scan
// plus the carry of the preceding chunks. Rows padded to 65 floats: the scan tasks of a wave, on consecutive columns,
// read without bank conflicts.
struct ScanLds {
    float x[HC][CH + 1];
};

// Two-level in-chunk scans: NSUB sub-chunks of SUB rows. Scan task t < NTASK owns (column t % HC, sub-chunk t / HC)
// and runs its SUB rows in order; thread NTASK + l folds the carry of column l meanwhile (carry_of below).
constexpr int SUB = 16, NSUB = CH / SUB, NTASK = HC * NSUB;
static_assert(NTASK + HC <= NT, "scan tasks and carry lanes on distinct threads");
template <class Acc>
struct SubLds {
    Acc sub[NSUB][HC];   // sub-chunk totals
    Acc carry[HC];       // carry of the preceding (forward) or following (reverse) chunks
};

// Forward scan, phase 1, in place: x[SUB*s + r] <- v_r = x[SUB*s] + ... + x[SUB*s + r] summed in row order; the
// sub-chunk total is v_{SUB-1}.
SISA_DEV void fwd_sub_scan(ScanLds& sm, SubLds<float>& sl, int t) {
    const int col = t % HC, s = t / HC;
    float* x = sm.x[col] + SUB * s;
    float v[SUB];
#pragma unroll
    for (int r = 0; r < SUB; ++r) v[r] = x[r];
#pragma unroll
    for (int r = 1; r < SUB; ++r) v[r] += v[r - 1];
#pragma unroll
    for (int r = 1; r < SUB; ++r) x[r] = v[r];
    sl.sub[s][col] = v[SUB - 1];
}
// P_n: the left fold, from 0, of the first n sub-chunk totals of column col. The chunk total is P_NSUB.
SISA_DEV float fwd_sub_prefix(const SubLds<float>& sl, int col, int n) {
    float p = 0.f;
#pragma unroll
    for (int j = 0; j < NSUB; ++j)
        if (j < n) p += sl.sub[j][col];
    return p;
}
// Forward scan, phase 2: x[SUB*s + r] = carry + (P_s + v_r). For non-positive inputs each level is non-increasing
// and ends on the first partial sum of the level above (v[SUB-1] + P_s = P_{s+1}; carry_c + P_NSUB = carry_{c+1}),
// so the result is non-increasing over the chunk and across chunk boundaries.
SISA_DEV void fwd_sub_finish(ScanLds& sm, const SubLds<float>& sl, int t) {
    const int col = t % HC, s = t / HC;
    const float p = fwd_sub_prefix(sl, col, s), carry = sl.carry[col];
    float* x = sm.x[col] + SUB * s;
#pragma unroll
    for (int r = 0; r < SUB; ++r) x[r] = carry + (p + x[r]);
}

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

// Workgroup barrier that orders LDS only: global loads and buffer->LDS transfers a wave has in flight stay in flight
// across it (a plain barrier waits for all of them first).
SISA_DEV void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
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
// The carry of column li (when `lane`) over chunks [c0, c1). The caller has loaded the first batch into v with
// tot_load(v, ..., c0, min(c1, c0 + TB)), stored it (tot_store) and passed a barrier. Further batches are loaded and
// folded here; every thread of the workgroup calls this (it has barriers when c1 - c0 > TB).
template <class Acc>
SISA_DEV Acc carry_of(TotLds<Acc>& tl, Acc (&v)[TPT], const Acc* tot, int bh0, int hn, int NCH, int c0, int c1,
                      bool lane, int li, int tid) {
    const int hl = li / NCOMP, comp = li % NCOMP;
    Acc acc = lane ? tot_fold(tl, hl, comp, (c1 - c0 < TB) ? c1 - c0 : TB, (Acc)0) : (Acc)0;
    for (int cb = c0 + TB; cb < c1; cb += TB) {
        const int ce = (c1 - cb < TB) ? c1 : cb + TB;
        tot_load(v, tot, bh0, hn, NCH, cb, ce, tid);
        lds_barrier();   // every lane is done with the previous batch
        tot_store(tl, v, tid);
        lds_barrier();
        if (lane) acc = tot_fold(tl, hl, comp, ce - cb, acc);
    }
    return acc;
}

// ------------------------------------------------------------------------------------------------ total exchange
// The backward's workgroups hand their fp64 chunk totals to each other through the workspace instead of through a
// second launch. A total travels as two 64-bit words (its low and high 32 bits) whose upper halves are the launch's
// tag, written and polled with relaxed device-scope atomics: a word is read whole, so a half and its tag always belong
// together and no fence is needed, and a word left by an earlier launch carries an older tag. The tag is the
// workspace's epoch + 1. Every workgroup reads the epoch before it counts itself in `arrivals` (at its end); the last
// to arrive resets the count and advances the epoch, which the next launch on the stream then reads. A zeroed
// workspace starts at epoch 0 with no word tagged 1.
//
// Progress: the workgroups are numbered chunk-major from the last chunk down (the last chunk of every sequence before
// the one below it), each publishes its totals before it waits, and it waits only for workgroups of lower number,
// which the hardware dispatches first, so the lowest unfinished workgroup never waits. The wait is bounded all the
// same: after SPIN_LIMIT polls the `error` word is set, the missing totals count as zero and the launch ends (the
// environment variable SISA_PREP_SPIN_LIMIT lowers the bound, so that a test can take that path on purpose).
struct XchHeader {
    uint32_t epoch, arrivals, error;
};
constexpr int64_t XCH_HEADER = 256;   // bytes before the words
constexpr int SPIN_LIMIT = 1 << 15;
constexpr int XW = 2;                 // words per total

__host__ __device__ inline int64_t xch_bytes(int B, int L, int H) {
    const int64_t seqs = (int64_t)B * ((H + HG - 1) / HG), chunks = (L + CH - 1) / CH;
    return XCH_HEADER + seqs * chunks * HC * XW * (int64_t)sizeof(uint64_t);
}

SISA_DEV uint64_t tagged(uint32_t tag, uint32_t bits) { return ((uint64_t)tag << 32) | bits; }
SISA_DEV void xch_put(uint64_t* w, uint32_t tag, double v) {
    const uint64_t u = (uint64_t)__double_as_longlong(v);
    __hip_atomic_store(w, tagged(tag, (uint32_t)u), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(w + 1, tagged(tag, (uint32_t)(u >> 32)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// A poll of a word: the first of a gather at workgroup scope (a plain load, which the caches may serve and which may
// return an older copy of the line), every later one at device scope (coherent across the XCDs' L2s). Either way a
// word carrying this launch's tag holds its final value (each word is written once per launch), so a cached copy is
// used when it is current and polled again coherently when it is not.
SISA_DEV uint64_t xch_load(const uint64_t* w, bool coherent) {
    return coherent ? __hip_atomic_load(const_cast<uint64_t*>(w), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                    : __hip_atomic_load(const_cast<uint64_t*>(w), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Exchanged totals of up to TB chunks, [chunk - first][column].
struct XLds {
    double t[TB][HC];
};
constexpr int GPT = (TB * HC) / NT;   // totals per thread and batch
static_assert(GPT * NT == TB * HC && GPT <= 32 && (TB & (TB - 1)) == 0, "gathered totals split evenly");

// The totals of chunks [c0, c1) (at most TB) of one sequence's words (laid out [chunk][column][2]) into xl (zero for
// columns of absent heads), each polled until both its words carry `tag`; thread t takes the totals t, t + NT, ... of
// the range. All loads of a poll are issued before the first is examined; a total goes to LDS as soon as it has
// arrived. The first poll may be served by the caches (the totals of chunks whose workgroups finished before this
// one started are then read from L2 rather than from memory, once per XCD).
SISA_DEV void xch_gather(XLds& xl, const uint64_t* seqw, int hn, int c0, int c1, uint32_t tag, uint32_t* err, int t,
                         int spin_limit) {
    const int n = (c1 - c0) * HC;
    double* dst = &xl.t[0][0];
    const uint64_t* src = seqw + ((int64_t)c0 * HC + t) * XW;
    uint32_t pending = 0;
#pragma unroll
    for (int q = 0; q < GPT; ++q) {
        const int e = t + NT * q;
        if (e < n && (e % HC) / NCOMP < hn)
            pending |= 1u << q;
        else
            dst[e] = 0.0;
    }
    for (int it = 0; pending != 0; ++it) {
        uint64_t lo[GPT], hi[GPT];
#pragma unroll
        for (int q = 0; q < GPT; ++q)
            if (pending & (1u << q)) {
                lo[q] = xch_load(src + NT * XW * q, it > 0);
                hi[q] = xch_load(src + NT * XW * q + 1, it > 0);
            }
#pragma unroll
        for (int q = 0; q < GPT; ++q)
            if ((pending & (1u << q)) && (uint32_t)(lo[q] >> 32) == tag && (uint32_t)(hi[q] >> 32) == tag) {
                dst[t + NT * q] = __longlong_as_double((long long)((hi[q] << 32) | (lo[q] & 0xffffffffull)));
                pending &= ~(1u << q);
            }
        if (pending == 0) break;
        if (it >= spin_limit) {
            __hip_atomic_fetch_or(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
            for (int q = 0; q < GPT; ++q)
                if (pending & (1u << q)) dst[t + NT * q] = 0.0;
            break;
        }
        __builtin_amdgcn_s_sleep(4);
    }
}

// The left fold, in chunk order, of the exchanged totals of chunks [c0, c1) for column li (when `lane`). Every thread
// of the workgroup calls this: it gathers through LDS, TB chunks per batch; the reads of FB chunks are issued before
// their adds.
SISA_DEV double carry_xch(XLds& xl, const uint64_t* seqw, int hn, int c0, int c1, uint32_t tag, uint32_t* err,
                          int spin_limit, bool lane, int li, int tid) {
    constexpr int FB = 16;
    double acc = 0.0;
    for (int cb = c0; cb < c1; cb += TB) {
        const int ce = (c1 - cb < TB) ? c1 : cb + TB;
        if (cb > c0) __syncthreads();   // every lane is done with the previous batch
        xch_gather(xl, seqw, hn, cb, ce, tag, err, tid, spin_limit);
        __syncthreads();
        if (lane) {
            for (int k0 = 0; k0 < ce - cb; k0 += FB) {
                double buf[FB];
#pragma unroll
                for (int k = 0; k < FB; ++k) buf[k] = xl.t[(k0 + k) & (TB - 1)][li];
#pragma unroll
                for (int k = 0; k < FB; ++k) acc += (k0 + k < ce - cb) ? buf[k] : 0.0;
            }
        }
    }
    return acc;
}

// The launch's arrival (thread 0, at its end): the last workgroup to arrive resets the count and advances the epoch.
SISA_DEV void xch_arrive(XchHeader* xh, uint32_t epoch, unsigned nwg) {
    const uint32_t before = __hip_atomic_fetch_add(&xh->arrivals, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (before == nwg - 1) {
        __hip_atomic_store(&xh->arrivals, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&xh->epoch, epoch + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Workgroup w of the backward's launch: sequence seq = w % NSEQ (batch row seq / NHG, heads of group seq % NHG),
// chunk NCH - 1 - w / NSEQ (chunk-major from the last chunk down, the order the total exchange waits in).
struct Geo {
    int c, b, h0, hn, nrows, NCH, seq;
};
SISA_DEV Geo bwd_geo(int B, int L, int H) {
    Geo g;
    const int NHG = (H + HG - 1) / HG, NSEQ = B * NHG;
    g.NCH = (L + CH - 1) / CH;
    g.seq = (int)blockIdx.x % NSEQ;
    g.c = g.NCH - 1 - (int)blockIdx.x / NSEQ;
    g.b = g.seq / NHG;
    g.h0 = (g.seq % NHG) * HG;
    g.hn = (H - g.h0 < HG) ? H - g.h0 : HG;
    g.nrows = (L - g.c * CH < CH) ? L - g.c * CH : CH;
    return g;
}

// Stores of outputs that no later step of the launch reads: non-temporal, so that they stream to memory while the
// kernel runs instead of waiting in L2 for the write-back at its end (1.5 us of the forward pass at the north-star
// shape).
template <class V>
SISA_DEV void store_nt(V* p, const V& v) {
    __builtin_nontemporal_store(v, p);
}

// Buffer->LDS staging of a chunk's C and B columns of the workgroup's heads into cbl = [C, B][CH rows][CB_ROW]: wave
// instruction k (0..31, eight for each of waves 0..3) moves 1 KB, four rows of one block, lane i one 16-byte piece.
// Rows past the chunk's valid rows read as zero (the buffer's extent ends there).
constexpr int CB_ROW = HG * DS;   // elements of a staged row
template <int KERNEL, class T>
SISA_DEV void cb_dma(const T* P, int64_t s_pl, int nrows, const Layout& off, int h0, T* cbl, int tid) {
    const __amdgpu_buffer_rsrc_t r = make_rsrc(P, (int64_t)nrows * s_pl * (int64_t)sizeof(T));
    const int w = tid >> 6, lane = tid & 63;
#pragma unroll
    for (int p = 0; p < 8; ++p) {
        const int k = w + 4 * p;
        const int pi = 64 * (k & 15) + lane;   // piece of the block: row pi / 16, 16-byte column pi % 16
        const int voff = (int)(((pi >> 4) * s_pl + ((k >> 4) ? off.B : off.C) + h0 * DS) * (int64_t)sizeof(T)) +
                         16 * (pi & 15);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            r, (__attribute__((address_space(3))) void*)(cbl + k * (1024 / (int)sizeof(T))), 16, voff, 0, 0, 0);
    }
}

// ------------------------------------------------------------------------------------------------ forward
// Two launches. Pass 1: TOT[bh][c][comp] = the chunk total P_NSUB of the element values, formed by the code of the
// pass-2 scan, so that it equals the chunk's last scanned value bit for bit.
template <class T>
__global__ __launch_bounds__(NT) void prep_sums_kernel(sisa_prep_fwd_args a) {
    __shared__ ScanLds sm;
    __shared__ SubLds<float> sl;
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
    if (tid < NTASK) fwd_sub_scan(sm, sl, tid);
    __syncthreads();
    if (tid < HC && tid / NCOMP < hn)
        a.tot[((int64_t)(b * H + h0 + tid / NCOMP) * NCH + c) * NCOMP + tid % NCOMP] = fwd_sub_prefix(sl, tid, NSUB);
}

// Pass 2: scans (carry of the preceding chunks + the two-level in-chunk scan), g/F/rowf/colf, rotation of C and B.
// The totals and scan inputs (cached by pass 1) are loaded first, then waves 0..3 move C and B straight into LDS;
// every barrier until the rotation orders LDS only, so the carry fold and the scans run while C and B are in flight.
template <class T>
__global__ __launch_bounds__(NT) void prep_fwd_kernel(sisa_prep_fwd_args a) {
    __shared__ ScanLds sm;
    __shared__ TotLds<float> tl;
    __shared__ SubLds<float> sl;
    __shared__ __attribute__((aligned(16))) T cbl[2 * CH * CB_ROW];
    const int c = blockIdx.x, b = blockIdx.y, h0 = blockIdx.z * HG;
    const int H = a.H, L = a.L, NCH = gridDim.x;
    const int hn = (H - h0 < HG) ? H - h0 : HG;
    const int nrows = (L - c * CH < CH) ? L - c * CH : CH;
    const Layout off = layout_of(H);
    const int tid = threadIdx.x;
    const T* P = (const T*)a.proj + (int64_t)b * a.s_pb + (int64_t)c * CH * a.s_pl;
    const float* Z = a.z ? a.z + (int64_t)b * a.s_zb + (int64_t)c * CH * a.s_zl : nullptr;
    float tv[TPT];
    tot_load(tv, a.tot, b * H + h0, hn, NCH, 0, c < TB ? c : TB, tid);
    const StageVals<T> sv = stage_load<T>(P, a.s_pl, Z, a.s_zl, nrows, hn, off, h0, tid);
    if (tid < 256) cb_dma<0, T>(P, a.s_pl, nrows, off, h0, cbl, tid);
    stage_store<T, true>(sm, sv, nrows, hn, Z != nullptr, tid);
    tot_store(tl, tv, tid);
    lds_barrier();
    if (tid < NTASK) fwd_sub_scan(sm, sl, tid);
    const int li = tid - NTASK;   // carry lane of column li
    const bool lane = li >= 0 && li < HC && li / NCOMP < hn;
    const float carry = carry_of(tl, tv, a.tot, b * H + h0, hn, NCH, 0, c, lane, li, tid);
    if (li >= 0 && li < HC) sl.carry[li] = carry;
    lds_barrier();
    if (tid < NTASK) fwd_sub_finish(sm, sl, tid);
    lds_barrier();
    // g, F, rowf, colf: (B,H,L) rows, one (head, row) per thread, coalesced along L
    {
        const int hh = tid >> 6, r = tid & 63;
        if (hh < hn && r < nrows) {   // hh >= HG for the upper half of the workgroup
            const int64_t o = ((int64_t)(b * H + h0 + hh)) * L + c * CH + r;
            const float* gx = sm.x[hh * NCOMP];
            const float g = gx[r];
            store_nt(a.g + o, g);
            store_nt(a.rowf + o, exp2_le0((g - gx[0]) * LOG2E));
            store_nt(a.colf + o, exp2_le0((gx[CH - 1] - g) * LOG2E));   // rows >= L added 0: the last valid g
            if (a.z) store_nt(a.f + o, sm.x[hh * NCOMP + 1][r]);
        }
    }
    __syncthreads();   // C and B have landed in LDS
    // rotation of C and B by Phi (fp32, one rounding to T); 4 pairs per vector
    T* CR = (T*)a.cr;
    T* BR = (T*)a.br;
#pragma unroll
    for (int i = 0; i < NU; ++i) {
        const Unit u = cb_unit(tid + NT * i);
        if (u.row >= nrows || u.hl >= hn) continue;
        const T* src = cbl + u.row * CB_ROW + u.hl * DS + 8 * u.q;
        const frag8<T> cv = load8<T>(src), bv = load8<T>(src + CH * CB_ROW);
        f32x4 clo, chi, blo, bhi;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            float sn, cs;
            sincos_rev(sm.x[u.hl * NCOMP + 2 + 4 * u.q + p][u.row], &sn, &cs);
            const float ce = (float)cv[2 * p], co = (float)cv[2 * p + 1];
            const float be = (float)bv[2 * p], bo = (float)bv[2 * p + 1];
            const float c0 = ce * cs - co * sn, c1 = ce * sn + co * cs;
            const float b0 = be * cs - bo * sn, b1 = be * sn + bo * cs;
            if (p < 2) {
                clo[2 * p] = c0; clo[2 * p + 1] = c1; blo[2 * p] = b0; blo[2 * p + 1] = b1;
            } else {
                chi[2 * p - 4] = c0; chi[2 * p - 3] = c1; bhi[2 * p - 4] = b0; bhi[2 * p - 3] = b1;
            }
        }
        const int64_t o = (((int64_t)b * L + c * CH + u.row) * H + h0 + u.hl) * DS + 8 * u.q;
        store_nt(reinterpret_cast<frag8<T>*>(CR + o), pack8<T>(clo, chi));
        store_nt(reinterpret_cast<frag8<T>*>(BR + o), pack8<T>(blo, bhi));
    }
}

// ------------------------------------------------------------------------------------------------ backward
// One launch, the chunks in reverse order: Phi recomputed (the forward scan of theta, its carry folded from the
// forward's TOT), then per (row, head, 4 pairs) dPhi = sum over {C, B} of dout_odd * out_even - dout_even * out_odd and
// the inverse rotation dC = R(-Phi) dC~, dB = R(-Phi) dB~ into dproj; the fp64 chunk totals of (dg, dF, dPhi[16])
// published; their carry folded from the following chunks; the reverse scans into d alpha, dz, d theta; pad columns
// set to zero. d alpha = -suffix * softplus'(alpha) and dz = suffix * logsigmoid'(z) are formed by the threads that
// loaded alpha and z.
template <class T>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(4, 8))) void prep_bwd_kernel(sisa_prep_bwd_args a,
                                                                                               int spin_limit) {
    __shared__ ScanLds sm;   // theta, then Phi
    __shared__ ScanLds sq;   // dg, dF and dPhi, then their reverse scans
    __shared__ union {
        TotLds<float> f;   // forward totals of the preceding chunks (Phi carry)
        XLds d;            // exchanged totals of the following chunks (reverse carry)
    } tu;
    __shared__ SubLds<float> sl;
    __shared__ SubLds<double> sd;
    __shared__ uint32_t s_tag;
    const int H = a.H, L = a.L;
    const Geo G = bwd_geo(a.B, L, H);
    const int c = G.c, b = G.b, h0 = G.h0, hn = G.hn, nrows = G.nrows, NCH = G.NCH;
    const Layout off = layout_of(H);
    const int tid = threadIdx.x;
    XchHeader* xh = (XchHeader*)a.workspace;
    uint64_t* seqw = (uint64_t*)((char*)a.workspace + XCH_HEADER) + (int64_t)G.seq * NCH * HC * XW;
    const T* P = (const T*)a.proj + (int64_t)b * a.s_pb + (int64_t)c * CH * a.s_pl;
    // Every global load but alpha and z is issued before the first wait, in the order of use: the epoch, theta, dg
    // and dF, the forward totals of the preceding chunks, then the C, B, dC~ and dB~ vectors of this thread. Alpha and
    // z are loaded while the workgroup waits for the following chunks' totals.
    uint32_t epoch = 0;
    if (tid == 0) epoch = __hip_atomic_load(&xh->epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const StageVals<T> sv = stage_load<T, false>(P, a.s_pl, nullptr, 0, nrows, hn, off, h0, tid);
    float dgv = 0.f, dfv = 0.f;
    if (tid < CH * HG) {
        const int hh = tid >> 6, r = tid & 63;   // dg, dF of (head hh, row r): coalesced along L
        if (hh < hn && r < nrows) {
            const int64_t o = (int64_t)(b * H + h0 + hh) * L + c * CH + r;
            dgv = a.dg[o];
            if (a.df) dfv = a.df[o];
        }
    }
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
        sq.x[hh * NCOMP + 0][r] = dgv;
        sq.x[hh * NCOMP + 1][r] = dfv;
    }
    tot_store(tu.f, tv, tid);
    if (tid == 0) s_tag = epoch + 1;
    // LDS-only barriers until the rotation: the Phi scan runs while C, B, dC~ and dB~ are in flight (issued last, so
    // the waits for theta, dg, dF and the totals do not wait for them).
    lds_barrier();
    const int li = tid - NTASK;   // carry lane of column li
    {   // Phi: the forward scan of theta (components 2..17), by the forward's code
        const bool phi_task = tid < NTASK && (tid % HC) % NCOMP >= 2;
        const bool phi_lane = li >= 0 && li < HC && li / NCOMP < hn && li % NCOMP >= 2;
        if (phi_task) fwd_sub_scan(sm, sl, tid);
        const float carry = carry_of(tu.f, tv, a.tot, b * H + h0, hn, NCH, 0, c, phi_lane, li, tid);
        if (li >= 0 && li < HC) sl.carry[li] = carry;
        lds_barrier();
        if (phi_task) fwd_sub_finish(sm, sl, tid);
    }
    lds_barrier();
    T* DP = (T*)a.dproj + (int64_t)b * a.s_db + (int64_t)c * CH * a.s_dl;
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
            sq.x[u.hl * NCOMP + 2 + 4 * u.q + p][u.row] = ok ? d1 + d2 : 0.f;
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
        }
    }
    __syncthreads();
    if (tid < NTASK) {   // fp64 sub-chunk sums
        const float* x = sq.x[tid % HC] + SUB * (tid / HC);
        double acc = 0.0;
#pragma unroll
        for (int r = 0; r < SUB; ++r) acc += (double)x[r];
        sd.sub[tid / HC][tid % HC] = acc;
    }
    __syncthreads();
    const uint32_t tag = s_tag;
    if (tid < HC && tid / NCOMP < hn) {   // chunk totals, in a fixed order, published
        double t = 0.0;
#pragma unroll
        for (int j = 0; j < NSUB; ++j) t += sd.sub[j][tid];
        xch_put(seqw + ((int64_t)c * HC + tid) * XW, tag, t);
    }
    float al = 0.f, zv = 0.f;   // alpha, z of (row tid>>2, head tid&3): contiguous in the row
    if (tid < CH * HG) {
        const int row = tid >> 2, hl = tid & 3;
        if (row < nrows && hl < hn) {
            al = (float)P[(int64_t)row * a.s_pl + off.A + h0 + hl];
            if (a.z) zv = a.z[(int64_t)b * a.s_zb + (int64_t)(c * CH + row) * a.s_zl + h0 + hl];
        }
    }
    // Reverse scans in two levels (fp64, fixed order): the carry of the following chunks, then each value = (carry +
    // following sub-chunk totals) + its suffix within the sub-chunk.
    const bool lane = li >= 0 && li < HC && li / NCOMP < hn;
    const double sa = carry_xch(tu.d, seqw, hn, c + 1, NCH, tag, &xh->error, spin_limit, lane, li, tid);
    if (li >= 0 && li < HC) sd.carry[li] = sa;
    __syncthreads();
    if (tid < NTASK) {
        const int col = tid % HC, s0 = tid / HC;
        double p = sd.carry[col];
#pragma unroll
        for (int j = NSUB - 1; j > 0; --j)
            if (j > s0) p += sd.sub[j][col];
        float* x = sq.x[col] + SUB * s0;
        double acc = 0.0;
#pragma unroll
        for (int r = SUB - 1; r >= 0; --r) {
            acc += (double)x[r];
            x[r] = (float)(p + acc);   // the suffix sum; d alpha and dz take their element derivative below
        }
    }
    __syncthreads();
    // d theta: 8 columns per vector
#pragma unroll
    for (int i = 0; i < 512 / NT; ++i) {
        const int v = tid + NT * i;
        const int row = v >> 3, hl = (v >> 1) & 3, half = v & 1;
        if (row >= nrows || hl >= hn) continue;
        f32x4 lo, hi;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            lo[j] = sq.x[hl * NCOMP + 2 + 8 * half + j][row];
            hi[j] = sq.x[hl * NCOMP + 6 + 8 * half + j][row];
        }
        *reinterpret_cast<frag8<T>*>(DP + (int64_t)row * a.s_dl + off.TH + (h0 + hl) * S2 + 8 * half) =
            pack8<T>(lo, hi);
    }
    if (tid < CH * HG) {
        const int row = tid >> 2, hl = tid & 3;
        if (row < nrows && hl < hn) {
            DP[(int64_t)row * a.s_dl + off.A + h0 + hl] = cvt<T>(-sq.x[hl * NCOMP + 0][row] * softplus_grad(al));
            if (a.dz)
                a.dz[(int64_t)b * a.s_dzb + (int64_t)(c * CH + row) * a.s_dzl + h0 + hl] =
                    sq.x[hl * NCOMP + 1][row] * logsigmoid_grad(zv);
        }
    }
    // zero padding columns (they multiply the zero rows of W_cat; keeps NaN out of dX)
    if (h0 == 0 && off.NPAD > off.NTOT) {
        const int npad = off.NPAD - off.NTOT;
        for (int idx = tid; idx < CH * npad; idx += NT) {
            const int r = idx / npad, j = idx % npad;
            if (r < nrows) DP[(int64_t)r * a.s_dl + off.NTOT + j] = cvt<T>(0.f);
        }
    }
    if (tid == 0) xch_arrive(xh, epoch, gridDim.x);
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

// The backward's grid: one workgroup per (chunk, sequence), numbered as bwd_geo reads them.
inline unsigned prep_grid(int B, int L, int H) {
    return (unsigned)((int64_t)sisa::cdiv(L, CH) * B * sisa::cdiv(H, HG));
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
    const char* env = getenv("SISA_PREP_SPIN_LIMIT");
    const int spin_limit = env ? atoi(env) : SPIN_LIMIT;
    prep_bwd_kernel<T><<<prep_grid(a->B, a->L, a->H), NT, 0, st>>>(*a, spin_limit < 0 ? 0 : spin_limit);
    return sisa::launch_status("sisa_prep_bwd");
}

// Shapes whose backward grid stays below 2^31 workgroups.
inline bool prep_shape_ok(int B, int L, int H) {
    return (int64_t)sisa::cdiv(L, CH) * B * sisa::cdiv(H, HG) < (int64_t)1 << 31;
}

}  // namespace

extern "C" int sisa_prep_fwd(const sisa_prep_fwd_args* a, void* stream) {
    SISA_REQUIRE(a != nullptr, "sisa_prep_fwd: null args");
    SISA_REQUIRE(a->B >= 1 && a->L >= 1 && a->H >= 1 && prep_shape_ok(a->B, a->L, a->H),
                 "sisa_prep_fwd: bad shape B=%d L=%d H=%d", a->B, a->L, a->H);
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
    return (B >= 1 && L >= 1 && H >= 1) ? xch_bytes(B, L, H) : 0;
}

extern "C" int sisa_prep_bwd(const sisa_prep_bwd_args* a, void* stream) {
    SISA_REQUIRE(a != nullptr, "sisa_prep_bwd: null args");
    SISA_REQUIRE(a->B >= 1 && a->L >= 1 && a->H >= 1 && prep_shape_ok(a->B, a->L, a->H),
                 "sisa_prep_bwd: bad shape B=%d L=%d H=%d", a->B, a->L, a->H);
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
