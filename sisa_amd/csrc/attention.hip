// SISA attention for gfx950: decay factors, forward, exact-delta backward (query-owned and key-owned kernels) and
// the deterministic fp64 dlambda reduction.
//
//   s_ij = q_i.k_j / 8 + lam * exp(g_i - g_j) * (c_i.b_j) + (F_i - F_j)        (j <= i)
//   o_i  = sum_j softmax_j(s_ij) v_j
//
// Reference: src/sisa/kernels/attention.py (Triton). The arithmetic follows the reference's numerics notes
// (attention.py:9-78): chunk-factored decay exp(g_i-g_j) = rowf_i * mid * colf_j over 64-row blocks for key blocks
// strictly before the query block, pairwise exp2(min((g_i-g_j)*log2e, 0)) inside the query's own block, differences
// before log2e, the self-normalised fp32 o'' for the exact delta, and the delta-free diagonal dS_tt. The kernel
// structure (tiles, wave ownership, MFMA layouts, LDS staging) is this library's own.
//
// Work decomposition (16 rows per wave: one column group of the 16x16 MFMA blocks; no atomics):
//   forward: a workgroup of 8 waves owns 128 consecutive queries; key tiles of 64 positions are staged row-major in
//     LDS while the next tile's global loads are in flight; at most 128 VGPRs, so 4 waves per SIMD.
//   dq kernel: a workgroup of 4 waves owns one 64-query decay block; every key tile before the block is an
//     off-block tile for all four waves and the block's own tile comes last, in its own code region.
//   dkv kernel: a workgroup of 4 waves owns one 64-key block; query tiles are visited from the last one down to the
//     block's own tile. Both backward kernels run 3 waves per SIMD.
//   Operands of the sequence-contracted products (P V, dS K, ...) are read from the row-major tiles with the gfx950
//   LDS transpose read, so no transposed copy is ever stored.
//   Ownership is exclusive: dq/dc by query blocks, dk/dv/db/dg/dF by key blocks.
#include "common.h"
#include "host.h"

namespace {

constexpr int DH = 64;   // d_head
constexpr int DS = 32;   // d_state
constexpr int BLK = 64;  // decay-factor block (rowf/colf anchors)
constexpr float RESCALE_LOG2 = 8.f;   // forward: largest exponent of an unrescaled softmax weight (2^8)
constexpr float M_FLOOR = -1e30f;     // forward: initial running maximum (finite, so exp2(-inf - m) = 0)

// Forward: 8 waves per workgroup, 16 rows (one column group of the MFMA block) per wave, 128 rows per workgroup,
// 64-position tiles of the other operand staged row-major in LDS.
constexpr int NW = 8;
constexpr int NTH = 64 * NW;
// Backward kernels: 4 waves x 16 rows = one 64-row decay block per workgroup, so that every tile before the block is
// an off-block tile for all waves and the block's own tile comes last (two code regions with small register sets;
// three workgroups per CU).
constexpr int NWB = 4;
constexpr int NTHB = 64 * NWB;

// ------------------------------------------------------------------------------------------------ factors
// rowf_t = exp2(min((g_t - g_{block start})*log2e, 0)), colf_t = exp2(min((g_{block end} - g_t)*log2e, 0)), and the
// maximum increase g_t - g_{t-1} per block. Reference: attention.py:129-153.
__global__ __launch_bounds__(64) void factors_kernel(sisa_factors_args a) {
    const int p = blockIdx.x;
    const int bh = blockIdx.y;
    const int H = a.H, L = a.L;
    const int b = bh / H, h = bh % H;
    const float* G = (const float*)a.g.ptr + (int64_t)b * a.g.sb + (int64_t)h * a.g.sh;
    const int64_t sgl = a.g.sl;
    const int t0 = p * BLK;
    const int t = t0 + threadIdx.x;
    const bool msk = t < L;
    const int tc = t < L ? t : L - 1;
    const float g = G[(int64_t)tc * sgl];
    const float gs = G[(int64_t)t0 * sgl];
    const int last = (t0 + BLK - 1 < L - 1) ? t0 + BLK - 1 : L - 1;
    const float ge = G[(int64_t)last * sgl];
    const float rowf = exp2_le0((g - gs) * LOG2E);
    const float colf = exp2_le0((ge - g) * LOG2E);
    if (msk) {
        a.rowf[(int64_t)bh * L + t] = rowf;
        a.colf[(int64_t)bh * L + t] = colf;
    }
    const int tp = tc - 1 > 0 ? tc - 1 : 0;
    const float prv = G[(int64_t)tp * sgl];
    float inc = (msk && t > 0) ? g - prv : -__builtin_inff();
    for (int o = 32; o > 0; o >>= 1) inc = nmax(inc, __shfl_xor(inc, o));
    if (threadIdx.x == 0) a.mono[(int64_t)bh * gridDim.x + p] = inc;
}

template <class T, class TO>
SISA_DEV void store_row4(TO* p, f32x4 v) {
    store4<TO>(p, to_vec4<TO>(v));
}

// Workgroup i of a 1-D grid of nrank * BH workgroups -> (bh, rank); rank 0 is the heaviest workgroup of a head.
// Workgroups are dispatched round-robin over the 8 XCDs (workgroup i runs on XCD i % 8), each with its own L2, so
// every XCD gets whole heads: the workgroups sharing one head's K/V (or Q/dO) tiles run on one XCD and read them
// from HBM once. When BH is a multiple of 8, XCD x owns heads [x BH/8, (x+1) BH/8) and dispatches them rank-major
// (rank 0 of each of its heads, then rank 1, ...): the XCD's queue is heaviest-first, which a greedy in-order
// dispatcher packs with a short tail (head after head, the last head's heavy workgroups would start late).
// Otherwise each XCD gets a contiguous range of (bh, rank), or the plain order when the grid does not split in 8.
SISA_DEV void xcd_map(int i, int nrank, int BH, int& bh, int& rank) {
    if (BH % 8 == 0) {
        const int hp = BH / 8;
        const int s = i / 8;
        bh = (i % 8) * hp + s % hp;
        rank = s / hp;
        return;
    }
    const int total = nrank * BH;
    const int j = (total % 8 == 0) ? (i % 8) * (total / 8) + i / 8 : i;
    bh = j / nrank;
    rank = j % nrank;
}

// ------------------------------------------------------------------------------------------------ forward
// Scores are computed transposed (S^T = K Q^T): a lane owns one query's softmax state and the 16x16 C blocks of S^T
// are directly the B fragments of O^T += V^T P^T. Per tile and wave one of two code paths runs (uniform branch):
// off-block tiles (every key in an earlier 64-block than the wave's queries; chunk-factored decay, no masks) or the
// wave's own block (pairwise decay and the causal mask).
//
// Score arithmetic (16-bit inputs). Off-block tiles use the key block's last F as an anchor: with F_e = F at the
// tile's last key, s_ij = s''_ij + (F_i - F_e), where s''_ij = q.k/8 + (F_e - F_j) + decay term and F_i - F_e is one
// scalar per (query, tile) that goes into the exponent offset and the tile maximum. Both parts are differences of
// F values no farther apart than F_i - F_j, so errors keep scaling with F differences, never with |F| (shift
// invariance); the diagonal tile, where F_i - F_e can exceed F_i - F_j, uses the reference's per-element F_i - F_j.
// Then
//   * q is pre-scaled by 1/8 = 1/sqrt(d_head) (a power of two: exact), and the per-key F_e - F_j enters the q.k MFMA
//     as its accumulator input, so that product block is already q.k/8 + F_e - F_j;
//   * off-block tiles: for bf16 the query factor lam*rowf_i is folded into the c~ operand as an unevaluated bf16 pair
//     hi + lo = lam*rowf_i*c~_i (relative error <= 2^-17, two MFMAs), for fp32 as one fp32 operand; the decayed
//     side term is then one FMA with the per-key colf_j*mid. fp16 (too little exponent range for the split) keeps
//     the fp32 products lam*rowf_i * (cb_ij * colf_j*mid).
// Per off-block score element that leaves one FMA (two for fp16) before the softmax. fp32 (the accuracy path) keeps
// the reference's per-element F_i - F_j everywhere.
constexpr float QSCALE = 0.125f;   // 1/sqrt(DH), exact in every input type
template <class T> struct FoldC { static constexpr bool on = sizeof(T) != 2 || __is_same(T, __bf16); };
template <class T> struct SplitC { static constexpr bool on = __is_same(T, __bf16); };
template <class T> struct Anchor { static constexpr bool on = sizeof(T) == 2; };

template <class T>
struct __attribute__((aligned(16))) FwdLds {
    T ks[64 * DH];               // K tile
    T bs[64 * DS];               // B~ tile
    T vs[64 * DH];               // V tile
    float fk[64], gk[64];        // F and g at the tile's keys
    float nfe[64];               // F_e - F_j (F_e = F at the tile's last key)
    float cfm[2][64];            // colf * mid for the workgroup's two query blocks
};

// The 8 values of a fragment multiplied by s (fp32) and rounded back to T.
template <class T> SISA_DEV frag8<T> scale_frag(const frag8<T>& f, float s) {
    return __builtin_convertvector(__builtin_convertvector(f, f32x8) * s, frag8<T>);
}
// hi + lo = s * f with hi, lo in T (lo = 0 where the split is off).
template <class T> SISA_DEV void split_frag(const frag8<T>& f, float s, frag8<T>& hi, frag8<T>& lo) {
    const f32x8 x = __builtin_convertvector(f, f32x8) * s;
    hi = __builtin_convertvector(x, frag8<T>);
    if constexpr (SplitC<T>::on) lo = __builtin_convertvector(x - __builtin_convertvector(hi, f32x8), frag8<T>);
    else lo = zero8<T>();
}

// One 64-key tile for a wave's 16 queries. cx0/cx1: for off-block tiles the folded c~ operand (hi, lo; FoldC types)
// or the plain c~ (fp16, cx1 unused); for the diagonal tile the plain c~ (cx1 unused).
template <class T, bool DIAG>
SISA_DEV void fwd_tile(const FwdLds<T>& sm, int qblk, int lane, int n0, int q0, int L, const frag8<T> (&qf)[2],
                       const frag8<T>& cx0, const frag8<T>& cx1, const frag8<T>& onesf, float fq, float rs, float gq,
                       float lam, float& m, float& l, f32x4 (&acc)[5]) {
    constexpr bool ANCH = Anchor<T>::on && !DIAG;
    const int grp = lane >> 4, lc = lane & 15;
    const int qq = q0 + lc;
    const float* cfm = sm.cfm[qblk];
    f32x4 sc[4], cb[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
        const frag8<T> k0 = frag_rows<T, DH>(sm.ks, kb * 16, 0, lane);
        const frag8<T> k1 = frag_rows<T, DH>(sm.ks, kb * 16, 1, lane);
        const frag8<T> bf = frag_rows<T, DS>(sm.bs, kb * 16, 0, lane);
        if constexpr (ANCH) sc[kb] = mma(k1, qf[1], mma(k0, qf[0], lds4f(&sm.nfe[kb * 16 + 4 * grp])));
        else sc[kb] = mma(k1, qf[1], mma(k0, qf[0], zero4()));
        if constexpr (!DIAG && SplitC<T>::on) cb[kb] = mma(bf, cx1, mma(bf, cx0, zero4()));
        else cb[kb] = mma(bf, cx0, zero4());
    }
    float mloc = -__builtin_inff();
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
        const int j0 = kb * 16 + 4 * grp;
        if constexpr (!ANCH) {   // the reference's difference F_i - F_j per element
            const f32x4 fk = lds4f(&sm.fk[j0]);
#pragma unroll
            for (int i = 0; i < 4; ++i) sc[kb][i] = sc[kb][i] + (fq - fk[i]);
        }
        if (DIAG) {
            const f32x4 gk = lds4f(&sm.gk[j0]);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int jj = n0 + j0 + i;
                const bool valid = jj <= qq && jj < L;
                const float dec = valid ? exp2_le0((gq - gk[i]) * LOG2E) : 0.f;
                float s = sc[kb][i] + lam * (dec * cb[kb][i]);
                s = valid ? s : -__builtin_inff();
                sc[kb][i] = s;
                mloc = fmaxf(mloc, s);
            }
        } else {
            const f32x4 cf = lds4f(&cfm[j0]);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float s;
                if constexpr (FoldC<T>::on) s = fmaf(cb[kb][i], cf[i], sc[kb][i]);
                else s = sc[kb][i] + rs * (cb[kb][i] * cf[i]);
                sc[kb][i] = s;
                mloc = fmaxf(mloc, s);
            }
        }
    }
    // anchored tiles: sc holds s'' = s - (F_i - F_e); ft = (F_i - F_e) * log2e restores s in the exponent and max
    const float ft = ANCH ? (fq - sm.fk[63]) * LOG2E : 0.f;
    // Online softmax in log2 units with lazy rescaling: a query's running offset m moves (and its l, acc are
    // rescaled) only when its tile maximum exceeds m by more than RESCALE_LOG2, so the exponentials stay below
    // 2^RESCALE_LOG2. The decision is per query (a query's results never depend on its neighbours); the wave skips
    // the rescale when no query needs it, and queries that do not need it multiply by exactly 1. m starts at a
    // finite floor, so fully masked rows give exp2(-inf) = 0. A NaN score reaches l through its exponential.
    const float mt = ANCH ? fmaf(group_max(mloc), LOG2E, ft) : group_max(mloc) * LOG2E;
    const bool need = mt > m + RESCALE_LOG2;
    if (__builtin_amdgcn_ballot_w64(need) != 0) {
        const float mn = need ? fmaxf(m, mt) : m;
        const float corr = fast_exp2(m - mn);
        m = mn;
        l *= corr;
#pragma unroll
        for (int db = 0; db < 5; ++db) acc[db] *= corr;
    }
    float ls = 0.f;
    const float off = ANCH ? ft - m : -m;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float pe = fast_exp2(fmaf(sc[kb][i], LOG2E, off));
            sc[kb][i] = pe;
            ls += pe;
        }
    l += ls;
#pragma unroll
    for (int st = 0; st < 2; ++st) {
        const frag8<T> pf = pack8<T>(sc[2 * st], sc[2 * st + 1]);
#pragma unroll
        for (int db = 0; db < 4; ++db) acc[db] = mma(frag_tr<T, DH>(sm.vs, db * 16, st, lane), pf, acc[db]);
        acc[4] = mma(onesf, pf, acc[4]);   // row 0 of block 4: the sum of the rounded weights (o'' normaliser)
    }
}

template <class T>
__global__ __launch_bounds__(NTH) __attribute__((amdgpu_waves_per_eu(4))) void attn_fwd_kernel(sisa_attn_fwd_args a) {
    constexpr int NBUF = sizeof(T) == 2 ? 2 : 1;
    __shared__ FwdLds<T> smb[NBUF];
    const int tid = threadIdx.x, lane = tid & 63, grp = lane >> 4, lc = lane & 15;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int NQT = (a.L + 127) / 128;
    int bh, rank;
    xcd_map(blockIdx.x, NQT, a.B * a.H, bh, rank);
    const int tile = NQT - 1 - rank;               // heavy (late) query tiles first
    const int H = a.H, L = a.L;
    const int b = bh / H, h = bh % H;
    const bool has_f = a.f.ptr != nullptr;
    const T* Q = (const T*)a.q.ptr + (int64_t)b * a.q.sb + (int64_t)h * a.q.sh;
    const T* K = (const T*)a.k.ptr + (int64_t)b * a.k.sb + (int64_t)h * a.k.sh;
    const T* V = (const T*)a.v.ptr + (int64_t)b * a.v.sb + (int64_t)h * a.v.sh;
    const T* C = (const T*)a.c.ptr + (int64_t)b * a.c.sb + (int64_t)h * a.c.sh;
    const T* Bm = (const T*)a.b.ptr + (int64_t)b * a.b.sb + (int64_t)h * a.b.sh;
    const float* G = (const float*)a.g.ptr + (int64_t)b * a.g.sb + (int64_t)h * a.g.sh;
    const float* FF = has_f ? (const float*)a.f.ptr + (int64_t)b * a.f.sb + (int64_t)h * a.f.sh : nullptr;
    const float* ROWF = a.rowf + (int64_t)bh * L;
    const float* COLF = a.colf + (int64_t)bh * L;
    const float lam = a.lam[(int64_t)h * a.s_lam];
    const int64_t sql = a.q.sl, skl = a.k.sl, svl = a.v.sl, scl = a.c.sl, sbl = a.b.sl, sgl = a.g.sl;
    const int64_t sfl = has_f ? a.f.sl : 0;

    const int tile0 = tile * 128;
    const int q0 = tile0 + 16 * w;
    const int qblk = w >> 2;                       // which of the workgroup's two query blocks
    const bool live = q0 < L;
    const int ta0 = tile0 < L ? tile0 : L - 1, ta1 = tile0 + 64 < L ? tile0 + 64 : L - 1;   // block anchors
    const float ga0 = G[(int64_t)ta0 * sgl];
    const float ga1 = G[(int64_t)ta1 * sgl];

    // qf: q/8 (exact). cx0/cx1: the c~ operand of off-block tiles (folded with lam*rowf_i where FoldC).
    frag8<T> qf[2], cx0, cx1;
    float fq, rs, gq;
    {
        const int qq = q0 + lc;
        const bool ok = qq < L;
        qf[0] = ok ? scale_frag<T>(load8<T>(Q + (int64_t)qq * sql + 8 * grp), QSCALE) : zero8<T>();
        qf[1] = ok ? scale_frag<T>(load8<T>(Q + (int64_t)qq * sql + 32 + 8 * grp), QSCALE) : zero8<T>();
        const frag8<T> cfr = ok ? load8<T>(C + (int64_t)qq * scl + 8 * grp) : zero8<T>();
        fq = (has_f && ok) ? FF[(int64_t)qq * sfl] : 0.f;
        rs = lam * (ok ? ROWF[qq] : 0.f);
        gq = G[(int64_t)(ok ? qq : L - 1) * sgl];
        if constexpr (FoldC<T>::on) split_frag<T>(cfr, rs, cx0, cx1);
        else { cx0 = cfr; cx1 = zero8<T>(); }
    }
    // the plain c~ operand of the diagonal tile (loaded there: the loop does not keep it in registers)
    auto diag_c = [&]() -> frag8<T> {
        const int qq = q0 + lc;
        return qq < L ? load8<T>(C + (int64_t)qq * scl + 8 * grp) : zero8<T>();
    };
    const frag8<T> onesf = ones_row_frag<T>(lane);

    float m = M_FLOOR, l = 0.f;
    f32x4 acc[5];
#pragma unroll
    for (int db = 0; db < 5; ++db) acc[db] = zero4();

    // Key tiles go straight from global memory into LDS (DMA buffer loads). 16-bit types double-buffer the tiles:
    // tile t+1 is issued into the idle buffer while tile t is computed, one barrier per tile. fp32 tiles do not fit
    // twice and use one buffer with a barrier on each side of the issue. The per-key scalars of the next tile are
    // fetched into registers by the first wave one tile ahead.
    DmaStage<T, DH, NW> dk, dv;
    DmaStage<T, DS, NW> dbt;
    const int64_t xk = ((int64_t)(L - 1) * skl + DH) * (int64_t)sizeof(T);   // view extents (bytes)
    const int64_t xv = ((int64_t)(L - 1) * svl + DH) * (int64_t)sizeof(T);
    const int64_t xb = ((int64_t)(L - 1) * sbl + DS) * (int64_t)sizeof(T);
    dk.init(skl, w, lane);
    dv.init(svl, w, lane);
    dbt.init(sbl, w, lane);
    const int kend = (tile0 + 128 < L) ? tile0 + 128 : L;
    float pf_f = 0.f, pf_g = 0.f, pf_cf = 0.f, pf_ge = 0.f, pf_fe = 0.f;
    auto fetch_scalars = [&](int n0) {
        if (tid < 64) {
            const int j = n0 + tid;
            const int jc = j < L ? j : L - 1;
            const int je = n0 + 63 < L ? n0 + 63 : L - 1;   // end of the key block
            pf_f = (has_f && j < L) ? FF[(int64_t)j * sfl] : 0.f;
            pf_g = G[(int64_t)jc * sgl];
            pf_cf = j < L ? COLF[j] : 0.f;
            pf_ge = G[(int64_t)je * sgl];
            pf_fe = has_f ? FF[(int64_t)je * sfl] : 0.f;
        }
    };
    auto issue_tile = [&](FwdLds<T>& d, int n0) {
        dma_issue<0>(dk, K, xk, (int)(n0 * skl * (int64_t)sizeof(T)), d.ks, w);
        dma_issue<0>(dv, V, xv, (int)(n0 * svl * (int64_t)sizeof(T)), d.vs, w);
        dma_issue<0>(dbt, Bm, xb, (int)(n0 * sbl * (int64_t)sizeof(T)), d.bs, w);
        if (tid < 64) {
            d.fk[tid] = pf_f;
            d.nfe[tid] = pf_fe - pf_f;
            d.gk[tid] = pf_g;
            d.cfm[0][tid] = pf_cf * exp2_le0((ga0 - pf_ge) * LOG2E);
            d.cfm[1][tid] = pf_cf * exp2_le0((ga1 - pf_ge) * LOG2E);
        }
    };
    // Advance to tile t (key offset 64 t): afterwards (and after the caller's barrier for two buffers) the tile is in
    // LDS buffer t & (NBUF-1).
    auto advance = [&](int t) {
        const int n0 = 64 * t;
        if (NBUF == 2) {
            if (n0 + 64 < kend) {
                issue_tile(smb[(t + 1) & (NBUF - 1)], n0 + 64);
                if (n0 + 128 < kend) fetch_scalars(n0 + 128);
            }
        } else if (t > 0) {
            __syncthreads();
            issue_tile(smb[0], n0);
            __syncthreads();
            if (n0 + 64 < kend) fetch_scalars(n0 + 64);
        }
    };
    fetch_scalars(0);
    issue_tile(smb[0], 0);
    if (64 < kend) fetch_scalars(64);
    __syncthreads();
    // tiles before the workgroup's first query block: off-block for every wave (one code path in the loop)
    const int nfull = tile0 / 64;
    for (int t = 0; t < nfull; ++t) {
        advance(t);
        if (live) {
            const FwdLds<T>& sm = smb[t & (NBUF - 1)];
            fwd_tile<T, false>(sm, qblk, lane, 64 * t, q0, L, qf, cx0, cx1, onesf, fq, rs, gq, lam, m, l, acc);
        }
        if (NBUF == 2) __syncthreads();
    }
    // the workgroup's own tiles: block 0's (off-block for block 1's waves), then block 1's
    advance(nfull);
    if (live) {
        const FwdLds<T>& sm = smb[nfull & (NBUF - 1)];
        if (qblk == 0)
            fwd_tile<T, true>(sm, 0, lane, tile0, q0, L, qf, diag_c(), cx1, onesf, fq, rs, gq, lam, m, l, acc);
        else
            fwd_tile<T, false>(sm, 1, lane, tile0, q0, L, qf, cx0, cx1, onesf, fq, rs, gq, lam, m, l, acc);
    }
    if (tile0 + 64 < kend) {
        if (NBUF == 2) __syncthreads();
        advance(nfull + 1);
        if (live && qblk == 1) {
            const FwdLds<T>& sm = smb[(nfull + 1) & (NBUF - 1)];
            fwd_tile<T, true>(sm, 1, lane, tile0 + 64, q0, L, qf, diag_c(), cx1, onesf, fq, rs, gq, lam, m, l, acc);
        }
    }
    if (!live) return;
    T* O = (T*)a.o.ptr + (int64_t)b * a.o.sb + (int64_t)h * a.o.sh;
    const float lt = group_sum(l);
    const float lbt = group_bcast0(acc[4][0], lane);   // row 0 of block 4: sum of the rounded weights
    const int qq = q0 + lc;
    if (qq >= L) return;
    const float ls = (lt == 0.f) ? 1.f : lt;
#pragma unroll
    for (int db = 0; db < 4; ++db) store4<T>(O + (int64_t)qq * a.o.sl + db * 16 + 4 * grp, to_vec4<T>(acc[db] / ls));
    if (a.o32) {
        const float lbs = (lbt == 0.f) ? 1.f : lbt;
        float* O32 = a.o32 + ((int64_t)bh * L + qq) * DH;
#pragma unroll
        for (int db = 0; db < 4; ++db) *reinterpret_cast<f32x4*>(O32 + db * 16 + 4 * grp) = acc[db] / lbs;
    }
    // lse of the true scores s = s' + (F_i - F_a), in log2 units
    if (grp == 0) a.lse[(int64_t)bh * L + qq] = m + __builtin_amdgcn_logf(ls);
}

// ------------------------------------------------------------------------------------------------ backward: dq
// Row buffers handed from the dq kernel to the dkv kernel (workspace, each (B,H,L) fp32).
enum { WS_DELTA = 0, WS_DDEL, WS_DSD, WS_RG, WS_RL, WS_RF, WS_N };

template <class T>
struct __attribute__((aligned(16))) DqLds {
    T ks[64 * DH];               // K (scores; transposed reads for dq)
    T vs[64 * DH];               // V (dP)
    T bs[64 * DS];               // B~ (scores; transposed reads for dc)
    float fk[64], gk[64];
    float nfe[64];               // F_e - F_j (F_e = F at the tile's last key; anchored off-block scores)
    float cfm[64];               // colf * mid for the workgroup's query block
};

// Per-query row sums of the dq kernel (diagonal excluded): xa = sum dS^ u, ya = sum P u, wa = D = sum dS^,
// za = Z = sum P, ptt = P_tt, dptt = dP_tt, xd = cb_tt. Off-block tiles accumulate xa, ya without the row factor
// rowf; a wave's own-block tile is its last one, and rowf (lam*rowf for dc) is applied once before it.
struct RowSums {
    float xa, ya, wa, za, ptt, dptt, xd;
};

// Score arithmetic as in the forward: q is pre-scaled by 1/8; for 16-bit inputs off-block tiles are anchored at the
// key tile's last F (F_e - F_j enters the q.k MFMA as its accumulator input, (F_i - F_e) log2e - lse is one offset
// per query and tile) and dP - Delta comes out of the dO.V MFMA (-Delta as its accumulator input). The dkv kernel
// evaluates the same pairs with the same anchors and the same accumulator inputs.
template <class T, bool DIAG>
SISA_DEV void dq_tile(const DqLds<T>& sm, int lane, int n0, int q0, int L, const frag8<T> (&qf)[2],
                      const frag8<T>& cfr, const frag8<T> (&dof)[2], float fq, float rs, float gq, float lse,
                      float dhat, float lam, RowSums& R, f32x4 (&dqa)[4], f32x4 (&dca)[2]) {
    constexpr bool F16 = Anchor<T>::on;
    constexpr bool ANCH = F16 && !DIAG;
    const int grp = lane >> 4, lc = lane & 15;
    const int qq = q0 + lc;
    const float* cfm = sm.cfm;
    const float ftl = ANCH ? fmaf(fq - sm.fk[63], LOG2E, -lse) : -lse;
    const f32x4 ndh = F16 ? f32x4{-dhat, -dhat, -dhat, -dhat} : zero4();
#pragma unroll
    for (int st = 0; st < 2; ++st) {           // 32 keys (one K-step of the dq/dc products) at a time
        f32x4 dsv[2], wv[2];                   // dq and dc operands of the two 16-key blocks (before rounding)
#pragma unroll
        for (int hb = 0; hb < 2; ++hb) {       // one 16-key block at a time keeps the live set small
            __builtin_amdgcn_sched_barrier(0);
            const int kb = 2 * st + hb;
            const int j0 = kb * 16 + 4 * grp;
            const f32x4 sc = mma(frag_rows<T, DH>(sm.ks, kb * 16, 1, lane), qf[1],
                                 mma(frag_rows<T, DH>(sm.ks, kb * 16, 0, lane), qf[0],
                                     ANCH ? lds4f(&sm.nfe[j0]) : zero4()));
            const f32x4 cb = mma(frag_rows<T, DS>(sm.bs, kb * 16, 0, lane), cfr, zero4());
            const f32x4 dp = mma(frag_rows<T, DH>(sm.vs, kb * 16, 1, lane), dof[1],
                                 mma(frag_rows<T, DH>(sm.vs, kb * 16, 0, lane), dof[0], ndh));
            const f32x4 fk = lds4f(&sm.fk[j0]);
            if (DIAG) {
                const f32x4 gk = lds4f(&sm.gk[j0]);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int jj = n0 + j0 + i;
                    const bool valid = jj <= qq && jj < L && qq < L;
                    const bool eye = valid && jj == qq;
                    const float dec = valid ? exp2_le0((gq - gk[i]) * LOG2E) : 0.f;
                    const float cbv = cb[i];
                    const float u = dec * cbv;
                    float s = sc[i] + (fq - fk[i]);
                    s = s + lam * u;
                    const float pr = valid ? fast_exp2(fmaf(s, LOG2E, -lse)) : 0.f;
                    const float dpd = F16 ? dp[i] : dp[i] - dhat;   // dP - Delta
                    const float ds = pr * dpd;
                    const float dso = eye ? 0.f : ds;
                    R.ptt += eye ? pr : 0.f;
                    R.dptt += eye ? dpd : 0.f;
                    R.xd += eye ? cbv : 0.f;
                    const float po = eye ? 0.f : pr;
                    R.za += po;
                    R.ya += po * u;
                    R.wa += dso;
                    R.xa += dso * u;
                    dsv[hb][i] = dso;
                    wv[hb][i] = dso * (lam * dec);
                }
            } else {
                const f32x4 cf = lds4f(&cfm[j0]);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float uc = cb[i] * cf[i];
                    float s;
                    if constexpr (ANCH) s = fmaf(rs, uc, sc[i]);
                    else s = (sc[i] + (fq - fk[i])) + rs * uc;
                    const float pr = fast_exp2(fmaf(s, LOG2E, ftl));
                    const float ds = pr * (F16 ? dp[i] : dp[i] - dhat);
                    R.xa += ds * uc;
                    R.ya += pr * uc;
                    R.za += pr;
                    R.wa += ds;
                    dsv[hb][i] = ds;
                    wv[hb][i] = ds * cf[i];
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        const frag8<T> dsf = pack8<T>(dsv[0], dsv[1]);
        const frag8<T> wf = pack8<T>(wv[0], wv[1]);
#pragma unroll
        for (int db = 0; db < 4; ++db) dqa[db] = mma(frag_tr<T, DH>(sm.ks, db * 16, st, lane), dsf, dqa[db]);
#pragma unroll
        for (int sb = 0; sb < 2; ++sb) dca[sb] = mma(frag_tr<T, DS>(sm.bs, sb * 16, st, lane), wf, dca[sb]);
    }
}

template <class T>
__global__ __launch_bounds__(NTHB) __attribute__((amdgpu_waves_per_eu(3))) void attn_bwd_dq_kernel(sisa_attn_bwd_args a) {
    constexpr int NBUF = sizeof(T) == 2 ? 2 : 1;
    __shared__ DqLds<T> smb[NBUF];
    const int tid = threadIdx.x, lane = tid & 63, grp = lane >> 4, lc = lane & 15;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int NQT = (a.L + 63) / 64;
    int bh, rank;
    xcd_map(blockIdx.x, NQT, a.B * a.H, bh, rank);
    const int tile = NQT - 1 - rank;               // heavy (late) query blocks first
    const int H = a.H, L = a.L;
    const int b = bh / H, h = bh % H;
    const bool has_f = a.f.ptr != nullptr;
    const T* Q = (const T*)a.q.ptr + (int64_t)b * a.q.sb + (int64_t)h * a.q.sh;
    const T* K = (const T*)a.k.ptr + (int64_t)b * a.k.sb + (int64_t)h * a.k.sh;
    const T* V = (const T*)a.v.ptr + (int64_t)b * a.v.sb + (int64_t)h * a.v.sh;
    const T* C = (const T*)a.c.ptr + (int64_t)b * a.c.sb + (int64_t)h * a.c.sh;
    const T* Bm = (const T*)a.b.ptr + (int64_t)b * a.b.sb + (int64_t)h * a.b.sh;
    const T* O = (const T*)a.o.ptr + (int64_t)b * a.o.sb + (int64_t)h * a.o.sh;
    const T* DO = (const T*)a.dout.ptr + (int64_t)b * a.dout.sb + (int64_t)h * a.dout.sh;
    const float* G = (const float*)a.g.ptr + (int64_t)b * a.g.sb + (int64_t)h * a.g.sh;
    const float* FF = has_f ? (const float*)a.f.ptr + (int64_t)b * a.f.sb + (int64_t)h * a.f.sh : nullptr;
    const float* ROWF = a.rowf + (int64_t)bh * L;
    const float* COLF = a.colf + (int64_t)bh * L;
    const float* LSE = a.lse + (int64_t)bh * L;
    const float lam = a.lam[(int64_t)h * a.s_lam];
    const int64_t skl = a.k.sl, svl = a.v.sl, sbl = a.b.sl, sgl = a.g.sl;
    const int64_t sfl = has_f ? a.f.sl : 0;
    const int64_t BHL = (int64_t)a.B * H * L;
    float* WS = (float*)a.workspace;

    const int tile0 = tile * 64;                   // the workgroup's 64-row decay block
    const int q0 = tile0 + 16 * w;
    const bool live = q0 < L;
    const float ga = G[(int64_t)tile0 * sgl];      // anchor: g at the start of the block

    frag8<T> qf[2], cfr, dof[2];
    float fq, rowfq, rs, gq, lse, dhat;
    {
        const int qq = q0 + lc;
        const bool ok = qq < L;
        float part = 0.f;
#pragma unroll
        for (int st = 0; st < 2; ++st) {
            qf[st] = ok ? scale_frag<T>(load8<T>(Q + (int64_t)qq * a.q.sl + 32 * st + 8 * grp), QSCALE) : zero8<T>();
            dof[st] = ok ? load8<T>(DO + (int64_t)qq * a.dout.sl + 32 * st + 8 * grp) : zero8<T>();
            if (ok) {
                const frag8<T> ov = load8<T>(O + (int64_t)qq * a.o.sl + 32 * st + 8 * grp);
                f32x4 o32a = zero4(), o32b = zero4();
                if (a.o32) {
                    const float* p32 = a.o32 + ((int64_t)bh * L + qq) * DH + 32 * st + 8 * grp;
                    o32a = *reinterpret_cast<const f32x4*>(p32);
                    o32b = *reinterpret_cast<const f32x4*>(p32 + 4);
                }
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    float o = (float)ov[j];
                    if (a.o32) {
                        // o'' agrees with the DT o to within 2^-15 relative: use the DT value (attention.py:341-349)
                        const float o2 = j < 4 ? o32a[j] : o32b[j - 4];
                        o = (fabsf(o2 - o) <= 3.0517578125e-05f * fabsf(o)) ? o : o2;
                    }
                    part += o * (float)dof[st][j];
                }
            }
        }
        dhat = group_sum(part);
        cfr = ok ? load8<T>(C + (int64_t)qq * a.c.sl + 8 * grp) : zero8<T>();
        fq = (has_f && ok) ? FF[(int64_t)qq * sfl] : 0.f;
        rowfq = ok ? ROWF[qq] : 0.f;
        rs = lam * rowfq;
        gq = G[(int64_t)(ok ? qq : L - 1) * sgl];
        lse = ok ? LSE[qq] : __builtin_inff();
    }

    f32x4 dqa[4], dca[2];
#pragma unroll
    for (int db = 0; db < 4; ++db) dqa[db] = zero4();
    dca[0] = dca[1] = zero4();
    RowSums R{0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};

    // Key tiles straight into LDS (DMA buffer loads); 16-bit types double-buffer them (one barrier per tile), fp32
    // uses one buffer. The per-key scalars (F_j, g_j, colf_j, g at the tile's last key) are fetched into registers by
    // the first wave one tile ahead.
    DmaStage<T, DH, NWB> dk, dv;
    DmaStage<T, DS, NWB> dbt;
    const int64_t xk = ((int64_t)(L - 1) * skl + DH) * (int64_t)sizeof(T);   // view extents (bytes)
    const int64_t xv = ((int64_t)(L - 1) * svl + DH) * (int64_t)sizeof(T);
    const int64_t xb = ((int64_t)(L - 1) * sbl + DS) * (int64_t)sizeof(T);
    dk.init(skl, w, lane);
    dv.init(svl, w, lane);
    dbt.init(sbl, w, lane);
    float pf_f = 0.f, pf_g = 0.f, pf_cf = 0.f, pf_ge = 0.f, pf_fe = 0.f;
    auto fetch_scalars = [&](int n0) {
        if (tid < 64) {
            const int j = n0 + tid;
            const int jc = j < L ? j : L - 1;
            const int je = n0 + 63 < L ? n0 + 63 : L - 1;   // end of the key block
            pf_f = (has_f && j < L) ? FF[(int64_t)j * sfl] : 0.f;
            pf_g = G[(int64_t)jc * sgl];
            pf_cf = j < L ? COLF[j] : 0.f;
            pf_ge = G[(int64_t)je * sgl];
            pf_fe = has_f ? FF[(int64_t)je * sfl] : 0.f;
        }
    };
    auto issue_tile = [&](DqLds<T>& d, int n0) {   // rows >= L read as zero
        dma_issue<1>(dk, K, xk, (int)(n0 * skl * (int64_t)sizeof(T)), d.ks, w);
        dma_issue<1>(dv, V, xv, (int)(n0 * svl * (int64_t)sizeof(T)), d.vs, w);
        dma_issue<1>(dbt, Bm, xb, (int)(n0 * sbl * (int64_t)sizeof(T)), d.bs, w);
        if (tid < 64) {
            d.fk[tid] = pf_f;
            d.nfe[tid] = pf_fe - pf_f;
            d.gk[tid] = pf_g;
            d.cfm[tid] = pf_cf * exp2_le0((ga - pf_ge) * LOG2E);
        }
    };
    // tile t (keys 64 t ..) is in buffer t & (NBUF-1) after advance(t) (and, for two buffers, the barrier before it)
    auto advance = [&](int t) {
        const int n0 = 64 * t;
        if (NBUF == 2) {
            if (n0 + 64 <= tile0) {
                issue_tile(smb[(t + 1) & (NBUF - 1)], n0 + 64);
                if (n0 + 128 <= tile0) fetch_scalars(n0 + 128);
            }
        } else if (t > 0) {
            __syncthreads();
            issue_tile(smb[0], n0);
            __syncthreads();
            if (n0 + 64 <= tile0) fetch_scalars(n0 + 64);
        }
    };
    fetch_scalars(0);
    issue_tile(smb[0], 0);
    if (64 <= tile0) fetch_scalars(64);
    __syncthreads();
    // key tiles before the block (all off-block), then the block's own tile
    const int nt = tile0 / 64;
    for (int t = 0; t < nt; ++t) {
        advance(t);
        if (live) {
            const DqLds<T>& sm = smb[t & (NBUF - 1)];
            dq_tile<T, false>(sm, lane, 64 * t, q0, L, qf, cfr, dof, fq, rs, gq, lse, dhat, lam, R, dqa, dca);
        }
        if (NBUF == 2) __syncthreads();
    }
    advance(nt);
    if (live) {
        // the block's own tile: apply the off-block row factors once, in fp32, then the diagonal path
        const DqLds<T>& sm = smb[nt & (NBUF - 1)];
        R.xa *= rowfq;
        R.ya *= rowfq;
        dca[0] *= rs;
        dca[1] *= rs;
        dq_tile<T, true>(sm, lane, tile0, q0, L, qf, cfr, dof, fq, rs, gq, lse, dhat, lam, R, dqa, dca);
    }
    if (!live) return;
    const float xat = group_sum(R.xa), yat = group_sum(R.ya), Wa = group_sum(R.wa), Za = group_sum(R.za);
    const float Ptt = group_sum(R.ptt), Dptt = group_sum(R.dptt), Xd = group_sum(R.xd);
    const int qq = q0 + lc;
    if (qq >= L) return;
    // self-normalised exact delta and the delta-free diagonal (attention.py:453-463)
    float ssum = Ptt + Za;
    ssum = ssum > 0.f ? ssum : 1.f;
    const float x0 = Dptt;   // dP_tt - Delta
    const float tt = dhat + (Ptt * x0 + Wa) / ssum;
    const float dstt = Ptt * (Za * x0 - Wa) / ssum;
    const float dl_row = xat + (dhat - tt) * yat;
    const float dsq = (float)cvt<T>(dstt);           // one DT rounding of the diagonal operands
    const float dsc = (float)cvt<T>(dstt * lam);
    const T* krow = K + (int64_t)qq * skl;
    const T* brow = Bm + (int64_t)qq * sbl;
    T* dqp = (T*)a.dq.ptr + (int64_t)b * a.dq.sb + (int64_t)h * a.dq.sh + (int64_t)qq * a.dq.sl;
#pragma unroll
    for (int db = 0; db < 4; ++db) {
        const int d = db * 16 + 4 * grp;
        const vec4<T> kv = load4<T>(krow + d);
        f32x4 r = dqa[db];
#pragma unroll
        for (int i = 0; i < 4; ++i) r[i] = fmaf(dsq, (float)kv[i], r[i]);
        store_row4<T, T>(dqp + d, r * QSCALE);
    }
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
        const int s0 = sb * 16 + 4 * grp;
        const vec4<T> bv = load4<T>(brow + s0);
        f32x4 r = dca[sb];
#pragma unroll
        for (int i = 0; i < 4; ++i) r[i] = fmaf(dsc, (float)bv[i], r[i]);
        if (a.dcb_dtype == SISA_F32) {
            float* dcp = (float*)a.dc.ptr + (int64_t)b * a.dc.sb + (int64_t)h * a.dc.sh + (int64_t)qq * a.dc.sl;
            *reinterpret_cast<f32x4*>(dcp + s0) = r;
        } else {
            T* dcp = (T*)a.dc.ptr + (int64_t)b * a.dc.sb + (int64_t)h * a.dc.sh + (int64_t)qq * a.dc.sl;
            store_row4<T, T>(dcp + s0, r);
        }
    }
    if (grp == 0) {
        const int64_t o = (int64_t)bh * L + qq;
        WS[WS_DELTA * BHL + o] = dhat;
        WS[WS_DDEL * BHL + o] = tt - dhat;
        WS[WS_DSD * BHL + o] = dstt;
        WS[WS_RG * BHL + o] = lam * dl_row;
        WS[WS_RL * BHL + o] = dl_row + dstt * Xd;
        WS[WS_RF * BHL + o] = Wa - Za * (tt - dhat);
    }
}

// ------------------------------------------------------------------------------------------------ backward: dk dv db
// Scores are computed as S = Q K^T (a lane owns one key's column sums); query tiles are visited in descending order
// so that the keys' own 64-block is every wave's last tile.
template <class T>
struct __attribute__((aligned(16))) DkvLds {
    T qs[64 * DH];               // Q (scores; transposed reads for dk)
    T cs[64 * DS];               // C~ (scores; transposed reads for db)
    T ds[64 * DH];               // dO (dP; transposed reads for dv)
    float lse[64], dhat[64], ddel[64], fq[64], gq[64];
    float rq[64];                // rowf * mid for the query block against the workgroup's key block
    float ftl[64];               // (F_i - F_e) log2e - lse_i (16-bit: anchored off-block scores)
    float ndh[64];               // -Delta_i (16-bit: the dO.V MFMA's accumulator input)
};

// kf holds k/8 (the same exact products as the dq kernel's q/8); for 16-bit inputs off-block tiles use the dq kernel's
// anchor (nfe = F_e - F_j of the workgroup's key block as the q.k accumulator input, ftl per query) and -Delta as the
// dO.V accumulator input, so both kernels evaluate every pair with the same operations.
template <class T, bool PAIR>
SISA_DEV void dkv_tile(const DkvLds<T>& sm, int lane, int m0, int k0, int L, const frag8<T> (&kf)[2],
                       const frag8<T> (&vf)[2], const frag8<T>& bfr, float fk, float nfe, float rk, float gk, float dsd,
                       float lam, float& dgu, float& dfs, f32x4 (&dva)[4], f32x4 (&dka)[4], f32x4 (&dba)[2]) {
    constexpr bool F16 = Anchor<T>::on;
    constexpr bool ANCH = F16 && !PAIR;
    const int grp = lane >> 4, lc = lane & 15;
    const int kk = k0 + lc;
    const float* rqm = sm.rq;
    const f32x4 nfe4 = ANCH ? f32x4{nfe, nfe, nfe, nfe} : zero4();
#pragma unroll
    for (int st = 0; st < 2; ++st) {           // 32 queries (one K-step of the dk/dv/db products) at a time
        f32x4 pv[2], kv[2], bv[2];             // dv, dk and db operands of the two 16-query blocks (before rounding)
#pragma unroll
        for (int hb = 0; hb < 2; ++hb) {       // one 16-query block at a time keeps the live set small
            __builtin_amdgcn_sched_barrier(0);
            const int qb = 2 * st + hb;
            const int i0 = qb * 16 + 4 * grp;
            const f32x4 sc = mma(frag_rows<T, DH>(sm.qs, qb * 16, 1, lane), kf[1],
                                 mma(frag_rows<T, DH>(sm.qs, qb * 16, 0, lane), kf[0], nfe4));
            const f32x4 cb = mma(frag_rows<T, DS>(sm.cs, qb * 16, 0, lane), bfr, zero4());
            const f32x4 dp = mma(frag_rows<T, DH>(sm.ds, qb * 16, 1, lane), vf[1],
                                 mma(frag_rows<T, DH>(sm.ds, qb * 16, 0, lane), vf[0],
                                     F16 ? lds4f(&sm.ndh[i0]) : zero4()));
            const f32x4 dd = lds4f(&sm.ddel[i0]);
            if (PAIR) {
                const f32x4 gq = lds4f(&sm.gq[i0]);
                const f32x4 lq = lds4f(&sm.lse[i0]), fq = lds4f(&sm.fq[i0]);
                const f32x4 dh = F16 ? zero4() : lds4f(&sm.dhat[i0]);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int qq = m0 + i0 + i;
                    const bool valid = qq >= kk && qq < L;
                    const bool strict = valid && qq > kk;
                    const bool eye = valid && qq == kk;
                    const float dec = valid ? exp2_le0((gq[i] - gk) * LOG2E) : 0.f;
                    const float u = dec * cb[i];
                    float s = sc[i] + (fq[i] - fk);
                    s = s + lam * u;
                    const float p = valid ? fast_exp2(fmaf(s, LOG2E, -lq[i])) : 0.f;
                    const float dsh = p * (F16 ? dp[i] : dp[i] - dh[i]);
                    const float dsx = dsh - p * dd[i];
                    const float dso = strict ? dsx : 0.f;
                    dgu += dso * u;
                    dfs += dso;
                    pv[hb][i] = p;
                    kv[hb][i] = eye ? dsd : dso;
                    bv[hb][i] = (eye ? dsd : (strict ? dsh : 0.f)) * (lam * dec);
                }
            } else {
                const f32x4 rq = lds4f(&rqm[i0]);
                const f32x4 off = ANCH ? lds4f(&sm.ftl[i0]) : zero4();
                const f32x4 lq = ANCH ? zero4() : lds4f(&sm.lse[i0]);
                const f32x4 fq = ANCH ? zero4() : lds4f(&sm.fq[i0]);
                const f32x4 dh = F16 ? zero4() : lds4f(&sm.dhat[i0]);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float uc = cb[i] * rq[i];
                    float s;
                    if constexpr (ANCH) s = fmaf(rk, uc, sc[i]);
                    else s = (sc[i] + (fq[i] - fk)) + rk * uc;
                    const float p = fast_exp2(fmaf(s, LOG2E, ANCH ? off[i] : -lq[i]));
                    const float dsh = p * (F16 ? dp[i] : dp[i] - dh[i]);
                    const float dsx = dsh - p * dd[i];
                    dgu += dsx * uc;
                    dfs += dsx;
                    pv[hb][i] = p;
                    kv[hb][i] = dsx;
                    bv[hb][i] = dsh * rq[i];
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        const frag8<T> pf = pack8<T>(pv[0], pv[1]);
        const frag8<T> kfr = pack8<T>(kv[0], kv[1]);
        const frag8<T> bf = pack8<T>(bv[0], bv[1]);
#pragma unroll
        for (int db = 0; db < 4; ++db) {
            dva[db] = mma(frag_tr<T, DH>(sm.ds, db * 16, st, lane), pf, dva[db]);
            dka[db] = mma(frag_tr<T, DH>(sm.qs, db * 16, st, lane), kfr, dka[db]);
        }
#pragma unroll
        for (int sb = 0; sb < 2; ++sb) dba[sb] = mma(frag_tr<T, DS>(sm.cs, sb * 16, st, lane), bf, dba[sb]);
    }
}

template <class T>
__global__ __launch_bounds__(NTHB) __attribute__((amdgpu_waves_per_eu(3))) void attn_bwd_dkv_kernel(sisa_attn_bwd_args a) {
    constexpr int NBUF = sizeof(T) == 2 ? 2 : 1;
    __shared__ DkvLds<T> smb[NBUF];
    const int tid = threadIdx.x, lane = tid & 63, grp = lane >> 4, lc = lane & 15;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    int bh, ktile;
    xcd_map(blockIdx.x, (a.L + 63) / 64, a.B * a.H, bh, ktile);   // early key blocks carry the most queries: first
    const int H = a.H, L = a.L;
    const int b = bh / H, h = bh % H;
    const bool has_f = a.f.ptr != nullptr;
    const T* Q = (const T*)a.q.ptr + (int64_t)b * a.q.sb + (int64_t)h * a.q.sh;
    const T* K = (const T*)a.k.ptr + (int64_t)b * a.k.sb + (int64_t)h * a.k.sh;
    const T* V = (const T*)a.v.ptr + (int64_t)b * a.v.sb + (int64_t)h * a.v.sh;
    const T* C = (const T*)a.c.ptr + (int64_t)b * a.c.sb + (int64_t)h * a.c.sh;
    const T* Bm = (const T*)a.b.ptr + (int64_t)b * a.b.sb + (int64_t)h * a.b.sh;
    const T* DO = (const T*)a.dout.ptr + (int64_t)b * a.dout.sb + (int64_t)h * a.dout.sh;
    const float* G = (const float*)a.g.ptr + (int64_t)b * a.g.sb + (int64_t)h * a.g.sh;
    const float* FF = has_f ? (const float*)a.f.ptr + (int64_t)b * a.f.sb + (int64_t)h * a.f.sh : nullptr;
    const float* ROWF = a.rowf + (int64_t)bh * L;
    const float* COLF = a.colf + (int64_t)bh * L;
    const float* LSE = a.lse + (int64_t)bh * L;
    const float lam = a.lam[(int64_t)h * a.s_lam];
    const int64_t sql = a.q.sl, scl = a.c.sl, sdl = a.dout.sl, sgl = a.g.sl;
    const int64_t sfl = has_f ? a.f.sl : 0;
    const int64_t BHL = (int64_t)a.B * H * L;
    const float* WS = (const float*)a.workspace;
    const float* DELTA = WS + WS_DELTA * BHL + (int64_t)bh * L;
    const float* DDEL = WS + WS_DDEL * BHL + (int64_t)bh * L;

    const int ktile0 = ktile * 64;                 // the workgroup's 64-key decay block
    const int k0 = ktile0 + 16 * w;
    const bool live = k0 < L;
    const int kend = ktile0 + 63 < L ? ktile0 + 63 : L - 1;
    const float ge = G[(int64_t)kend * sgl];       // anchors: g and F at the block end
    const float fe = has_f ? FF[(int64_t)kend * sfl] : 0.f;

    frag8<T> kf[2], vf[2], bfr;
    float fk, nfe, colf, rk, gk, dsd;
    {
        const int kk = k0 + lc;
        const bool ok = kk < L;
#pragma unroll
        for (int st = 0; st < 2; ++st) {
            kf[st] = ok ? scale_frag<T>(load8<T>(K + (int64_t)kk * a.k.sl + 32 * st + 8 * grp), QSCALE) : zero8<T>();
            vf[st] = ok ? load8<T>(V + (int64_t)kk * a.v.sl + 32 * st + 8 * grp) : zero8<T>();
        }
        bfr = ok ? load8<T>(Bm + (int64_t)kk * a.b.sl + 8 * grp) : zero8<T>();
        fk = (has_f && ok) ? FF[(int64_t)kk * sfl] : 0.f;
        nfe = fe - fk;
        colf = ok ? COLF[kk] : 0.f;
        rk = lam * colf;
        gk = G[(int64_t)(ok ? kk : L - 1) * sgl];
        dsd = ok ? WS[WS_DSD * BHL + (int64_t)bh * L + kk] : 0.f;
    }

    f32x4 dva[4], dka[4], dba[2];
#pragma unroll
    for (int db = 0; db < 4; ++db) dva[db] = dka[db] = zero4();
    dba[0] = dba[1] = zero4();
    // column sums (diagonal excluded); off-block tiles accumulate dgu without the column factor colf
    float dgu = 0.f, dfs = 0.f;

    // Query tiles straight into LDS (DMA buffer loads), from the last one down to the block's own tile; 16-bit types
    // double-buffer them (one barrier per tile), fp32 uses one buffer. The per-query scalars are fetched into
    // registers by the first wave one tile ahead.
    DmaStage<T, DH, NWB> dmq, dmd;
    DmaStage<T, DS, NWB> dmc;
    const int64_t xq = ((int64_t)(L - 1) * sql + DH) * (int64_t)sizeof(T);   // view extents (bytes)
    const int64_t xd = ((int64_t)(L - 1) * sdl + DH) * (int64_t)sizeof(T);
    const int64_t xc = ((int64_t)(L - 1) * scl + DS) * (int64_t)sizeof(T);
    dmq.init(sql, w, lane);
    dmd.init(sdl, w, lane);
    dmc.init(scl, w, lane);
    const int mlast = (L - 1) / 64 * 64;
    const int nt = (mlast - ktile0) / 64;         // query tiles after the block; tile t starts at mlast - 64 t
    float pf_lse = 0.f, pf_dh = 0.f, pf_dd = 0.f, pf_f = 0.f, pf_g = 0.f, pf_rowf = 0.f, pf_gm = 0.f;
    auto fetch_scalars = [&](int m0) {
        if (tid < 64) {
            const int i = m0 + tid;
            const bool ok = i < L;
            const int ic = ok ? i : L - 1;
            pf_lse = ok ? LSE[i] : __builtin_inff();
            pf_dh = ok ? DELTA[i] : 0.f;
            pf_dd = ok ? DDEL[i] : 0.f;
            pf_f = (has_f && ok) ? FF[(int64_t)i * sfl] : 0.f;
            pf_g = G[(int64_t)ic * sgl];
            pf_rowf = ok ? ROWF[i] : 0.f;
            pf_gm = G[(int64_t)m0 * sgl];           // start of the query block
        }
    };
    auto issue_tile = [&](DkvLds<T>& d, int m0) {   // rows >= L read as zero
        dma_issue<2>(dmq, Q, xq, (int)(m0 * sql * (int64_t)sizeof(T)), d.qs, w);
        dma_issue<2>(dmd, DO, xd, (int)(m0 * sdl * (int64_t)sizeof(T)), d.ds, w);
        dma_issue<2>(dmc, C, xc, (int)(m0 * scl * (int64_t)sizeof(T)), d.cs, w);
        if (tid < 64) {
            d.lse[tid] = pf_lse;
            d.dhat[tid] = pf_dh;
            d.ddel[tid] = pf_dd;
            d.fq[tid] = pf_f;
            d.gq[tid] = pf_g;
            d.rq[tid] = pf_rowf * exp2_le0((pf_gm - ge) * LOG2E);
            d.ftl[tid] = fmaf(pf_f - fe, LOG2E, -pf_lse);
            d.ndh[tid] = -pf_dh;
        }
    };
    auto advance = [&](int t) {
        const int m0 = mlast - 64 * t;
        if (NBUF == 2) {
            if (t < nt) {
                issue_tile(smb[(t + 1) & (NBUF - 1)], m0 - 64);
                if (t + 1 < nt) fetch_scalars(m0 - 128);
            }
        } else if (t > 0) {
            __syncthreads();
            issue_tile(smb[0], m0);
            __syncthreads();
            if (t < nt) fetch_scalars(m0 - 64);
        }
    };
    fetch_scalars(mlast);
    issue_tile(smb[0], mlast);
    if (nt > 0) fetch_scalars(mlast - 64);
    __syncthreads();
    for (int t = 0; t < nt; ++t) {
        advance(t);
        if (live) {
            const DkvLds<T>& sm = smb[t & (NBUF - 1)];
            dkv_tile<T, false>(sm, lane, mlast - 64 * t, k0, L, kf, vf, bfr, fk, nfe, rk, gk, dsd, lam, dgu, dfs, dva,
                               dka, dba);
        }
        if (NBUF == 2) __syncthreads();
    }
    advance(nt);
    if (live) {
        // the block's own tile: apply the off-block column factors once, in fp32, then the pair path
        const DkvLds<T>& sm = smb[nt & (NBUF - 1)];
        dgu *= colf;
        dba[0] *= rk;
        dba[1] *= rk;
        dkv_tile<T, true>(sm, lane, ktile0, k0, L, kf, vf, bfr, fk, nfe, rk, gk, dsd, lam, dgu, dfs, dva, dka, dba);
    }
    if (!live) return;
    const float Dgu = group_sum(dgu), Dfs = group_sum(dfs);
    const int kk = k0 + lc;
    if (kk >= L) return;
    T* dkp = (T*)a.dk.ptr + (int64_t)b * a.dk.sb + (int64_t)h * a.dk.sh + (int64_t)kk * a.dk.sl;
    T* dvp = (T*)a.dv.ptr + (int64_t)b * a.dv.sb + (int64_t)h * a.dv.sh + (int64_t)kk * a.dv.sl;
#pragma unroll
    for (int db = 0; db < 4; ++db) {
        const int d = db * 16 + 4 * grp;
        store_row4<T, T>(dkp + d, dka[db] * QSCALE);
        store_row4<T, T>(dvp + d, dva[db]);
    }
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
        const int s0 = sb * 16 + 4 * grp;
        if (a.dcb_dtype == SISA_F32) {
            float* p = (float*)a.db.ptr + (int64_t)b * a.db.sb + (int64_t)h * a.db.sh + (int64_t)kk * a.db.sl;
            *reinterpret_cast<f32x4*>(p + s0) = dba[sb];
        } else {
            T* p = (T*)a.db.ptr + (int64_t)b * a.db.sb + (int64_t)h * a.db.sh + (int64_t)kk * a.db.sl;
            store_row4<T, T>(p + s0, dba[sb]);
        }
    }
    if (grp == 0) {
        const int64_t o = (int64_t)bh * L + kk;
        a.dg[o] = WS[WS_RG * BHL + o] - lam * Dgu;
        if (has_f) a.df[o] = WS[WS_RF * BHL + o] - Dfs;
    }
}

// dlambda_h = sum over (b, t) of the per-row parts, in fp64 with a fixed reduction order (attention.py:781-783).
__global__ __launch_bounds__(1024) void dlam_kernel(const float* __restrict__ rl, float* __restrict__ dlam, int B,
                                                   int H, int L) {
    __shared__ double red[1024];
    const int h = blockIdx.x;
    const int64_t n = (int64_t)B * L;
    double s = 0.0;
    for (int64_t t = threadIdx.x; t < n; t += 1024) {
        const int64_t bb = t / L, l = t % L;
        s += (double)rl[(bb * H + h) * (int64_t)L + l];
    }
    red[threadIdx.x] = s;
    __syncthreads();
    for (int o = 512; o > 0; o >>= 1) {
        if ((int)threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
        __syncthreads();
    }
    if (threadIdx.x == 0) dlam[h] = (float)red[0];
}

template <class T>
int launch_fwd(const sisa_attn_fwd_args* a, hipStream_t st) {
    const dim3 grid((unsigned)(sisa::cdiv(a->L, 128) * a->B * a->H));
    attn_fwd_kernel<T><<<grid, NTH, 0, st>>>(*a);
    return sisa::launch_status("sisa_attn_fwd");
}

template <class T>
int launch_bwd(const sisa_attn_bwd_args* a, hipStream_t st) {
    const dim3 grid((unsigned)(sisa::cdiv(a->L, 64) * a->B * a->H));
    attn_bwd_dq_kernel<T><<<grid, NTHB, 0, st>>>(*a);
    int rc = sisa::launch_status("sisa_attn_bwd (dq)");
    if (rc) return rc;
    attn_bwd_dkv_kernel<T><<<grid, NTHB, 0, st>>>(*a);
    rc = sisa::launch_status("sisa_attn_bwd (dkv)");
    if (rc) return rc;
    const int64_t BHL = (int64_t)a->B * a->H * a->L;
    dlam_kernel<<<a->H, 1024, 0, st>>>((const float*)a->workspace + WS_RL * BHL, a->dlam, a->B, a->H, a->L);
    return sisa::launch_status("sisa_attn_bwd (dlam)");
}

bool g_view_ok(const sisa_view& v) {
    return v.ptr != nullptr;
}

}  // namespace

extern "C" int sisa_factors(const sisa_factors_args* a, void* stream) {
    SISA_REQUIRE(a != nullptr, "sisa_factors: null args");
    SISA_REQUIRE(a->B >= 1 && a->H >= 1 && a->L >= 1, "sisa_factors: bad shape B=%d H=%d L=%d", a->B, a->H, a->L);
    SISA_REQUIRE(g_view_ok(a->g) && a->rowf && a->colf && a->mono, "sisa_factors: null pointer");
    dim3 grid((unsigned)sisa::cdiv(a->L, BLK), (unsigned)(a->B * a->H));
    factors_kernel<<<grid, 64, 0, (hipStream_t)stream>>>(*a);
    return sisa::launch_status("sisa_factors");
}

// The sequence extent of one (batch, head) slice of a view, addressed through one buffer resource.
static bool extent_ok(const sisa_view& v, int L, int C, int dtype) {
    return v.sl >= 0 && ((int64_t)(L - 1) * v.sl + C) * sisa::elem_size(dtype) < ((int64_t)1 << 31);
}

extern "C" int sisa_attn_fwd(const sisa_attn_fwd_args* a, void* stream) {
    SISA_REQUIRE(a != nullptr, "sisa_attn_fwd: null args");
    SISA_REQUIRE(a->B >= 1 && a->H >= 1 && a->L >= 1, "sisa_attn_fwd: bad shape B=%d H=%d L=%d", a->B, a->H, a->L);
    SISA_REQUIRE((int64_t)a->B * a->H * sisa::cdiv(a->L, 64) * 512 < ((int64_t)1 << 31),
                 "sisa_attn_fwd: B*H*L too large for one launch");
    SISA_REQUIRE(a->dtype == SISA_BF16 || a->dtype == SISA_F16 || a->dtype == SISA_F32, "sisa_attn_fwd: dtype %d",
                 a->dtype);
    SISA_REQUIRE(sisa::view_ok(a->q, a->dtype) && sisa::view_ok(a->k, a->dtype) && sisa::view_ok(a->v, a->dtype) &&
                     sisa::view_ok(a->c, a->dtype) && sisa::view_ok(a->b, a->dtype) && sisa::view_ok(a->o, a->dtype),
                 "sisa_attn_fwd: q/k/v/c/b/o must be non-null with 16-byte aligned rows");
    SISA_REQUIRE(g_view_ok(a->g) && a->lam && a->rowf && a->colf && a->lse, "sisa_attn_fwd: null pointer");
    SISA_REQUIRE(a->o32 == nullptr || sisa::aligned16(a->o32), "sisa_attn_fwd: o32 not aligned");
    SISA_REQUIRE(extent_ok(a->k, a->L, DH, a->dtype) && extent_ok(a->v, a->L, DH, a->dtype) &&
                     extent_ok(a->b, a->L, DS, a->dtype),
                 "sisa_attn_fwd: a (batch, head) slice of k/v/b spans 2 GiB or more");
    hipStream_t st = (hipStream_t)stream;
    switch (a->dtype) {
        case SISA_BF16: return launch_fwd<__bf16>(a, st);
        case SISA_F16: return launch_fwd<_Float16>(a, st);
        default: {
            SISA_REQUIRE(a->o32 == nullptr, "sisa_attn_fwd: o32 is for bf16/fp16 inputs");
            return launch_fwd<float>(a, st);
        }
    }
}

extern "C" int64_t sisa_attn_bwd_workspace_bytes(int32_t B, int32_t H, int32_t L) {
    return (int64_t)WS_N * B * H * L * (int64_t)sizeof(float);
}

extern "C" int sisa_attn_bwd(const sisa_attn_bwd_args* a, void* stream) {
    SISA_REQUIRE(a != nullptr, "sisa_attn_bwd: null args");
    SISA_REQUIRE(a->B >= 1 && a->H >= 1 && a->L >= 1, "sisa_attn_bwd: bad shape B=%d H=%d L=%d", a->B, a->H, a->L);
    SISA_REQUIRE((int64_t)a->B * a->H * sisa::cdiv(a->L, 64) * 512 < ((int64_t)1 << 31),
                 "sisa_attn_bwd: B*H*L too large for one launch");
    SISA_REQUIRE(a->dtype == SISA_BF16 || a->dtype == SISA_F16 || a->dtype == SISA_F32, "sisa_attn_bwd: dtype %d",
                 a->dtype);
    SISA_REQUIRE(a->dcb_dtype == a->dtype || a->dcb_dtype == SISA_F32, "sisa_attn_bwd: dc/db dtype %d",
                 a->dcb_dtype);
    const int dt = a->dtype;
    SISA_REQUIRE(sisa::view_ok(a->q, dt) && sisa::view_ok(a->k, dt) && sisa::view_ok(a->v, dt) &&
                     sisa::view_ok(a->c, dt) && sisa::view_ok(a->b, dt) && sisa::view_ok(a->o, dt) &&
                     sisa::view_ok(a->dout, dt) && sisa::view_ok(a->dq, dt) && sisa::view_ok(a->dk, dt) &&
                     sisa::view_ok(a->dv, dt) && sisa::view_ok(a->dc, a->dcb_dtype) &&
                     sisa::view_ok(a->db, a->dcb_dtype),
                 "sisa_attn_bwd: tensors must be non-null with 16-byte aligned rows");
    SISA_REQUIRE(g_view_ok(a->g) && a->lam && a->rowf && a->colf && a->lse && a->dg && a->dlam && a->workspace,
                 "sisa_attn_bwd: null pointer");
    SISA_REQUIRE(extent_ok(a->q, a->L, DH, dt) && extent_ok(a->k, a->L, DH, dt) && extent_ok(a->v, a->L, DH, dt) &&
                     extent_ok(a->dout, a->L, DH, dt) && extent_ok(a->c, a->L, DS, dt) &&
                     extent_ok(a->b, a->L, DS, dt),
                 "sisa_attn_bwd: a (batch, head) slice of q/k/v/do/c/b spans 2 GiB or more");
    SISA_REQUIRE((a->f.ptr == nullptr) == (a->df == nullptr), "sisa_attn_bwd: f and df must both be given or null");
    SISA_REQUIRE(a->o32 == nullptr || (sisa::aligned16(a->o32) && dt != SISA_F32), "sisa_attn_bwd: bad o32");
    hipStream_t st = (hipStream_t)stream;
    switch (dt) {
        case SISA_BF16: return launch_bwd<__bf16>(a, st);
        case SISA_F16: return launch_bwd<_Float16>(a, st);
        default: return launch_bwd<float>(a, st);
    }
}
