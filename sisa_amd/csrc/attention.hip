// SISA attention for gfx950: decay factors, forward and exact-delta backward (the query-owned kernel in
// attention_dq.hip, the key-owned one in attention_bwd.hip; they also hold the deterministic fp64 dlambda reduction),
// with the C entry points.
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
// One rounding point differs from the reference on purpose. The side-term operand of the dc and db products,
// W_ij = dS_ij * lam * exp(g_i - g_j), is rounded to the 16-bit type for the MFMA. The reference rounds
// dS * (colf * mid) in its dq kernel and dS * (rowf * mid) in its dkv kernel (attention.py:20-21): the same pair then
// enters dc_i and db_j with two different roundings. Each pair's rotation terms of dPhi (+ at the query, - at the key)
// cancel in the reverse scan dtheta_t = sum_{s >= t} dPhi_s only for pairs that straddle t, exactly, when both sides
// see the same operand value; otherwise every pair past t leaves a residue of the operand's rounding, and the error
// of dtheta grows with the sequence (measured against fp64: 1.3-2.1e-2 at T = 4096, 2.0-2.8e-2 at T = 16384). Here
// both kernels round the same fp32 value dS * (rowf_i * (colf_j * mid)) (pairwise lam * exp2(min(...)) inside the
// query's own block, as before) and apply lam to the sums: dtheta is then as accurate as every other gradient
// (2.4e-3 at both lengths), for one more multiply per off-block score in each backward kernel.
//
// Work decomposition (16 rows per wave: one column group of the 16x16 MFMA blocks; no atomics):
//   forward: a workgroup of 8 waves owns 128 consecutive queries; key tiles of 64 positions, nearest first, are
//     staged row-major in LDS while the next tile's global loads are in flight; at most 128 VGPRs, so 4 waves per
//     SIMD.
//   dq kernel: a workgroup of 8 waves owns 128 queries, two 64-query decay blocks; every key tile before them is an
//     off-block tile for all waves, then block 0's own tile (off-block for block 1's waves) and block 1's; at most
//     128 VGPRs (16-bit types), so 4 waves per SIMD.
//   dkv kernel: a workgroup of 4 waves owns one 64-key block; query tiles are visited from the last one down to the
//     block's own tile; 3 waves per SIMD.
//   Operands of the sequence-contracted products (P V, dS K, ...) are read from the row-major tiles with the gfx950
//   LDS transpose read, so no transposed copy is ever stored.
//   Ownership is exclusive: dq/dc by query blocks, dk/dv/db/dg/dF by key blocks.
#include <mutex>

#include "attention_common.h"

namespace {

// ------------------------------------------------------------------------------------------------ factors
// rowf_t = exp2(min((g_t - g_{block start})*log2e, 0)), colf_t = exp2(min((g_{block end} - g_t)*log2e, 0)), and the
// maximum increase g_t - g_{t-1} per block. Reference: attention.py:129-153.
__global__ __launch_bounds__(64) void factors_kernel(sisa_factors_args a, int NT) {
    // one-dimensional grid (B*H may exceed the 65,536 limit of the second grid dimension): block = bh * NT + p
    const int p = (int)(blockIdx.x % (unsigned)NT);
    const int bh = (int)(blockIdx.x / (unsigned)NT);
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
    if (threadIdx.x == 0) a.mono[(int64_t)bh * NT + p] = inc;
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
template <class T>
struct __attribute__((aligned(16))) FwdLds {
    T ks[64 * DH];               // K tile
    T bs[64 * DS];               // B~ tile
    T vs[64 * DH];               // V tile
    float fk[64], gk[64];        // F and g at the tile's keys
    float nfe[64];               // F_e - F_j (F_e = F at the tile's last key)
    float cfm[2][64];            // colf * mid for the workgroup's two query blocks
};


// One 64-key tile for a wave's 16 queries. cx0/cx1: for off-block tiles the folded c~ operand (hi, lo; FoldC types)
// or the plain c~ (fp16, cx1 unused); for the diagonal tile the plain c~ (cx1 unused). nkb (diagonal tile only,
// wave-uniform): the 16-key blocks at or before the wave's last query; later blocks are masked for all 16 queries
// and are skipped (zero weights).
template <class T, bool DIAG>
SISA_DEV void fwd_tile(const FwdLds<T>& sm, int qblk, int lane, int n0, int q0, int L, const frag8<T> (&qf)[2],
                       const frag8<T>& cx0, const frag8<T>& cx1, const frag8<T>& onesf, float fq, float rs, float gq,
                       float lam, float& m, float& l, f32x4 (&acc)[5], int nkb = 4) {
    constexpr bool ANCH = Anchor<T>::on && !DIAG;
    const int grp = lane >> 4, lc = lane & 15;
    const int qq = q0 + lc;
    const float* cfm = sm.cfm[qblk];
    f32x4 sc[4], cb[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
        if (DIAG && kb >= nkb) continue;
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
        if (DIAG && kb >= nkb) continue;
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
    for (int kb = 0; kb < 4; ++kb) {
        if (DIAG && kb >= nkb) {
            sc[kb] = zero4();
            continue;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float pe = fast_exp2(fmaf(sc[kb][i], LOG2E, off));
            sc[kb][i] = pe;
            ls += pe;
        }
    }
    l += ls;
#pragma unroll
    for (int st = 0; st < 2; ++st) {
        if (DIAG && 2 * st >= nkb) break;
        const frag8<T> pf = pack8<T>(sc[2 * st], sc[2 * st + 1]);
#pragma unroll
        for (int db = 0; db < 4; ++db) acc[db] = mma(frag_tr<T, DH>(sm.vs, db * 16, st, lane), pf, acc[db]);
        acc[4] = mma(onesf, pf, acc[4]);   // block 4: every row holds the sum of the rounded weights
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
    const frag8<T> onesf = ones_frag<T>();

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
    // Key tiles are visited from the workgroup's last one down to key 0: the nearest keys, which usually hold a row's
    // largest scores, come first, so that the running maximum is set early and the lazy rescale seldom fires again.
    // Position k holds tile tlast - k, in LDS buffer k & (NBUF-1); advance_into(k, nxt) issues position k + 1 into
    // nxt, the buffer idle during position k (two buffers), or loads position k (one buffer).
    const int nfull = tile0 / 64;                  // tiles before the workgroup's first query block
    const int tlast = (tile0 + 64 < kend) ? nfull + 1 : nfull;
    auto advance_into = [&](int k, FwdLds<T>& nxt) {
        const int t = tlast - k;
        if (NBUF == 2) {
            if (t > 0) {
                issue_tile(nxt, 64 * (t - 1));
                if (t > 1) fetch_scalars(64 * (t - 2));
            }
        } else if (k > 0) {
            __syncthreads();
            issue_tile(smb[0], 64 * t);
            __syncthreads();
            if (t > 0) fetch_scalars(64 * (t - 1));
        }
    };
    fetch_scalars(64 * tlast);
    issue_tile(smb[0], 64 * tlast);
    if (tlast > 0) fetch_scalars(64 * (tlast - 1));
    // 16-bit types with both query blocks in range: block 0's tile goes into the second buffer in the prologue too, so
    // that the two blocks' diagonal tiles run in the same position (each wave group still sees its tiles in the same
    // order: block 1's waves T1, T0, T-1, ...; block 0's waves T0, T-1, ...)
    const bool both = NBUF == 2 && tlast == nfull + 1;
    if (both) {
        issue_tile(smb[NBUF - 1], 64 * (tlast - 1));
        if (tlast > 1) fetch_scalars(64 * (tlast - 2));
    }
    __syncthreads();
    int k = 0;
    if (both) {
        if (live) {
            if (qblk == 1)
                fwd_tile<T, true>(smb[0], 1, lane, tile0 + 64, q0, L, qf, diag_c(), cx1, onesf, fq, rs, gq, lam, m, l,
                                  acc, (w & 3) + 1);
            else
                fwd_tile<T, true>(smb[NBUF - 1], 0, lane, tile0, q0, L, qf, diag_c(), cx1, onesf, fq, rs, gq, lam, m, l,
                                  acc, (w & 3) + 1);
        }
        __syncthreads();
        // block 1's waves take block 0's tile (off-block for them) while the next tile's DMA fills the first buffer
        advance_into(1, smb[0]);
        if (live && qblk == 1)
            fwd_tile<T, false>(smb[NBUF - 1], 1, lane, tile0, q0, L, qf, cx0, cx1, onesf, fq, rs, gq, lam, m, l, acc);
        __syncthreads();
        k = 2;
    } else {
        // the workgroup's own tiles first: block 1's (its waves' diagonal), then block 0's (diagonal for block 0's
        // waves, off-block for block 1's)
        if (tlast == nfull + 1) {
            advance_into(0, smb[NBUF - 1]);
            if (live && qblk == 1)
                fwd_tile<T, true>(smb[0], 1, lane, tile0 + 64, q0, L, qf, diag_c(), cx1, onesf, fq, rs, gq, lam, m, l,
                                  acc, (w & 3) + 1);
            if (NBUF == 2) __syncthreads();
            k = 1;
        }
        {
            const FwdLds<T>& sm = smb[k & (NBUF - 1)];
            advance_into(k, smb[(k + 1) & (NBUF - 1)]);
            if (live) {
                if (qblk == 0)
                    fwd_tile<T, true>(sm, 0, lane, tile0, q0, L, qf, diag_c(), cx1, onesf, fq, rs, gq, lam, m, l,
                                      acc, (w & 3) + 1);
                else
                    fwd_tile<T, false>(sm, 1, lane, tile0, q0, L, qf, cx0, cx1, onesf, fq, rs, gq, lam, m, l, acc);
            }
            if (NBUF == 2) __syncthreads();
            ++k;
        }
    }
    // then the tiles before the workgroup's first block, nearest first: off-block for every wave
    auto off_tile = [&](int kk, const FwdLds<T>& sm, FwdLds<T>& nxt) {
        advance_into(kk, nxt);
        if (live)
            fwd_tile<T, false>(sm, qblk, lane, 64 * (tlast - kk), q0, L, qf, cx0, cx1, onesf, fq, rs, gq, lam, m, l,
                               acc);
        if (NBUF == 2) __syncthreads();
    };
    if constexpr (NBUF == 2) {
        // two tiles per iteration, so that each names its LDS buffers statically (no per-tile address arithmetic);
        // the first off-block position is even or odd depending on whether block 1 had a tile
        if (k & 1) {
            for (; k + 2 <= tlast + 1; k += 2) {
                off_tile(k, smb[1], smb[0]);
                off_tile(k + 1, smb[0], smb[1]);
            }
            if (k <= tlast) off_tile(k, smb[1], smb[0]);
        } else {
            for (; k + 2 <= tlast + 1; k += 2) {
                off_tile(k, smb[0], smb[1]);
                off_tile(k + 1, smb[1], smb[0]);
            }
            if (k <= tlast) off_tile(k, smb[0], smb[1]);
        }
    } else {
        for (; k <= tlast; ++k) off_tile(k, smb[0], smb[0]);
    }
    if (!live) return;
    T* O = (T*)a.o.ptr + (int64_t)b * a.o.sb + (int64_t)h * a.o.sh;
    // o and lse are normalised by the fp32 sum of the weights (the backward recomputes weights that sum to 1 in fp32
    // with this lse); o'' by the sum of the rounded weights, which every element of block 4 holds.
    const float lt = group_sum(l);
    const float lbt = acc[4][0];
    const int qq = q0 + lc;
    if (qq >= L) return;
    const float ls = (lt == 0.f) ? 1.f : lt;
    // one correctly rounded reciprocal per normaliser, then products (within 1.5 ulp of the quotients); 32 IEEE
    // divisions per lane cost the forward ~2 % at the north-star shape
    const float rls = 1.f / ls;
#pragma unroll
    for (int db = 0; db < 4; ++db) store4<T>(O + (int64_t)qq * a.o.sl + db * 16 + 4 * grp, to_vec4<T>(acc[db] * rls));
    if (a.o32) {
        const float rlb = 1.f / ((lbt == 0.f) ? 1.f : lbt);
        float* O32 = a.o32 + ((int64_t)bh * L + qq) * DH;
#pragma unroll
        for (int db = 0; db < 4; ++db) *reinterpret_cast<f32x4*>(O32 + db * 16 + 4 * grp) = acc[db] * rlb;
    }
    // lse of the true scores s = s' + (F_i - F_a), in log2 units
    if (grp == 0) a.lse[(int64_t)bh * L + qq] = m + __builtin_amdgcn_logf(ls);
}

template <class T>
int launch_fwd(const sisa_attn_fwd_args* a, hipStream_t st) {
    const dim3 grid((unsigned)(sisa::cdiv(a->L, 128) * a->B * a->H));
    attn_fwd_kernel<T><<<grid, NTH, 0, st>>>(*a);
    return sisa::launch_status("sisa_attn_fwd");
}


bool g_view_ok(const sisa_view& v) {
    return v.ptr != nullptr;
}

}  // namespace

extern "C" int sisa_factors(const sisa_factors_args* a, void* stream) {
    SISA_REQUIRE(a != nullptr, "sisa_factors: null args");
    SISA_REQUIRE(a->B >= 1 && a->H >= 1 && a->L >= 1, "sisa_factors: bad shape B=%d H=%d L=%d", a->B, a->H, a->L);
    SISA_REQUIRE(g_view_ok(a->g) && a->rowf && a->colf && a->mono, "sisa_factors: null pointer");
    const int64_t nt = sisa::cdiv(a->L, BLK);
    SISA_REQUIRE(nt * a->B * a->H < ((int64_t)1 << 31), "sisa_factors: B*H*ceil(L/64) exceeds the grid limit");
    factors_kernel<<<dim3((unsigned)(nt * a->B * a->H)), 64, 0, (hipStream_t)stream>>>(*a, (int)nt);
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

// Five (B,H,L) fp32 row buffers, then (B*H, ceil(L/16)) fp64 group sums of dlambda (8-byte aligned).
static int64_t bwd_workspace_bytes(int64_t B, int64_t H, int64_t L) {
    const int64_t BHL = B * H * L;
    return (WS_N * BHL + (BHL & 1)) * (int64_t)sizeof(float) + B * H * ((L + 15) / 16) * (int64_t)sizeof(double);
}

extern "C" int64_t sisa_attn_bwd_workspace_bytes(int32_t B, int32_t H, int32_t L) {
    return bwd_workspace_bytes(B, H, L);
}

// Argument checks shared by sisa_attn_bwd and sisa_attn_bwd_noalloc (the workspace pointer included).
static int check_bwd(const sisa_attn_bwd_args* a) {
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
    return SISA_OK;
}

// the dq and dkv kernels (attention_dq.hip, attention_bwd.hip); dlambda is summed inside them
static int launch_bwd_any(const sisa_attn_bwd_args* a, hipStream_t st) { return sisa::detail::attn_bwd_dq_dkv(a, st); }

extern "C" int sisa_attn_bwd(const sisa_attn_bwd_args* a, void* stream) {
    SISA_REQUIRE(a != nullptr, "sisa_attn_bwd: null args");
    const int rc = check_bwd(a);
    return rc ? rc : launch_bwd_any(a, (hipStream_t)stream);
}

// ------------------------------------------------------------------------------------------------ no-alloc backward
// The backward's workspace (five (B,H,L) fp32 row buffers and the fp64 dlambda group sums, at most 2^20 of them for
// B*H*L <= 2^20) in a file-scope device array, for callers that cannot allocate. Every GPU the library runs on holds
// its own copy (28 MiB) until the process ends. In host code `scratch` names a host-side
// stand-in, not device memory: its device address is looked up once per device (hipGetSymbolAddress, with that
// device current) and only that address is ever handed to kernels.
static __device__ __align__(256) float scratch[(WS_N + 2) * (int64_t)SISA_NOALLOC_MAX_BHL];   // 28 MiB

namespace {
constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
float* g_scratch_dev[MAX_DEVICES] = {};   // device address of `scratch`, per device ordinal

// The device address of `scratch` on the current device (looked up on the first call on that device). The stream
// must belong to the current device.
int scratch_address(hipStream_t st, float** out) {
    int dev = -1;
    SISA_REQUIRE(hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < MAX_DEVICES,
                 "sisa_attn_bwd_noalloc: no current device (or ordinal %d >= %d)", dev, MAX_DEVICES);
    if (st != nullptr) {
        hipDevice_t sdev = -1;
        SISA_REQUIRE(hipStreamGetDevice(st, &sdev) == hipSuccess && sdev == dev,
                     "sisa_attn_bwd_noalloc: the stream belongs to device %d, the current device is %d", (int)sdev,
                     dev);
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_dev[dev] == nullptr) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr) {
            sisa::set_error("sisa_attn_bwd_noalloc: hipGetSymbolAddress of the scratch array failed on device %d: %s",
                            dev, hipGetErrorString(e));
            return SISA_ERR_LAUNCH;
        }
        g_scratch_dev[dev] = static_cast<float*>(p);
    }
    *out = g_scratch_dev[dev];
    return SISA_OK;
}
}  // namespace

extern "C" int sisa_attn_bwd_noalloc(const sisa_attn_bwd_args* a, void* stream) {
    SISA_REQUIRE(a != nullptr, "sisa_attn_bwd_noalloc: null args");
    SISA_REQUIRE(a->workspace == nullptr, "sisa_attn_bwd_noalloc: workspace must be NULL (the library's scratch is "
                                          "used)");
    SISA_REQUIRE(a->B >= 1 && a->H >= 1 && a->L >= 1 &&
                     (int64_t)a->B * a->H * a->L <= (int64_t)SISA_NOALLOC_MAX_BHL,
                 "sisa_attn_bwd_noalloc: B*H*L = %lld exceeds the scratch limit SISA_NOALLOC_MAX_BHL = %d",
                 (long long)a->B * a->H * a->L, SISA_NOALLOC_MAX_BHL);
    hipStream_t st = (hipStream_t)stream;
    float* ws = nullptr;
    int rc = scratch_address(st, &ws);
    if (rc) return rc;
    sisa_attn_bwd_args b = *a;
    b.workspace = ws;      // every entry the kernels read is written earlier in the same call: nothing to clear
    rc = check_bwd(&b);
    return rc ? rc : launch_bwd_any(&b, st);
}
