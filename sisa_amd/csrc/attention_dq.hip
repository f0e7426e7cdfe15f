// SISA attention backward for gfx950, the query-owned dq kernel of the exact-delta backward (the decomposition, score
// arithmetic and reference citations are described in attention.hip; the key-owned dkv kernel is in
// attention_bwd.hip). A translation unit of its own so that the build can give it its own machine scheduler.
#include "attention_common.h"

namespace {

// ------------------------------------------------------------------------------------------------ backward: dq

template <class T>
struct __attribute__((aligned(16))) DqLds {
    T ks[64 * DH];               // K (scores; transposed reads for dq)
    T vs[64 * DH];               // V (dP)
    T bs[64 * DS];               // B~ (scores; transposed reads for dc)
    float fk[64], gk[64];
    float nfe[64];               // F_e - F_j (F_e = F at the tile's last key; anchored off-block scores)
    float cfm[2][64];            // colf * mid for the workgroup's two query blocks
};

// Per-query row sums of the dq kernel (diagonal excluded): xa = sum dS^ u, ya = sum P u, wa = D = sum dS^,
// za = Z = sum P, ptt = P_tt, dptt = dP_tt, xd = cb_tt. Off-block tiles accumulate xa, ya without the row factor
// rowf; a wave's own-block tile is its last one, and rowf (lam for dc) is applied once before it.
struct RowSums {
    float xa, ya, wa, za, ptt, dptt, xd;
};

// Score arithmetic as in the forward: q is pre-scaled by 1/8; for 16-bit inputs off-block tiles are anchored at the
// key tile's last F (F_e - F_j enters the q.k MFMA as its accumulator input, (F_i - F_e) log2e - lse is one offset
// per query and tile) and dP - Delta comes out of the dO.V MFMA (-Delta as its accumulator input). The dkv kernel
// evaluates the same pairs with the same anchors and the same accumulator inputs.
// nkb (own-block tile only, wave-uniform): the 16-key blocks at or before the wave's last query; later blocks are
// masked for all 16 queries and are skipped.
template <class T, bool DIAG>
SISA_DEV void dq_tile(const DqLds<T>& sm, int qblk, int lane, int n0, int q0, int L, const frag8<T> (&qf)[2],
                      const frag8<T>& cfr, const frag8<T> (&dof)[2], float fq, float rf, float gq, float lse,
                      float dhat, float lam, bool exact, RowSums& R, f32x4 (&dqa)[4], f32x4 (&dca)[2], int nkb = 4) {
    constexpr bool F16 = Anchor<T>::on;
    constexpr bool ANCH = F16 && !DIAG;
    const int grp = lane >> 4, lc = lane & 15;
    const int qq = q0 + lc;
    const float* cfm = sm.cfm[qblk];
    const float rs = lam * rf;                 // row scale lambda * rowf of the off-block scores
    const float ftl = ANCH ? fmaf(fq - sm.fk[63], LOG2E, -lse) : -lse;
    const f32x4 ndh = F16 ? f32x4{-dhat, -dhat, -dhat, -dhat} : zero4();
#pragma unroll
    for (int st = 0; st < 2; ++st) {           // 32 keys (one K-step of the dq/dc products) at a time
        if (DIAG && 2 * st >= nkb) break;
        f32x4 dsv[2], wv[2];                   // dq and dc operands of the two 16-key blocks (before rounding)
#pragma unroll
        for (int hb = 0; hb < 2; ++hb) {       // one 16-key block at a time keeps the live set small
            __builtin_amdgcn_sched_barrier(0);
            const int kb = 2 * st + hb;
            if (DIAG && kb >= nkb) {
                dsv[hb] = wv[hb] = zero4();
                continue;
            }
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
                    // exact: the diagonal enters the dq/dc products after the loop (delta-free dS_tt);
                    // FlashAttention-standard mode keeps P_tt (dP_tt - delta) in the GEMM operands
                    const float dsg = exact ? dso : ds;
                    R.ptt += eye ? pr : 0.f;
                    R.dptt += eye ? dpd : 0.f;
                    R.xd += eye ? (exact ? cbv : ds * u) : 0.f;
                    const float po = eye ? 0.f : pr;
                    R.za += po;
                    R.ya += po * u;
                    R.wa += dso;
                    R.xa += dso * u;
                    dsv[hb][i] = dsg;
                    wv[hb][i] = dsg * (lam * dec);
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
                    // the dc operand dS * (rowf_i * (colf_j * mid)): the same fp32 value the dkv kernel rounds for
                    // the pair's db term, so that the pair's two rotation terms of dPhi cancel exactly in the
                    // reverse scan of dtheta (lambda is applied to the sums)
                    wv[hb][i] = ds * (rf * cf[i]);
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
__global__ __launch_bounds__(NTH) __attribute__((amdgpu_waves_per_eu(sizeof(T) == 2 ? 4 : 2)))
void attn_bwd_dq_kernel(sisa_attn_bwd_args a) {
    constexpr int NBUF = sizeof(T) == 2 ? 2 : 1;
    __shared__ DqLds<T> smb[NBUF];
    const int tid = threadIdx.x, lane = tid & 63, grp = lane >> 4, lc = lane & 15;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int NQT = (a.L + 127) / 128;
    int bh, rank;
    xcd_map(blockIdx.x, NQT, a.B * a.H, bh, rank);
    const int tile = NQT - 1 - rank;               // heavy (late) query tiles first
    const int H = a.H, L = a.L;
    const int b = bh / H, h = bh % H;
    const bool has_f = a.f.ptr != nullptr;
    const bool exact = a.exact != 0;
    const float* O32 = exact ? a.o32 : nullptr;
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

    const int tile0 = tile * 128;                  // the workgroup's two 64-row decay blocks
    const int q0 = tile0 + 16 * w;
    const int qblk = w >> 2;                       // the wave's block
    const bool live = q0 < L;
    const int ta0 = tile0 < L ? tile0 : L - 1, ta1 = tile0 + 64 < L ? tile0 + 64 : L - 1;
    const float ga0 = G[(int64_t)ta0 * sgl];       // anchors: g at the start of each block
    const float ga1 = G[(int64_t)ta1 * sgl];

    frag8<T> qf[2], cfr, dof[2];
    float fq, rowfq, rs, gq, lse, dhat;
    {
        // every load from a row in range (rows past L read row L - 1 and are masked), all in flight together
        const int qq = q0 + lc;
        const bool ok = qq < L;
        const int64_t qc = ok ? qq : L - 1;
        frag8<T> qr[2], dr[2];
#pragma unroll
        for (int st = 0; st < 2; ++st) {
            qr[st] = load8<T>(Q + qc * a.q.sl + 32 * st + 8 * grp);
            dr[st] = load8<T>(DO + qc * a.dout.sl + 32 * st + 8 * grp);
        }
        const frag8<T> cr = load8<T>(C + qc * a.c.sl + 8 * grp);
        const float fr = has_f ? FF[qc * sfl] : 0.f;
        const float rr = ROWF[qc];
        gq = G[qc * sgl];
        const float lr = LSE[qc];
        // exact mode: Delta'' = o''.do with the fp32 o'' as stored (no snapping to the DT o: a snapped element
        // carries up to the snap threshold of error, not proportional to the non-dominant mass of the row)
        f32x4 oa[2], ob[2];
        if (O32) {
            const float* p32 = O32 + ((int64_t)bh * L + qc) * DH + 8 * grp;
#pragma unroll
            for (int st = 0; st < 2; ++st) {
                oa[st] = *reinterpret_cast<const f32x4*>(p32 + 32 * st);
                ob[st] = *reinterpret_cast<const f32x4*>(p32 + 32 * st + 4);
            }
        } else {
#pragma unroll
            for (int st = 0; st < 2; ++st) {
                const frag8<T> ov = load8<T>(O + qc * a.o.sl + 32 * st + 8 * grp);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    oa[st][j] = (float)ov[j];
                    ob[st][j] = (float)ov[j + 4];
                }
            }
        }
        float part = 0.f;
#pragma unroll
        for (int st = 0; st < 2; ++st) {
            qf[st] = ok ? scale_frag<T>(qr[st], QSCALE) : zero8<T>();
            dof[st] = ok ? dr[st] : zero8<T>();
#pragma unroll
            for (int j = 0; j < 4; ++j) part += oa[st][j] * (float)dof[st][j] + ob[st][j] * (float)dof[st][j + 4];
        }
        dhat = group_sum(part);
        cfr = ok ? cr : zero8<T>();
        fq = ok ? fr : 0.f;
        rowfq = ok ? rr : 0.f;
        rs = lam * rowfq;
        lse = ok ? lr : __builtin_inff();
    }

    f32x4 dqa[4], dca[2];
#pragma unroll
    for (int db = 0; db < 4; ++db) dqa[db] = zero4();
    dca[0] = dca[1] = zero4();
    RowSums R{0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};

    // Key tiles straight into LDS (DMA buffer loads); 16-bit types double-buffer them (one barrier per tile), fp32
    // uses one buffer. The per-key scalars (F_j, g_j, colf_j, g at the tile's last key) are fetched into registers by
    // the first wave one tile ahead.
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
    auto issue_tile = [&](DqLds<T>& d, int n0) {   // rows >= L read as zero
        dma_issue<1>(dk, K, xk, (int)(n0 * skl * (int64_t)sizeof(T)), d.ks, w);
        dma_issue<1>(dv, V, xv, (int)(n0 * svl * (int64_t)sizeof(T)), d.vs, w);
        dma_issue<1>(dbt, Bm, xb, (int)(n0 * sbl * (int64_t)sizeof(T)), d.bs, w);
        if (tid < 64) {
            d.fk[tid] = pf_f;
            d.nfe[tid] = pf_fe - pf_f;
            d.gk[tid] = pf_g;
            d.cfm[0][tid] = pf_cf * exp2_le0((ga0 - pf_ge) * LOG2E);
            d.cfm[1][tid] = pf_cf * exp2_le0((ga1 - pf_ge) * LOG2E);
        }
    };
    // tile t (keys 64 t ..) is in buffer t & (NBUF-1) after advance_into(t, ...) (and, for two buffers, the barrier
    // before it)
    auto advance_into = [&](int t, DqLds<T>& nxt) {   // nxt: the buffer that is idle during tile t
        const int n0 = 64 * t;
        if (NBUF == 2) {
            if (n0 + 64 < kend) {
                issue_tile(nxt, n0 + 64);
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
    // key tiles before the workgroup's first block (off-block for every wave), then the blocks' own tiles
    const int nt = tile0 / 64;
    auto off_tile = [&](int t, const DqLds<T>& sm, DqLds<T>& nxt) {
        advance_into(t, nxt);
        if (live)
            dq_tile<T, false>(sm, qblk, lane, 64 * t, q0, L, qf, cfr, dof, fq, rowfq, gq, lse, dhat, lam, exact, R, dqa,
                              dca);
        if (NBUF == 2) __syncthreads();
    };
    if constexpr (NBUF == 2) {
        // two tiles per iteration, so that each names its LDS buffers statically (no per-tile address arithmetic)
        int t = 0;
        for (; t + 2 <= nt; t += 2) {
            off_tile(t, smb[0], smb[NBUF - 1]);
            off_tile(t + 1, smb[NBUF - 1], smb[0]);
        }
        if (t < nt) off_tile(t, smb[0], smb[NBUF - 1]);
    } else {
        for (int t = 0; t < nt; ++t) off_tile(t, smb[0], smb[0]);
    }
    // block 0's own tile (its waves' last tile; an off-block tile for block 1's waves), then block 1's own tile. The
    // off-block row factors (rowf for the row sums, lam for dc) are applied once, in fp32, before a wave's own tile.
    auto own_tile = [&](const DqLds<T>& sm, int n0) {
        R.xa *= rowfq;
        R.ya *= rowfq;
        dca[0] *= lam;
        dca[1] *= lam;
        dq_tile<T, true>(sm, qblk, lane, n0, q0, L, qf, cfr, dof, fq, rowfq, gq, lse, dhat, lam, exact, R, dqa, dca,
                         (w & 3) + 1);
    };
    advance_into(nt, smb[(nt + 1) & (NBUF - 1)]);
    if (live) {
        const DqLds<T>& sm = smb[nt & (NBUF - 1)];
        if (qblk == 0) own_tile(sm, tile0);
        else dq_tile<T, false>(sm, 1, lane, tile0, q0, L, qf, cfr, dof, fq, rowfq, gq, lse, dhat, lam, exact, R, dqa, dca);
    }
    if (tile0 + 64 < kend) {
        if (NBUF == 2) __syncthreads();
        advance_into(nt + 1, smb[nt & (NBUF - 1)]);
        if (live && qblk == 1) own_tile(smb[(nt + 1) & (NBUF - 1)], tile0 + 64);
    }
    if (!live) return;
    const float xat = group_sum(R.xa), yat = group_sum(R.ya), Wa = group_sum(R.wa), Za = group_sum(R.za);
    const float Ptt = group_sum(R.ptt), Dptt = group_sum(R.dptt), Xd = group_sum(R.xd);
    const int qq = q0 + lc;
    // Self-normalised exact delta T^ = Delta + ddel and the delta-free diagonal (attention.py:453-463). ddel is kept
    // as its own quantity: forming T^ = Delta + ddel and taking T^ - Delta again would quantise ddel to the fp32 ulp
    // of Delta, an absolute error that dominates every dS of rows whose mass sits on one key. The
    // FlashAttention-standard mode keeps Delta (ddel = 0) and has the diagonal inside the products already.
    float ssum = Ptt + Za;
    ssum = ssum > 0.f ? ssum : 1.f;
    const float x0 = Dptt;   // dP_tt - Delta
    const float ddel = exact ? (Ptt * x0 + Wa) / ssum : 0.f;
    const float dstt = exact ? Ptt * (Za * x0 - Wa) / ssum : 0.f;
    const float dl_row = xat - ddel * yat;
    const float rl = exact ? dl_row + dstt * Xd : dl_row + Xd;   // the row's dlambda part (FA: Xd = dS_tt cb_tt)
    {
        // the wave's 16 rows summed in fp64 in a fixed butterfly order (lanes of group 0; rows past L add zero)
        double v = (grp == 0 && qq < L) ? (double)rl : 0.0;
#pragma unroll
        for (int o = 8; o > 0; o >>= 1) v += __shfl_xor(v, o);
        if (lane == 0) ws_block_dlam(a.workspace, BHL)[(int64_t)bh * ((L + 15) / 16) + (q0 >> 4)] = v;
    }
    if (qq >= L) return;
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
        WS[WS_DDEL * BHL + o] = ddel;
        WS[WS_DSD * BHL + o] = dstt;
        WS[WS_RG * BHL + o] = lam * dl_row;
        WS[WS_RF * BHL + o] = Wa - Za * ddel;
    }
}

}  // namespace

namespace sisa {
namespace detail {

template <class T>
static int launch_dq(const sisa_attn_bwd_args* a, hipStream_t st) {
    const dim3 qgrid((unsigned)(sisa::cdiv(a->L, 128) * a->B * a->H));
    attn_bwd_dq_kernel<T><<<qgrid, NTH, 0, st>>>(*a);
    return sisa::launch_status("sisa_attn_bwd (dq)");
}

int attn_bwd_dq(const sisa_attn_bwd_args* a, hipStream_t st) {
    switch (a->dtype) {
        case SISA_BF16: return launch_dq<__bf16>(a, st);
        case SISA_F16: return launch_dq<_Float16>(a, st);
        default: return launch_dq<float>(a, st);
    }
}

}  // namespace detail
}  // namespace sisa
