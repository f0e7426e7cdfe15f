// SISA attention backward for gfx950: the query-owned dq kernel and the key-owned dkv kernel of the exact-delta
// backward (the decomposition, score arithmetic and reference citations are described in attention.hip). A
// translation unit of its own so that the build can give these two kernels their own machine scheduler.
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
    float rf[64];                // rowf (the db operand's row factor)
    float ftl[64];               // (F_i - F_e) log2e - lse_i (16-bit: anchored off-block scores)
    float ndh[64];               // -Delta_i (16-bit: the dO.V MFMA's accumulator input)
};

// kf holds k/8 (the same exact products as the dq kernel's q/8); for 16-bit inputs off-block tiles use the dq kernel's
// anchor (nfe = F_e - F_j of the workgroup's key block as the q.k accumulator input, ftl per query) and -Delta as the
// dO.V accumulator input, so both kernels evaluate every pair with the same operations.
// q0b (own-block tile only, wave-uniform): the first 16-query block at or after the wave's first key; earlier blocks
// are masked for all 16 keys and are skipped (16-bit types; the fp32 kernel, at its register limit, computes them).
template <class T, bool PAIR>
SISA_DEV void dkv_tile(const DkvLds<T>& sm, int lane, int m0, int k0, int L, const frag8<T> (&kf)[2],
                       const frag8<T> (&vf)[2], const frag8<T>& bfr, float fk, float nfe, float rk, float cmk, float gk,
                       float dsd, float lam, bool exact, float& dgu, float& dfs, f32x4 (&dva)[4], f32x4 (&dka)[4],
                       f32x4 (&dba)[2], int q0b = 0) {
    constexpr bool F16 = Anchor<T>::on;
    constexpr bool ANCH = F16 && !PAIR;
    constexpr bool SKIP = PAIR && sizeof(T) == 2;
    const int grp = lane >> 4, lc = lane & 15;
    const int kk = k0 + lc;
    const float* rqm = sm.rq;
    const f32x4 nfe4 = ANCH ? f32x4{nfe, nfe, nfe, nfe} : zero4();
#pragma unroll
    for (int st = 0; st < 2; ++st) {           // 32 queries (one K-step of the dk/dv/db products) at a time
        if (SKIP && 2 * st + 1 < q0b) continue;
        f32x4 pv[2], kv[2], bv[2];             // dv, dk and db operands of the two 16-query blocks (before rounding)
#pragma unroll
        for (int hb = 0; hb < 2; ++hb) {       // one 16-query block at a time keeps the live set small
            __builtin_amdgcn_sched_barrier(0);
            const int qb = 2 * st + hb;
            if (SKIP && qb < q0b) {
                pv[hb] = kv[hb] = bv[hb] = zero4();
                continue;
            }
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
                    // the diagonal: the dq kernel's delta-free dS_tt (exact) or P_tt (dP_tt - delta) (FA mode,
                    // where T^ - delta = 0 makes dsx = dsh)
                    const float dse = exact ? dsd : dsh;
                    kv[hb][i] = eye ? dse : dso;
                    bv[hb][i] = (eye ? dse : (strict ? dsh : 0.f)) * (lam * dec);
                }
            } else {
                const f32x4 rq = lds4f(&rqm[i0]);
                const f32x4 rf = lds4f(&sm.rf[i0]);
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
                    bv[hb][i] = dsh * (rf[i] * cmk);   // dS * (rowf_i * (colf_j * mid)), as in the dq kernel
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

// Occupancy hint 2: the max-ILP schedule then takes 165 VGPRs for 16-bit types (still 3 waves per SIMD; the hint 3
// held it to 158 with a slower schedule, about 20 us more per backward at the north-star shape); fp32 takes 189 (2).
template <class T>
__global__ __launch_bounds__(NTHB) __attribute__((amdgpu_waves_per_eu(2))) void attn_bwd_dkv_kernel(sisa_attn_bwd_args a) {
    constexpr int NBUF = sizeof(T) == 2 ? 2 : 1;
    __shared__ DkvLds<T> smb[NBUF];
    const int tid = threadIdx.x, lane = tid & 63, grp = lane >> 4, lc = lane & 15;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    int bh, ktile;
    xcd_map(blockIdx.x, (a.L + 63) / 64, a.B * a.H, bh, ktile);   // early key blocks carry the most queries: first
    const int H = a.H, L = a.L;
    const int b = bh / H, h = bh % H;
    const bool has_f = a.f.ptr != nullptr;
    const bool exact = a.exact != 0;
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
            d.rf[tid] = pf_rowf;
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
            // colf_j * mid of this query tile: mid from the dq kernel's formula (g at the query block's start,
            // gq[0], against g at the key block's end)
            const float cmk = colf * exp2_le0((sm.gq[0] - ge) * LOG2E);
            dkv_tile<T, false>(sm, lane, mlast - 64 * t, k0, L, kf, vf, bfr, fk, nfe, rk, cmk, gk, dsd, lam, exact,
                               dgu, dfs, dva, dka, dba);
        }
        if (NBUF == 2) __syncthreads();
    }
    advance(nt);
    if (live) {
        // the block's own tile: apply the off-block column factors once, in fp32, then the pair path
        const DkvLds<T>& sm = smb[nt & (NBUF - 1)];
        dgu *= colf;
        dba[0] *= lam;
        dba[1] *= lam;
        dkv_tile<T, true>(sm, lane, ktile0, k0, L, kf, vf, bfr, fk, nfe, rk, 0.f, gk, dsd, lam, exact, dgu, dfs, dva,
                          dka, dba, w);
    }
    if (w == 0 && b == 0 && ktile == 0) {
        // dlambda_h: the B * ceil(L/16) group sums of head h (written by the dq kernel) added in a fixed order,
        // lane-strided then a butterfly, by the workgroup of (batch 0, key block 0) (attention.py:781-783)
        const int ng = (L + 15) / 16, n = a.B * ng;
        const double* blk = ws_block_dlam(a.workspace, BHL);
        double sum = 0.0;
        for (int t = lane; t < n; t += 64) {
            const int bb = t / ng, s = t - bb * ng;
            sum += blk[((int64_t)bb * H + h) * ng + s];
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o);
        if (lane == 0) a.dlam[h] = (float)sum;
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

}  // namespace

namespace sisa {
namespace detail {

template <class T>
static int launch_dq_dkv(const sisa_attn_bwd_args* a, hipStream_t st) {
    const dim3 qgrid((unsigned)(sisa::cdiv(a->L, 128) * a->B * a->H));
    attn_bwd_dq_kernel<T><<<qgrid, NTH, 0, st>>>(*a);
    const int rc = sisa::launch_status("sisa_attn_bwd (dq)");
    if (rc) return rc;
    const dim3 kgrid((unsigned)(sisa::cdiv(a->L, 64) * a->B * a->H));
    attn_bwd_dkv_kernel<T><<<kgrid, NTHB, 0, st>>>(*a);
    return sisa::launch_status("sisa_attn_bwd (dkv)");
}

int attn_bwd_dq_dkv(const sisa_attn_bwd_args* a, hipStream_t st) {
    switch (a->dtype) {
        case SISA_BF16: return launch_dq_dkv<__bf16>(a, st);
        case SISA_F16: return launch_dq_dkv<_Float16>(a, st);
        default: return launch_dq_dkv<float>(a, st);
    }
}

}  // namespace detail
}  // namespace sisa
