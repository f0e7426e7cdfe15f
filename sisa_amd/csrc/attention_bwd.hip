// SISA attention backward for gfx950: the key-owned dkv kernel of the exact-delta backward and the launch of both
// backward kernels (the decomposition, score arithmetic and reference citations are described in attention.hip; the
// query-owned dq kernel is in attention_dq.hip). Translation units of their own so that the build can give the two
// kernels different machine schedulers.
#include "attention_common.h"

namespace {

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
static int launch_dkv(const sisa_attn_bwd_args* a, hipStream_t st) {
    const dim3 kgrid((unsigned)(sisa::cdiv(a->L, 64) * a->B * a->H));
    attn_bwd_dkv_kernel<T><<<kgrid, NTHB, 0, st>>>(*a);
    return sisa::launch_status("sisa_attn_bwd (dkv)");
}

int attn_bwd_dq_dkv(const sisa_attn_bwd_args* a, hipStream_t st) {
    const int rc = attn_bwd_dq(a, st);
    if (rc) return rc;
    switch (a->dtype) {
        case SISA_BF16: return launch_dkv<__bf16>(a, st);
        case SISA_F16: return launch_dkv<_Float16>(a, st);
        default: return launch_dkv<float>(a, st);
    }
}

}  // namespace detail
}  // namespace sisa
