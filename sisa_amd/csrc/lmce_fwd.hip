// Fused forward of the linear cross-entropy for gfx950: logits = x W_pad^T computed tile by tile on bf16/fp16 MFMA
// and reduced on the fly to each row's log-sum-exp and label logit. The (N x Vp) logits never exist in memory.
//
// Reference: the forward of `_LinearCrossEntropyFn` (src/sisa/kernels/linear_ce.py:138-191: logits chunk GEMM, then
// `_lmce_row_kernel`'s online max / sum-exp and the label pick, linear_ce.py:60-96). The reference materialises a
// (chunk, Vp) logits buffer; here the GEMM's output tiles never leave registers. As there, each logit (an fp32 MFMA
// accumulation) is rounded once to the compute dtype before the reduction, so lse and the loss are those of the
// reference's stored logits.
//
// Decomposition: a workgroup of 2 x 4 waves owns 256 rows of x and walks a range of 256-column vocabulary tiles (one
// of S vocabulary splits). Per tile, K = D is streamed through LDS in 64-wide stages (buffer loads straight into
// LDS, double-buffered, XOR-swizzled 16-byte chunks); a wave computes a 128 (vocabulary) x 64 (rows) block as 8 x 4
// v_mfma_f32_16x16x32 blocks with W as the A operand, so that a lane holds 32 logits of one row per block column
// (12 operand fragments per 32 MFMAs, to keep the LDS reads below the matrix rate). After a tile's last stage each
// wave takes every row's maximum over its 128 columns of the tile (log2 units, shared by the row's four lane groups),
// sums the row's exponentials relative to it and folds that sum into the row's running (max, sum of exponentials);
// when the tile holds a row's label it keeps that logit. At the end the lane groups and the two waves sharing rows
// combine their partials; a second launch combines the S splits of each row in a fixed order.
//
// The training pass (sisa_lmce_train, lmce_train.hip) runs the same kernel with STORE: each exponential
// p~ = exp2(logit*log2e - m_t), m_t the row's maximum over the wave's half of the tile, is also stored in the compute
// dtype into a (N, Vp) buffer, and m_t into a (2 * tiles, N) table; the gradient GEMMs later form
// G = p~ * exp2(m_t - lse) * scale - onehot from them. Both passes therefore give bitwise the same loss rows.
// Deterministic: no atomics. Workgroup i runs on XCD i % 8; each XCD takes a set of row blocks with all their
// splits, so its L2 keeps those rows of x for every vocabulary tile.
#include "common.h"
#include "host.h"

namespace {

constexpr int NWC = 8;            // waves per workgroup: 2 along the vocabulary x 4 along the rows
constexpr int TR = 256;           // rows of x per workgroup
constexpr int TV = 256;           // vocabulary columns per tile
constexpr int WV = 128;           // vocabulary columns of a wave (8 MFMA blocks)
constexpr int WR = 64;            // rows of a wave (4 MFMA blocks)
constexpr int IB = WV / 16, JB = WR / 16;
constexpr int TK = 64;            // hidden elements per LDS stage
constexpr float M_FLOOR_CE = -1e30f;
constexpr float LN2 = 0.69314718055994531f;

template <class T>
struct __attribute__((aligned(16))) CeLds {
    T x[2][TR * TK];
    T w[2][TV * TK];
    float red_m[TR], red_s[TR];   // the second wave of each row pair hands over its row partials
};

// Outputs of the training pass (STORE): exponentials relative to the tile-half maxima and those maxima.
template <class T>
struct CeStore {
    T* probs;                     // (N, Vp) in the compute dtype, row stride Vp; columns >= V hold 0
    float* mtab;                  // (2 * tiles, N): m_t of (tile t, half h) at row (2 t + h) * N + n, log2 units
};

// The vocabulary splits of one problem: S splits of `per` consecutive tiles (the last ones may be shorter or empty).
struct Split {
    int64_t tiles, S, per;
};
inline Split ce_split(int64_t N, int64_t Vp) {
    const int64_t nrb = sisa::cdiv(N, TR), tiles = sisa::cdiv(Vp, TV);
    int64_t S = sisa::cdiv(512, nrb);            // about 512 workgroups: two rounds of one per CU
    S = S < 1 ? 1 : (S > tiles ? tiles : S);
    return {tiles, S, sisa::cdiv(tiles, S)};
}

template <class T, bool STORE>
__global__ __launch_bounds__(64 * NWC) void lmce_fwd_kernel(sisa_lmce_fwd_args a, int S, int per, CeStore<T> out) {
    __shared__ CeLds<T> sm;
    const int tid = threadIdx.x, lane = tid & 63, grp = lane >> 4, lc = lane & 15;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t N = a.N, V = a.V;
    const int nrb = (int)((N + TR - 1) / TR), rbx = (nrb + 7) / 8;
    const int xcd = blockIdx.x % 8, q = blockIdx.x / 8;
    const int split = q % S, rb = xcd * rbx + q / S;
    if (rb >= nrb) return;
    const int tiles = (int)((a.Vp + TV - 1) / TV);
    const int t_begin = split * per;
    const int t_end = t_begin + per < tiles ? t_begin + per : tiles;
    const int ntiles = t_end > t_begin ? t_end - t_begin : 0;
    const int nks = a.D / TK;
    const int64_t row0 = (int64_t)rb * TR;
    const int wv = WV * (w & 1), wn = WR * (w >> 1);   // the wave's vocabulary and row offsets in the tile

    // staging: a 256-row tile is four 64-row DMA groups; rows past the data read as zero
    DmaStage<T, TK, NWC> sx, sw;
    sx.init(a.ldx, w, lane);
    sw.init(a.ldw, w, lane);
    const int64_t xbytes = ((N - 1) * a.ldx + a.D) * (int64_t)sizeof(T);
    const int64_t wbytes = ((a.Vp - 1) * a.ldw + a.D) * (int64_t)sizeof(T);
    const T* X = (const T*)a.x;
    const T* W = (const T*)a.w;
    auto issue = [&](int g, int buf) {   // stage g of the workgroup: vocabulary tile g / nks, K block g % nks
        const int64_t v0 = (int64_t)(t_begin + g / nks) * TV;
        const int k0 = (g % nks) * TK;
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            dma_issue<STORE ? 8 : 4>(sx, X, xbytes, (int)(((row0 + 64 * h) * a.ldx + k0) * (int64_t)sizeof(T)),
                         sm.x[buf] + 64 * h * TK, w);
            dma_issue<STORE ? 9 : 5>(sw, W, wbytes, (int)(((v0 + 64 * h) * a.ldw + k0) * (int64_t)sizeof(T)),
                         sm.w[buf] + 64 * h * TK, w);
        }
    };

    // the label of each of the lane's 4 rows: which tile, and whether this lane holds it (and where)
    int lab_tile[JB], lab_idx[JB];
#pragma unroll
    for (int j = 0; j < JB; ++j) {
        const int64_t n = row0 + wn + 16 * j + lc;
        lab_tile[j] = -1;
        lab_idx[j] = 0;
        if (n < N) {
            const int64_t y = a.labels[n];
            if (y != a.ignore_index && y >= 0 && y < V) {
                const int pos = (int)(y % TV);
                const bool mine = (pos / WV) * WV == wv && ((pos % 16) >> 2) == grp;
                lab_tile[j] = mine ? (int)(y / TV) : -1;
                lab_idx[j] = ((pos % WV) >> 4) * 4 + (pos & 3);   // block i, register r
            }
        }
    }
    float m[JB], s[JB], zlab[JB];
#pragma unroll
    for (int j = 0; j < JB; ++j) {
        m[j] = M_FLOOR_CE;
        s[j] = 0.f;
        zlab[j] = 0.f;
    }
    bool got[JB] = {false, false, false, false};

    f32x4 acc[IB][JB];
#pragma unroll
    for (int i = 0; i < IB; ++i)
#pragma unroll
        for (int j = 0; j < JB; ++j) acc[i][j] = zero4();

    // STORE: the exponentials go out through one buffer resource over (N, Vp) (below 2 GiB, checked by the host)
    const __amdgpu_buffer_rsrc_t prs =
        make_rsrc(STORE ? (const void*)out.probs : (const void*)a.x, STORE ? N * a.Vp * (int64_t)sizeof(T) : 0);
    const int total = ntiles * nks;
    if (total > 0) issue(0, 0);
    __syncthreads();
    for (int g = 0; g < total; ++g) {
        const int buf = g & 1;
        if (g + 1 < total) issue(g + 1, buf ^ 1);
        __builtin_amdgcn_sched_barrier(0);   // the next stage's DMA stays ahead of this stage's stores
        // all 12 operand fragments of a 32-deep step are read before its 32 MFMAs (two waves per SIMD leave room
        // for them), so one LDS wait per step instead of one per 4 MFMAs
#pragma unroll
        for (int step = 0; step < TK / 32; ++step) {
            frag8<T> xf[JB], wf[IB];
#pragma unroll
            for (int j = 0; j < JB; ++j) xf[j] = frag_rows<T, TK>(sm.x[buf], wn + 16 * j, step, lane);
#pragma unroll
            for (int i = 0; i < IB; ++i) wf[i] = frag_rows<T, TK>(sm.w[buf], wv + 16 * i, step, lane);
#pragma unroll
            for (int i = 0; i < IB; ++i)
#pragma unroll
                for (int j = 0; j < JB; ++j) acc[i][j] = mma(wf[i], xf[j], acc[i][j]);
        }
        if (g % nks == nks - 1) {
            // the tile is complete: lane holds logits of rows wn + 16 j + lc at columns v0 + wv + 16 i + 4 grp + r,
            // rounded once to the compute dtype (the logits the reference's row kernel reads)
            const int vt = t_begin + g / nks;
#pragma unroll
            for (int i = 0; i < IB; ++i)
#pragma unroll
                for (int j = 0; j < JB; ++j) acc[i][j] = __builtin_convertvector(to_vec4<T>(acc[i][j]), f32x4);
            if ((int64_t)(vt + 1) * TV > V) {   // the last tile: padding columns do not enter the sums
                const int lim = (int)(V - (int64_t)vt * TV) - wv - 4 * grp;
#pragma unroll
                for (int i = 0; i < IB; ++i)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
#pragma unroll
                        for (int j = 0; j < JB; ++j)
                            acc[i][j][r] = 16 * i + r < lim ? acc[i][j][r] : -__builtin_inff();
            }
#pragma unroll
            for (int j = 0; j < JB; ++j) {
                float mt = -__builtin_inff();   // the row's maximum over the wave's 128 columns, in log2 units
#pragma unroll
                for (int i = 0; i < IB; ++i)
#pragma unroll
                    for (int r = 0; r < 4; ++r) mt = fmaxf(mt, acc[i][j][r]);
                mt = group_max(mt) * LOG2E;
                // a half made only of padding columns (-inf) takes the reference 0: its exponentials are 0
                const float mref = mt == -__builtin_inff() ? 0.f : mt;
                const int64_t n = row0 + wn + 16 * j + lc;
                float ls = 0.f;
#pragma unroll
                for (int i = 0; i < IB; ++i) {
                    f32x4 e;
#pragma unroll
                    for (int r = 0; r < 4; ++r) e[r] = fast_exp2(fmaf(acc[i][j][r], LOG2E, -mref));
                    ls += (e[0] + e[1]) + (e[2] + e[3]);
                    if constexpr (STORE) {   // unconditional: positions past the data go past the resource
                        const int64_t v = (int64_t)vt * TV + wv + 16 * i + 4 * grp;
                        const int off = (n < N && v < a.Vp) ? (int)((n * a.Vp + v) * (int64_t)sizeof(T)) : 0x7ffffff8;
                        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, to_vec4<T>(e)), prs, off, 0, 0);
                    }
                }
                if constexpr (STORE) {
                    if (grp == 0 && n < N) out.mtab[(int64_t)(2 * vt + (w & 1)) * N + n] = mref;
                }
                if (mt > m[j]) {
                    s[j] = fmaf(s[j], fast_exp2(m[j] - mt), ls);
                    m[j] = mt;
                } else {
                    s[j] = fmaf(ls, fast_exp2(mt - m[j]), s[j]);
                }
                if (lab_tile[j] == vt) {   // rare: pick the label's logit (natural units)
                    float z = 0.f;
#pragma unroll
                    for (int i = 0; i < IB; ++i)
#pragma unroll
                        for (int r = 0; r < 4; ++r) z = (lab_idx[j] == 4 * i + r) ? acc[i][j][r] : z;
                    zlab[j] = z;
                    got[j] = true;
                }
            }
#pragma unroll
            for (int i = 0; i < IB; ++i)
#pragma unroll
                for (int j = 0; j < JB; ++j) acc[i][j] = zero4();
            if constexpr (STORE) {
                // The barrier after a tile's stores waits only until the next stage's DMA (issued before them) has
                // landed: vector memory operations complete in issue order, and at least the 32 exponential stores
                // (unconditional instructions) follow it, so vmcnt <= 32 implies the DMA is done; the stores
                // themselves complete under the next stage (its barrier waits for everything).
                __builtin_amdgcn_sched_barrier(0);
                __builtin_amdgcn_s_waitcnt(0x8070);   // vmcnt(32) expcnt(7) lgkmcnt(0)
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
                __builtin_amdgcn_s_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
                continue;
            }
        }
        __syncthreads();
    }

    // combine the four lane groups of each row, then the two waves sharing the rows (w and w ^ 1)
    float rm[JB], rsum[JB];
#pragma unroll
    for (int j = 0; j < JB; ++j) {
        rm[j] = group_max(m[j]);
        rsum[j] = group_sum(s[j] * fast_exp2(m[j] - rm[j]));
        if (got[j]) a.workspace[2 * (int64_t)S * N + row0 + wn + 16 * j + lc] = zlab[j];
    }
    if ((w & 1) && grp == 0) {
#pragma unroll
        for (int j = 0; j < JB; ++j) {
            sm.red_m[wn + 16 * j + lc] = rm[j];
            sm.red_s[wn + 16 * j + lc] = rsum[j];
        }
    }
    __syncthreads();
    if ((w & 1) == 0 && grp == 0) {
#pragma unroll
        for (int j = 0; j < JB; ++j) {
            const int64_t n = row0 + wn + 16 * j + lc;
            if (n >= N) continue;
            const float m2 = sm.red_m[wn + 16 * j + lc], s2 = sm.red_s[wn + 16 * j + lc];
            const float mm = fmaxf(rm[j], m2);
            a.workspace[(int64_t)split * N + n] = mm;
            a.workspace[(int64_t)(S + split) * N + n] = rsum[j] * fast_exp2(rm[j] - mm) + s2 * fast_exp2(m2 - mm);
        }
    }
}

// Per row: the S split partials combined in split order; lse (natural log) and the loss row. The training pass also
// keeps lse in log2 units and the row's gradient scale (0 for an ignored row, else inv_n * gscale).
struct CeTrainRows {
    float* lse2;                  // (N,) or nullptr (the no-gradient pass)
    float2* rinfo;                // (N,): s_n, and the label as the bit pattern of an int (-1 outside [0, V))
    const float* inv_n;           // device scalar 1 / N_valid
    float gscale;
};

__global__ __launch_bounds__(256) void lmce_combine_kernel(sisa_lmce_fwd_args a, int S, CeTrainRows tr) {
    const int64_t n = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (n >= a.N) return;
    const int64_t N = a.N;
    float mm = M_FLOOR_CE;
    for (int sp = 0; sp < S; ++sp) mm = fmaxf(mm, a.workspace[(int64_t)sp * N + n]);
    float ss = 0.f;
    for (int sp = 0; sp < S; ++sp)
        ss += a.workspace[(int64_t)(S + sp) * N + n] * fast_exp2(a.workspace[(int64_t)sp * N + n] - mm);
    const float l2 = mm + __builtin_amdgcn_logf(ss);
    const float lse = l2 * LN2;
    const int64_t y = a.labels[n];
    float loss;
    if (y == a.ignore_index) loss = 0.f;
    else if (y < 0 || y >= a.V) loss = __builtin_nanf("");
    else loss = lse - a.workspace[2 * (int64_t)S * N + n];
    a.loss_rows[n] = loss;
    if (a.lse) a.lse[n] = lse;
    if (tr.lse2) {
        tr.lse2[n] = l2;
        const int lab = (y >= 0 && y < a.V) ? (int)y : -1;
        tr.rinfo[n] = float2{y == a.ignore_index ? 0.f : tr.inv_n[0] * tr.gscale, __int_as_float(lab)};
    }
}

template <class T>
int launch_lmce_fwd(const sisa_lmce_fwd_args* a, hipStream_t st) {
    const Split sp = ce_split(a->N, a->Vp);
    const int64_t nrb = sisa::cdiv(a->N, TR), rbx = sisa::cdiv(nrb, 8);
    const unsigned grid = (unsigned)(8 * rbx * sp.S);
    lmce_fwd_kernel<T, false><<<grid, 64 * NWC, 0, st>>>(*a, (int)sp.S, (int)sp.per, CeStore<T>{nullptr, nullptr});
    const int rc = sisa::launch_status("sisa_lmce_fwd");
    if (rc) return rc;
    lmce_combine_kernel<<<(unsigned)sisa::cdiv(a->N, 256), 256, 0, st>>>(*a, (int)sp.S,
                                                                        CeTrainRows{nullptr, nullptr, nullptr, 0.f});
    return sisa::launch_status("sisa_lmce_fwd (combine)");
}

}  // namespace

namespace sisa {
namespace detail {

int64_t lmce_fwd_splits(int64_t N, int64_t Vp) { return ce_split(N, Vp).S; }

// The training pass's forward: the logits GEMM storing the exponentials and tile-half maxima (probs: (N, Vp) in the
// compute dtype; mtab: (2 * ceil(Vp / 256), N) fp32), then the split combine writing the loss rows, lse in log2 units
// and each row's gradient scale. a->workspace holds the (2 S + 1) N split partials.
int lmce_train_forward(const sisa_lmce_fwd_args* a, void* probs, float* mtab, float* lse2, float2* rinfo,
                       const float* inv_n, float gscale, hipStream_t st) {
    const Split sp = ce_split(a->N, a->Vp);
    const int64_t nrb = sisa::cdiv(a->N, TR), rbx = sisa::cdiv(nrb, 8);
    const unsigned grid = (unsigned)(8 * rbx * sp.S);
    if (a->dtype == SISA_BF16)
        lmce_fwd_kernel<__bf16, true><<<grid, 64 * NWC, 0, st>>>(*a, (int)sp.S, (int)sp.per,
                                                                  CeStore<__bf16>{(__bf16*)probs, mtab});
    else
        lmce_fwd_kernel<_Float16, true><<<grid, 64 * NWC, 0, st>>>(*a, (int)sp.S, (int)sp.per,
                                                                    CeStore<_Float16>{(_Float16*)probs, mtab});
    const int rc = sisa::launch_status("sisa_lmce_train (logits)");
    if (rc) return rc;
    lmce_combine_kernel<<<(unsigned)sisa::cdiv(a->N, 256), 256, 0, st>>>(*a, (int)sp.S,
                                                                        CeTrainRows{lse2, rinfo, inv_n, gscale});
    return sisa::launch_status("sisa_lmce_train (combine)");
}

}  // namespace detail
}  // namespace sisa

extern "C" int64_t sisa_lmce_fwd_workspace_bytes(int64_t N, int64_t Vp) {
    if (N < 1 || Vp < 1) return 0;
    return (2 * ce_split(N, Vp).S + 1) * N * (int64_t)sizeof(float);
}

extern "C" int sisa_lmce_fwd(const sisa_lmce_fwd_args* a, void* stream) {
    SISA_REQUIRE(a != nullptr, "sisa_lmce_fwd: null args");
    if (a->N == 0) return SISA_OK;
    SISA_REQUIRE(a->N >= 1 && a->V >= 1 && a->Vp >= a->V, "sisa_lmce_fwd: bad shape N=%lld V=%lld Vp=%lld",
                 (long long)a->N, (long long)a->V, (long long)a->Vp);
    SISA_REQUIRE(a->D >= TK && a->D % TK == 0, "sisa_lmce_fwd: hidden size %d must be a positive multiple of %d", a->D,
                 TK);
    SISA_REQUIRE(a->dtype == SISA_BF16 || a->dtype == SISA_F16, "sisa_lmce_fwd: dtype %d (bf16 or fp16)", a->dtype);
    SISA_REQUIRE(a->x && a->w && a->labels && a->loss_rows && a->workspace && sisa::aligned16(a->x) &&
                     sisa::aligned16(a->w) && a->ldx >= a->D && a->ldw >= a->D && a->ldx % 8 == 0 && a->ldw % 8 == 0,
                 "sisa_lmce_fwd: x, w must be 16-byte aligned with row strides >= D (multiples of 8); labels, "
                 "loss_rows, workspace given");
    // one buffer resource per operand: both extents below 2 GiB
    SISA_REQUIRE(((sisa::cdiv(a->N, TR) * TR - 1) * a->ldx + a->D) * 2 < ((int64_t)1 << 31) &&
                     ((sisa::cdiv(a->Vp, TV) * TV - 1) * a->ldw + a->D) * 2 < ((int64_t)1 << 31),
                 "sisa_lmce_fwd: x or w spans 2 GiB or more");
    hipStream_t st = (hipStream_t)stream;
    return a->dtype == SISA_BF16 ? launch_lmce_fwd<__bf16>(a, st) : launch_lmce_fwd<_Float16>(a, st);
}
