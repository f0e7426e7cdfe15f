// Training pass of the linear cross-entropy for gfx950, on hand-written MFMA kernels only.
//
// Reference: the chunk loop of `_LinearCrossEntropyFn.forward` (src/sisa/kernels/linear_ce.py:138-217): per chunk of
// rows, logits = x W_pad^T (library GEMM), `_lmce_row_kernel` (linear_ce.py:60-96: lse, loss row, and
// G = (softmax - onehot) / N_valid * gscale written over the logits in the compute dtype), then dx = G W_pad and
// dW += G^T x (library GEMMs, fp32 results). The contract (loss rows, fp32 dx and dW of a G rounded once to the
// compute dtype, ignored rows contributing nothing) is the reference's; the arrangement is this library's own:
//
//   1. the logits GEMM of sisa_lmce_fwd (lmce_fwd.hip) with its STORE epilogue: each exponential
//      p~ = exp2(logit * log2e - m_t), m_t the row's maximum over one 128-column half of a 256-column vocabulary
//      tile, goes to a (N, Vp) buffer in the compute dtype and m_t to a (2 * tiles, N) table; the split partials
//      are combined into the loss rows (bitwise those of sisa_lmce_fwd), lse2 = lse / ln 2 and, per row, the scale
//      s_n = inv_n * gscale (0 for ignored rows) with the label (-1 when outside [0, V));
//   2. lmce_scale_kernel turns the m_t table into c = exp2(m_t - lse2) * s_n in place, so that
//      G[n, v] = p~[n, v] * c[n, tile half of v] - s_n [v == label_n], and writes each row's label entry of G;
//   3. one launch of lmce_grad_kernel runs two kinds of output tiles: dW tiles (256 vocabulary x 256 hidden, all
//      rows of the chunk as K) first, then dx tiles (256 rows x 256 hidden, K = a range of the vocabulary: dx is
//      split over the vocabulary so that both kinds of workgroup run about equally long and the last round of the
//      grid is short). Both form G from p~ and c while staging it into LDS (16-byte loads, 8 multiplies, the rare
//      label subtraction, one rounding to the compute dtype, one 16-byte LDS store per 8 values); the dense operand
//      (W_pad rows for dx, x rows for dW) is staged by buffer loads straight into LDS; both are double-buffered;
//   4. lmce_dx_reduce_kernel adds the dx splits in split order.
// G and the logits are never written to memory; the only large buffer is the chunk's exponentials (read once per
// output column tile). Deterministic: no atomics.
//
// Tile arithmetic: a workgroup of 2 x 4 waves, two waves per SIMD (247 VGPRs); a wave owns 128 hidden x 64 rows
// (dx) or 128 hidden x 64 vocabulary (dW) as 8 x 4 blocks of v_mfma_f32_16x16x32 (128 accumulators; all 12 operand
// fragments of a 32-deep step are read before its 32 MFMAs), hidden on the A side so that a lane's 4 results are 4
// consecutive hidden values (16-byte stores). The next stage's exponentials are loaded into registers before a
// stage's MFMAs and formed into G in LDS after them. dx reads W_pad as A with the feature-map transpose read (K = vocabulary, W_pad
// rows) and G as B with direct 16-byte fragment reads (K = vocabulary along G rows); dW reads x and G both with the
// sequence-map transpose read (K = rows). Workgroup i runs on XCD i % 8; each XCD takes consecutive work items, so
// the three hidden tiles that share a G tile run on one L2.
#include "common.h"
#include "host.h"

namespace sisa {
namespace detail {
int64_t lmce_fwd_splits(int64_t N, int64_t Vp);
int lmce_train_forward(const sisa_lmce_fwd_args* a, void* probs, float* mtab, float* lse2, float2* rinfo,
                       const float* inv_n, float gscale, hipStream_t st);
}  // namespace detail
}  // namespace sisa

namespace {

constexpr int NWG = 8;              // waves per workgroup: 2 along the hidden size x 4 along rows / vocabulary
constexpr int TD = 256;             // hidden columns of an output tile
constexpr int TO = 256;             // rows (dx) or vocabulary columns (dW) of an output tile
constexpr int TK = 64;              // K per LDS stage: vocabulary columns (dx) or rows (dW)
constexpr int TV = 256;             // vocabulary tile of the logits pass (two m_t halves of 128 columns)
constexpr int WD = 128, WO = 64;    // wave tile: hidden x rows / vocabulary (two waves per SIMD)
constexpr int IB = WD / 16, JB = WO / 16;
constexpr int GL = TO * TK / 8 / (64 * NWG);   // 16-byte G loads per thread and stage (4)

template <class T>
struct __attribute__((aligned(16))) GradLds {
    T dense[2][TK * TD];            // W_pad rows (dx) or x rows (dW): 64 K-rows x 256 hidden, toff<T, 256>
    T g[2][TO * TK];                // dx: 256 rows x 64 vocabulary (toff<T, 64>); dW: 64 rows x 256 vocabulary
};

struct GradArgs {
    const void* probs;              // (N, Vp) exponentials p~ in the compute dtype, row stride Vp
    const float* cs;                // (2 * tiles, N): c = exp2(m_t - lse2) * s_n
    const float2* rinfo;            // (N,) per row: s_n, and the label (bit pattern of an int; -1 if none)
    const float* glab;              // (N,) per row: G at the label, p~ * c - s_n rounded once to the compute dtype
    const int64_t* labels;
    const void* x;
    const void* w;
    float* dxo;                     // dx partials (dx_splits, N, D) or dx itself (one split)
    float* dw;
    int64_t N, V, Vp, ldx, ldw, lddxo, split_stride, lddw;
    int D, dts;                     // hidden size and its 256-column tiles
    int dx_splits, dx_per;          // vocabulary splits of dx, 64-column stages per split
    int n_dw, n_dw_pad, n_dx;       // dW items (blocks padded to a multiple of 8), dx items
    int accumulate;
};

// Work item of block i of a part of n items laid over 8 * ceil(n / 8) blocks (block i runs on XCD i % 8): XCD x
// takes a contiguous range of items. -1 for a spare block.
SISA_DEV int xcd_item(int i, int n) {
    const int x = i & 7, k = i >> 3, q = n >> 3, r = n & 7;
    if (k >= q + (x < r ? 1 : 0)) return -1;
    return x * q + (x < r ? x : r) + k;
}

SISA_DEV int64_t clamp_bytes(int64_t b) {
    return b < 0 ? 0 : (b > (int64_t)0x7ffffff0 ? (int64_t)0x7ffffff0 : b);
}

// G for 8 consecutive vocabulary columns of one row: p~ * c rounded once to T, stored as one 16-byte chunk; when the
// row's label lies in these columns (rel in [0, 8), rare) that element is replaced by the row's precomputed label
// entry gl = p~ * c - s_n, rounded once (a 2-byte store after the 16-byte one, by the same thread, so it lands last).
template <class T>
SISA_DEV void g_store(T* dst, const frag8<T>& raw, float c, int rel, float gl) {
    f32x8 e = __builtin_convertvector(raw, f32x8);
#pragma unroll
    for (int j = 0; j < 8; ++j) e[j] *= c;
    *reinterpret_cast<frag8<T>*>(dst) = __builtin_convertvector(e, frag8<T>);
    if ((unsigned)rel < 8u) dst[rel] = cvt<T>(gl);
}

template <class T>
SISA_DEV frag8<T> load16(__amdgpu_buffer_rsrc_t r, int voff) {
    return __builtin_bit_cast(frag8<T>, __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, 0));
}

// One output tile: DW (dW tile u = vocabulary tile * dts + hidden tile) or dx (u = (row block * dx_splits + split)
// * dts + hidden tile).
template <class T, bool DW>
SISA_DEV void grad_tile(const GradArgs& a, GradLds<T>& sm, int u) {
    const int tid = threadIdx.x, lane = tid & 63, grp = lane >> 4, lc = lane & 15;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t N = a.N, Vp = a.Vp;
    const int dt = u % a.dts, rest = u / a.dts;
    const int d0 = dt * TD;
    // DW: vocabulary tile vt, K = all rows; dx: row block rb, K = vocabulary stages [k0, k0 + total) of split sp
    const int vt = rest, sp = rest % a.dx_splits, rb = rest / a.dx_splits;
    const int64_t n0 = DW ? 0 : (int64_t)rb * TO;
    const int k0 = DW ? 0 : sp * a.dx_per;
    const int kstages = DW ? (int)((N + TK - 1) / TK) : (int)(Vp / TK);
    const int k1 = DW ? kstages : (k0 + a.dx_per < kstages ? k0 + a.dx_per : kstages);
    const int total = k1 > k0 ? k1 - k0 : 0;
    const int wd = WD * (w & 1), wo = WO * (w >> 1);

    // dense operand: 64 K-rows x 256 hidden columns straight into LDS (rows past the data read as zero)
    DmaStage<T, TD, NWG> dma;
    const T* dsrc = DW ? (const T*)a.x + d0 : (const T*)a.w + d0;
    const int64_t dld = DW ? a.ldx : a.ldw;
    const int64_t drows = DW ? N : Vp;
    const int64_t dbytes = ((drows - 1) * dld + a.D - d0) * (int64_t)sizeof(T);
    dma.init(dld, w, lane);

    // G staging: thread tid handles GL 16-byte chunks per stage
    //   dx: rows rr[p] = tid / 8 + 32 p of the row block, vocabulary columns 8 (tid % 8) of the stage
    //   dW: rows rr[p] = tid / 32 + 8 p of the stage, vocabulary columns 8 (tid % 32) of the tile
    constexpr int RSTEP = 64 * NWG / (DW ? 32 : 8);
    const int gc = DW ? (tid & 31) : (tid & 7);
    int rr[GL];
#pragma unroll
    for (int p = 0; p < GL; ++p) rr[p] = (DW ? (tid >> 5) : (tid >> 3)) + RSTEP * p;
    const T* P = (const T*)a.probs;
    // dx: the rows are fixed for the whole tile -- labels and row scales once
    int lab[GL];
    float gl[GL];                   // G at the row's label (already rounded once to T), converted when stored
    if constexpr (!DW) {
#pragma unroll
        for (int p = 0; p < GL; ++p) {
            const int64_t n = n0 + rr[p] < N ? n0 + rr[p] : N - 1;   // rows past N: G is 0 (their p~ read as 0)
            lab[p] = n0 + rr[p] < N ? __float_as_int(a.rinfo[n].y) : -1;
            gl[p] = a.glab[n];
        }
    }
    frag8<T> raw[GL];
    float cv[GL];
    auto load_g = [&](int g) {   // stage g of the tile into registers (exponentials, c, and for dW labels)
        if constexpr (DW) {
            const int64_t m0 = (int64_t)(k0 + g) * TK;
            const __amdgpu_buffer_rsrc_t rs = make_rsrc(P + m0 * Vp, clamp_bytes((N - m0) * Vp * (int64_t)sizeof(T)));
            const int h = gc >= 16;
#pragma unroll
            for (int p = 0; p < GL; ++p) {
                raw[p] = load16<T>(rs, (int)((rr[p] * Vp + (int64_t)vt * TV + 8 * gc) * (int64_t)sizeof(T)));
                const int64_t n = m0 + rr[p] < N ? m0 + rr[p] : N - 1;   // rows past N: their p~ read as 0
                cv[p] = a.cs[(int64_t)(2 * vt + h) * N + n];
                lab[p] = m0 + rr[p] < N ? __float_as_int(a.rinfo[n].y) : -1;
                gl[p] = a.glab[n];
            }
        } else {
            const int64_t v0 = (int64_t)(k0 + g) * TK;
            const __amdgpu_buffer_rsrc_t rs = make_rsrc(P + n0 * Vp, clamp_bytes((N - n0) * Vp * (int64_t)sizeof(T)));
            const int64_t ci = 2 * (v0 / TV) + ((v0 % TV) >= TV / 2);
#pragma unroll
            for (int p = 0; p < GL; ++p) {
                raw[p] = load16<T>(rs, (int)((rr[p] * Vp + v0 + 8 * gc) * (int64_t)sizeof(T)));
                const int64_t n = n0 + rr[p] < N ? n0 + rr[p] : N - 1;   // rows past N: their p~ read as 0
                cv[p] = a.cs[ci * N + n];
            }
        }
    };
    auto store_g = [&](int g, int buf) {
        if constexpr (DW) {
            const int vc = vt * TV + 8 * gc;
#pragma unroll
            for (int p = 0; p < GL; ++p)
                g_store<T>(sm.g[buf] + toff<T, TO>(rr[p], gc), raw[p], cv[p], lab[p] < 0 ? -1 : lab[p] - vc, gl[p]);
        } else {
            const int vc = (k0 + g) * TK + 8 * gc;
#pragma unroll
            for (int p = 0; p < GL; ++p)
                g_store<T>(sm.g[buf] + toff<T, TK>(rr[p], gc), raw[p], cv[p], lab[p] < 0 ? -1 : lab[p] - vc, gl[p]);
        }
    };
    auto issue_dense = [&](int g, int buf) {
        const int64_t k = (int64_t)(k0 + g) * TK;
        if constexpr (DW) dma_issue<7>(dma, dsrc, dbytes, (int)(k * dld * (int64_t)sizeof(T)), sm.dense[buf], w);
        else dma_issue<6>(dma, dsrc, dbytes, (int)(k * dld * (int64_t)sizeof(T)), sm.dense[buf], w);
    };

    f32x4 acc[IB][JB];
#pragma unroll
    for (int i = 0; i < IB; ++i)
#pragma unroll
        for (int j = 0; j < JB; ++j) acc[i][j] = zero4();

    if (total > 0) {
        issue_dense(0, 0);
        load_g(0);
        store_g(0, 0);
    }
    __syncthreads();
    for (int g = 0; g < total; ++g) {
        const int buf = g & 1;
        if (g + 1 < total) {   // G loads first: a wait for them then never covers the younger DMA
            load_g(g + 1);
            issue_dense(g + 1, buf ^ 1);
        }
        // the next stage's loads all go out before this stage's MFMAs, and its G is formed after them
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int step = 0; step < TK / 32; ++step) {
            // all 12 operand fragments of the 32-deep step are read before its 32 MFMAs: one LDS wait per step
            frag8<T> af[IB], bf[JB];
#pragma unroll
            for (int i = 0; i < IB; ++i)
                af[i] = DW ? frag_tr<T, TD>(sm.dense[buf], wd + 16 * i, step, lane)
                           : frag_trf<T, TD>(sm.dense[buf], wd + 16 * i, step, lane);
#pragma unroll
            for (int j = 0; j < JB; ++j)
                bf[j] = DW ? frag_tr<T, TO>(sm.g[buf], wo + 16 * j, step, lane)
                           : frag_rows<T, TK>(sm.g[buf], wo + 16 * j, step, lane);
#pragma unroll
            for (int i = 0; i < IB; ++i)
#pragma unroll
                for (int j = 0; j < JB; ++j) acc[i][j] = mma(af[i], bf[j], acc[i][j]);
        }
        __builtin_amdgcn_sched_barrier(0);
        if (g + 1 < total) store_g(g + 1, buf ^ 1);
        __syncthreads();
    }

    // lane l, register r of block (i, j): hidden d0 + wd + 16 i + 4 (l / 16) + r, row / vocabulary wo + 16 j + l % 16
    if constexpr (DW) {
        if (a.accumulate) {   // all of the lane's earlier partial sums in flight at once, then the sums
#pragma unroll
            for (int j = 0; j < JB; ++j) {
                const int64_t o = (int64_t)vt * TO + wo + 16 * j + lc;
#pragma unroll
                for (int i = 0; i < IB; ++i) {
                    const int d = d0 + wd + 16 * i + 4 * grp;
                    if (o < Vp && d < a.D) acc[i][j] += *reinterpret_cast<const f32x4*>(a.dw + o * a.lddw + d);
                }
            }
        }
    }
#pragma unroll
    for (int j = 0; j < JB; ++j) {
        const int64_t o = (DW ? (int64_t)vt * TO : n0) + wo + 16 * j + lc;
        if (o >= (DW ? Vp : N)) continue;
#pragma unroll
        for (int i = 0; i < IB; ++i) {
            const int d = d0 + wd + 16 * i + 4 * grp;
            if (d >= a.D) continue;
            if constexpr (DW) *reinterpret_cast<f32x4*>(a.dw + o * a.lddw + d) = acc[i][j];
            else *reinterpret_cast<f32x4*>(a.dxo + (int64_t)sp * a.split_stride + o * a.lddxo + d) = acc[i][j];
        }
    }
}

template <class T>
__global__ __launch_bounds__(64 * NWG) void lmce_grad_kernel(GradArgs a) {
    __shared__ GradLds<T> sm;
    const int i = blockIdx.x;
    if (i < a.n_dw_pad) {
        const int u = xcd_item(i, a.n_dw);
        if (u >= 0) grad_tile<T, true>(a, sm, u);
    } else {
        const int u = xcd_item(i - a.n_dw_pad, a.n_dx);
        if (u >= 0) grad_tile<T, false>(a, sm, u);
    }
}

// c[k, n] = exp2(m_t[k, n] - lse2[n]) * s_n, in place over the (2 * tiles, N) table
// c[k, n] = exp2(m_t[k, n] - lse2[n]) * s_n, in place over the (2 * tiles, N) table; the entry k that holds the
// row's label also writes G at the label, p~ * c - s_n, rounded once to T (glab, kept in fp32)
template <class T>
__global__ __launch_bounds__(256) void lmce_scale_kernel(float* cs, const float* lse2, const float2* rinfo,
                                                         const T* probs, int64_t Vp, float* glab, int64_t N) {
    const int64_t n = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (n >= N) return;
    const int k = blockIdx.y;
    float* p = cs + (int64_t)k * N + n;
    const float2 ri = rinfo[n];
    const float c = fast_exp2(*p - lse2[n]) * ri.x;
    *p = c;
    const int lab = __float_as_int(ri.y);
    if (lab >= 0 && 2 * (lab / TV) + ((lab % TV) >= TV / 2) == k)
        glab[n] = (float)cvt<T>(fmaf((float)probs[n * Vp + lab], c, -ri.x));
}

// dx[n, :] = sum over the splits, in split order, of the partial rows
__global__ __launch_bounds__(256) void lmce_dx_reduce_kernel(const float* part, float* dx, int64_t N, int D, int S,
                                                             int64_t lddx) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int q = D / 4;
    if (idx >= N * q) return;
    const int64_t n = idx / q, d = 4 * (idx % q);
    f32x4 s = lds4f(part + n * D + d);
    for (int sp = 1; sp < S; ++sp) s += lds4f(part + ((int64_t)sp * N + n) * D + d);
    *reinterpret_cast<f32x4*>(dx + n * lddx + d) = s;
}

struct Layout {
    int64_t probs, cs, part, lse2, srow, glab, dxp, total;
};

int64_t align256(int64_t b) { return (b + 255) / 256 * 256; }

int default_dx_splits(int64_t N, int64_t Vp) {
    // dx workgroups about as long as dW workgroups (whose K is all N rows)
    const int64_t sv = Vp / TK, sn = sisa::cdiv(N, TK);
    int64_t s = (sv + sn / 2) / (sn > 0 ? sn : 1);
    return (int)(s < 1 ? 1 : (s > 16 ? 16 : s));
}

Layout layout(int64_t N, int64_t Vp, int D, int dx_splits) {
    Layout l{};
    const int64_t tiles = sisa::cdiv(Vp, TV);
    l.probs = 0;
    l.cs = align256(N * Vp * 2);
    l.part = l.cs + align256(2 * tiles * N * 4);
    l.lse2 = l.part + align256((2 * sisa::detail::lmce_fwd_splits(N, Vp) + 1) * N * 4);
    l.srow = l.lse2 + align256(N * 4);
    l.glab = l.srow + align256(N * 8);
    l.dxp = l.glab + align256(N * 4);
    l.total = l.dxp + (dx_splits > 1 ? align256((int64_t)dx_splits * N * D * 4) : 0);
    return l;
}

}  // namespace

extern "C" int64_t sisa_lmce_train_workspace_bytes(int64_t N, int64_t Vp, int32_t D, int32_t dx_splits) {
    if (N < 1 || Vp < 1 || D < 1) return 0;
    const int s = dx_splits > 0 ? dx_splits : default_dx_splits(N, Vp);
    return layout(N, Vp, D, s).total;
}

extern "C" int sisa_lmce_train(const sisa_lmce_train_args* a, void* stream) {
    SISA_REQUIRE(a != nullptr, "sisa_lmce_train: null args");
    if (a->N == 0) return SISA_OK;
    SISA_REQUIRE(a->N >= 1 && a->V >= 1 && a->Vp >= a->V && a->Vp % 128 == 0,
                 "sisa_lmce_train: bad shape N=%lld V=%lld Vp=%lld (Vp >= V, a multiple of 128)", (long long)a->N,
                 (long long)a->V, (long long)a->Vp);
    SISA_REQUIRE(a->D >= 64 && a->D % 64 == 0, "sisa_lmce_train: hidden size %d must be a positive multiple of 64",
                 a->D);
    SISA_REQUIRE(a->dtype == SISA_BF16 || a->dtype == SISA_F16, "sisa_lmce_train: dtype %d (bf16 or fp16)",
                 a->dtype);
    SISA_REQUIRE(a->x && a->w && a->labels && a->loss_rows && a->inv_n && a->workspace && sisa::aligned16(a->x) &&
                     sisa::aligned16(a->w) && ((uintptr_t)a->workspace & 255) == 0 && a->ldx >= a->D &&
                     a->ldw >= a->D && a->ldx % 8 == 0 && a->ldw % 8 == 0,
                 "sisa_lmce_train: x, w 16-byte aligned with row strides >= D (multiples of 8); labels, loss_rows, "
                 "inv_n and a 256-byte aligned workspace given");
    SISA_REQUIRE(a->dx == nullptr || (sisa::aligned16(a->dx) && a->lddx >= a->D && a->lddx % 4 == 0),
                 "sisa_lmce_train: dx 16-byte aligned with row stride >= D (multiple of 4)");
    SISA_REQUIRE(a->dw == nullptr || (sisa::aligned16(a->dw) && a->lddw >= a->D && a->lddw % 4 == 0),
                 "sisa_lmce_train: dw 16-byte aligned with row stride >= D (multiple of 4)");
    SISA_REQUIRE(a->dx_splits >= 0 && a->dx_splits <= 16, "sisa_lmce_train: dx_splits %d (0..16)", a->dx_splits);
    // one buffer resource per dense operand: extents below 2 GiB
    SISA_REQUIRE(((sisa::cdiv(a->N, 256) * 256 - 1) * a->ldx + a->D) * 2 < ((int64_t)1 << 31) &&
                     ((sisa::cdiv(a->Vp, 256) * 256 - 1) * a->ldw + a->D) * 2 < ((int64_t)1 << 31),
                 "sisa_lmce_train: x or w spans 2 GiB or more");
    hipStream_t st = (hipStream_t)stream;
    const int S = a->dx_splits > 0 ? a->dx_splits : default_dx_splits(a->N, a->Vp);
    const Layout l = layout(a->N, a->Vp, a->D, S);
    char* ws = (char*)a->workspace;
    float* cs = (float*)(ws + l.cs);
    float* lse2 = (float*)(ws + l.lse2);
    float2* rinfo = (float2*)(ws + l.srow);
    float* glab = (float*)(ws + l.glab);
    sisa_lmce_fwd_args f{a->N, a->V, a->Vp, a->D, a->dtype, a->x, a->ldx, a->w, a->ldw, a->labels, a->ignore_index,
                         a->lse, a->loss_rows, (float*)(ws + l.part)};
    int rc = sisa::detail::lmce_train_forward(&f, ws + l.probs, cs, lse2, rinfo, a->inv_n, a->gscale, st);
    if (rc || (a->dx == nullptr && a->dw == nullptr)) return rc;

    const int64_t tiles = sisa::cdiv(a->Vp, TV);
    const dim3 sgrid((unsigned)sisa::cdiv(a->N, 256), (unsigned)(2 * tiles));
    if (a->dtype == SISA_BF16)
        lmce_scale_kernel<__bf16><<<sgrid, 256, 0, st>>>(cs, lse2, rinfo, (const __bf16*)(ws + l.probs), a->Vp, glab, a->N);
    else
        lmce_scale_kernel<_Float16><<<sgrid, 256, 0, st>>>(cs, lse2, rinfo, (const _Float16*)(ws + l.probs), a->Vp, glab,
                                                           a->N);
    rc = sisa::launch_status("sisa_lmce_train (scale)");
    if (rc) return rc;

    GradArgs g{};
    g.probs = ws + l.probs;
    g.cs = cs;
    g.rinfo = rinfo;
    g.glab = glab;
    g.labels = a->labels;
    g.x = a->x;
    g.w = a->w;
    g.N = a->N;
    g.V = a->V;
    g.Vp = a->Vp;
    g.ldx = a->ldx;
    g.ldw = a->ldw;
    g.D = a->D;
    g.dts = (int)sisa::cdiv(a->D, TD);
    g.dx_splits = S;
    g.dx_per = (int)sisa::cdiv(a->Vp / TK, S);
    g.n_dw = a->dw ? (int)(tiles * g.dts) : 0;
    g.n_dw_pad = (int)(sisa::cdiv(g.n_dw, 8) * 8);
    g.n_dx = a->dx ? (int)(sisa::cdiv(a->N, TO) * S * g.dts) : 0;
    g.dw = a->dw;
    g.lddw = a->lddw;
    g.accumulate = a->dw_accumulate != 0;
    if (S > 1) {
        g.dxo = (float*)(ws + l.dxp);
        g.lddxo = a->D;
        g.split_stride = a->N * a->D;
    } else {
        g.dxo = a->dx;
        g.lddxo = a->lddx;
        g.split_stride = 0;
    }
    const unsigned grid = (unsigned)(g.n_dw_pad + sisa::cdiv(g.n_dx, 8) * 8);
    if (a->dtype == SISA_BF16) lmce_grad_kernel<__bf16><<<grid, 64 * NWG, 0, st>>>(g);
    else lmce_grad_kernel<_Float16><<<grid, 64 * NWG, 0, st>>>(g);
    rc = sisa::launch_status("sisa_lmce_train (gradients)");
    if (rc || a->dx == nullptr || S == 1) return rc;
    lmce_dx_reduce_kernel<<<(unsigned)sisa::cdiv(a->N * (a->D / 4), 256), 256, 0, st>>>(g.dxo, a->dx, a->N, a->D, S,
                                                                                       a->lddx);
    return sisa::launch_status("sisa_lmce_train (dx splits)");
}
