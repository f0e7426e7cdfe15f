// Weight-gradient GEMM for gfx950: C[N x K] (fp32) = A^T B, with A (M x N) and B (M x K) row-major 16-bit matrices
// and M the long dimension (the tokens of a batch). This is dW = dY^T X of a linear layer y = x W^T, the product the
// libraries run slowest in the decoder training step (small outputs, M = B*T = 16,384 reduction): 240-690 TFLOP/s
// for the W_cat, W_O, gate/up and down projections of sisa-152m.
//
// Reference: the weight gradients autograd computes for the nn.Linear layers of src/sisa/modeling.py:79-291 (bf16
// products under autocast, rounded to bf16 and cast to the fp32 parameter's dtype); here the result is written in
// fp32 directly (no bf16 rounding of dW, no cast pass).
//
// Decomposition: a workgroup of 4 waves (2 x 2) computes a 128 x 128 output tile over a range of M (split-K; the
// partial tiles are summed in split order by a second launch, so results are bitwise reproducible). A wave owns 64 x
// 64 outputs as 4 x 4 blocks of v_mfma_f32_16x16x32_bf16. Both operands are staged as 32- or 64-row tiles (rows = M)
// straight from global memory into LDS (buffer loads with the LDS destination, double-buffered, 16-byte chunks
// XOR-swizzled per row) and read as MFMA fragments with the LDS transpose read (8 consecutive M of one column per
// lane), the same sequence map for both operands. Workgroup i runs on XCD i % 8; split = i % nsplit (a power of two)
// keeps each XCD on one split, whose rows of A and B its L2 then serves to all the split's tiles.
#include "common.h"
#include "host.h"

namespace {

constexpr int NW = 4;               // waves per workgroup (2 x 2)
constexpr int BN = 128, BK = 128;   // workgroup output tile
constexpr int WTN = 64, WTK = 64;   // wave quarter

// Staging of a TM-row tile of C 16-bit columns straight into LDS: wave instruction k fills tile bytes
// [1024 k, 1024 k + 1024), lane i the 16-byte chunk 64 k + i; the per-lane offsets are fixed, the tile's first row
// enters as the scalar offset.
template <class T, int C, int TM>
struct Stage {
    static constexpr int CPR = C * (int)sizeof(T) / 16;
    static constexpr int INSTR = TM * CPR / 64;
    static constexpr int PER = (INSTR + NW - 1) / NW;
    int voff[PER];

    SISA_DEV void init(int64_t srow, int w, int lane) {
#pragma unroll
        for (int p = 0; p < PER; ++p) {
            const int ci = 64 * (w + NW * p) + lane;
            const int row = ci / CPR, phys = ci % CPR;
            voff[p] = (int)(row * srow * (int64_t)sizeof(T) + 16 * (phys ^ swz<T, C>(row)));
        }
    }
};

// ID: one specialization per kernel instantiation (see dma_issue in common.h)
template <int ID, class T, int C, int TM>
SISA_DEV void stage_issue(const Stage<T, C, TM>& st, const void* base, int64_t bytes, int soff, T* X, int w) {
    const __amdgpu_buffer_rsrc_t r = make_rsrc(base, bytes);
#pragma unroll
    for (int p = 0; p < Stage<T, C, TM>::PER; ++p) {
        const int k = w + NW * p;
        if (k < Stage<T, C, TM>::INSTR)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                r, (__attribute__((address_space(3))) void*)(X + k * (1024 / (int)sizeof(T))), 16, st.voff[p], soff, 0,
                0);
    }
}

template <class T, int TM>
struct __attribute__((aligned(16))) WgLds {
    T a[2][TM * BN];
    T b[2][TM * BK];
};

// TM: M rows per LDS tile (32: more workgroups per CU; 64: fewer barriers, for grids of few tiles)
template <class T, int TM>
__global__ __launch_bounds__(64 * NW) void wgrad_kernel(sisa_wgrad_args g) {
    __shared__ WgLds<T, TM> sm;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int split = blockIdx.x % g.nsplit;           // workgroup i runs on XCD i % 8: one split per XCD
    const int tile = blockIdx.x / g.nsplit;
    const int tiles_k = (g.K + BK - 1) / BK;
    const int n0 = (tile / tiles_k) * BN, k0 = (tile % tiles_k) * BK;
    const int64_t m_begin = (int64_t)split * g.m_per_split;
    const int64_t m_end = m_begin + g.m_per_split < g.M ? m_begin + g.m_per_split : g.M;
    const int ntiles = m_end > m_begin ? (int)((m_end - m_begin + TM - 1) / TM) : 0;

    Stage<T, BN, TM> sa;
    Stage<T, BK, TM> sb;
    sa.init(g.lda, w, lane);
    sb.init(g.ldb, w, lane);
    const T* A = (const T*)g.a + n0;
    const T* B = (const T*)g.b + k0;
    // extents end at the last element of row M-1: columns past N (K) of that row read as zero, never past the data;
    // rows at or beyond M read as zero
    const int64_t abytes = ((g.M - 1) * g.lda + g.N - n0) * (int64_t)sizeof(T);
    const int64_t bbytes = ((g.M - 1) * g.ldb + g.K - k0) * (int64_t)sizeof(T);
    auto issue = [&](int t, int buf) {
        const int64_t row0 = m_begin + (int64_t)t * TM;
        stage_issue<2 * TM + 0>(sa, A, abytes, (int)(row0 * g.lda * (int64_t)sizeof(T)), sm.a[buf], w);
        stage_issue<2 * TM + 1>(sb, B, bbytes, (int)(row0 * g.ldb * (int64_t)sizeof(T)), sm.b[buf], w);
    };

    const int wn = WTN * (w >> 1), wk = WTK * (w & 1);
    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = zero4();

    if (ntiles > 0) issue(0, 0);
    __syncthreads();
    for (int t = 0; t < ntiles; ++t) {
        const int buf = t & 1;
        if (t + 1 < ntiles) issue(t + 1, buf ^ 1);
#pragma unroll
        for (int step = 0; step < TM / 32; ++step) {
            frag8<T> af[4], bf[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) af[i] = frag_tr<T, BN>(sm.a[buf], wn + 16 * i, step, lane);
#pragma unroll
            for (int j = 0; j < 4; ++j) bf[j] = frag_tr<T, BK>(sm.b[buf], wk + 16 * j, step, lane);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = mma(af[i], bf[j], acc[i][j]);
        }
        __syncthreads();
    }

    // D layout: lane l, register r -> row 4 (l / 16) + r of the block (n), column l % 16 (k)
    float* out = g.nsplit > 1 ? g.workspace + (int64_t)split * g.N * g.K : g.c;
    const int64_t ldo = g.nsplit > 1 ? g.K : g.ldc;
    const int grp = lane >> 4, col = lane & 15;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int kk = k0 + wk + 16 * j + col;
            if (kk >= g.K) continue;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int nn = n0 + wn + 16 * i + 4 * grp + r;
                if (nn < g.N) out[(int64_t)nn * ldo + kk] = acc[i][j][r];
            }
        }
}

// C[n][k] = sum over the splits in order of the partial tiles
__global__ __launch_bounds__(256) void wgrad_reduce_kernel(sisa_wgrad_args g) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t nk = (int64_t)g.N * g.K;
    if (idx >= nk) return;
    float s = 0.f;
    constexpr int BATCH = 8;
    int sp = 0;
    for (; sp + BATCH <= g.nsplit; sp += BATCH) {
        float t[BATCH];
#pragma unroll
        for (int e = 0; e < BATCH; ++e) t[e] = __builtin_nontemporal_load(g.workspace + (int64_t)(sp + e) * nk + idx);
#pragma unroll
        for (int e = 0; e < BATCH; ++e) s += t[e];
    }
    for (; sp < g.nsplit; ++sp) s += g.workspace[(int64_t)sp * nk + idx];
    const int64_t n = idx / g.K, k = idx % g.K;
    g.c[n * g.ldc + k] = s;
}

template <class T>
int launch_wgrad(const sisa_wgrad_args* g, hipStream_t st) {
    const int tiles = (int)(sisa::cdiv(g->N, BN) * sisa::cdiv(g->K, BK));
    const unsigned grid = (unsigned)(tiles * g->nsplit);
    if (tiles < 64) wgrad_kernel<T, 64><<<grid, 64 * NW, 0, st>>>(*g);
    else wgrad_kernel<T, 32><<<grid, 64 * NW, 0, st>>>(*g);
    int rc = sisa::launch_status("sisa_wgrad");
    if (rc || g->nsplit == 1) return rc;
    wgrad_reduce_kernel<<<(unsigned)sisa::cdiv((int64_t)g->N * g->K, 256), 256, 0, st>>>(*g);
    return sisa::launch_status("sisa_wgrad (split reduction)");
}

}  // namespace

extern "C" int32_t sisa_wgrad_splits(int64_t M, int32_t N, int32_t K) {
    // the smallest power of two up to 8 (it divides the 8 XCDs: one split per XCD) that gives about two workgroups
    // per CU, each split at least 1024 rows
    const int64_t tiles = sisa::cdiv(N, BN) * sisa::cdiv(K, BK);
    int64_t s = 1;
    while (s < 8 && tiles * s < 500 && M / (s * 2) >= 1024) s *= 2;
    return (int32_t)s;
}

extern "C" int64_t sisa_wgrad_workspace_bytes(int64_t M, int32_t N, int32_t K, int32_t nsplit) {
    return nsplit > 1 ? (int64_t)nsplit * N * K * (int64_t)sizeof(float) : 0;
}

extern "C" int sisa_wgrad(const sisa_wgrad_args* g, void* stream) {
    SISA_REQUIRE(g != nullptr, "sisa_wgrad: null args");
    SISA_REQUIRE(g->M >= 1 && g->N >= 1 && g->K >= 1, "sisa_wgrad: bad shape M=%lld N=%d K=%d", (long long)g->M, g->N,
                 g->K);
    SISA_REQUIRE(g->dtype == SISA_BF16 || g->dtype == SISA_F16, "sisa_wgrad: dtype %d (bf16 or fp16 operands)",
                 g->dtype);
    SISA_REQUIRE(g->a && g->b && g->c && sisa::aligned16(g->a) && sisa::aligned16(g->b),
                 "sisa_wgrad: a, b must be 16-byte aligned and c given");
    SISA_REQUIRE(g->lda >= g->N && g->ldb >= g->K && g->lda % 8 == 0 && g->ldb % 8 == 0 && g->ldc >= g->K,
                 "sisa_wgrad: row strides lda >= N, ldb >= K (multiples of 8), ldc >= K");
    SISA_REQUIRE(g->M * g->lda * 2 < ((int64_t)1 << 31) && g->M * g->ldb * 2 < ((int64_t)1 << 31),
                 "sisa_wgrad: operands must be below 2 GiB");
    SISA_REQUIRE(g->nsplit >= 1 && g->nsplit <= 64 && g->m_per_split >= 1 &&
                     (int64_t)g->nsplit * g->m_per_split >= g->M && g->m_per_split % 64 == 0,
                 "sisa_wgrad: nsplit in [1, 64] and m_per_split (a multiple of 64) covering M");
    SISA_REQUIRE(g->nsplit == 1 || (g->workspace && sisa::aligned16(g->workspace)),
                 "sisa_wgrad: split-K needs a workspace of sisa_wgrad_workspace_bytes");
    hipStream_t st = (hipStream_t)stream;
    return g->dtype == SISA_BF16 ? launch_wgrad<__bf16>(g, st) : launch_wgrad<_Float16>(g, st);
}
