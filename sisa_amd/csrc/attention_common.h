// Definitions shared by the SISA attention translation units: attention.hip (decay factors, forward, dlambda and the
// C entry points), attention_dq.hip and attention_bwd.hip (the dq and the dkv kernel of the exact-delta backward,
// each compiled with a scheduler of its own). Reference: src/sisa/kernels/attention.py.
#pragma once
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
// dkv kernel: 4 waves x 16 rows = one 64-row decay block per workgroup, so that every tile before the block is an
// off-block tile for all waves and the block's own tile comes last (two code regions with small register sets; three
// workgroups per CU). The dq kernel uses the forward's 8-wave workgroups (two decay blocks).
constexpr int NWB = 4;
constexpr int NTHB = 64 * NWB;

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

constexpr float QSCALE = 0.125f;   // 1/sqrt(DH), exact in every input type
template <class T> struct FoldC { static constexpr bool on = sizeof(T) != 2 || __is_same(T, __bf16); };
template <class T> struct SplitC { static constexpr bool on = __is_same(T, __bf16); };
template <class T> struct Anchor { static constexpr bool on = sizeof(T) == 2; };


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

// Row buffers handed from the dq kernel to the dkv kernel (workspace, each (B,H,L) fp32), followed by the fp64 sums
// of the per-row dlambda parts over each 16-row group of queries, (B*H, ceil(L/16)), written by the dq kernel's waves
// and added up per head by one dkv workgroup.
enum { WS_DELTA = 0, WS_DDEL, WS_DSD, WS_RG, WS_RF, WS_N };
__host__ __device__ inline double* ws_block_dlam(void* ws, int64_t BHL) {
    return reinterpret_cast<double*>(static_cast<float*>(ws) + WS_N * BHL + (BHL & 1));   // 8-byte aligned
}

}  // namespace

namespace sisa {
namespace detail {
// The dq and dkv launches of sisa_attn_bwd (attention_bwd.hip), after the entry point's checks; 0 or an error code.
__attribute__((visibility("hidden"))) int attn_bwd_dq_dkv(const sisa_attn_bwd_args* a, hipStream_t st);
// The dq launch alone (attention_dq.hip).
__attribute__((visibility("hidden"))) int attn_bwd_dq(const sisa_attn_bwd_args* a, hipStream_t st);
}  // namespace detail
}  // namespace sisa
