// SISA decode attention for gfx950: a few new query rows (decode steps) against a long key cache, split over the keys
// (flash-decoding) with a deterministic combine.
//
//   s_mj = q_m.k_j / 8 + lam * exp(g_m - g_j) * (c_m.b_j) + (F_m - F_j),   j <= q_start + m
//   out_m = softmax_j(s_mj) v_j                                              (fp32)
//
// Reference: `_attend_rows` (src/sisa/functional.py:69-93) as called by `SISAAttention._forward_cached`
// (src/sisa/modeling.py:224-238): the exact score in float32, the decay exponent of masked keys set to 0 before the
// exponential, softmax over the valid keys. The reference materialises the (M, N) score matrix with torch GEMMs; here
// the cache is read once: the work is memory-bound (328 bytes per cached bf16 key and head: k, v, b~, g, F).
//
// Work decomposition: one workgroup of 4 waves per (query row, chunk of 256 keys); each wave owns 64 keys. Within a
// wave, 8 consecutive lanes share a key: lane (slot kq, group fg) reads features 8 fg .. 8 fg + 7 of the k, v (and b~)
// rows of keys kq + 8 i, i < 8, so every load instruction covers whole 128-byte rows. The lane's partial score is
// summed over the 8 lanes of its key; the weighted sum of V over the key slots. Each workgroup writes its chunk's
// (max, sum, unnormalised output) in fixed wave order; a second kernel combines the chunks of a row in chunk order.
// No atomics: bitwise reproducible.
#include "common.h"
#include "host.h"

namespace {

constexpr int DH = 64, DS = 32;
constexpr int DW = 4;                 // waves per workgroup
constexpr int KCH = 64 * DW;          // keys per chunk (workgroup)
constexpr int PART = DH + 2;          // chunk partial: max, sum, out[64]

SISA_DEV float wave_max(float x) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
    return x;
}

SISA_DEV float wave_sum(float x) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
    return x;
}

// Occupancy hint 3 (the 132 registers allow three waves per SIMD either way): the schedule made for that register
// target runs the config-4 decode step 2-4 % faster than the one made without the hint; forcing four waves (128
// registers) makes it 15 % slower.
template <class T>
__global__ __launch_bounds__(64 * DW) __attribute__((amdgpu_waves_per_eu(3)))
void decode_chunk_kernel(sisa_decode_args a) {
    __shared__ float wm[DW], wl[DW], wo[DW][DH];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int fg = lane & 7, kq = lane >> 3;           // feature group (8 features), key slot within a group of 8
    const int chunk = blockIdx.x;
    const int row = blockIdx.y;                        // (b, h, m) flattened
    const int M = a.M, H = a.H;
    const int m = row % M, bh = row / M, h = bh % H, b = bh / H;
    const T* Q = (const T*)a.q.ptr + (int64_t)b * a.q.sb + (int64_t)h * a.q.sh + (int64_t)m * a.q.sl;
    const T* C = (const T*)a.c.ptr + (int64_t)b * a.c.sb + (int64_t)h * a.c.sh + (int64_t)m * a.c.sl;
    const float gq = ((const float*)a.gq.ptr)[(int64_t)b * a.gq.sb + (int64_t)h * a.gq.sh + (int64_t)m * a.gq.sl];
    const bool has_f = a.fq.ptr != nullptr;
    const float fq =
        has_f ? ((const float*)a.fq.ptr)[(int64_t)b * a.fq.sb + (int64_t)h * a.fq.sh + (int64_t)m * a.fq.sl] : 0.f;
    const float lam = a.lam[(int64_t)h * a.s_lam];
    const int last = a.q_start + m;                    // the row's last visible key
    const int jw = chunk * KCH + w * 64;               // the wave's first key
    const T* kbase = (const T*)a.k.ptr + (int64_t)b * a.k.sb + (int64_t)h * a.k.sh;
    const T* bbase = (const T*)a.b.ptr + (int64_t)b * a.b.sb + (int64_t)h * a.b.sh;
    const T* vbase = (const T*)a.v.ptr + (int64_t)b * a.v.sb + (int64_t)h * a.v.sh;

    // Row loads first (all independent): the lane's 8 features of k and v (and of b~ for fg < 4) for the keys
    // jw + kq + 8 i, i < 8; 8 consecutive lanes cover one 128-byte (bf16) row.
    frag8<T> kr[8], vr[8], br[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int jj = jw + kq + 8 * i;
        if (jj < a.N && jj <= last) {
            kr[i] = load8<T>(kbase + (int64_t)jj * a.k.sl + 8 * fg);
            vr[i] = load8<T>(vbase + (int64_t)jj * a.v.sl + 8 * fg);
            if (fg < DS / 8) br[i] = load8<T>(bbase + (int64_t)jj * a.b.sl + 8 * fg);
        }
    }
    // per-key scalars with lane = key: lam * exp(g_m - g_j) and F_m - F_j
    const int j = jw + lane;
    float dec = 0.f, fd = 0.f;
    if (j < a.N && j <= last) {
        dec = lam * expf(gq - ((const float*)a.gk.ptr)[(int64_t)b * a.gk.sb + (int64_t)h * a.gk.sh +
                                                       (int64_t)j * a.gk.sl]);
        if (has_f)
            fd = fq - ((const float*)a.fk.ptr)[(int64_t)b * a.fk.sb + (int64_t)h * a.fk.sh + (int64_t)j * a.fk.sl];
    }
    const f32x8 qv = load_f32x8<T>(Q + 8 * fg);
    f32x8 cv;
    if (fg < DS / 8) cv = load_f32x8<T>(C + 8 * fg);
    else
#pragma unroll
        for (int e = 0; e < 8; ++e) cv[e] = 0.f;

    // scores: per key, the lane's share q.k/8 + dec * c.b over its 8 features, summed over the 8 lanes of the key
    float s[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int jj = jw + kq + 8 * i;
        const bool ok = jj < a.N && jj <= last;
        const float di = __shfl(dec, kq + 8 * i), fi = __shfl(fd, kq + 8 * i);
        float qk = 0.f, cb = 0.f;
        if (ok) {
            const f32x8 kv = __builtin_convertvector(kr[i], f32x8);
#pragma unroll
            for (int e = 0; e < 8; ++e) qk = fmaf(qv[e], kv[e], qk);
            if (fg < DS / 8) {
                const f32x8 bv = __builtin_convertvector(br[i], f32x8);
#pragma unroll
                for (int e = 0; e < 8; ++e) cb = fmaf(cv[e], bv[e], cb);
            }
        }
        float part = fmaf(qk, 0.125f, di * cb);
#pragma unroll
        for (int o = 1; o < 8; o <<= 1) part += __shfl_xor(part, o);
        s[i] = ok ? part + fi : -__builtin_inff();
    }
    // wave softmax statistics over its 64 keys (NaN scores propagate through the sum)
    float mx = s[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) mx = fmaxf(mx, s[i]);
#pragma unroll
    for (int o = 8; o < 64; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    float p[8], l = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int jj = jw + kq + 8 * i;
        p[i] = (jj < a.N && jj <= last) ? expf(s[i] - mx) : 0.f;
        l += p[i];
    }
#pragma unroll
    for (int o = 8; o < 64; o <<= 1) l += __shfl_xor(l, o);
    // weighted sum of V: the lane's 8 features over its 8 keys, then over the 8 key slots (fixed xor order)
    f32x8 acc;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        if (p[i] != 0.f) {
            const f32x8 vv = __builtin_convertvector(vr[i], f32x8);
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[e] = fmaf(p[i], vv[e], acc[e]);
        }
    }
#pragma unroll
    for (int o = 8; o < 64; o <<= 1)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] += __shfl_xor(acc[e], o);
    if (lane == 0) {
        wm[w] = mx;
        wl[w] = l;
    }
    if (kq == 0) {
#pragma unroll
        for (int e = 0; e < 8; ++e) wo[w][8 * fg + e] = acc[e];
    }
    __syncthreads();
    if (w != 0) return;
    // combine the 4 waves in order into the chunk partial
    float cm = wm[0];
#pragma unroll
    for (int k = 1; k < DW; ++k) cm = fmaxf(cm, wm[k]);
    float cl = 0.f, co = 0.f;
#pragma unroll
    for (int k = 0; k < DW; ++k) {
        const float sc = (wm[k] == -__builtin_inff()) ? 0.f : expf(wm[k] - cm);
        cl = fmaf(wl[k], sc, cl);
        co = fmaf(wo[k][lane], sc, co);
    }
    float* part = a.workspace + ((int64_t)row * gridDim.x + chunk) * PART;
    part[2 + lane] = co;
    if (lane == 0) {
        part[0] = cm;
        part[1] = cl;
    }
}

// out[row] = sum_c exp(m_c - M) o_c / sum_c exp(m_c - M) l_c. One wave per row: chunk c's max and sum are read by
// lane c mod 64, its output row by lane = feature, chunks in order, 8 row loads issued ahead of their FMAs.
__global__ __launch_bounds__(64) void decode_combine_kernel(sisa_decode_args a, int nchunk) {
    const int row = blockIdx.x, lane = threadIdx.x;
    const float* part = a.workspace + (int64_t)row * nchunk * PART;
    float M = -__builtin_inff();
    for (int c = lane; c < nchunk; c += 64) M = fmaxf(M, part[(int64_t)c * PART]);
    M = wave_max(M);
    float L = 0.f, o = 0.f;
    for (int c0 = 0; c0 < nchunk; c0 += 64) {
        const int c = c0 + lane, nc = nchunk - c0 < 64 ? nchunk - c0 : 64;
        float sc = 0.f;
        if (c < nchunk) {
            const float mc = part[(int64_t)c * PART];
            sc = (mc == -__builtin_inff()) ? 0.f : expf(mc - M);
            L = fmaf(part[(int64_t)c * PART + 1], sc, L);
        }
        for (int i0 = 0; i0 < nc; i0 += 8) {
            float t[8];
#pragma unroll
            for (int e = 0; e < 8; ++e)
                t[e] = i0 + e < nc ? __builtin_nontemporal_load(part + (int64_t)(c0 + i0 + e) * PART + 2 + lane) : 0.f;
#pragma unroll
            for (int e = 0; e < 8; ++e) o = fmaf(t[e], __shfl(sc, i0 + e), o);
        }
    }
    L = wave_sum(L);
    a.out[(int64_t)row * DH + lane] = o / L;
}

template <class T>
int launch_decode(const sisa_decode_args* a, hipStream_t st) {
    const int nchunk = (int)sisa::cdiv(a->N, KCH);
    const int rows = a->B * a->H * a->M;
    decode_chunk_kernel<T><<<dim3((unsigned)nchunk, (unsigned)rows), 64 * DW, 0, st>>>(*a);
    const int rc = sisa::launch_status("sisa_decode_attn");
    if (rc) return rc;
    decode_combine_kernel<<<(unsigned)rows, 64, 0, st>>>(*a, nchunk);
    return sisa::launch_status("sisa_decode_attn (combine)");
}

bool rows_ok(const sisa_view& v, int dtype, int width) {
    const int es = sisa::elem_size(dtype);
    if (!v.ptr || !sisa::aligned16(v.ptr)) return false;
    return (v.sb * es) % 16 == 0 && (v.sh * es) % 16 == 0 && (v.sl * es) % 16 == 0 && width % 8 == 0;
}

}  // namespace

extern "C" int64_t sisa_decode_workspace_bytes(int32_t B, int32_t H, int32_t M, int32_t N) {
    return (int64_t)B * H * M * sisa::cdiv(N, KCH) * PART * (int64_t)sizeof(float);
}

extern "C" int sisa_decode_attn(const sisa_decode_args* a, void* stream) {
    SISA_REQUIRE(a != nullptr, "sisa_decode_attn: null args");
    SISA_REQUIRE(a->B >= 1 && a->H >= 1 && a->M >= 1 && a->N >= 1, "sisa_decode_attn: bad shape B=%d H=%d M=%d N=%d",
                 a->B, a->H, a->M, a->N);
    SISA_REQUIRE(a->q_start >= 0 && a->q_start + a->M <= a->N,
                 "sisa_decode_attn: rows q_start=%d .. +M=%d must lie inside the N=%d cached positions", a->q_start,
                 a->M, a->N);
    SISA_REQUIRE((int64_t)a->B * a->H * a->M < 65536, "sisa_decode_attn: B*H*M must be below 65536");
    SISA_REQUIRE(a->dtype == SISA_BF16 || a->dtype == SISA_F16 || a->dtype == SISA_F32, "sisa_decode_attn: dtype %d",
                 a->dtype);
    SISA_REQUIRE(rows_ok(a->k, a->dtype, DH) && rows_ok(a->v, a->dtype, DH) && rows_ok(a->b, a->dtype, DS) && a->q.ptr &&
                     a->c.ptr,
                 "sisa_decode_attn: q/c must be given; k/v/b must be 16-byte aligned with 16-byte row strides");
    SISA_REQUIRE(a->gq.ptr && a->gk.ptr && a->lam && a->out && a->workspace, "sisa_decode_attn: null pointer");
    SISA_REQUIRE((a->fq.ptr == nullptr) == (a->fk.ptr == nullptr), "sisa_decode_attn: fq and fk given together");
    hipStream_t st = (hipStream_t)stream;
    switch (a->dtype) {
        case SISA_BF16: return launch_decode<__bf16>(a, st);
        case SISA_F16: return launch_decode<_Float16>(a, st);
        default: return launch_decode<float>(a, st);
    }
}
