/*
 * sisa_hip.h -- C ABI of the MI355X (gfx950) SISA hot-path library libsisa_hip.so.
 *
 * Every entry point takes one argument struct and a hipStream_t (passed as void*), launches its kernels on that
 * stream, never allocates device memory and never synchronises the host. The caller owns every buffer (inputs,
 * outputs and workspaces). Return value: SISA_OK or an error code; sisa_last_error() gives the message of the last
 * failing call on the calling thread.
 *
 * Conventions
 *   - (B,H,L,.) views: pointer + element strides (sb, sh, sl) of the batch, head and sequence axes; the last axis is
 *     contiguous. (B,H,L) views: pointer + (sb, sh, sl).
 *   - d_head = 64, d_state = 32 (the shapes the reference's kernels are written for, src/sisa/config.py:15-16).
 *   - Attention element types: SISA_BF16, SISA_F16, SISA_F32. g, F, lambda, lse, factors: fp32.
 *   - lse is stored in log2 units (max(s)*log2(e) + log2(sum)), as the reference's kernels do
 *     (src/sisa/kernels/attention.py:296).
 *   - Deterministic: no atomics; results are bitwise reproducible for a given shape.
 *
 * Each declaration names the reference interface it replaces (path:line in tlstngud/sisa).
 */
#ifndef SISA_HIP_H
#define SISA_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SISA_ABI_VERSION 4

enum sisa_dtype { SISA_F32 = 0, SISA_BF16 = 1, SISA_F16 = 2, SISA_F64 = 3 };

enum sisa_status {
    SISA_OK = 0,
    SISA_ERR_INVALID = 1,      /* bad argument (shape, stride, null pointer, dtype) */
    SISA_ERR_UNSUPPORTED = 2,  /* valid but not implemented for this configuration */
    SISA_ERR_LAUNCH = 3        /* a HIP launch failed */
};

/* A (B,H,L,.) tensor view with a contiguous last axis, or a (B,H,L) view. Strides are in elements. */
typedef struct {
    void* ptr;
    int64_t sb, sh, sl;
} sisa_view;

/* ------------------------------------------------------------------------------------------------ attention */

/* rowf/colf decay factors over 64-row blocks and the per-block maximum increase of g (monotonicity check).
 * Replaces `_factors` (src/sisa/kernels/attention.py:129-153), launched at attention.py:709. */
typedef struct {
    int32_t B, H, L;
    sisa_view g;         /* (B,H,L) fp32 */
    float* rowf;         /* (B,H,L) contiguous */
    float* colf;         /* (B,H,L) contiguous */
    float* mono;         /* (B*H*ceil(L/64)) */
} sisa_factors_args;

/* Forward attention: o, lse and (optionally) the self-normalised fp32 o'' used by the exact-delta backward.
 * Replaces `_fwd` (src/sisa/kernels/attention.py:177-296) and the host core `attn_forward` (attention.py:686-727).
 * rowf/colf must come from sisa_factors or sisa_prep_fwd (64-row blocks). */
typedef struct {
    int32_t B, H, L;
    int32_t dtype;             /* of q, k, v, c, b, o */
    sisa_view q, k, v;         /* (B,H,L,64) */
    sisa_view c, b;            /* (B,H,L,32) rotated C~, B~ */
    sisa_view g;               /* (B,H,L) fp32 cumulative log-decay */
    sisa_view f;               /* (B,H,L) fp32 cumulative log-sigmoid forget gate; ptr NULL = no forget term */
    const float* lam;          /* (H,) fp32 */
    int64_t s_lam;
    const float* rowf;         /* (B,H,L) contiguous */
    const float* colf;         /* (B,H,L) contiguous */
    sisa_view o;               /* (B,H,L,64) output, dtype */
    float* lse;                /* (B,H,L) contiguous output, log2 units */
    float* o32;                /* (B,H,L,64) contiguous fp32 output or NULL (bf16/fp16 only) */
} sisa_attn_fwd_args;

/* Workspace (bytes) of sisa_attn_bwd: five (B,H,L) fp32 row buffers, then B*H*ceil(L/16) fp64 dlambda sums of
 * 16-row groups. Always size the buffer with this function (it is not a multiple of the row-buffer size). */
int64_t sisa_attn_bwd_workspace_bytes(int32_t B, int32_t H, int32_t L);

/* Backward: dq, dk, dv, dc, db, dg, dF and dlambda, exact-delta scheme by default (`exact`). Two launches; the
 * first writes fp64 dlambda sums of 16-row groups, the second adds each head's groups in a fixed order.
 * Replaces `_bwd_dq` (src/sisa/kernels/attention.py:300-491), `_bwd_dkv` (attention.py:495-663), the fp64 dlambda
 * reduction (attention.py:781-783) and the host core `attn_backward` (attention.py:730-784). */
typedef struct {
    int32_t B, H, L;
    int32_t dtype;             /* of q, k, v, c, b, o, do, dq, dk, dv */
    int32_t dcb_dtype;         /* of dc, db: dtype or SISA_F32 */
    sisa_view q, k, v, c, b, g, f;
    const float* lam;
    int64_t s_lam;
    const float* rowf;
    const float* colf;
    sisa_view o;               /* forward output (dtype) */
    const float* o32;          /* (B,H,L,64) contiguous fp32 o'' or NULL (then delta = o.do) */
    const float* lse;          /* (B,H,L) contiguous */
    sisa_view dout;            /* (B,H,L,64) upstream gradient (dtype) */
    sisa_view dq, dk, dv;      /* outputs (dtype), any strides with contiguous last axis */
    sisa_view dc, db;          /* outputs (dcb_dtype) */
    float* dg;                 /* (B,H,L) contiguous output */
    float* df;                 /* (B,H,L) contiguous output, NULL when f.ptr is NULL */
    float* dlam;               /* (H,) output */
    void* workspace;           /* sisa_attn_bwd_workspace_bytes(B,H,L) bytes */
    int32_t exact;             /* nonzero: exact-delta scheme (the public path); 0: FlashAttention-standard delta
                                  o.do everywhere, diagonal included (comparison mode of the reference's kernels,
                                  EXACT=False, attention.py:47-48); o32 is ignored when 0 */
} sisa_attn_bwd_args;

int sisa_factors(const sisa_factors_args* a, void* stream);
int sisa_attn_fwd(const sisa_attn_fwd_args* a, void* stream);
int sisa_attn_bwd(const sisa_attn_bwd_args* a, void* stream);

/* Largest B*H*L that sisa_attn_bwd_noalloc takes: its scratch holds the backward workspace for it (28 MiB). */
#define SISA_NOALLOC_MAX_BHL (1 << 20)

/* sisa_attn_bwd without a caller workspace and without any allocation: `workspace` must be NULL, and the five row
 * buffers live in the library's static device scratch (one 28 MiB copy per GPU, held until the process ends).
 * No counterpart in the reference: for callers that cannot allocate (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). Limits: B*H*L <= SISA_NOALLOC_MAX_BHL (else SISA_ERR_INVALID); the stream
 * must belong to the current device. All calls on one GPU share its scratch: calls that overlap on one GPU (on
 * different streams, or from different threads) race; calls ordered on one stream do not. Results are bitwise those
 * of sisa_attn_bwd. */
int sisa_attn_bwd_noalloc(const sisa_attn_bwd_args* a, void* stream);

/* ------------------------------------------------------------------------------------------------ fused prep */

/* proj column layout (src/sisa/kernels/fused_prep.py:71-96): [Q H*64 | K H*64 | V H*64 | B H*32 | C H*32 |
 * theta H*16 | alpha H | zero pad to NPAD = ceil(273H/16)*16]. */

/* Forward prep: g = cumsum(-softplus(alpha)), F = cumsum(logsigmoid(z)), Phi = cumsum(theta), C~ = R(Phi)C,
 * B~ = R(Phi)B, rowf/colf, and the per-64-row block totals TOT (B*H, ceil(L/64), 18).
 * Replaces `_prep_sums` + `_prep_fwd` (src/sisa/kernels/fused_prep.py:247-352), host `_launch_prep_forward`
 * (fused_prep.py:527-564). q and k are not copied (they are read as strided views of proj). */
typedef struct {
    int32_t B, L, H;
    int32_t dtype;             /* of proj, cr, br: SISA_BF16 or SISA_F16 */
    const void* proj;          /* (B,L,NPAD) */
    int64_t s_pb, s_pl;
    const float* z;            /* (B,L,H) fp32, contiguous last axis, or NULL (no forget gate) */
    int64_t s_zb, s_zl;
    void* cr;                  /* (B,L,H,32) contiguous, dtype */
    void* br;                  /* (B,L,H,32) contiguous, dtype */
    float* g;                  /* (B,H,L) contiguous */
    float* f;                  /* (B,H,L) contiguous, ignored when z is NULL */
    float* rowf;               /* (B,H,L) contiguous */
    float* colf;               /* (B,H,L) contiguous */
    float* tot;                /* (B*H, ceil(L/64), 18) contiguous block totals */
} sisa_prep_fwd_args;

/* Workspace of sisa_prep_bwd. The backward runs as one launch whose workgroups hand their 64-row block totals to each
 * other through the workspace, so it must be zero-filled once before its first use and then kept: it carries a launch
 * counter from call to call (no per-call clearing). One workspace serves any shape up to its size; calls that overlap
 * in time on one workspace race. Bytes 8..11 (uint32) are nonzero after a call in which a workgroup's bounded wait for
 * another's totals ran out (results invalid; not expected to happen). */
int64_t sisa_prep_bwd_workspace_bytes(int32_t B, int32_t L, int32_t H);

/* Backward prep: reverse scans (fp64) for d alpha, dz, d theta; inverse rotation of dC~/dB~; zero pad columns.
 * Replaces `_prep_bsums` + `_prep_bwd` (src/sisa/kernels/fused_prep.py:385-494). The Q/K/V columns of dproj are
 * written by sisa_attn_bwd (views); this call writes the B, C, theta, alpha and pad columns. */
typedef struct {
    int32_t B, L, H;
    int32_t dtype;             /* of proj and dproj */
    const void* proj;
    int64_t s_pb, s_pl;
    const float* z;            /* or NULL */
    int64_t s_zb, s_zl;
    const float* tot;          /* from sisa_prep_fwd */
    const float* dg;           /* (B,H,L) contiguous */
    const float* df;           /* (B,H,L) contiguous or NULL */
    const float* dcr;          /* (B,L,H,32) contiguous fp32 */
    const float* dbr;          /* (B,L,H,32) contiguous fp32 */
    void* dproj;               /* (B,L,NPAD) dtype */
    int64_t s_db, s_dl;
    float* dz;                 /* (B,L,H) fp32 or NULL */
    int64_t s_dzb, s_dzl;
    void* workspace;           /* sisa_prep_bwd_workspace_bytes(B,L,H) bytes, 16-byte aligned, zero-filled once */
} sisa_prep_bwd_args;

int sisa_prep_fwd(const sisa_prep_fwd_args* a, void* stream);
int sisa_prep_bwd(const sisa_prep_bwd_args* a, void* stream);

/* Non-finite input check of the fused path: *ok (one byte on the device) = 1 if sum(a[0..na)) + sum(b[0..nb)) is
 * finite, else 0, summed in fp32 in a fixed order in one launch; a and b 16-byte aligned. Replaces the torch
 * reductions of `_nan_guard` (src/sisa/kernels/fused_prep.py:502-523), whose result feeds `torch._assert_async`. */
int sisa_finite_sum(const float* a, int64_t na, const float* b, int64_t nb, uint8_t* ok, void* stream);

/* ------------------------------------------------------------------------------------------------ linear CE */

/* Row pass of the chunked linear cross-entropy over one chunk of low-precision logits (logits = x W_pad^T from the
 * caller's GEMM, padded columns V..Vp-1 present but ignored on read):
 *   lse_r   = log sum_{c<V} exp(logit[r,c])            (fp32; a NaN logit makes the row NaN)
 *   loss_r  = lse_r - logit[r, label_r], or 0 when label_r == ignore_index (NaN for a label outside [0, V))
 *   G[r,c]  = (exp(logit[r,c] - lse_r) - [c == label_r]) * (*inv_n) * gscale, 0 for ignored rows and for c >= V,
 *             rounded once to the buffer dtype and written over the logits (when compute_grad != 0).
 * Replaces `_lmce_row_kernel` + `_launch_rows` (src/sisa/kernels/linear_ce.py:60-104). Rows of up to 65,536 columns
 * are read once (held in registers); longer rows are read twice. */
typedef struct {
    int64_t T;                 /* rows of the chunk (0 is a no-op) */
    int64_t V;                 /* real vocabulary columns, >= 1 */
    int64_t Vp;                /* padded columns, >= V, multiple of 8 */
    int64_t stride;            /* row stride of logits in elements, >= Vp, multiple of 8 */
    int32_t dtype;             /* SISA_BF16 or SISA_F16 */
    int32_t compute_grad;      /* nonzero: overwrite columns 0..Vp-1 of each row with G */
    void* logits;              /* (T, stride), 16-byte aligned */
    const int64_t* labels;     /* (T,) */
    int64_t ignore_index;
    const float* inv_n;        /* device scalar 1 / N_valid (read only when compute_grad) */
    float gscale;              /* extra multiplier of G (1, or the promised backward seed) */
    float* loss_rows;          /* (T,) fp32 output */
    float* lse;                /* (T,) fp32 output, natural log, or NULL */
} sisa_lmce_rows_args;

int sisa_lmce_rows(const sisa_lmce_rows_args* a, void* stream);

/* Fused forward of the linear cross-entropy: lse_r = log sum_{c<V} exp(x_r . w_c) and loss_r = lse_r - x_r . w_{label_r}
 * (0 for ignore_index, NaN for a label outside [0, V)) from x (N, D) and the padded weight w (Vp, D) on MFMA, without
 * a logits buffer: the logits are fp32 MFMA accumulations reduced tile by tile (online max / sum-exp over vocabulary
 * splits, combined in a fixed order). Replaces the forward of the reference's chunk loop for callers that need no
 * gradient -- the logits GEMM + `_lmce_row_kernel` pass of `_LinearCrossEntropyFn.forward`
 * (src/sisa/kernels/linear_ce.py:138-191, 60-96). */
typedef struct {
    int64_t N;                 /* rows (0 is a no-op) */
    int64_t V;                 /* real vocabulary rows of w, >= 1 */
    int64_t Vp;                /* rows of w, >= V (rows >= V are ignored) */
    int32_t D;                 /* hidden size, a positive multiple of 64 */
    int32_t dtype;             /* of x and w: SISA_BF16 or SISA_F16 */
    const void* x;             /* (N, D), 16-byte aligned, row stride ldx (multiple of 8) */
    int64_t ldx;
    const void* w;             /* (Vp, D), 16-byte aligned, row stride ldw (multiple of 8) */
    int64_t ldw;
    const int64_t* labels;     /* (N,) */
    int64_t ignore_index;
    float* lse;                /* (N,) fp32 output, natural log, or NULL */
    float* loss_rows;          /* (N,) fp32 output */
    float* workspace;          /* sisa_lmce_fwd_workspace_bytes(N, Vp) bytes */
} sisa_lmce_fwd_args;

int64_t sisa_lmce_fwd_workspace_bytes(int64_t N, int64_t Vp);
int sisa_lmce_fwd(const sisa_lmce_fwd_args* a, void* stream);

/* Training pass of the linear cross-entropy over one chunk of rows, on MFMA kernels only: the loss rows and, as
 * requested, dL/dx and dL/dW_pad in fp32 for G = (softmax - onehot) * (*inv_n) * gscale, i.e. for a backward seed of
 * gscale. The logits GEMM is sisa_lmce_fwd's kernel, which here also stores every exponential relative to its row's
 * maximum over a 128-column half of a 256-column vocabulary tile (compute dtype, in the workspace) and those maxima;
 * the loss rows are bitwise those of sisa_lmce_fwd. One launch then runs the dW tiles (dW = G^T x, all rows of the
 * chunk) and the dx tiles (dx = G W_pad, split over the vocabulary, the splits added in a fixed order); both form G
 * = exp * exp2(max - lse) * scale - onehot, rounded once to the compute dtype, while staging it into LDS. No logits
 * and no G are ever written. Replaces the chunk loop of `_LinearCrossEntropyFn.forward`
 * (src/sisa/kernels/linear_ce.py:138-217: the logits GEMM, `_lmce_row_kernel` (linear_ce.py:60-96) and the dx and
 * dW GEMMs of linear_ce.py:171-191). Deterministic: no atomics. */
typedef struct {
    int64_t N;                 /* rows of the chunk (0 is a no-op) */
    int64_t V;                 /* real vocabulary rows of w, >= 1 */
    int64_t Vp;                /* rows of w, a multiple of 128, >= V (rows >= V never enter a sum) */
    int32_t D;                 /* hidden size, a positive multiple of 64 */
    int32_t dtype;             /* of x and w: SISA_BF16 or SISA_F16 */
    const void* x;             /* (N, D), 16-byte aligned, row stride ldx (multiple of 8) */
    int64_t ldx;
    const void* w;             /* (Vp, D), 16-byte aligned, row stride ldw (multiple of 8) */
    int64_t ldw;
    const int64_t* labels;     /* (N,) */
    int64_t ignore_index;
    const float* inv_n;        /* device scalar 1 / N_valid of the whole problem (all chunks) */
    float gscale;              /* multiplier of G: 1, or the promised backward seed */
    float* loss_rows;          /* (N,) fp32 output */
    float* lse;                /* (N,) fp32 output, natural log, or NULL */
    float* dx;                 /* (N, D) fp32 output, row stride lddx (multiple of 4), or NULL */
    int64_t lddx;
    float* dw;                 /* (Vp, D) fp32 output, row stride lddw (multiple of 4), or NULL */
    int64_t lddw;
    int32_t dw_accumulate;     /* nonzero: dw += this chunk's part; zero: dw = it */
    int32_t dx_splits;         /* vocabulary splits of the dx product, 1..16 (0: the library's choice) */
    void* workspace;           /* sisa_lmce_train_workspace_bytes(N, Vp, D, dx_splits) bytes, 256-byte aligned */
} sisa_lmce_train_args;

int64_t sisa_lmce_train_workspace_bytes(int64_t N, int64_t Vp, int32_t D, int32_t dx_splits);
int sisa_lmce_train(const sisa_lmce_train_args* a, void* stream);

/* ------------------------------------------------------------------------------------------------ decoder block */

/* RMSNorm over the last axis: y = (x * rsqrt(mean(x^2) + eps)) * w in fp32, stored in the input dtype; rstd (N) fp32
 * saved for the backward. Backward: dx = rstd * (dy*w - n * mean(dy*w*n)) with n = x*rstd, and dw = sum over rows of
 * dy*n, reduced deterministically through dw_partial (sisa_rmsnorm_bwd_workspace_bytes). Replaces the eager float32
 * `RMSNorm.forward` and its autograd (src/sisa/modeling.py:26-36). */
typedef struct {
    int64_t N;                 /* rows */
    int32_t D;                 /* row length, multiple of 8, <= 4096 */
    int32_t dtype;             /* of x, y, dy, dx: SISA_BF16, SISA_F16 or SISA_F32 */
    float eps;
    const void* x; int64_t sx;         /* (N, D), row stride sx */
    const float* w;                    /* (D) fp32 */
    void* y; int64_t sy;               /* forward output */
    float* rstd;                       /* (N) fp32: written by the forward (may be NULL), read by the backward */
    const void* dy; int64_t sdy;       /* backward: incoming gradient */
    void* dx; int64_t sdx;             /* backward: gradient of x */
    float* dw;                         /* backward: (D) fp32 gradient of w */
    float* dw_partial;                 /* backward workspace */
} sisa_rmsnorm_args;

int64_t sisa_rmsnorm_bwd_workspace_bytes(int64_t N, int32_t D);
int sisa_rmsnorm_fwd(const sisa_rmsnorm_args* a, void* stream);
int sisa_rmsnorm_bwd(const sisa_rmsnorm_args* a, void* stream);

/* RMSNorm with an optional fused projection of the normalised rows, as the SISA attention sublayer uses it: the
 * normalised input n feeds the concatenated projection GEMM (in the autocast dtype) and the forget-gate logits
 * z = n W_f^T + b_f in fp32 (src/sisa/modeling.py:166-169, 217-220; RMSNorm modeling.py:26-36):
 *   forward:  rstd = 1/sqrt(mean(x^2) + eps), n = round_x((x * rstd) * w), y = round_y(n), z = n . W_f^T + b_f
 *   backward: dn = dy + dz W_f (summed in x's dtype as autograd does), dx = rstd * (du - u * mean(du * u)) with
 *             u = x * rstd, du = dn * w; dw = sum_rows dn * u; dW_f = dz^T n; db_f = sum_rows dz
 * Replaces RMSNorm.forward, the autocast cast of its output, `_forget_logits` and their autograd. H = 0 is a plain
 * RMSNorm with an output dtype of its own. Weight gradients are reduced deterministically through the workspace
 * (sisa_norm_bwd_workspace_bytes).
 * Residual (optional, replaces the residual add before the norm, `x = x + sublayer(...)`, modeling.py:288-291):
 *   forward with res:  h = round_x(x + res) is written to h and normalised in place of x;
 *   backward with dh:  dx = round_x(dx_norm) + dh, the gradient of h summed over its two consumers (the norm and
 *   the residual stream), as autograd sums them; x is then the h of the forward. */
typedef struct {
    int64_t N;                 /* rows */
    int32_t D;                 /* row length, multiple of 8, <= 4096 */
    int32_t H;                 /* projection outputs, 0..64 (0: none) */
    int32_t xdtype;            /* of x, dx and of n as the projection reads it: SISA_F32, SISA_BF16 or SISA_F16 */
    int32_t ydtype;            /* of y and dy: any of the three for an fp32 x, else xdtype */
    float eps;
    int32_t reserved;
    const void* x; int64_t sx;         /* (N, D), row stride sx */
    const float* w;                    /* (D) fp32 norm weight */
    const float* wf;                   /* (H, D) fp32 projection weight, row stride D */
    const float* bf;                   /* (H) fp32 projection bias */
    void* y; int64_t sy;               /* forward output (N, D) */
    float* rstd;                       /* (N): written by the forward (may be NULL without a backward), read back */
    float* z;                          /* (N, H) fp32 forward output, row stride H */
    const void* dy; int64_t sdy;       /* backward: gradient of y */
    const float* dz;                   /* backward: (N, H) gradient of z */
    void* dx; int64_t sdx;             /* backward: gradient of x */
    float* dw;                         /* backward: (D) */
    float* dwf;                        /* backward: (H, D) */
    float* dbf;                        /* backward: (H) */
    float* workspace;                  /* backward scratch, 16-byte aligned */
    const void* res; int64_t sres;     /* forward: residual (N, D) in ydtype, or NULL */
    void* h; int64_t sh;               /* forward: x + res (N, D) in xdtype; required with res */
    const void* dh; int64_t sdh;       /* backward: (N, D) gradient of h from the residual stream, xdtype, or NULL */
} sisa_norm_args;

int64_t sisa_norm_bwd_workspace_bytes(int64_t N, int32_t D, int32_t H);
int sisa_norm_fwd(const sisa_norm_args* a, void* stream);
int sisa_norm_bwd(const sisa_norm_args* a, void* stream);

/* SwiGLU activation h = silu(a) * b (fp32 arithmetic, one rounding) and its backward da = dh * b * silu'(a),
 * db = dh * silu(a), over n contiguous elements (n a multiple of 8). Replaces `F.silu(self.w_gate(x)) * self.w_up(x)`
 * and its autograd (src/sisa/modeling.py:48-49). With pairs = 1, a and b are one array of interleaved 8-element
 * chunks (a_8k..a_8k+7, b_8k..b_8k+7), the output of one GEMM against the gate and up weights interleaved in 8-row
 * chunks; the backward then writes the interleaved (da, db) chunks to da (b and db unused). */
typedef struct {
    int64_t n;                 /* elements of h */
    int32_t dtype;             /* SISA_BF16, SISA_F16 or SISA_F32 */
    int32_t pairs;             /* 0: separate a and b; 1: interleaved chunk pairs in a (and da) */
    const void* a;             /* gate pre-activation */
    const void* b;             /* up projection */
    void* h;                   /* forward output */
    const void* dh;            /* backward: incoming gradient */
    void* da;                  /* backward outputs */
    void* db;
} sisa_swiglu_args;

int sisa_swiglu_fwd(const sisa_swiglu_args* a, void* stream);
int sisa_swiglu_bwd(const sisa_swiglu_args* a, void* stream);

/* ------------------------------------------------------------------------------------------------ weight gradients */

/* C[N x K] (fp32) = A^T B with A (M x N) and B (M x K) row-major bf16/fp16: the weight gradient dW = dY^T X of a
 * linear layer y = x W^T over M tokens. Replaces the bf16 weight-gradient GEMMs autograd runs for the nn.Linear
 * projections of the decoder block (src/sisa/modeling.py:79-291) and the cast of their result to the fp32
 * parameter dtype. Split-K over M (nsplit splits of m_per_split rows, a multiple of 64; sisa_wgrad_splits gives the
 * default) with a fixed-order reduction through the workspace (sisa_wgrad_workspace_bytes). */
typedef struct {
    int64_t M;                 /* reduction length (rows of A and B) */
    int32_t N, K;              /* output rows and columns */
    int32_t dtype;             /* of A and B: SISA_BF16 or SISA_F16 */
    int32_t nsplit;            /* splits of M, 1..64 */
    int64_t m_per_split;       /* rows per split, multiple of 64, nsplit * m_per_split >= M */
    const void* a; int64_t lda;        /* (M, N), row stride lda >= N, multiple of 8 */
    const void* b; int64_t ldb;        /* (M, K), row stride ldb >= K, multiple of 8 */
    float* c; int64_t ldc;             /* (N, K) fp32 output, row stride ldc >= K */
    float* workspace;                  /* nsplit * N * K fp32 when nsplit > 1 */
} sisa_wgrad_args;

int32_t sisa_wgrad_splits(int64_t M, int32_t N, int32_t K);
int64_t sisa_wgrad_workspace_bytes(int64_t M, int32_t N, int32_t K, int32_t nsplit);
int sisa_wgrad(const sisa_wgrad_args* a, void* stream);

/* ------------------------------------------------------------------------------------------------ decoding */

/* Attention of M new query rows (positions q_start .. q_start+M-1) against the N cached positions of a decode
 * cache, exact fp32 score and softmax, fp32 output (B,H,M,64) contiguous:
 *   s_mj = q_m.k_j/8 + lam_h * exp(g_m - g_j) * (c_m.b_j) + (F_m - F_j) for j <= q_start + m.
 * Replaces `_attend_rows` (src/sisa/functional.py:69-93) in the decode step of `SISAAttention._forward_cached`
 * (src/sisa/modeling.py:224-238). Split over 256-key chunks; workspace sisa_decode_workspace_bytes(B,H,M,N). */
typedef struct {
    int32_t B, H, M, N;
    int32_t dtype;             /* of q, k, v, c, b: SISA_BF16, SISA_F16 or SISA_F32 */
    int32_t q_start;           /* position of query row 0; q_start + M <= N */
    sisa_view q, k, v;         /* (B,H,M,64), (B,H,N,64), (B,H,N,64) */
    sisa_view c, b;            /* (B,H,M,32), (B,H,N,32) */
    sisa_view gq, gk;          /* (B,H,M), (B,H,N) fp32 */
    sisa_view fq, fk;          /* (B,H,M), (B,H,N) fp32, or both null */
    const float* lam;          /* (H) fp32, element stride s_lam */
    int64_t s_lam;
    float* out;                /* (B,H,M,64) fp32 contiguous */
    float* workspace;
} sisa_decode_args;

int64_t sisa_decode_workspace_bytes(int32_t B, int32_t H, int32_t M, int32_t N);
int sisa_decode_attn(const sisa_decode_args* a, void* stream);

/* ------------------------------------------------------------------------------------------------ misc */

/* The library's 16-bit operand rounding over a flat buffer: y[i] = x[i] rounded to nearest even in dtype (the
 * kernels' pair conversion), and back[i] = y[i] widened to fp32 by the kernels' load conversion (back may be NULL).
 * Replaces nothing on the call path: it exposes `_bf16x2` / `_bf16x2_f32` (src/sisa/kernels/attention.py:156-173),
 * which the kernels inline, so that they can be compared bit for bit with tensor.to(dtype) / .float(). */
typedef struct {
    int64_t n;                 /* elements (0 is a no-op) */
    int32_t dtype;             /* SISA_BF16 or SISA_F16 */
    const float* x;            /* (n,) fp32, 16-byte aligned */
    void* y;                   /* (n,) dtype output, 16-byte aligned */
    float* back;               /* (n,) fp32 output or NULL, 16-byte aligned */
} sisa_round16_args;

int sisa_round16(const sisa_round16_args* a, void* stream);

int sisa_abi_version(void);
const char* sisa_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* SISA_HIP_H */
