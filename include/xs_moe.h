/*
 * xs_moe.h -- C ABI of the MI355X (gfx950) MoE operator library libxs_moe.so.
 *
 * Plain C: pointers, sizes, enums.  No torch or HIP types appear in any
 * signature; a stream is passed as `void *` (a hipStream_t, NULL = the null
 * stream).  Every entry point returns 0 on success or a non-zero xs_status;
 * xs_last_error() then holds a message for the calling thread.  The C++ Tensor
 * layer converts non-zero codes into std::runtime_error, as CHECK_CUDA does in
 * the reference (xstar_cpp/include/cuda/cuda_check.h:23-31).
 *
 * All device pointers must be device-resident (hipMalloc'd or torch CUDA
 * tensors).  Activations, outputs and weights are moved with 16-byte vector
 * loads and stores: their base pointers must be 16-byte aligned (f32 scales 4,
 * FP8 codes written by the quantizers 8); a misaligned pointer is rejected
 * with XS_ERR_INVALID ("misaligned operand ...").  xs_rmsnorm without its FP8
 * output accepts any alignment (it falls back to a scalar kernel).  Compute entry points enqueue work on `stream` and return without
 * synchronising; callers that need results on the host synchronise the stream
 * (the C++ Tensor ops do, matching the reference's synchronous launchers,
 * xstar_cpp/src/ops/gemm.cu:238-239).
 *
 * Reference interfaces each group replaces are cited per declaration
 * (paths relative to the reference repository root).
 */
#ifndef XS_MOE_H
#define XS_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    XS_OK = 0,
    XS_ERR_INVALID = 1,      /* bad argument (shape, dtype, null pointer, alignment) */
    XS_ERR_HIP = 2,          /* a HIP runtime call or kernel launch failed */
    XS_ERR_UNSUPPORTED = 3,  /* valid request this build does not implement */
    XS_ERR_WORKSPACE = 4     /* workspace too small */
} xs_status;

/* Element types.  The first two values match the reference's DType
 * (xstar_cpp/include/dtype.h:8-12). */
typedef enum {
    XS_F32 = 0,
    XS_BF16 = 1,
    XS_FP8_E4M3 = 2,   /* OCP E4M3FN, 1 byte */
    XS_FP4_E2M1X2 = 3, /* OCP E2M1, two per byte, element 2i in the low nibble */
    XS_E8M0 = 4,       /* OCP E8M0 scale byte: 2^(b-127) */
    XS_I32 = 5
} xs_dtype;

/* Thread-local message of the last failing call on this thread. */
const char *xs_last_error(void);

/* ---------------------------------------------------------------------------
 * Runtime shim.  Replaces cuda_alloc / cuda_free / cuda_memcpy_h2d / _d2h /
 * _d2d / cuda_free_bytes (xstar_cpp/include/cuda/cuda_allocator.h:32-69,
 * xstar_cpp/src/cuda/cuda_allocator.cu:7-45).
 * ------------------------------------------------------------------------- */
int xs_device_count(int *count);
int xs_malloc(void **ptr, size_t bytes);
int xs_free(void *ptr);
int xs_memcpy_h2d(void *dst, const void *src, size_t bytes);
int xs_memcpy_d2h(void *dst, const void *src, size_t bytes);
int xs_memcpy_d2d(void *dst, const void *src, size_t bytes);
int xs_free_bytes(size_t *free_bytes);
int xs_stream_synchronize(void *stream);

/* ---------------------------------------------------------------------------
 * Stage entry points.  The reference has no MoE code (README.md:28,45); each
 * stage replaces the op it would otherwise be composed from, noted per entry.
 * ------------------------------------------------------------------------- */

/* Router logits = x . router_w^T in f32 (replaces linear(x, router_w, nullptr),
 * xstar_cpp/src/ops/linear.cpp:9-66 over gemm_launch, xstar_cpp/include/ops/gemm.h:165-176).
 * x [T, H], router_w [E, H], dtype XS_F32 or XS_BF16 (both the same);
 * logits [T, E] f32.  exact != 0: sequential-k f32 accumulation with separately
 * rounded products, bit-identical to gemm_cpu (gemm.h:57-83).  exact = 0 (bf16
 * only): bf16 MFMA with f32 accumulation.  H % 128 == 0; x and router_w
 * 16-byte aligned. */
int xs_moe_router_logits(const void *x, const void *router_w, int dtype, int64_t T, int64_t E,
                         int64_t H, int exact, float *logits, void *stream);

/* Top-k routing (no reference counterpart; contract: sigmoid scores
 * s = sigmoid(logit) with the branched form of xstar_cpp/src/ops/mlp.cpp:10-21,
 * selection key s + bias (bias may be NULL), optional group-limited selection
 * (n_group > 1 keeps the topk_group groups with the largest top-2 key sum),
 * top-k with ties to the lower expert index, weights s_j / sum(s) * scaling
 * when renormalize, else s_j * scaling).  logits [T, E] f32, idx [T, k] i32,
 * w [T, k] f32.  E <= 1024, k <= 16, n_group <= 64. */
int xs_moe_route(const float *logits, const float *bias, int64_t T, int64_t E, int64_t k,
                 int64_t n_group, int64_t topk_group, int renormalize, float scaling,
                 int32_t *idx, float *w, void *stream);

/* Stable counting sort of the T*k slots (slot = t*k + j) by expert.
 * counts [E], offsets [E+1] (exclusive scan), perm [T*k] (position -> slot),
 * inv [T*k] (slot -> position).  workspace: xs_moe_permute_workspace_size()
 * bytes of device memory.  Precondition, checked: every idx is in [0, E) and no
 * row names an expert twice (the router's output always is).  Otherwise the
 * call returns XS_ERR_INVALID ("idx: expert index outside [0, E)" / "idx:
 * expert named twice in one row") and the outputs are unspecified.  The check
 * waits for the stream once, so this stage entry point is synchronous. */
size_t xs_moe_permute_workspace_size(int64_t T, int64_t E);
int xs_moe_permute(const int32_t *idx, int64_t T, int64_t E, int64_t k, int32_t *counts,
                   int32_t *offsets, int32_t *perm, int32_t *inv, void *workspace,
                   size_t workspace_bytes, void *stream);

/* Activation quantization (no reference counterpart).
 * FP8: per (row, 128-column group) scale = amax/448 (amax == 0 -> 1),
 *      q = e4m3_rne(v * (448/amax)); q [rows, cols] bytes, s [rows, cols/128] f32.
 * MXFP8 (OCP MX v1.0): per (row, 32-column block) exponent se = floor(log2 amax) - 8,
 *      q = e4m3_rne_sat(v * 2^-se); s [rows, cols/32] e8m0 bytes.
 * x dtype XS_F32 or XS_BF16. */
int xs_quant_act_fp8(const void *x, int dtype, int64_t rows, int64_t cols, uint8_t *q, float *s,
                     void *stream);
int xs_quant_act_mxfp8(const void *x, int dtype, int64_t rows, int64_t cols, uint8_t *q,
                       uint8_t *s, void *stream);

/* RMSNorm, optionally fused with the FP8 1x128 activation quantization of its
 * output.  Replaces rmsnorm(x, weight, eps) (xstar_cpp/include/ops/rmsnorm.h,
 * xstar_cpp/src/ops/rmsnorm.cpp:6-81; device launcher rmsnorm_launch,
 * xstar_cpp/src/ops/rmsnorm.cu:57-81) and, with q/s, the rmsnorm -> activation
 * quant pair ahead of the MoE layer (xstar_cpp/src/ops/transformer_block.cpp:353).
 * x, y [rows, hidden] and weight [hidden] of `dtype` (XS_F32 or XS_BF16).
 * y = x * inv * weight with inv = 1 / sqrt(mean(x^2) + eps) in f32 (correctly
 * rounded sqrt and divisions); bf16 rounds x * inv to bf16 before the weight
 * multiply, as the reference CPU path does (rmsnorm.cpp:72).  q [rows, hidden]
 * e4m3 and s [rows, hidden/128] f32 (both NULL, or both set with
 * hidden % 128 == 0) receive xs_quant_act_fp8(y). */
int xs_rmsnorm(const void *x, const void *weight, int dtype, int64_t rows, int64_t hidden, float eps,
               void *y, uint8_t *q, float *s, void *stream);

/* Weight quantization for loading dense checkpoints (no reference counterpart;
 * the reference loads F32/BF16 only, xstar_cpp/src/weight_io.cpp:122-127).
 * FP8 128x128 blocks: w [batch, n, k] -> q [batch, n, k], s [batch, n/128, k/128] f32,
 *   scale = amax/448 over the block (amax == 0 -> 1), q = e4m3_rne(v * 448/amax).
 * MXFP4: w [batch, n, k] -> q [batch, n, k/2] packed, s [batch, n, k/32] e8m0,
 *   se = floor(log2 amax) - 2, q = e2m1_rne_sat(v * 2^-se). */
int xs_quant_weight_fp8_block(const void *w, int dtype, int64_t batch, int64_t n, int64_t k,
                              uint8_t *q, float *s, void *stream);
int xs_quant_weight_mxfp4(const void *w, int dtype, int64_t batch, int64_t n, int64_t k,
                          uint8_t *q, uint8_t *s, void *stream);

/* Fragment-order copy of e4m3 weights for the weight-direct prefill GEMMs.
 * No counterpart in the reference (a layout of this library, made once when a
 * layer's weights are loaded).  w [batch, n, k] row-major e4m3 -> out, same
 * size: 16-byte chunk c = ((b * n/16 + t) * k/128 + kb) * 128 + 64 h + l holds
 * w[b][16 t + l % 16][128 kb + 64 h + 16 (l / 16) .. + 16) (h = 0, 1; l = 0..63),
 * the operand layout of v_mfma_f32_16x16x128_f8f6f4.  n % 16 == 0,
 * k % 128 == 0, 16-byte aligned, out not overlapping w. */
int xs_pack_weight_fp8_frag(const uint8_t *w, int64_t batch, int64_t n, int64_t k, uint8_t *out, void *stream);

/* MXFP4 weights w [batch, n, k/2] (e2m1 pairs) and their e8m0 scales
 * s [batch, n, k/32] -> out_w (same bytes as w) and out_s (same bytes as s) in
 * the operand layout of v_mfma_scale_f32_16x16x128_f8f6f4 with an FP4 A
 * operand: per 16-row tile and 128-K slice, lane 16 g + r's 16 bytes (row r,
 * K = [32 g, 32 g + 32)) and its scale byte (row r, 32-block g).
 * n % 16 == 0, k % 128 == 0, w and out_w 16-byte aligned, outputs not
 * overlapping inputs.  No reference counterpart: the storage format of the
 * weight-direct MXFP4 GEMMs. */
int xs_pack_weight_mxfp4_frag(const uint8_t *w, const uint8_t *s, int64_t batch, int64_t n, int64_t k,
                              uint8_t *out_w, uint8_t *out_s, void *stream);

/* Single FP8 block-scaled GEMM: C = dequant(A) . dequant(B)^T, bf16 out.
 * Replaces gemm_launch(C, A, B, nullptr, m, k, n, transB=true, ...)
 * (xstar_cpp/include/ops/gemm.h:165-176) for FP8 operands.
 * A [M, K] bf16 activations (quantized per 1x128 inside, workspace holds them),
 * B [N, K] e4m3 with Bs [N/128, K/128] f32 block scales, C [M, N] bf16.
 * K % 128 == 0, N % 128 == 0. */
size_t xs_gemm_fp8_blockscale_workspace_size(int64_t M, int64_t K);
int xs_gemm_fp8_blockscale(const void *A, const uint8_t *B, const float *Bs, int64_t M,
                           int64_t N, int64_t K, void *C, void *workspace,
                           size_t workspace_bytes, void *stream);

/* The same GEMM with B given in fragment order (xs_pack_weight_fp8_frag with
 * batch 1, n = N, k = K), loaded straight into registers by the weight-direct
 * kernel: 64-row tiles of A x 256-column slabs of B, no K split.  Same
 * arguments and workspace (xs_gemm_fp8_blockscale_workspace_size) as
 * xs_gemm_fp8_blockscale otherwise; N % 256 == 0, K % 512 == 0.  No
 * reference counterpart of its own: it stands in for the same gemm_launch
 * call when the caller keeps a packed copy of the weights.  Results agree
 * with xs_gemm_fp8_blockscale within f32 rounding (its K split sums the
 * partial products in another order).  Opt-in: without XS_WEIGHT_DIRECT=1
 * in the environment it returns XS_ERR_UNSUPPORTED. */
int xs_gemm_fp8_blockscale_packed(const void *A, const uint8_t *Bp, const float *Bs, int64_t M,
                                  int64_t N, int64_t K, void *C, void *workspace,
                                  size_t workspace_bytes, void *stream);

/* Router of the MoE layer (xs_moe_params.router_exact).  The reference's
 * router logits are gemm_cpu's sequential f32 sums (gemm.h:57-83); the
 * routing contract asks for its top-k indices bit for bit.
 *   XS_ROUTER_MFMA: bf16 MFMA logits, f32 accumulate.  Fast, not bit-exact:
 *     a token whose top-k keys lie within rounding of each other may route
 *     differently.
 *   XS_ROUTER_CERTIFIED: bit-exact routing.  The MFMA logits come with a
 *     proven bound on their distance from the gemm_cpu sums; tokens whose
 *     top-k the bound settles are routed on them, and for the others the
 *     logits whose key interval meets another's (the undecided experts) are
 *     recomputed in gemm_cpu order before routing.  Indices, order, counts
 *     and the permutation are the reference's; logits (and so the routing
 *     weights) of settled experts are the MFMA's.  f32 inputs take the chain
 *     router.
 *   XS_ROUTER_CHAIN: every logit in gemm_cpu order (bit-exact logits too). */
enum { XS_ROUTER_MFMA = 0, XS_ROUTER_CERTIFIED = 1, XS_ROUTER_CHAIN = 2 };

/* ---------------------------------------------------------------------------
 * The whole MoE layer.  Replaces mlp(x, gate_up_weight, down_weight)
 * (xstar_cpp/include/ops/mlp.h:51) at its call sites in transformer_block
 * (xstar_cpp/src/ops/transformer_block.cpp:75,142,204,353).
 * ------------------------------------------------------------------------- */
typedef struct {
    int64_t T;            /* tokens (T x E < 2^31; T x H and T x (top_k + 1) x I < 2^32) */
    int64_t H;            /* hidden (multiple of 256) */
    int64_t I;            /* expert intermediate (multiple of 128) */
    int64_t E;            /* routed experts (<= 1024) */
    int64_t top_k;        /* <= 16 */
    int64_t n_group;      /* 1 = no group-limited routing */
    int64_t topk_group;
    int renormalize;      /* 1: w = s / sum(s) */
    float routed_scaling; /* multiplies the routed weights */
    int x_dtype;          /* XS_BF16 or XS_F32: x, router_w and out */
    int routed_format;    /* XS_FP8_E4M3 (128x128 f32 scales) or XS_FP4_E2M1X2 (MXFP4) */
    int has_shared;       /* 1: shared expert weights present (FP8 128x128) */
    int router_exact;     /* XS_ROUTER_MFMA (0), XS_ROUTER_CERTIFIED (1) or XS_ROUTER_CHAIN (2) */
    int has_norm;         /* 1: RMSNorm x with norm_weight first (the block's pre-norm) */
    float norm_eps;       /* RMSNorm epsilon when has_norm */
} xs_moe_params;

typedef struct {
    const void *x;             /* [T, H] x_dtype */
    const void *router_w;      /* [E, H] x_dtype */
    const float *router_bias;  /* [E] f32 or NULL */
    /* routed experts.  FP8: w13 [E, 2I, H] e4m3, w13_scale [E, 2I/128, H/128] f32,
     *                       w2 [E, H, I] e4m3,   w2_scale [E, H/128, I/128] f32.
     *                  FP4: w13 [E, 2I, H/2], w13_scale [E, 2I, H/32] e8m0,
     *                       w2 [E, H, I/2],   w2_scale [E, H, I/32] e8m0.
     * w13 rows are [gate ; up] (xstar_cpp/include/ops/mlp.h:4-14). */
    const void *w13; const void *w13_scale;
    const void *w2;  const void *w2_scale;
    /* shared expert, FP8 128x128 (E = 1 shapes), or NULL when !has_shared */
    const void *shared_w13; const float *shared_w13_scale;
    const void *shared_w2;  const float *shared_w2_scale;
    void *out;                 /* [T, H] x_dtype */
    /* optional device outputs for inspection (NULL = not written) */
    float *logits;             /* [T, E] */
    int32_t *topk_idx;         /* [T, k] */
    float *topk_w;             /* [T, k] */
    int32_t *counts;           /* [E] */
    int32_t *offsets;          /* [E+1] */
    int32_t *perm;             /* [T*k] */
    int32_t *inv;              /* [T*k] */
    /* RMSNorm weight [H] x_dtype when has_norm (else ignored) */
    const void *norm_weight;
    /* optional [T, H] x_dtype added to the output before its one rounding
     * (the block's residual, xstar_cpp/src/ops/transformer_block.cpp:75,353:
     * add(h, mlp(rmsnorm(h)))); may equal out (in place); NULL = none */
    const void *residual;
    /* optional inspection outputs of the expert stages (NULL = not written),
     * rows in position order: the routed rows sorted by (expert, token), then
     * the shared segment's T rows; R = T*k (+ T with the shared expert).
     * act_q / act_s: FP8 routed format only (ignored for MXFP4). */
    uint8_t *act_q;            /* [R, I] e4m3: SwiGLU output after its FP8 1x128 re-quant */
    float *act_s;              /* [R, I/128] f32 scales of act_q */
    float *y_rows;             /* [R, H] f32: each row's down projection, before the combine */
    /* optional: the weights again, packed in MFMA fragment order.  FP8 layers:
     * xs_pack_weight_fp8_frag (w13 as [E, 2I, H], w2 as [E, H, I], the shared
     * expert's as E = 1; same byte counts as the row-major tensors).  When the
     * layer gives all it has (FP8 routed experts, and the shared expert's if
     * present), the prefill and decode GEMMs load their weights straight into
     * registers from these copies, with the same results bit for bit.  MXFP4
     * layers: w13_frag / w2_frag and w13_scale_frag / w2_scale_frag from
     * xs_pack_weight_mxfp4_frag (routed experts; the shared expert is FP8, its
     * packed copy from xs_pack_weight_fp8_frag).  NULL = not given.
     * Packed-only layer: w13 and w2 (and shared_w13 / shared_w2) NULL, the
     * packed copies given; the block scales (FP8) stay required.  Every GEMM
     * is then a weight-direct one, and a shape they do not take (K a multiple
     * of 512, N of 512) is refused with XS_ERR_UNSUPPORTED.
     * The weight-direct GEMMs are opt-in: they run only when the environment
     * sets XS_WEIGHT_DIRECT=1 (read per call).  Otherwise the packed copies
     * are ignored when the row-major weights are given, and a packed-only
     * layer is refused with XS_ERR_UNSUPPORTED. */
    const void *w13_frag;
    const void *w2_frag;
    const void *shared_w13_frag;
    const void *shared_w2_frag;
    const void *w13_scale_frag;
    const void *w2_scale_frag;
} xs_moe_tensors;

/* Device workspace the forward needs for these params (bytes, 256-aligned). */
size_t xs_moe_workspace_size(const xs_moe_params *p);

/* The kernels xs_moe_forward chooses for these params and tensors: the same
 * decision, environment switches included, without launching anything or
 * touching a GPU.  No reference counterpart: for callers and tests that check
 * the dispatch.  T >= 1. */
typedef enum {
    XS_GEMM_TILED = 0,            /* one block per tile, operands through an LDS ring */
    XS_GEMM_STREAM = 1,           /* persistent stream-K */
    XS_GEMM_TALL = 2,             /* tall tiles, operands through LDS rings */
    XS_GEMM_DIRECT_PREFILL = 3,   /* weight-direct, 128-row tiles */
    XS_GEMM_DIRECT_DECODE = 4,    /* weight-direct, 16-row tiles */
    XS_GEMM_DIRECT_MXFP4 = 5      /* weight-direct MXFP4, 64- or 128-row tiles */
} xs_gemm_kind;
typedef struct {
    int tile_rows;       /* rows per tile of the routed GEMMs */
    int routed_gemm;     /* xs_gemm_kind of the routed experts' gate_up and down */
    int shared_gemm;     /* xs_gemm_kind of the shared expert (FP8 layers: the routed launch); -1: none */
    int fused_combine;   /* 1: the down GEMM sums each token's rows itself; 2: the shared
                          * expert's down launch sums them (XS_SHARED_COMBINE=1) */
} xs_moe_plan_t;
int xs_moe_plan(const xs_moe_params *p, const xs_moe_tensors *t, xs_moe_plan_t *out);

/* Diagnostics of the certified router (no reference counterpart: for
 * benchmarks and tests).  After a forward with these params on this workspace
 * (NULL: the no-allocation scratch) has been enqueued on `stream`: out[0] =
 * the (token, expert) logits its exact pass recomputed in gemm_cpu order,
 * out[1] = the tokens it routed after that pass.  Waits for the stream.  Other
 * routers report 0, 0. */
int xs_moe_router_stats(const xs_moe_params *p, const void *workspace, int64_t out[2], void *stream);

/* [RMSNorm] + activation quant -> router -> top-k -> permute -> grouped gate_up
 * GEMM with SwiGLU and FP8 re-quant -> grouped down GEMM -> weighted combine
 * (+ shared).  With has_norm the layer computes moe(rmsnorm(x, norm_weight,
 * norm_eps)) (xstar_cpp/src/ops/transformer_block.cpp:353 with the MoE in place
 * of mlp()): one kernel writes the normalized rows the router reads and their
 * FP8 quantization the expert GEMMs read (xs_rmsnorm semantics).  With a
 * residual the combine adds it in f32 before the one cast, so has_norm plus
 * residual = x computes the block's whole FFN half, x + moe(rmsnorm(x)).
 * Stream-ordered, no host synchronisation inside.  T = 0 returns XS_OK after
 * validating the params; its tensor pointers may then be null. */
int xs_moe_forward(const xs_moe_params *p, const xs_moe_tensors *t, void *workspace,
                   size_t workspace_bytes, void *stream);

/* ---------------------------------------------------------------------------
 * xs_moe_forward without a caller workspace.  No counterpart in the reference:
 * for callers that cannot allocate device memory -- code under HIP graph
 * capture, tight serving loops, harnesses that forbid allocation.  The layer's
 * scratch lives in a static device array of XS_NOALLOC_SCRATCH_BYTES per GPU
 * (held until the process ends, by every process that loads this library,
 * whether or not it calls this entry); params whose workspace
 * (xs_moe_workspace_size) exceeds it are rejected with XS_ERR_WORKSPACE.
 * Callers compare xs_moe_workspace_size(p) with xs_moe_noalloc_scratch_bytes():
 * the size is not monotonic in T (tile and stream-K regions change with the
 * kernels chosen), so no token count is a bound.  Examples at the V4-Flash
 * shape with the default router: FP8 T = 256 needs 53.5 MiB, MXFP4 T = 200 62.2 MiB.  Calls nothing that
 * allocates.  Every call on one GPU shares that GPU's array: calls that
 * overlap on one GPU (different streams, or threads) race; calls in one
 * stream order are safe, because each forward re-arms what must start at zero.
 * Same semantics and outputs as xs_moe_forward.
 * ------------------------------------------------------------------------- */
#define XS_NOALLOC_SCRATCH_BYTES (64u * 1024u * 1024u)
size_t xs_moe_noalloc_scratch_bytes(void);
int xs_moe_forward_noalloc(const xs_moe_params *p, const xs_moe_tensors *t, void *stream);

/* ---------------------------------------------------------------------------
 * Per-stage timing hook (no reference counterpart; the reference times ops with
 * torch.cuda.Event around whole calls, bench/bench_splitkv.py:86-105).  While
 * enabled, xs_moe_forward records a HIP event at each stage boundary on its
 * stream (activation quant with the optional RMSNorm, router logits, route,
 * permute, gate_up GEMM, down GEMM, combine).  xs_moe_profile_read waits for the recorded forwards, writes
 * the summed milliseconds of up to 7 stages and the number of forwards, and
 * clears the record.  Process-wide state: not for concurrent callers.
 * ------------------------------------------------------------------------- */
int xs_moe_profile_enable(int enable);
int xs_moe_profile_read(float *stage_ms, int n_stages, int *n_calls);

#ifdef __cplusplus
}
#endif
#endif
