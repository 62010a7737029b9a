/*
 * moe_oracle.h -- CPU restatement of the MoE operator's numerics.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (the HIP library, the
 * C++ Tensor ops, the pybind11 module) may link, load or call this code.  It is
 * used by tests/ (as the checker), by __graft_entry__.smoke() (as the checker)
 * and by bench.py's cpu_baseline leg (as the timed CPU baseline).
 *
 * Reference anchors (paths relative to the reference repository root):
 *   - f32 GEMM accumulation order (i -> kk -> j, f32 row accumulator, one
 *     output cast):                     xstar_cpp/include/ops/gemm.h:57-83
 *   - bias-free linear over gemm_cpu:   xstar_cpp/src/ops/linear.cpp:9-66
 *   - branched sigmoid, silu, f32 silu*up with one downcast:
 *                                       xstar_cpp/src/ops/mlp.cpp:10-45
 *   - [gate ; up] fused row order:      xstar_cpp/include/ops/mlp.h:4-14,
 *                                       xstar_cpp/src/qwen2_model.cpp:187-206
 *   - f32 -> bf16 RNE by bias add:      xstar_cpp/src/bfloat16.cpp:5-25
 *   - elementwise add via f32:          xstar_cpp/src/ops/add.cpp:38-49
 * The MoE-specific stages (router top-k, permute, FP8/FP4 codecs, block-scaled
 * GEMM, combine) have no implementation in the reference (README.md:28,45);
 * their contract is defined here and pinned by the tests listed in each
 * function's comment.
 */
#ifndef XSTAR_MOE_ORACLE_H
#define XSTAR_MOE_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------- scalar codecs ---------------- */
uint16_t xo_bf16_from_f32(float f);          /* RNE by bias add, bfloat16.cpp:5-25 */
float    xo_f32_from_bf16(uint16_t b);       /* zero-extend, bfloat16.cpp:27-36 */
float    xo_e4m3_decode(uint8_t b);          /* OCP FP8 E4M3FN */
uint8_t  xo_e4m3_encode(float f);            /* RNE, saturate to +-448, NaN -> 0x7f */
float    xo_e2m1_decode(uint8_t nib);        /* OCP FP4 E2M1 (low 4 bits) */
uint8_t  xo_e2m1_encode(float f);            /* RNE, saturate to +-6 */
float    xo_e8m0_decode(uint8_t b);          /* 2^(b-127); 255 -> NaN */

/* ---------------- scalar math ---------------- */
float xo_expf(float x);      /* Cody-Waite + degree-7 Taylor; bit-identical on the GPU */
float xo_sigmoid(float x);   /* branched form of mlp.cpp:10-21 over xo_expf */
float xo_silu(float x);      /* mlp.cpp:23-26 */

/* ---------------- quantizers ---------------- */
/* Activation FP8: per (row, 128-column group) amax; inv = 448/amax,
 * scale = amax/448 (amax == 0 -> scale 1, q 0); q = e4m3(v * inv).
 * x is f32 [rows, cols], cols % 128 == 0.  q [rows, cols], s [rows, cols/128]. */
void xo_quant_act_fp8(const float *x, int64_t rows, int64_t cols, uint8_t *q, float *s);
/* Activation MXFP8 (OCP MX v1.0): per (row, 32-column block) shared exponent
 * se = floor(log2(amax)) - 8, scale byte = se + 127 (clamped to [0,254]),
 * q = e4m3(v * 2^-se) saturating.  s [rows, cols/32] e8m0 bytes. */
void xo_quant_act_mxfp8(const float *x, int64_t rows, int64_t cols, uint8_t *q, uint8_t *s);
/* Weight FP8 128x128 block scales: scale = amax/448 over the block (amax == 0
 * -> 1), q = e4m3(v * (448/amax)).  w f32 [n, k] (n, k % 128 == 0),
 * q [n, k], s [n/128, k/128]. */
void xo_quant_weight_fp8_block(const float *w, int64_t n, int64_t k, uint8_t *q, float *s);
/* Weight MXFP4: per (row, 32-column block) se = floor(log2(amax)) - 2,
 * q = e2m1(v * 2^-se).  q packed [n, k/2] (element 2i in the low nibble),
 * s [n, k/32] e8m0 bytes. */
void xo_quant_weight_mxfp4(const float *w, int64_t n, int64_t k, uint8_t *q, uint8_t *s);

/* ---------------- RMSNorm ---------------- */
/* y = x * inv_rms * w per row of `hidden` values, following the reference CPU
 * path xstar_cpp/src/ops/rmsnorm.cpp:27-73: sum of squares in f32 over the row
 * in order (product rounded, then sum rounded), inv_rms = 1 / sqrt(sum/hidden + eps)
 * with IEEE sqrt and division; f32: y = (x * inv_rms) * w; bf16:
 * y = bf16(f32(bf16(x * inv_rms)) * w).  x, w, y are f32 (is_bf16 = 0) or bf16
 * bits (is_bf16 = 1). */
void xo_rmsnorm(const void *x, const void *w, int is_bf16, int64_t rows, int64_t hidden, float eps, void *y);

/* ---------------- router ---------------- */
/* logits[t, e] = sum_kk x[t,kk] * Wr[e,kk] in gemm_cpu order (sequential kk,
 * separate multiply then add, f32).  x/Wr are f32 (is_bf16 = 0) or bf16 bits
 * (is_bf16 = 1).  gemm.h:57-83 with transB = true, linear.cpp:9-66. */
void xo_router_logits(const void *x, const void *wr, int is_bf16, int64_t T, int64_t E,
                      int64_t H, float *logits);

/* Top-k routing on f32 logits.
 * s_e = sigmoid(logit_e) (xo_sigmoid); key_e = s_e + bias_e (bias may be NULL).
 * Optional group-limited selection (n_group > 1): experts split into n_group
 * contiguous groups; group score = largest key + second largest key of the
 * group; keep the topk_group best groups (ties -> lower group index); other
 * experts are excluded.
 * Select the k largest keys (ties -> lower expert index), in descending order.
 * weights: w_j = s_j / (s_0 + ... + s_{k-1}) * scaling if renormalize,
 * else s_j * scaling.  idx [T,k] int32, w [T,k] f32. */
void xo_route(const float *logits, const float *bias, int64_t T, int64_t E, int64_t k,
              int64_t n_group, int64_t topk_group, int renormalize, float scaling,
              int32_t *idx, float *w);

/* Stable counting sort of the T*k slots (slot = t*k + j) by expert.
 * counts [E], offsets [E+1] (exclusive scan), perm [T*k] (position -> slot),
 * inv [T*k] (slot -> position). */
void xo_permute(const int32_t *idx, int64_t T, int64_t E, int64_t k, int32_t *counts,
                int32_t *offsets, int32_t *perm, int32_t *inv);

/* ---------------- full layer ---------------- */
typedef struct {
    int64_t T, H, I, E, k;
    int64_t n_group, topk_group;
    int renormalize;
    float scaling;
    int x_is_bf16;            /* x and router_w dtype: 1 = bf16 bits, 0 = f32 */
    int routed_fp4;           /* 0: routed experts FP8 128x128; 1: MXFP4 */
    int has_shared;
    int nthreads;             /* OpenMP threads for the expert GEMMs (1 = serial) */
} xo_moe_cfg;

typedef struct {
    const void *x;            /* [T, H] */
    const void *router_w;     /* [E, H] */
    const float *router_bias; /* [E] or NULL */
    const float *logits_in;   /* optional [T, E]: route on these instead of computing them */
    /* routed experts, FP8: w13 [E, 2I, H] e4m3, s13 [E, 2I/128, H/128] f32,
     *                      w2 [E, H, I] e4m3,  s2 [E, H/128, I/128] f32
     *                 FP4: w13 [E, 2I, H/2] e2m1x2, s13 [E, 2I, H/32] e8m0,
     *                      w2 [E, H, I/2] e2m1x2,  s2 [E, H, I/32] e8m0 */
    const uint8_t *w13; const void *s13;
    const uint8_t *w2;  const void *s2;
    /* shared expert, always FP8 128x128 (E = 1 shapes) */
    const uint8_t *sw13; const float *ss13;
    const uint8_t *sw2;  const float *ss2;
} xo_moe_inputs;

typedef struct {
    float *logits;    /* [T, E] (optional) */
    int32_t *idx;     /* [T, k] (optional) */
    float *w;         /* [T, k] (optional) */
    int32_t *counts;  /* [E]   (optional) */
    int32_t *offsets; /* [E+1] (optional) */
    int32_t *perm;    /* [T*k] (optional) */
    int32_t *inv;     /* [T*k] (optional) */
    float *out_f32;   /* [T, H] f32 combine before the final cast (optional) */
    void *out;        /* [T, H] bf16 bits (x_is_bf16) or f32 */
} xo_moe_outputs;

/* Quantized-path oracle ("dequantize then f32"): router -> route -> permute ->
 * per slot: a = dequant(xq) (FP8 1x128, or MXFP8 1x32 for FP4 experts),
 * [g ; u] = a . dequant(W13[e])^T (sequential-k f32), act = silu(g)*u (f32),
 * act quantized like the activations, y = act . dequant(W2[e])^T ->
 * out[t] = shared(t) + sum_j w_tj * y_tj (f32, in slot order), one final
 * cast (bf16 RNE or f32).  Returns 0 on success. */
int xo_moe_forward(const xo_moe_cfg *cfg, const xo_moe_inputs *in, xo_moe_outputs *out);

/* Reference-path fp32 MoE: the reference's CPU ops composed as a MoE layer.
 * Weights are dense f32, one pointer per expert (w13_tab[e] -> [2I,H],
 * w2_tab[e] -> [H,I]; NULL allowed for experts the tokens do not route to;
 * shared sw13 [2I,H] / sw2 [H,I] or NULL);
 * x f32 [T,H].  Router = linear (gemm_cpu order), route as xo_route, each
 * routed/shared expert = mlp() numerics (gemm_cpu i->kk->j loop with strided
 * transB reads, f32 silu*up), combine in f32.  This is the timed CPU baseline;
 * it runs single-threaded like the reference.  Only tokens [t0, t1) are
 * computed (bounded samples); routing still covers those tokens only. */
void xo_moe_ref_f32(const float *x, const float *router_w, const float *router_bias,
                    const float *const *w13_tab, const float *const *w2_tab, const float *sw13, const float *sw2,
                    int64_t T, int64_t H, int64_t I, int64_t E, int64_t k, int renormalize,
                    float scaling, int64_t t0, int64_t t1, float *out);

#ifdef __cplusplus
}
#endif
#endif
