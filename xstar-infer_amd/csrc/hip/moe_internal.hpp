// moe_internal.hpp -- declarations shared by the MoE translation units.
#pragma once

#include "xs_device.hpp"

namespace xs {

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(uint16_t v) { return f32_from_bf16(v); }

// 8 consecutive elements -> f32 (16-byte aligned for bf16, 32-byte for f32).
__device__ __forceinline__ void load8(const uint16_t *p, float *v)
{
    v4i r = *reinterpret_cast<const v4i *>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[2 * i] = __uint_as_float((uint32_t)r[i] << 16);
        v[2 * i + 1] = __uint_as_float((uint32_t)r[i] & 0xFFFF0000u);
    }
}
__device__ __forceinline__ void load8(const float *p, float *v)
{
    v4f a = *reinterpret_cast<const v4f *>(p);
    v4f b = *reinterpret_cast<const v4f *>(p + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[i] = a[i];
        v[4 + i] = b[i];
    }
}

// 4 consecutive elements -> f32 (8-byte aligned for bf16, 16-byte for f32).
__device__ __forceinline__ void load4(const uint16_t *p, float *v)
{
    v2i r = *reinterpret_cast<const v2i *>(p);
    v[0] = __uint_as_float((uint32_t)r[0] << 16);
    v[1] = __uint_as_float((uint32_t)r[0] & 0xFFFF0000u);
    v[2] = __uint_as_float((uint32_t)r[1] << 16);
    v[3] = __uint_as_float((uint32_t)r[1] & 0xFFFF0000u);
}
__device__ __forceinline__ void load4(const float *p, float *v)
{
    v4f a = *reinterpret_cast<const v4f *>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = a[i];
}

// 8 f32 values -> 8 consecutive outputs (bf16 RNE or f32).
__device__ __forceinline__ void store8(uint16_t *p, const float *v)
{
    v4i r;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        r[i] = (int)((uint32_t)bf16_from_f32(v[2 * i]) | ((uint32_t)bf16_from_f32(v[2 * i + 1]) << 16));
    *reinterpret_cast<v4i *>(p) = r;
}
__device__ __forceinline__ void store8(float *p, const float *v)
{
    *reinterpret_cast<v4f *>(p) = v4f{v[0], v[1], v[2], v[3]};
    *reinterpret_cast<v4f *>(p + 4) = v4f{v[4], v[5], v[6], v[7]};
}

// FP8 1x128 activation quant of 8 consecutive values held by one lane; the
// 16 lanes of an aligned 16-lane group hold one 128-column group.  amax over
// the group, inv = 448/amax, q = e4m3_rne(v * inv) (amax == 0: q = 0, scale 1),
// scale = amax/448 written through `s` by the group's first lane (s != null);
// q == null: the shuffles run, nothing is stored (lanes past the data).
__device__ __forceinline__ void quant8_fp8(const float *v, uint8_t *__restrict__ q, float *__restrict__ s)
{
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, __builtin_fabsf(v[i]));
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, WAVE));
    float inv = amax == 0.0f ? 0.0f : __fdiv_rn(448.0f, amax);
    // |v * inv| <= 448 (1 + 2^-22): clamped to the e4m3 range, the hardware
    // RNE converter gives the software encoder's codes (pinned by the GPU tests)
    float r[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = fminf(fmaxf(__fmul_rn(v[i], inv), -448.0f), 448.0f);
    uint32_t lo = e4m3_pack2_hw(r[0], r[1]) | (e4m3_pack2_hw(r[2], r[3]) << 16);
    uint32_t hi = e4m3_pack2_hw(r[4], r[5]) | (e4m3_pack2_hw(r[6], r[7]) << 16);
    if (amax == 0.0f) lo = hi = 0u;   // an all-zero group is code 0, also where its values are -0
    if (q) *reinterpret_cast<v2i *>(q) = v2i{(int)lo, (int)hi};
    if (s) *s = amax == 0.0f ? 1.0f : __fdiv_rn(amax, 448.0f);
}

struct CertState;
// ---- launchers (stream-ordered, no synchronisation) ----
// Router kind (XS_ROUTER_*) for params.router_exact and the input dtype.
int router_kind(int exact, int dtype);
// Number of K slices the bf16 MFMA router uses for T tokens (1 = no split).
int router_logits_splits(int64_t T, int64_t H, int exact, int dtype);
// Writes nsplit partial logit slices [nsplit][T][E] (nsplit = 1: the logits).
// mask_clear (optional): a [mask_words] bitmask zeroed by the same launch.
// q/qs (optional, decode path only: router_quantizes()): the FP8 1x128
// quantization of x, written by the same launch.
bool router_quantizes(int64_t T, int exact, int dtype);
// cert (certified router only): its dpart is written and its counters zeroed.
int launch_router_logits(const void *x, const void *wr, int dtype, int64_t T, int64_t E, int64_t H,
                         int exact, float *logits, int nsplit, hipStream_t st,
                         uint32_t *mask_clear = nullptr, int64_t mask_words = 0, uint8_t *q = nullptr,
                         float *qs = nullptr, const CertState *cert = nullptr);
// The certified router's device state for one forward (moe_router.hip):
// dpart [nsplit][T][E] error-bound terms of the MFMA logit slices, flog [T][E]
// logit rows of the tokens it could not settle, pairs [T*E][2] the (token,
// expert) logits to recompute exactly, cnt[2] {pairs, flagged tokens}
// (zeroed by the logits launch), flagged [T] with each token's pair range.
struct CertState {
    float *dpart;
    int kblocks;          // 32-wide K blocks per logit slice (H / nsplit / 32)
    float *flog;
    int32_t *pairs;
    int32_t *cnt;
    int32_t *flagged;
    int32_t *fbase;       // [T] first pair of flagged token j
    int32_t *fcnt;        // [T] its number of pairs
    float margin_scale;   // 1 (XS_ROUTER_MARGIN scales it: tests of the exact path)
};
// Routes on the sum (in slice order) of nsplit partial logit slices; writes the
// summed logits to logits_out when it is not NULL.  mode 0: plain; 1:
// certified (with cert: tokens it cannot settle are listed for the exact
// pass and left unrouted); 2: routes the listed tokens on cert->flog.
int launch_route(const float *logits, const float *bias, int64_t T, int64_t E, int64_t k,
                 int64_t n_group, int64_t topk_group, int renorm, float scaling, int32_t *idx,
                 float *w, uint32_t *mask, int mask_words, int nsplit, float *logits_out,
                 hipStream_t st, const CertState *cert = nullptr, int mode = 0);
// Certified routing of decode batches (T <= 256) in one launch, in place of
// launch_route: a block per token routes it and, when the bound leaves
// experts undecided, computes their logits in gemm_cpu order and routes again.
int launch_route_block(const void *x, const void *wr, int dtype, const float *logits, const float *bias, int64_t T,
                       int64_t E, int64_t H, int64_t k, int64_t n_group, int64_t topk_group, int renorm, float scaling,
                       int32_t *idx, float *w, uint32_t *mask, int mask_words, int nsplit, float *logits_out,
                       const CertState &cert, hipStream_t st);
// The exact (gemm_cpu order) logits of the listed pairs into cert->flog.
int launch_router_fix(const void *x, const void *wr, int dtype, int64_t T, int64_t E, int64_t H,
                      const CertState &cert, hipStream_t st);
// zero[0 .. zero_n) is cleared by the same launch (counters of a following kernel).
int launch_quant_act(const void *x, int dtype, int64_t rows, int64_t cols, uint8_t *q, void *s,
                     int mx, hipStream_t st, int32_t *zero = nullptr, int zero_n = 0);
// Dense FP8 block-scaled GEMM (gemm_dense.hip): C [M, N] bf16 = A [M, K] (e4m3,
// f32 1x128 row scales) . B [N, K]^T (e4m3, f32 128x128 block scales).  part
// (dense_part_bytes(M), the last 1 KB the counters) is used when the tiles do
// not fill the chip; the counters (dense_counters(M, N) of them) are zero on entry.
size_t dense_part_bytes(int64_t M);
int dense_counters(int64_t M, int64_t N);
int launch_gemm_dense(const uint8_t *A, const float *As, const uint8_t *B, const float *Bs, uint16_t *C,
                      int64_t M, int64_t N, int64_t K, float *part, int32_t *cnt, hipStream_t st);

// RMSNorm of rows x [rows, hidden] -> y (same dtype); with q/s non-null also the
// FP8 1x128 quantization of y (hidden % 128 == 0).
int launch_rmsnorm(const void *x, const void *w, int dtype, int64_t rows, int64_t hidden, float eps, void *y,
                   uint8_t *q, float *s, hipStream_t st);

// Permute.  Inputs: idx [T, k] and the per-expert token bitmasks built by the
// route kernel (mask [E+?][mask_words]).  Outputs positions sorted by
// (expert, token); a trailing shared-expert segment of T rows (identity) when
// shared_rows != 0.
struct PermuteOut {
    int32_t *counts;      // [E]
    int32_t *offsets;     // [E+1], or [E+2] with offsets_ext (shared-segment end at [E+1])
    int32_t *perm;        // position -> slot (or NULL)
    int32_t *inv;         // slot -> position (or NULL)
    int32_t *row_token;   // position -> token, routed then shared rows (or NULL)
    int32_t *tile_off;    // [E+2] exclusive scan of ceil(count / tile_bm), shared tiles last (or NULL)
    int32_t *tab;         // tile table (or NULL): entry 0 {tiles, shared tiles}, then
                          // {expert, first position, rows, t | nt << 16} (t: tile index within
                          // the expert, nt: the expert's tiles, both below 2^15 where used),
                          // the shared segment's tiles first
    int tile_bm;
    int offsets_ext;
    int32_t *zero;        // int32 words cleared by the scatter (or NULL): GEMM counters
    int64_t zero_n;
};
int mask_words_for(int64_t T);
int launch_mask_clear(uint32_t *mask, int64_t words, hipStream_t st);
size_t tile_table_bytes(int64_t rows_routed, int64_t rows_shared, int64_t E, int bm);
int launch_permute(const int32_t *idx, const uint32_t *mask, int64_t T, int64_t E, int64_t k,
                   int shared_rows, int32_t *wordprefix, const PermuteOut &o, hipStream_t st);

}  // namespace xs
