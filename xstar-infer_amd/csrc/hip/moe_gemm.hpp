// moe_gemm.hpp -- argument block and launchers of the grouped expert GEMMs.
#pragma once

#include "moe_internal.hpp"

namespace xs {

struct GemmArgs {
    const uint8_t *A;          // FP8 activation rows [*, K]
    const void *As;            // f32 [*, K/128] (FP8) or e8m0 [*, K/32] (MXFP8)
    const int32_t *row_token;  // position -> A row (NULL: A row = position)
    const uint8_t *B;          // routed weights [E, Nrows, K] (FP4: [E, Nrows, K/2])
    const void *Bs;            // routed scales
    const uint8_t *Bsh;        // shared expert weights (FP8), used for e == E
    const uint8_t *Bp;         // routed FP8 weights packed in fragment order (weight-direct kernels) or NULL
    const uint8_t *Bshp;       // shared expert weights packed in fragment order
    const uint8_t *Bsp;        // MXFP4: routed weight scales packed in fragment order (weight-direct kernels)
    const float *Bssh;         // shared expert scales
    const int32_t *offsets;    // [E+2] row offsets per expert (E = shared segment)
    const int32_t *tile_off;   // [E+2] tile offsets for tile height bm
    const int32_t *tile_tab;   // tile table (PermuteOut::tab) for tile height bm
    int e_lo, e_hi;            // experts covered by this launch: [e_lo, e_hi)
    int E;
    int K;                     // reduction length
    int N;                     // gate_up: I (output act columns); down: H
    int bm;                    // tile rows: 16, 32, 64 or 128
    int stream_w;              // tiled kernels: non-temporal weight loads (large launches)
    int xcd_order;             // tall-tile kernels: work grouped per XCD (set by launch_gemm_wide)
    int short_deep;            // tall-tile kernels: tiles of <= 64 rows run 64-row stages, 4 weight stages
    uint8_t *Cq;               // gate_up: act rows [*, I] FP8
    void *Cs;                  // gate_up: f32 [*, I/128] or e8m0 [*, I/32]
    uint16_t *Cy;              // down: bf16 rows [*, ldc] (the single GEMM's output)
    float *Cf;                 // down: f32 rows [*, ldc] (the MoE layer's per-slot outputs); set: used instead of Cy
    int64_t ldc;
    // down GEMM with the weighted combine fused into its epilogue (tall tiles):
    // each (token, 256-column slab) counter counts the token's rows stored so
    // far; the block whose rows complete a token sums them in f32 in the fixed
    // order (shared, then slots 0..k-1, then residual) and writes out.
    int fuse_combine;
    const int32_t *pos_token;  // position -> token (routed rows, then the shared segment)
    const int32_t *inv;        // [T, k] slot -> position
    const float *cw;           // [T, k] combine weights
    int topk;
    int has_shared;            // shared row of token t at position shared_base + t
    int64_t shared_base;
    // weight-direct prefill GEMM: > 0 = the launch covers the shared segment alone
    // (positions shared_base .., this many rows) in 128-row tiles of its own,
    // without a tile table
    int64_t sh_rows;
    int32_t *ccnt;             // [T, H/256] counters, zero on entry
    // tall-tile down GEMM over the shared segment alone, with the weighted
    // combine in its epilogue: each shared row's f32 result is summed with
    // its token's routed rows (Cf, written by the routed launch before) in
    // the combine's order and written to out; the shared row is not stored.
    // Uses inv, cw, topk, shared_base, out, residual, out_dtype.
    int shared_combine;
    void *out;                 // [T, H] of out_dtype
    const void *residual;      // [T, H] of out_dtype or NULL (may alias out)
    int out_dtype;
    // persistent (stream-K) kernels, moe_gemm_stream.hip:
    float *part;               // partial tiles of split items: stream_part_bytes()
    int32_t *cnt;              // per-item arrival counters, zero on entry
    int32_t *zero_cnt;         // counters of the next launch, zeroed here (or NULL)
    int zero_n;
};

int launch_gemm(const GemmArgs &a, bool gateup, bool fp4, int grid_y, hipStream_t st);
// Tall-tile FP8 GEMMs (moe_gemm_wide.hip): a.bm must be wide_tile_rows() and
// a.tile_tab the tile table for that height.
int wide_tile_rows();
int launch_gemm_wide(const GemmArgs &a, bool gateup, int grid_y, hipStream_t st);
// Weight-direct tall-tile FP8 GEMMs (moe_gemm_wd.hip): the same tiles and
// results as launch_gemm_wide, from fragment-packed weights (a.Bp, a.Bshp);
// gate_up, or down with f32 rows (a.Cf).
int launch_gemm_wd(const GemmArgs &a, bool gateup, int grid_y, hipStream_t st);
int wd_tile_rows();
// The single FP8 GEMM from fragment-packed B (moe_gemm_wd.hip): C [M, N] bf16 =
// A . B^T, 64-row tiles x 256-column slabs.  N a multiple of 256, K of 512.
int launch_gemm_wd_dense(const uint8_t *A, const float *As, const uint8_t *Bp, const float *Bs, uint16_t *C,
                         int64_t M, int64_t N, int64_t K, hipStream_t st);
bool wd_supported(int64_t H, int64_t I);   // the layer shapes the weight-direct kernels take
// Weight-direct decode GEMMs (moe_gemm_wdd.hip): 16-row tiles (a.bm 16), the
// same results as launch_gemm at that height, from fragment-packed weights;
// gate_up, or down with f32 rows (a.Cf).  K of 512, 1024, 2048 or 4096.
int launch_gemm_wdd(const GemmArgs &a, bool gateup, int grid_y, hipStream_t st);
bool wdd_supported(int64_t H, int64_t I);
// Weight-direct MXFP4 GEMMs (moe_gemm_wd4.hip): the routed tiles of a 64- or
// 128-row tile table, the same results as launch_gemm's MXFP4 tiles, from
// packed weights and scales (a.Bp, a.Bsp); gate_up, or down with f32 rows.
int launch_gemm_wd4(const GemmArgs &a, bool gateup, int grid_y, hipStream_t st);
bool wd4_supported(int64_t H, int64_t I);
// Persistent stream-K GEMMs (moe_gemm_stream.hip): FP8 with a.bm 16 or 32,
// MXFP4 with a.bm 16, 32 or 64.  tiles_max bounds the tile count of the
// launch's range of the tile table, rows_max the positions; a.cnt holds one
// counter per item, zero on entry.
int stream_blocks();
bool stream_fits(int bm, bool fp4, int64_t tiles_max, int64_t rows_max);
int64_t stream_items(bool gateup, int N, int64_t tiles_max);
size_t stream_part_bytes(int64_t items_max, int K, int bm);
int launch_gemm_stream(const GemmArgs &a, bool gateup, bool fp4, int tiles_max, int64_t rows_max, hipStream_t st);
int launch_combine(const float *y, const int32_t *inv, const float *w, int64_t T, int64_t k,
                   int64_t H, int64_t shared_base, int has_shared, void *out, int out_dtype,
                   hipStream_t st, const void *residual = nullptr);

}  // namespace xs
