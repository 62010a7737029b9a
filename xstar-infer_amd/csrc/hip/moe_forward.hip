// moe_forward.hip -- the whole MoE layer behind xs_moe_forward, and the single
// FP8 block-scaled GEMM behind xs_gemm_fp8_blockscale.
//
// Replaces mlp(x, gate_up_weight, down_weight) (xstar_cpp/src/ops/mlp.cpp:47-86)
// at the transformer_block call sites.  Every stage is enqueued on one stream
// with no host synchronisation.  Device memory comes only from the caller's
// workspace, laid out by WsLayout below.
#include "moe_gemm.hpp"

#include <cstdlib>
#include <cstring>
#include <mutex>

namespace xs {

static size_t al(size_t b) { return (b + 255) & ~(size_t)255; }

// ---- optional per-stage timing (xs_moe_profile_*) ----
// Stage boundaries: 0 act quant (+ RMSNorm) | 1 logits | 2 route | 3 permute | 4 gate_up |
// 5 down | 6 combine | 7 end.  One set of 8 events per forward, up to kProfMax
// forwards between two reads.
static constexpr int kStages = 7, kProfMax = 512;
static bool g_prof = false;
static int g_prof_n = 0;
static hipEvent_t g_prof_ev[kProfMax][kStages + 1];
static bool g_prof_made[kProfMax] = {};

static int prof_mark(int stage, hipStream_t st)
{
    if (!g_prof || g_prof_n >= kProfMax) return XS_OK;
    int s = g_prof_n;
    if (!g_prof_made[s]) {
        for (int i = 0; i <= kStages; ++i) XS_HIP(hipEventCreate(&g_prof_ev[s][i]));
        g_prof_made[s] = true;
    }
    XS_HIP(hipEventRecord(g_prof_ev[s][stage], st));
    if (stage == kStages) ++g_prof_n;
    return XS_OK;
}

struct WsLayout {
    size_t logits, dpart, flog, pairs, ccert, flagged, fbase, fcnt, idx, w, mask, wordprefix, counts, offsets, perm, inv, row_token, tiles, tiletab, part, cnt1, cnt2;
    size_t xn, xq, xs, xmq, xms, actq, acts, actms, y, ccnt;
    size_t total;
};

static int pick_bm(double rows_per_tile_group)
{
    if (rows_per_tile_group >= 96) return 128;
    if (rows_per_tile_group >= 48) return 64;
    if (rows_per_tile_group >= 24) return 32;
    return 16;
}

// GEMM family for the FP8 layer: the tall-tile kernels (moe_gemm_wide.hip) once
// experts average 32+ rows, else the 16..128-row tiles.  XS_MOE_GEMM=wide|tiled
// overrides (benchmarks, tests); read per call, since tests switch it.
static bool use_wide(const xs_moe_params *p)
{
    if (p->routed_format != XS_FP8_E4M3) return false;
    const char *force = getenv("XS_MOE_GEMM");
    if (force && !strcmp(force, "wide")) return true;
    if (force && !strcmp(force, "tiled")) return false;
    return p->T * p->top_k >= 32 * p->E;
}

// The routed (FP8: and shared) GEMMs may run the persistent kernels
// (moe_gemm_stream.hip) when the tall-tile FP8 kernels are not used:
// 0 never, 1 by size, 2 always.  XS_MOE_STREAM=0|1 forces (benchmarks, tests).
// An on/off switch from the environment, read per call (tests switch it).
static bool getenv_flag(const char *name, bool dflt)
{
    const char *v = getenv(name);
    return v ? v[0] != '0' : dflt;
}

// XS_FUSE_COMBINE=1: the tall-tile down GEMM sums each token's rows itself
// (moe_gemm_wide.hip, store_f32_tile) instead of the separate combine launch.
// Same bits; measured slower at prefill (the block that completes a token
// holds its CU through the gather), so it is off by default.
// The weight-direct GEMMs (moe_gemm_wd.hip, moe_gemm_wdd.hip, moe_gemm_wd4.hip
// and the packed single GEMM) run only when XS_WEIGHT_DIRECT=1: they have not
// yet passed a run on the card.  Off, a layer that also gives its row-major
// weights ignores the packed copies, and a packed-only layer or a packed GEMM
// is refused with XS_ERR_UNSUPPORTED.
static bool weight_direct_enabled() { return getenv_flag("XS_WEIGHT_DIRECT", false); }

// XS_ROUTER_MARGIN=<f>: scales the certified router's key margins (tests of
// the exact pass: a large value sends every token through it).  Default 1.
static float router_margin_scale()
{
    const char *v = getenv("XS_ROUTER_MARGIN");
    const float f = v ? strtof(v, nullptr) : 1.0f;
    return f >= 1.0f ? f : 1.0f;
}

static bool fuse_combine(const xs_moe_params *p)
{
    return use_wide(p) && getenv_flag("XS_FUSE_COMBINE", false);
}

static int use_stream(const xs_moe_params *p)
{
    if (p->routed_format == XS_FP8_E4M3 && use_wide(p)) return 0;
    const char *force = getenv("XS_MOE_STREAM");   // read per call: tests switch it
    if (force && !strcmp(force, "0")) return 0;
    if (force && !strcmp(force, "1")) return 2;
    return 1;
}

// Upper bound of the tile count at 16-row tiles (the smallest height).
static int64_t tiles16_max(const xs_moe_params *p)
{
    const int64_t S = p->T * p->top_k;
    return S / 16 + (p->E < S ? p->E : S) + (p->has_shared ? (p->T + 15) / 16 : 0);
}

static WsLayout layout(const xs_moe_params *p)
{
    const size_t T = (size_t)p->T, H = (size_t)p->H, I = (size_t)p->I, E = (size_t)p->E, k = (size_t)p->top_k;
    const size_t S = T * k, R = S + (p->has_shared ? T : 0);
    const size_t W = (size_t)mask_words_for(p->T);
    const bool fp4 = p->routed_format == XS_FP4_E2M1X2;
    WsLayout L = {};
    size_t o = 0;
    auto take = [&](size_t &field, size_t bytes) { field = o; o += al(bytes); };
    const size_t nsplit = (size_t)router_logits_splits(p->T, p->H, p->router_exact, p->x_dtype);
    take(L.logits, 4 * T * E * nsplit);
    // the certified router: bound terms, logit rows and pairs of the tokens it
    // lists (at most every logit), its two counters
    const bool cert = router_kind(p->router_exact, p->x_dtype) == XS_ROUTER_CERTIFIED;
    take(L.dpart, cert ? 4 * T * E * nsplit : 0);
    take(L.flog, cert ? 4 * T * E : 0);
    take(L.pairs, cert ? 8 * T * E : 0);
    take(L.ccert, cert ? 8 : 0);
    take(L.flagged, cert ? 4 * T : 0);
    take(L.fbase, cert ? 4 * T : 0);
    take(L.fcnt, cert ? 4 * T : 0);
    take(L.idx, 4 * S);
    take(L.w, 4 * S);
    take(L.mask, 4 * W * E);
    take(L.wordprefix, 4 * W * E);
    take(L.counts, 4 * E);
    take(L.offsets, 4 * (E + 2));
    take(L.perm, 4 * S);
    take(L.inv, 4 * S);
    take(L.row_token, 4 * R);
    take(L.tiles, 4 * (E + 2));
    take(L.tiletab, tile_table_bytes((int64_t)S, p->has_shared ? (int64_t)T : 0, (int64_t)E, 16));
    {
        const bool st = use_stream(p);
        const int64_t n1 = st ? stream_items(true, (int)I, tiles16_max(p)) : 0;
        const int64_t n2 = st ? stream_items(false, (int)H, tiles16_max(p)) : 0;
        const int pbm = fp4 ? 64 : 32;
        const size_t p1 = st ? stream_part_bytes(n1, (int)H, pbm) : 0, p2 = st ? stream_part_bytes(n2, (int)I, pbm) : 0;
        take(L.part, p1 > p2 ? p1 : p2);
        take(L.cnt1, st ? 4 * (size_t)(n1 + 1) : 0);
        take(L.cnt2, st ? 4 * (size_t)(n2 + 1) : 0);
    }
    take(L.xn, p->has_norm ? T * H * (p->x_dtype == XS_BF16 ? 2 : 4) : 0);
    take(L.xq, T * H);
    take(L.xs, 4 * T * (H / 128));
    take(L.xmq, fp4 ? T * H : 0);
    take(L.xms, fp4 ? T * (H / 32) : 0);
    take(L.actq, R * I);
    take(L.acts, 4 * R * (I / 128));
    take(L.actms, fp4 ? S * (I / 32) : 0);
    take(L.y, 4 * R * H);
    take(L.ccnt, fuse_combine(p) ? 4 * T * (H / 256) : 0);
    L.total = o;
    return L;
}

static int check_params(const xs_moe_params *p)
{
    XS_REQUIRE(p != nullptr, "params is null");
    XS_REQUIRE(p->T >= 0 && p->T < (1 << 24), "T out of range");
    XS_REQUIRE(p->H >= 256 && p->H % 256 == 0, "shape mismatch: H must be a multiple of 256");
    XS_REQUIRE(p->I >= 128 && p->I % 128 == 0, "shape mismatch: I must be a multiple of 128");
    XS_REQUIRE(p->E >= 1 && p->E <= 1024, "E must be in [1, 1024]");
    XS_REQUIRE(p->top_k >= 1 && p->top_k <= 16 && p->top_k <= p->E, "top_k must be in [1, min(16, E)]");
    XS_REQUIRE(p->x_dtype == XS_BF16 || p->x_dtype == XS_F32, "unsupported dtype");
    XS_REQUIRE(p->routed_format == XS_FP8_E4M3 || p->routed_format == XS_FP4_E2M1X2,
               "unsupported routed expert format");
    XS_REQUIRE(p->T * p->top_k + p->T < ((int64_t)1 << 31), "too many rows");
    // the certified router lists (token, expert) pairs with 32-bit counters
    XS_REQUIRE(p->T * p->E < ((int64_t)1 << 31), "too many logits: T x E must stay below 2^31 (split the batch)");
    // the GEMMs address gathered activation rows with 32-bit lane offsets:
    // token x H bytes (gate_up) and position x I bytes (down) stay below 4 GiB
    XS_REQUIRE(p->T * p->H < ((int64_t)1 << 32) && (p->T * p->top_k + p->T) * p->I < ((int64_t)1 << 32),
               "too many rows: T x H and T x (top_k + 1) x I must stay below 2^32 (split the batch)");
    XS_REQUIRE(p->has_norm == 0 || p->has_norm == 1, "has_norm must be 0 or 1");
    XS_REQUIRE(p->router_exact >= XS_ROUTER_MFMA && p->router_exact <= XS_ROUTER_CHAIN,
               "router_exact must be XS_ROUTER_MFMA, XS_ROUTER_CERTIFIED or XS_ROUTER_CHAIN");
    XS_REQUIRE(p->routed_format != XS_FP4_E2M1X2 || p->I % 256 == 0,
               "shape mismatch: MXFP4 experts need I to be a multiple of 256");
    if (p->n_group > 1) {
        XS_REQUIRE(p->n_group <= 64 && p->E % p->n_group == 0 && p->E / p->n_group >= 2,
                   "n_group must divide E into groups of >= 2 (n_group <= 64)");
        XS_REQUIRE(p->topk_group >= 1 && p->topk_group <= p->n_group &&
                       p->topk_group * (p->E / p->n_group) >= p->top_k,
                   "topk_group must keep at least top_k experts");
    }
    return XS_OK;
}

// The kernels of one forward: the tile height and each GEMM's family.
struct Plan {
    int bm;
    bool wide, fused, direct, ddirect, direct4, sdirect, stream;
    bool shcomb;   // tall-tile down GEMM: routed launch, then the shared segment with the combine in its epilogue
};

static int make_plan(const xs_moe_params *p, const xs_moe_tensors *t, Plan &pl)
{
    const int64_t T = p->T, H = p->H, I = p->I, E = p->E, k = p->top_k;
    const int64_t S = T * k;
    const bool fp4 = p->routed_format == XS_FP4_E2M1X2;
    const int shared_rows = p->has_shared ? (int)T : 0;
    const bool packed_only = !t->w13 && !t->w2;
    const bool wide = use_wide(p);
    const bool fused = fuse_combine(p) && !packed_only;
    // Weight-direct GEMMs (fragment-packed weights loaded straight into
    // registers) when the layer gives the packed copies: the tall tiles of
    // prefill (moe_gemm_wd.hip), the 16-row decode tiles (moe_gemm_wdd.hip),
    // MXFP4 routed experts on 64- and 128-row tiles (moe_gemm_wd4.hip) with
    // their FP8 shared expert on the prefill kernel in 128-row tiles of its
    // own.  XS_WIDE_DIRECT / XS_DECODE_DIRECT / XS_FP4_DIRECT = 0 keep the
    // LDS-ring, tiled and stream-K kernels (measurements, tests).  A
    // packed-only layer always takes them: FP8 batches that are not 16-row
    // decode go to the 128-row prefill kernel (the extra rows of short tiles
    // cost MFMA time that the weight stream hides), MXFP4 batches to 64-row
    // tiles at least.
    const bool sh_frag = !p->has_shared || (t->shared_w13_frag && t->shared_w2_frag);
    const bool frag8 = !fp4 && t->w13_frag && t->w2_frag && sh_frag;
    const bool frag4 = fp4 && t->w13_frag && t->w2_frag && t->w13_scale_frag && t->w2_scale_frag;
    int bm = pick_bm((double)S / (double)E);
    bool direct, ddirect, direct4;
    if (packed_only && !weight_direct_enabled())
        return set_error(XS_ERR_UNSUPPORTED,
                         "packed-only layer: the weight-direct GEMMs are off (XS_WEIGHT_DIRECT=1 enables them)");
    if (packed_only) {
        if (fp4 && bm < 64) bm = 64;
        ddirect = !fp4 && bm == 16 && wdd_supported(H, I);
        direct = !fp4 && !ddirect && wd_supported(H, I);
        direct4 = fp4 && wd4_supported(H, I);
        if (!direct && !ddirect && !direct4)
            return set_error(XS_ERR_UNSUPPORTED, "packed-only layer: no weight-direct GEMM for H=%lld I=%lld",
                             (long long)H, (long long)I);
    } else {
        const bool wd_on = weight_direct_enabled();
        direct = wd_on && wide && !fused && frag8 && wd_supported(H, I) && getenv_flag("XS_WIDE_DIRECT", true);
        ddirect = wd_on && !wide && frag8 && bm == 16 && wdd_supported(H, I) && getenv_flag("XS_DECODE_DIRECT", true);
        direct4 = wd_on && frag4 && (bm == 64 || bm == 128) && wd4_supported(H, I) && getenv_flag("XS_FP4_DIRECT", true);
    }
    const bool sdirect = direct4 && shared_rows && t->shared_w13_frag && t->shared_w2_frag && wd_supported(H, I);
    if (packed_only && fp4 && shared_rows && !sdirect)
        return set_error(XS_ERR_UNSUPPORTED, "packed-only layer: no weight-direct GEMM for the shared expert");
    if (direct) bm = wd_tile_rows();
    else if (wide && !packed_only) bm = wide_tile_rows();
    const int routed_tiles = (int)(S / bm + (E < S ? E : S));
    const int shared_tiles = (int)((shared_rows + bm - 1) / bm);
    // Persistent GEMMs once the gate_up work (items of one tile x one 256-row
    // slab) fills every CU twice; below that, whole items per block split
    // less and the one-block-per-tile kernels are faster.
    const int sm = use_stream(p);
    const int64_t rows_all = S + shared_rows;
    // FP8: all tiles in one launch; MXFP4: the routed tiles (the FP8 shared
    // expert runs a launch of its own: tiled, or weight-direct)
    const int stream_tiles = fp4 ? routed_tiles : routed_tiles + shared_tiles;
    const bool stream = !direct && !ddirect && !direct4 && stream_fits(bm, fp4, stream_tiles, rows_all) && (!fp4 || (H % 512 == 0 && I % 512 == 0)) &&
                        (sm == 2 || (sm == 1 && stream_items(true, (int)I, stream_tiles) >= 2 * (int64_t)stream_blocks()));
    // XS_SHARED_COMBINE=1: the combine in the shared expert's down epilogue
    // (tall tiles; not with the y_rows inspection output, which needs the
    // shared rows stored)
    const bool shcomb = wide && !packed_only && !fused && !direct && shared_rows && !t->y_rows &&
                        getenv_flag("XS_SHARED_COMBINE", false);
    pl = Plan{bm, wide, fused, direct, ddirect, direct4, sdirect, stream, shcomb};
    return XS_OK;
}

// The tensors of a forward: present where the params need them, aligned.
static int check_tensors(const xs_moe_params *p, const xs_moe_tensors *t)
{
    XS_REQUIRE(t && t->x && t->router_w && t->out, "null pointer");
    // packed-only layer: the routed weights are given only in fragment order
    // (w13 / w2 NULL, w13_frag / w2_frag set; MXFP4: with their packed scales)
    const bool packed_only = !t->w13 && !t->w2;
    const bool fp4_layer = p->routed_format == XS_FP4_E2M1X2;
    if (packed_only) {
        XS_REQUIRE(t->w13_frag && t->w2_frag && (!fp4_layer || (t->w13_scale_frag && t->w2_scale_frag)) &&
                       (fp4_layer || (t->w13_scale && t->w2_scale)),
                   "null pointer: a layer without w13 / w2 needs their packed copies (and scales)");
        XS_REQUIRE(!p->has_shared || (t->shared_w13_frag && t->shared_w2_frag && t->shared_w13_scale &&
                                      t->shared_w2_scale),
                   "null shared expert pointer: a packed-only layer needs the shared expert's packed copies");
    } else {
        XS_REQUIRE(t->w13 && t->w13_scale && t->w2 && t->w2_scale, "null pointer");
        XS_REQUIRE(!p->has_shared || (t->shared_w13 && t->shared_w13_scale && t->shared_w2 && t->shared_w2_scale),
                   "null shared expert pointer");
    }
    XS_REQUIRE(!p->has_norm || t->norm_weight, "null norm weight");
    XS_REQUIRE(((uintptr_t)t->x & 15) == 0 && ((uintptr_t)t->out & 15) == 0 &&
                   ((uintptr_t)t->residual & 15) == 0,
               "misaligned operand: x, out and residual need 16-byte alignment");
    XS_REQUIRE(((uintptr_t)t->w13 & 15) == 0 && ((uintptr_t)t->w2 & 15) == 0 &&
                   ((uintptr_t)t->shared_w13 & 15) == 0 && ((uintptr_t)t->shared_w2 & 15) == 0 &&
                   ((uintptr_t)t->router_w & 15) == 0,
               "misaligned operand: weights need 16-byte alignment");
    XS_REQUIRE(((uintptr_t)t->w13_frag & 15) == 0 && ((uintptr_t)t->w2_frag & 15) == 0 &&
                   ((uintptr_t)t->shared_w13_frag & 15) == 0 && ((uintptr_t)t->shared_w2_frag & 15) == 0,
               "misaligned operand: packed weights need 16-byte alignment");
    return XS_OK;
}

int moe_forward(const xs_moe_params *p, const xs_moe_tensors *t, void *ws, size_t ws_bytes,
                hipStream_t st)
{
    int rc = check_params(p);
    if (rc) return rc;
    if (p->T == 0) return XS_OK;   // empty input: nothing is read or written (its tensors may be null)
    if ((rc = check_tensors(p, t))) return rc;
    const WsLayout L = layout(p);
    XS_REQUIRE(ws != nullptr || L.total == 0, "workspace is null");
    if (ws_bytes < L.total) return set_error(XS_ERR_WORKSPACE, "workspace too small: %zu < %zu", ws_bytes, L.total);
    XS_REQUIRE(((uintptr_t)ws & 255) == 0, "workspace must be 256-byte aligned");
    const int64_t T = p->T, H = p->H, I = p->I, E = p->E, k = p->top_k;
    if (T == 0) return XS_OK;
    const int64_t S = T * k;
    const bool fp4 = p->routed_format == XS_FP4_E2M1X2;
    const int shared_rows = p->has_shared ? (int)T : 0;
    char *base = (char *)ws;
#define WS(type, field) reinterpret_cast<type *>(base + L.field)
    float *logits = WS(float, logits);
    int32_t *idx = WS(int32_t, idx);
    float *w = WS(float, w);
    uint32_t *mask = WS(uint32_t, mask);
    int32_t *offsets = WS(int32_t, offsets);
    int32_t *inv = WS(int32_t, inv);
    int32_t *tiles = WS(int32_t, tiles);
    const int Wd = mask_words_for(T);

    // 1. activation quantization (once per token, gathered by the GEMMs),
    //    with the optional RMSNorm fused in front of it
    if ((rc = prof_mark(0, st))) return rc;
    const void *xin = t->x;
    const bool fp8_act = !fp4 || p->has_shared;
    if (p->has_norm) {
        void *xn = WS(void, xn);
        rc = launch_rmsnorm(t->x, t->norm_weight, p->x_dtype, T, H, p->norm_eps, xn,
                            fp8_act ? WS(uint8_t, xq) : nullptr, fp8_act ? WS(float, xs) : nullptr, st);
        if (rc) return rc;
        xin = xn;
    }
    // small batches: the decode router writes the FP8 activations in its own launch
    const bool fold_quant = !p->has_norm && fp8_act && router_quantizes(T, p->router_exact, p->x_dtype) &&
                            getenv_flag("XS_FOLD_QUANT", true);
    if (!p->has_norm && fp8_act && !fold_quant) {
        rc = launch_quant_act(xin, p->x_dtype, T, H, WS(uint8_t, xq), WS(float, xs), 0, st);
        if (rc) return rc;
    }
    if (fp4) {
        rc = launch_quant_act(xin, p->x_dtype, T, H, WS(uint8_t, xmq), WS(uint8_t, xms), 1, st);
        if (rc) return rc;
    }
    // 2. router: logits -> top-k + per-expert token masks
    if ((rc = prof_mark(1, st))) return rc;
    const int nsplit = router_logits_splits(T, H, p->router_exact, p->x_dtype);
    const bool certified = router_kind(p->router_exact, p->x_dtype) == XS_ROUTER_CERTIFIED;
    CertState cs = {};
    if (certified) {
        cs.dpart = WS(float, dpart);
        cs.kblocks = (int)(H / nsplit / 32);
        cs.flog = WS(float, flog);
        cs.pairs = WS(int32_t, pairs);
        cs.cnt = WS(int32_t, ccert);
        cs.flagged = WS(int32_t, flagged);
        cs.fbase = WS(int32_t, fbase);
        cs.fcnt = WS(int32_t, fcnt);
        cs.margin_scale = router_margin_scale();
    }
    rc = launch_router_logits(xin, t->router_w, p->x_dtype, T, E, H, p->router_exact, logits, nsplit, st, mask,
                              (int64_t)Wd * E, fold_quant ? WS(uint8_t, xq) : nullptr,
                              fold_quant ? WS(float, xs) : nullptr, certified ? &cs : nullptr);
    if (rc) return rc;
    if ((rc = prof_mark(2, st))) return rc;
    if (certified && T <= 256) {
        // decode batches: routing, the exact pass of the pairs the bound
        // leaves undecided and the second routing in the one route launch
        rc = launch_route_block(xin, t->router_w, p->x_dtype, logits, t->router_bias, T, E, H, k, p->n_group,
                                p->topk_group, p->renormalize, p->routed_scaling, idx, w, mask, Wd, nsplit, t->logits,
                                cs, st);
        if (rc) return rc;
    } else {
        rc = launch_route(logits, t->router_bias, T, E, k, p->n_group, p->topk_group, p->renormalize,
                          p->routed_scaling, idx, w, mask, Wd, nsplit, t->logits, st, certified ? &cs : nullptr,
                          certified ? 1 : 0);
        if (rc) return rc;
    }
    if (certified && T > 256) {
        // prefill: the undecided pairs in gemm_cpu order spread over blocks,
        // then the listed tokens' routing on their patched logit rows
        if ((rc = launch_router_fix(xin, t->router_w, p->x_dtype, T, E, H, cs, st))) return rc;
        rc = launch_route(logits, t->router_bias, T, E, k, p->n_group, p->topk_group, p->renormalize,
                          p->routed_scaling, idx, w, mask, Wd, 1, t->logits, st, &cs, 2);
        if (rc) return rc;
    }
    // 3. permute: (expert, token)-sorted positions, tile offsets
    if ((rc = prof_mark(3, st))) return rc;
    Plan pl;
    if ((rc = make_plan(p, t, pl))) return rc;
    const bool wide = pl.wide, fused = pl.fused, direct = pl.direct, ddirect = pl.ddirect, direct4 = pl.direct4,
               sdirect = pl.sdirect;
    const int bm = pl.bm;
    PermuteOut po = {};
    po.counts = WS(int32_t, counts);
    po.offsets = offsets;
    po.perm = WS(int32_t, perm);
    po.inv = inv;
    po.row_token = WS(int32_t, row_token);
    po.tile_off = tiles;
    po.tab = WS(int32_t, tiletab);
    po.tile_bm = bm;
    po.offsets_ext = 1;

    const int routed_tiles = (int)(S / bm + (E < S ? E : S));
    const int shared_tiles = (int)((shared_rows + bm - 1) / bm);
    const int64_t rows_all = S + shared_rows;
    const int stream_tiles = fp4 ? routed_tiles : routed_tiles + shared_tiles;
    const bool stream = pl.stream;
    if (stream) {
        po.zero = WS(int32_t, cnt1);
        po.zero_n = stream_items(true, (int)I, tiles16_max(p)) + 1;
    } else if (fused) {
        po.zero = WS(int32_t, ccnt);
        po.zero_n = T * (H / 256);
    }
    rc = launch_permute(idx, mask, T, E, k, shared_rows, WS(int32_t, wordprefix), po, st);
    if (rc) return rc;

    // 4. gate_up GEMM + SwiGLU + activation re-quant
    GemmArgs g1 = {};
    g1.row_token = po.row_token;
    g1.B = (const uint8_t *)t->w13;
    g1.Bs = t->w13_scale;
    g1.Bsh = (const uint8_t *)t->shared_w13;
    g1.Bp = (const uint8_t *)t->w13_frag;
    g1.Bshp = (const uint8_t *)t->shared_w13_frag;
    g1.Bssh = t->shared_w13_scale;
    g1.offsets = offsets;
    g1.tile_off = tiles;
    g1.tile_tab = po.tab;
    g1.E = (int)E;
    g1.K = (int)H;
    g1.N = (int)I;
    g1.bm = bm;
    g1.Cq = WS(uint8_t, actq);
    GemmArgs g2 = {};
    g2.row_token = nullptr;
    g2.A = WS(uint8_t, actq);
    g2.B = (const uint8_t *)t->w2;
    g2.Bs = t->w2_scale;
    g2.Bsh = (const uint8_t *)t->shared_w2;
    g2.Bp = (const uint8_t *)t->w2_frag;
    g2.Bshp = (const uint8_t *)t->shared_w2_frag;
    g2.Bssh = t->shared_w2_scale;
    g2.offsets = offsets;
    g2.tile_off = tiles;
    g2.tile_tab = po.tab;
    g2.E = (int)E;
    g2.K = (int)I;
    g2.N = (int)H;
    g2.bm = bm;
    g2.Cf = WS(float, y);
    g2.ldc = H;
    if (fused) {
        g2.fuse_combine = 1;
        g2.pos_token = po.row_token;
        g2.inv = inv;
        g2.cw = w;
        g2.topk = (int)k;
        g2.has_shared = shared_rows ? 1 : 0;
        g2.shared_base = S;
        g2.ccnt = WS(int32_t, ccnt);
        g2.out = t->out;
        g2.residual = t->residual;
        g2.out_dtype = p->x_dtype;
    }

    if (stream) {
        g1.part = g2.part = WS(float, part);
        g1.cnt = WS(int32_t, cnt1);
        g2.cnt = g1.zero_cnt = WS(int32_t, cnt2);
        g1.zero_n = (int)stream_items(false, (int)H, tiles16_max(p)) + 1;
    }

    if ((rc = prof_mark(4, st))) return rc;
    if (!fp4) {
        g1.A = WS(uint8_t, xq);
        g1.As = WS(float, xs);
        g1.Cs = WS(float, acts);
        g1.e_lo = 0;
        g1.e_hi = (int)E + (shared_rows ? 1 : 0);
        rc = stream   ? launch_gemm_stream(g1, true, false, stream_tiles, rows_all, st)
             : direct ? launch_gemm_wd(g1, true, routed_tiles + shared_tiles, st)
             : ddirect ? launch_gemm_wdd(g1, true, routed_tiles + shared_tiles, st)
             : wide   ? launch_gemm_wide(g1, true, routed_tiles + shared_tiles, st)
                    : launch_gemm(g1, true, false, routed_tiles + shared_tiles, st);
        if (rc) return rc;
        if ((rc = prof_mark(5, st))) return rc;
        g2.As = WS(float, acts);
        g2.e_lo = 0;
        g2.e_hi = g1.e_hi;
        if (pl.shcomb) {
            // the routed rows first, then the shared segment, whose epilogue
            // sums each token's rows in the combine's order and writes out
            GemmArgs gr = g2;
            gr.e_hi = (int)E;
            if ((rc = launch_gemm_wide(gr, false, routed_tiles, st))) return rc;
            GemmArgs gs = g2;
            gs.e_lo = (int)E;
            gs.shared_combine = 1;
            gs.inv = inv;
            gs.cw = w;
            gs.topk = (int)k;
            gs.shared_base = S;
            gs.out = t->out;
            gs.residual = t->residual;
            gs.out_dtype = p->x_dtype;
            rc = launch_gemm_wide(gs, false, shared_tiles, st);
        } else
        rc = stream   ? launch_gemm_stream(g2, false, false, stream_tiles, rows_all, st)
             : direct ? launch_gemm_wd(g2, false, routed_tiles + shared_tiles, st)
             : ddirect ? launch_gemm_wdd(g2, false, routed_tiles + shared_tiles, st)
             : wide   ? launch_gemm_wide(g2, false, routed_tiles + shared_tiles, st)
                    : launch_gemm(g2, false, false, routed_tiles + shared_tiles, st);
        if (rc) return rc;
    } else {
        GemmArgs r1 = g1;
        r1.A = WS(uint8_t, xmq);
        r1.As = WS(uint8_t, xms);
        r1.Cs = WS(uint8_t, actms);
        r1.e_lo = 0;
        r1.e_hi = (int)E;
        r1.Bsp = (const uint8_t *)t->w13_scale_frag;
        rc = stream    ? launch_gemm_stream(r1, true, true, stream_tiles, rows_all, st)
             : direct4 ? launch_gemm_wd4(r1, true, routed_tiles, st)
                       : launch_gemm(r1, true, true, routed_tiles, st);
        if (rc) return rc;
        if (shared_rows) {
            GemmArgs s1 = g1;
            s1.A = WS(uint8_t, xq);
            s1.As = WS(float, xs);
            s1.Cs = WS(float, acts);
            s1.e_lo = (int)E;
            s1.e_hi = (int)E + 1;
            s1.Bp = nullptr;
            s1.sh_rows = sdirect ? shared_rows : 0;
            s1.shared_base = S;
            rc = sdirect ? launch_gemm_wd(s1, true, (int)((shared_rows + wd_tile_rows() - 1) / wd_tile_rows()), st)
                         : launch_gemm(s1, true, false, shared_tiles, st);
            if (rc) return rc;
        }
        if ((rc = prof_mark(5, st))) return rc;
        GemmArgs r2 = g2;
        r2.As = WS(uint8_t, actms);
        r2.e_lo = 0;
        r2.e_hi = (int)E;
        r2.Bsp = (const uint8_t *)t->w2_scale_frag;
        rc = stream    ? launch_gemm_stream(r2, false, true, stream_tiles, rows_all, st)
             : direct4 ? launch_gemm_wd4(r2, false, routed_tiles, st)
                       : launch_gemm(r2, false, true, routed_tiles, st);
        if (rc) return rc;
        if (shared_rows) {
            GemmArgs s2 = g2;
            s2.As = WS(float, acts);
            s2.e_lo = (int)E;
            s2.e_hi = (int)E + 1;
            s2.Bp = nullptr;
            s2.sh_rows = sdirect ? shared_rows : 0;
            s2.shared_base = S;
            rc = sdirect ? launch_gemm_wd(s2, false, (int)((shared_rows + wd_tile_rows() - 1) / wd_tile_rows()), st)
                         : launch_gemm(s2, false, false, shared_tiles, st);
            if (rc) return rc;
        }
    }
    // 5. weighted combine (+ shared), one cast to the output dtype
    if ((rc = prof_mark(6, st))) return rc;
    if (!fused && !pl.shcomb) {
        rc = launch_combine(WS(float, y), inv, w, T, k, H, S, shared_rows ? 1 : 0, t->out, p->x_dtype, st,
                            t->residual);
        if (rc) return rc;
    }
    if ((rc = prof_mark(7, st))) return rc;

    // optional inspection outputs
    auto cp = [&](void *dst, const void *src, size_t bytes) -> int {
        if (dst && bytes) XS_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, st));
        return XS_OK;
    };
    if ((rc = cp(t->topk_idx, idx, 4 * (size_t)S))) return rc;
    if ((rc = cp(t->topk_w, w, 4 * (size_t)S))) return rc;
    if ((rc = cp(t->counts, po.counts, 4 * (size_t)E))) return rc;
    if ((rc = cp(t->offsets, offsets, 4 * (size_t)(E + 1)))) return rc;
    if ((rc = cp(t->perm, po.perm, 4 * (size_t)S))) return rc;
    if ((rc = cp(t->inv, inv, 4 * (size_t)S))) return rc;
    const size_t R = (size_t)(S + shared_rows);
    if (!fp4) {
        if ((rc = cp(t->act_q, WS(uint8_t, actq), R * (size_t)I))) return rc;
        if ((rc = cp(t->act_s, WS(float, acts), 4 * R * (size_t)(I / 128)))) return rc;
    }
    if ((rc = cp(t->y_rows, WS(float, y), 4 * R * (size_t)H))) return rc;
#undef WS
    return XS_OK;
}

// --------------------------------------------------- single FP8 GEMM (C = A.B^T)
// Workspace: A quantized [M, K] e4m3 + [M, K/128] f32, then the dense kernel's
// partial tiles and counters (only when M is small enough for split-K).
static size_t gemm_ws(int64_t M, int64_t K, size_t *o_s, size_t *o_part)
{
    size_t q = al((size_t)M * K);
    size_t s = al(4 * (size_t)M * (K / 128));
    *o_s = q;
    *o_part = q + s;
    return q + s + al(dense_part_bytes(M));
}

// ------------------------------------------- forward without a caller workspace
// The workspace of xs_moe_forward_noalloc: a fixed device array in the code
// object, one copy per GPU, held until the process ends.  Host code never
// passes `scratch` itself (on the host it names a stand-in, not device
// memory): each device's address comes from hipGetSymbolAddress, taken once
// per device with that device current.
static constexpr size_t kNoallocScratch = (size_t)XS_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kNoallocScratch];

static constexpr int kMaxDevices = 64;
static void *g_scratch_ptr[kMaxDevices] = {};
static std::mutex g_scratch_mu;

static int scratch_for_current_device(void **out)
{
    int dev = 0;
    XS_HIP(hipGetDevice(&dev));
    XS_REQUIRE(dev >= 0 && dev < kMaxDevices, "device index %d beyond %d", dev, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        XS_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        XS_REQUIRE(p != nullptr && ((uintptr_t)p & 255) == 0, "scratch symbol address is null or misaligned");
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return XS_OK;
}

}  // namespace xs

using namespace xs;

extern "C" {

size_t xs_moe_noalloc_scratch_bytes(void) { return kNoallocScratch; }

int xs_moe_forward_noalloc(const xs_moe_params *p, const xs_moe_tensors *t, void *stream)
{
    int rc = check_params(p);
    if (rc) return rc;
    const size_t need = layout(p).total;
    if (need > kNoallocScratch)
        return set_error(XS_ERR_WORKSPACE,
                         "xs_moe_forward_noalloc: these params need %zu bytes of scratch; the static scratch holds %zu "
                         "(use xs_moe_forward with a workspace)",
                         need, kNoallocScratch);
    void *ws = nullptr;
    if ((rc = scratch_for_current_device(&ws))) return rc;
    return moe_forward(p, t, ws, kNoallocScratch, (hipStream_t)stream);
}

size_t xs_moe_workspace_size(const xs_moe_params *p)
{
    if (check_params(p)) return 0;
    return layout(p).total;
}

int xs_moe_router_stats(const xs_moe_params *p, const void *workspace, int64_t out[2], void *stream)
{
    XS_REQUIRE(out != nullptr, "null pointer");
    int rc = check_params(p);
    if (rc) return rc;
    out[0] = out[1] = 0;
    if (p->T == 0 || router_kind(p->router_exact, p->x_dtype) != XS_ROUTER_CERTIFIED) return XS_OK;
    const char *base = (const char *)workspace;
    if (!base) {
        void *sp = nullptr;
        if ((rc = scratch_for_current_device(&sp))) return rc;
        base = (const char *)sp;
    }
    int32_t c[2] = {0, 0};
    hipStream_t st = (hipStream_t)stream;
    XS_HIP(hipMemcpyAsync(c, base + layout(p).ccert, sizeof(c), hipMemcpyDeviceToHost, st));
    XS_HIP(hipStreamSynchronize(st));
    out[0] = c[0];
    out[1] = c[1];
    return XS_OK;
}

int xs_moe_plan(const xs_moe_params *p, const xs_moe_tensors *t, xs_moe_plan_t *out)
{
    XS_REQUIRE(out != nullptr, "null pointer");
    int rc = check_params(p);
    if (rc) return rc;
    XS_REQUIRE(p->T >= 1, "T must be at least 1");
    if ((rc = check_tensors(p, t))) return rc;
    Plan pl;
    if ((rc = make_plan(p, t, pl))) return rc;
    const bool fp4 = p->routed_format == XS_FP4_E2M1X2;
    out->tile_rows = pl.bm;
    out->routed_gemm = pl.stream    ? XS_GEMM_STREAM
                       : pl.direct  ? XS_GEMM_DIRECT_PREFILL
                       : pl.ddirect ? XS_GEMM_DIRECT_DECODE
                       : pl.direct4 ? XS_GEMM_DIRECT_MXFP4
                       : pl.wide    ? XS_GEMM_TALL
                                    : XS_GEMM_TILED;
    out->shared_gemm = !p->has_shared ? -1 : !fp4 ? out->routed_gemm : pl.sdirect ? XS_GEMM_DIRECT_PREFILL : XS_GEMM_TILED;
    out->fused_combine = pl.fused ? 1 : pl.shcomb ? 2 : 0;
    return XS_OK;
}

int xs_moe_forward(const xs_moe_params *p, const xs_moe_tensors *t, void *workspace,
                   size_t workspace_bytes, void *stream)
{
    return moe_forward(p, t, workspace, workspace_bytes, (hipStream_t)stream);
}

int xs_moe_profile_enable(int enable)
{
    g_prof = enable != 0;
    g_prof_n = 0;
    return XS_OK;
}

int xs_moe_profile_read(float *stage_ms, int n_stages, int *n_calls)
{
    XS_REQUIRE(stage_ms && n_stages >= 1, "null pointer");
    for (int i = 0; i < n_stages; ++i) stage_ms[i] = 0.f;
    for (int s = 0; s < g_prof_n; ++s) {
        XS_HIP(hipEventSynchronize(g_prof_ev[s][kStages]));
        for (int i = 0; i < kStages && i < n_stages; ++i) {
            float ms = 0.f;
            XS_HIP(hipEventElapsedTime(&ms, g_prof_ev[s][i], g_prof_ev[s][i + 1]));
            stage_ms[i] += ms;
        }
    }
    if (n_calls) *n_calls = g_prof_n;
    g_prof_n = 0;
    return XS_OK;
}

size_t xs_gemm_fp8_blockscale_workspace_size(int64_t M, int64_t K)
{
    size_t a, b;
    return gemm_ws(M, K, &a, &b);
}

int xs_gemm_fp8_blockscale(const void *A, const uint8_t *B, const float *Bs, int64_t M, int64_t N,
                           int64_t K, void *C, void *workspace, size_t workspace_bytes, void *stream)
{
    XS_REQUIRE(A && B && Bs && C, "null pointer");
    XS_REQUIRE(((uintptr_t)A & 15) == 0 && ((uintptr_t)B & 15) == 0 && ((uintptr_t)C & 15) == 0 &&
                   ((uintptr_t)Bs & 3) == 0,
               "misaligned operand: A, B and C need 16-byte, Bs 4-byte alignment");
    XS_REQUIRE(M * K < ((int64_t)1 << 32) && N * K < ((int64_t)1 << 32),
               "shape mismatch: M x K and N x K must stay below 2^32 (32-bit row offsets)");
    XS_REQUIRE(M >= 0 && M < (1 << 24) && N >= 128 && N % 128 == 0 && K >= 128 && K % 128 == 0,
               "shape mismatch: N and K must be multiples of 128");
    size_t o_s, o_part;
    size_t need = gemm_ws(M, K, &o_s, &o_part);
    if (!workspace || workspace_bytes < need)
        return set_error(XS_ERR_WORKSPACE, "workspace too small: %zu < %zu", workspace_bytes, need);
    if (M == 0) return XS_OK;
    hipStream_t st = (hipStream_t)stream;
    char *ws = (char *)workspace;
    float *part = dense_part_bytes(M) ? (float *)(ws + o_part) : nullptr;
    // the split counters sit in the last 1 KB of the partial region; the
    // quant launch clears them
    int32_t *cnt = part ? (int32_t *)(ws + o_part + dense_part_bytes(M) - 1024) : nullptr;
    const int ncnt = part ? dense_counters(M, N) : 0;
    int rc = launch_quant_act(A, XS_BF16, M, K, (uint8_t *)ws, ws + o_s, 0, st, cnt, ncnt);
    if (rc) return rc;
    return launch_gemm_dense((const uint8_t *)ws, (const float *)(ws + o_s), B, Bs, (uint16_t *)C, M, N, K, part,
                             cnt, st);
}

int xs_gemm_fp8_blockscale_packed(const void *A, const uint8_t *Bp, const float *Bs, int64_t M, int64_t N,
                                  int64_t K, void *C, void *workspace, size_t workspace_bytes, void *stream)
{
    XS_REQUIRE(A && Bp && Bs && C, "null pointer");
    XS_REQUIRE(((uintptr_t)A & 15) == 0 && ((uintptr_t)Bp & 15) == 0 && ((uintptr_t)C & 15) == 0 &&
                   ((uintptr_t)Bs & 3) == 0,
               "misaligned operand: A, Bp and C need 16-byte, Bs 4-byte alignment");
    XS_REQUIRE(M >= 0 && M < (1 << 24) && N >= 256 && N % 256 == 0 && K >= 512 && K % 512 == 0,
               "shape mismatch: N must be a multiple of 256 and K of 512");
    XS_REQUIRE(M * K < ((int64_t)1 << 32) && N * K < ((int64_t)1 << 32),
               "shape mismatch: M x K and N x K must stay below 2^32 (32-bit row offsets)");
    size_t o_s, o_part;
    const size_t need = gemm_ws(M, K, &o_s, &o_part);
    if (!workspace || workspace_bytes < need)
        return set_error(XS_ERR_WORKSPACE, "workspace too small: %zu < %zu", workspace_bytes, need);
    if (!xs::weight_direct_enabled())
        return set_error(XS_ERR_UNSUPPORTED, "packed GEMM: the weight-direct GEMMs are off (XS_WEIGHT_DIRECT=1 enables them)");
    if (M == 0) return XS_OK;
    hipStream_t st = (hipStream_t)stream;
    char *ws = (char *)workspace;
    int rc = launch_quant_act(A, XS_BF16, M, K, (uint8_t *)ws, ws + o_s, 0, st);
    if (rc) return rc;
    return launch_gemm_wd_dense((const uint8_t *)ws, (const float *)(ws + o_s), Bp, Bs, (uint16_t *)C, M, N, K, st);
}

}  // extern "C"
