// Whole-forward host emulation: the library's own C ABI (xs_moe_forward,
// xs_moe_forward_noalloc, xs_moe_plan), dispatch and launchers, with every
// kernel run from its source on the CPU (gen_fwd.py, hip_emu.hpp), against
// the CPU oracle on the same inputs.
// usage: fwd_emu T H I E k seed fp4 shared router x_f32 zipf norm residual noalloc [frag]
// frag: 1 also the weights in fragment order (xs_pack_weight_*_frag, run
// emulated), 2 only those (packed-only layer); with XS_WEIGHT_DIRECT=1 the
// forward then takes the weight-direct GEMMs.
// toggle NAME=VALUE: a second forward with that environment switch set must
// give the same output bits ("toggle mismatches N", its plan printed too).
// Prints the plan, then "idx mismatches N" etc. (routing, weights, counts,
// offsets, permutation and inverse against the oracle's routing of the logits
// the forward routed on), "ref idx mismatches N" (against the oracle's routing
// from x; required 0 for the certified and chain routers), "logit mismatches
// N" (chain router: required 0), and "max-abs-rel E" of the output against the
// oracle's dequantize-then-f32 layer.
#include "hip_emu.hpp"
#include <cmath>
#include <random>
#include <thread>

#include "moe_oracle.h"
#include "xs_moe.h"

int main(int argc, char **argv)
{
    auto arg = [&](int i, double d) { return argc > i ? atof(argv[i]) : d; };
    const int T = (int)arg(1, 64), H = (int)arg(2, 256), I = (int)arg(3, 256), E = (int)arg(4, 8), k = (int)arg(5, 2);
    const int seed = (int)arg(6, 1), fp4 = (int)arg(7, 0), shared = (int)arg(8, 1), router = (int)arg(9, 1);
    const int xf32 = (int)arg(10, 0);
    const double zipf = arg(11, 0);
    const int norm = (int)arg(12, 0), resid = (int)arg(13, 0), noalloc = (int)arg(14, 0), frag = (int)arg(15, 0);
    const char *toggle = argc > 16 ? argv[16] : nullptr;
    g_math = true;
    std::mt19937 rng(seed);
    std::normal_distribution<float> nd(0.f, 1.f);
    const size_t el = xf32 ? 4 : 2;
    auto fill_act = [&](void *p, size_t n, float sd) {
        for (size_t i = 0; i < n; ++i) {
            const float v = sd * nd(rng);
            if (xf32) ((float *)p)[i] = v; else ((uint16_t *)p)[i] = xo_bf16_from_f32(v);
        }
    };
    void *x = emu_alloc((size_t)T * H * el, "x");
    void *wr = emu_alloc((size_t)E * H * el, "router_w");
    float *bias = (float *)emu_alloc(4 * (size_t)E, "bias");
    fill_act(x, (size_t)T * H, 1.0f);
    // EMU_POISON=nan|inf: rows 0, T/2 and T-1 of x get that value (row 0 in
    // every element, the others every 97th); only those tokens' outputs may
    // be non-finite, and the routing must stay in range and the oracle's
    if (const char *pz = getenv("EMU_POISON")) {
        const float bad = !strcmp(pz, "nan") ? NAN : INFINITY;
        for (int t2 : {0, T / 2, T - 1})
            for (int c = 0; c < H; c += (t2 == 0 ? 1 : 97)) {
                if (xf32) ((float *)x)[(size_t)t2 * H + c] = bad;
                else ((uint16_t *)x)[(size_t)t2 * H + c] = xo_bf16_from_f32(bad);
            }
    }
    fill_act(wr, (size_t)E * H, 0.02f);
    for (int e = 0; e < E; ++e) bias[e] = 0.1f * nd(rng) + (zipf > 0 ? (float)(-zipf * std::log(1.0 + (e * 7919) % E)) : 0.f);
    void *nw = nullptr, *res = nullptr;
    if (norm) { nw = emu_alloc((size_t)H * el, "norm_w"); fill_act(nw, H, 1.0f); }
    if (resid) { res = emu_alloc((size_t)T * H * el, "residual"); fill_act(res, (size_t)T * H, 1.0f); }
    // weights: N(0, 0.02) quantized by the oracle's quantizers
    std::vector<float> w13f((size_t)2 * I * H), w2f((size_t)H * I);
    uint8_t *w13, *w2;
    void *s13, *s2;
    if (fp4) {
        w13 = (uint8_t *)emu_alloc((size_t)E * 2 * I * H / 2, "w13");
        s13 = emu_alloc((size_t)E * 2 * I * H / 32, "s13");
        w2 = (uint8_t *)emu_alloc((size_t)E * H * I / 2, "w2");
        s2 = emu_alloc((size_t)E * H * I / 32, "s2");
    } else {
        w13 = (uint8_t *)emu_alloc((size_t)E * 2 * I * H, "w13");
        s13 = emu_alloc(4 * (size_t)E * (2 * I / 128) * (H / 128), "s13");
        w2 = (uint8_t *)emu_alloc((size_t)E * H * I, "w2");
        s2 = emu_alloc(4 * (size_t)E * (H / 128) * (I / 128), "s2");
    }
    // each expert from its own generator (seed, e), over 8 host threads: the
    // same data however the experts are split (full-size layers take minutes
    // on one thread)
    {
        std::vector<std::thread> gen;
        for (int q = 0; q < 8; ++q)
            gen.emplace_back([&, q] {
                std::vector<float> a((size_t)2 * I * H), b((size_t)H * I);
                std::normal_distribution<float> g(0.f, 1.f);
                for (int e = q; e < E; e += 8) {
                    std::mt19937 r((uint32_t)seed * 2654435761u + (uint32_t)e);
                    for (auto &v : a) v = 0.02f * g(r);
                    for (auto &v : b) v = 0.02f * g(r);
                    if (fp4) {
                        xo_quant_weight_mxfp4(a.data(), 2 * I, H, w13 + (size_t)e * 2 * I * H / 2, (uint8_t *)s13 + (size_t)e * 2 * I * H / 32);
                        xo_quant_weight_mxfp4(b.data(), H, I, w2 + (size_t)e * H * I / 2, (uint8_t *)s2 + (size_t)e * H * I / 32);
                    } else {
                        xo_quant_weight_fp8_block(a.data(), 2 * I, H, w13 + (size_t)e * 2 * I * H, (float *)s13 + (size_t)e * (2 * I / 128) * (H / 128));
                        xo_quant_weight_fp8_block(b.data(), H, I, w2 + (size_t)e * H * I, (float *)s2 + (size_t)e * (H / 128) * (I / 128));
                    }
                }
            });
        for (auto &t : gen) t.join();
    }
    uint8_t *sw13 = nullptr, *sw2 = nullptr;
    float *ss13 = nullptr, *ss2 = nullptr;
    if (shared) {
        sw13 = (uint8_t *)emu_alloc((size_t)2 * I * H, "shared_w13");
        ss13 = (float *)emu_alloc(4 * (size_t)(2 * I / 128) * (H / 128), "shared_s13");
        sw2 = (uint8_t *)emu_alloc((size_t)H * I, "shared_w2");
        ss2 = (float *)emu_alloc(4 * (size_t)(H / 128) * (I / 128), "shared_s2");
        for (auto &v : w13f) v = 0.02f * nd(rng);
        for (auto &v : w2f) v = 0.02f * nd(rng);
        xo_quant_weight_fp8_block(w13f.data(), 2 * I, H, sw13, ss13);
        xo_quant_weight_fp8_block(w2f.data(), H, I, sw2, ss2);
    }

    // EMU_ROUTE="n_group,topk_group,renormalize,routed_scaling" (default 1,1,1,1)
    int ng = 1, tg = 1, renorm = 1;
    float scaling = 1.0f;
    if (const char *r = getenv("EMU_ROUTE")) sscanf(r, "%d,%d,%d,%f", &ng, &tg, &renorm, &scaling);
    xs_moe_params p = {};
    p.T = T; p.H = H; p.I = I; p.E = E; p.top_k = k; p.n_group = ng; p.topk_group = tg;
    p.renormalize = renorm; p.routed_scaling = scaling; p.x_dtype = xf32 ? XS_F32 : XS_BF16;
    p.routed_format = fp4 ? XS_FP4_E2M1X2 : XS_FP8_E4M3; p.has_shared = shared; p.router_exact = router;
    p.has_norm = norm; p.norm_eps = 1e-6f;
    void *out = emu_alloc((size_t)T * H * el, "out");
    float *lg = (float *)emu_alloc(4 * (size_t)T * E, "dbg logits");
    int32_t *idx = (int32_t *)emu_alloc(4 * (size_t)T * k, "dbg idx");
    float *w = (float *)emu_alloc(4 * (size_t)T * k, "dbg w");
    int32_t *counts = (int32_t *)emu_alloc(4 * (size_t)E, "dbg counts");
    int32_t *offsets = (int32_t *)emu_alloc(4 * (size_t)(E + 1), "dbg offsets");
    int32_t *perm = (int32_t *)emu_alloc(4 * (size_t)T * k, "dbg perm");
    int32_t *inv = (int32_t *)emu_alloc(4 * (size_t)T * k, "dbg inv");
    xs_moe_tensors t = {};
    t.x = x; t.router_w = wr; t.router_bias = bias;
    t.w13 = w13; t.w13_scale = s13; t.w2 = w2; t.w2_scale = s2;
    t.shared_w13 = sw13; t.shared_w13_scale = ss13; t.shared_w2 = sw2; t.shared_w2_scale = ss2;
    t.norm_weight = nw; t.residual = res; t.out = out;
    t.logits = lg; t.topk_idx = idx; t.topk_w = w; t.counts = counts; t.offsets = offsets; t.perm = perm; t.inv = inv;
    if (frag) {
        auto pack8 = [&](const uint8_t *w_, int64_t b, int64_t n, int64_t kk, const char *nm) {
            uint8_t *o_ = (uint8_t *)emu_alloc((size_t)(b * n * kk), nm);
            if (xs_pack_weight_fp8_frag(w_, b, n, kk, o_, nullptr)) { printf("pack failed: %s\n", xs_last_error()); exit(1); }
            return o_;
        };
        if (fp4) {
            uint8_t *p13 = (uint8_t *)emu_alloc((size_t)E * 2 * I * H / 2, "w13 packed");
            uint8_t *q13 = (uint8_t *)emu_alloc((size_t)E * 2 * I * H / 32, "s13 packed");
            uint8_t *p2 = (uint8_t *)emu_alloc((size_t)E * H * I / 2, "w2 packed");
            uint8_t *q2 = (uint8_t *)emu_alloc((size_t)E * H * I / 32, "s2 packed");
            if (xs_pack_weight_mxfp4_frag(w13, (uint8_t *)s13, E, 2 * I, H, p13, q13, nullptr) ||
                xs_pack_weight_mxfp4_frag(w2, (uint8_t *)s2, E, H, I, p2, q2, nullptr)) {
                printf("pack failed: %s\n", xs_last_error());
                return 1;
            }
            t.w13_frag = p13; t.w2_frag = p2; t.w13_scale_frag = q13; t.w2_scale_frag = q2;
        } else {
            t.w13_frag = pack8(w13, E, 2 * I, H, "w13 packed");
            t.w2_frag = pack8(w2, E, H, I, "w2 packed");
        }
        if (shared) {
            t.shared_w13_frag = pack8(sw13, 1, 2 * I, H, "shared w13 packed");
            t.shared_w2_frag = pack8(sw2, 1, H, I, "shared w2 packed");
        }
        if (frag == 2) t.w13 = t.w2 = t.shared_w13 = t.shared_w2 = nullptr;
    }
    if (T == 0) {
        // an empty batch: both forwards succeed without a workspace and launch
        // nothing (xs_moe_plan refuses T = 0: there is nothing to plan)
        int r1 = xs_moe_forward(&p, &t, nullptr, 0, nullptr), r2 = xs_moe_forward_noalloc(&p, &t, nullptr);
        printf("empty batch forward %d noalloc %d\nerrors %ld\n", r1, r2, (long)g_errors);
        return 0;
    }
    xs_moe_plan_t pl;
    if (xs_moe_plan(&p, &t, &pl)) { printf("plan failed: %s\n", xs_last_error()); return 1; }
    printf("plan tile_rows %d routed %d shared %d fused %d\n", pl.tile_rows, pl.routed_gemm, pl.shared_gemm, pl.fused_combine);
    int rc;
    void *last_ws = nullptr;
    if (noalloc) {
        rc = xs_moe_forward_noalloc(&p, &t, nullptr);
    } else {
        const size_t wsb = xs_moe_workspace_size(&p);
        void *ws = emu_alloc(wsb, "workspace");
        memset(ws, 0xA7, wsb);   // the forward must not rely on a zeroed workspace
        rc = xs_moe_forward(&p, &t, ws, wsb, nullptr);
        last_ws = ws;
    }
    if (rc) { printf("forward failed: %d %s\n", rc, xs_last_error()); return 1; }
    {
        int64_t st[2];
        if (xs_moe_router_stats(&p, noalloc ? nullptr : last_ws, st, nullptr)) { printf("stats failed\n"); return 1; }
        printf("exact pass logits %lld tokens %lld\n", (long long)st[0], (long long)st[1]);
    }

    if (toggle) {
        std::string kv(toggle);
        const size_t eq = kv.find('=');
        setenv(kv.substr(0, eq).c_str(), kv.substr(eq + 1).c_str(), 1);
        xs_moe_plan_t pl2;
        if (xs_moe_plan(&p, &t, &pl2)) { printf("plan failed: %s\n", xs_last_error()); return 1; }
        printf("toggle plan tile_rows %d routed %d shared %d fused %d\n", pl2.tile_rows, pl2.routed_gemm, pl2.shared_gemm,
               pl2.fused_combine);
        std::vector<uint8_t> first((uint8_t *)out, (uint8_t *)out + (size_t)T * H * el);
        memset(out, 0xEE, (size_t)T * H * el);
        if (resid && res == out) { printf("toggle with an in-place residual is not supported\n"); return 1; }
        const size_t wsb = xs_moe_workspace_size(&p);
        void *ws2 = emu_alloc(wsb, "workspace 2");
        memset(ws2, 0xA7, wsb);
        if ((rc = xs_moe_forward(&p, &t, ws2, wsb, nullptr))) { printf("forward failed: %d %s\n", rc, xs_last_error()); return 1; }
        long bad = 0;
        for (size_t i = 0; i < first.size(); ++i) bad += first[i] != ((uint8_t *)out)[i];
        printf("toggle mismatches %ld\n", bad);
    }
    // the oracle on the (normalized) x the router read.  With the pre-norm
    // that is xs_rmsnorm's output (the forward runs the same kernel): its sum
    // order differs from the oracle's sequential one, so a row can differ by
    // an ulp of inv, which can move an FP8 group scale; the row is checked
    // against the oracle's norm separately ("norm max code diff N": bf16 codes
    // or f32 bit patterns)
    std::vector<uint8_t> xin((size_t)T * H * el);
    if (norm) {
        void *xn = emu_alloc((size_t)T * H * el, "x normalized");
        if (xs_rmsnorm(x, nw, xf32 ? XS_F32 : XS_BF16, T, H, 1e-6f, xn, nullptr, nullptr, nullptr)) {
            printf("xs_rmsnorm failed: %s\n", xs_last_error());
            return 1;
        }
        memcpy(xin.data(), xn, xin.size());
        std::vector<uint8_t> rn(xin.size());
        xo_rmsnorm(x, nw, xf32 ? 0 : 1, T, H, 1e-6f, rn.data());
        long dmax_code = 0;
        for (size_t i = 0; i < (size_t)T * H; ++i) {
            const long a = xf32 ? (long)((const int32_t *)xn)[i] : (long)((const int16_t *)xn)[i];
            const long b = xf32 ? (long)((const int32_t *)rn.data())[i] : (long)((const int16_t *)rn.data())[i];
            dmax_code = std::max(dmax_code, std::labs(a - b));
        }
        printf("norm max code diff %ld\n", dmax_code);
    } else {
        memcpy(xin.data(), x, xin.size());
    }
    xo_moe_cfg cfg = {T, H, I, E, k, ng, tg, renorm, scaling, xf32 ? 0 : 1, fp4, shared, 8};   // 8 OpenMP threads
    xo_moe_inputs in = {xin.data(), wr, bias, lg, w13, s13, w2, s2, sw13, ss13, sw2, ss2};
    std::vector<int32_t> ridx((size_t)T * k), rc_((size_t)E), ro((size_t)E + 1), rp((size_t)T * k), ri((size_t)T * k);
    std::vector<float> rw((size_t)T * k), rout((size_t)T * H);
    std::vector<uint8_t> rob((size_t)T * H * el);
    xo_moe_outputs o = {nullptr, ridx.data(), rw.data(), rc_.data(), ro.data(), rp.data(), ri.data(), rout.data(), rob.data()};
    xo_moe_forward(&cfg, &in, &o);
    long b_idx = 0, b_w = 0, b_c = 0, b_o = 0, b_p = 0, b_i = 0;
    for (size_t i = 0; i < (size_t)T * k; ++i) {
        b_idx += idx[i] != ridx[i];
        b_w += memcmp(&w[i], &rw[i], 4) != 0;
        b_p += perm[i] != rp[i];
        b_i += inv[i] != ri[i];
    }
    for (int e = 0; e < E; ++e) b_c += counts[e] != rc_[e];
    for (int e = 0; e <= E; ++e) b_o += offsets[e] != ro[e];
    // routing from x (the reference's gemm_cpu logits)
    std::vector<float> xl((size_t)T * E);
    xo_router_logits(xin.data(), wr, xf32 ? 0 : 1, T, E, H, xl.data());
    std::vector<int32_t> xidx((size_t)T * k);
    std::vector<float> xw((size_t)T * k);
    xo_route(xl.data(), bias, T, E, k, ng, tg, renorm, scaling, xidx.data(), xw.data());
    long b_xidx = 0, b_lg = 0;
    for (size_t i = 0; i < (size_t)T * k; ++i) b_xidx += idx[i] != xidx[i];
    for (size_t i = 0; i < (size_t)T * E; ++i) b_lg += memcmp(&lg[i], &xl[i], 4) != 0;
    // poisoned tokens (EMU_POISON) are left out of the error: each output row
    // of one must be wholly non-finite, every other row finite.  (The
    // oracle's requantization drops NaN from a group's amax, so it can turn a
    // poisoned token's output into zeros; it is not compared there.)
    double amax = 0, dmax = 0;
    long poison_finite = 0, clean_nonfinite = 0, npoison = 0;
    for (int t2 = 0; t2 < T; ++t2) {
        bool gf_all = true, gf_any = false;
        for (int c = 0; c < H; ++c) {
            const bool f = std::isfinite(xf32 ? ((float *)out)[(size_t)t2 * H + c]
                                              : xo_f32_from_bf16(((uint16_t *)out)[(size_t)t2 * H + c]));
            gf_all &= f;
            gf_any |= f;
        }
        const bool poisoned = getenv("EMU_POISON") && (t2 == 0 || t2 == T / 2 || t2 == T - 1);
        npoison += poisoned;
        poison_finite += poisoned && gf_any;
        clean_nonfinite += !poisoned && !gf_all;
        if (poisoned) continue;
        for (int c = 0; c < H; ++c) {
            const size_t i = (size_t)t2 * H + c;
            double r = rout[i], g;
            if (resid) r += xf32 ? ((float *)res)[i] : xo_f32_from_bf16(((uint16_t *)res)[i]);
            g = xf32 ? ((float *)out)[i] : xo_f32_from_bf16(((uint16_t *)out)[i]);
            amax = std::max(amax, std::fabs(r));
            dmax = std::max(dmax, std::fabs(g - r));
        }
    }
    long bad_idx = 0;
    for (size_t i = 0; i < (size_t)T * k; ++i) {
        bad_idx += idx[i] < 0 || idx[i] >= E;
        for (size_t j = i - i % k; j < i; ++j) bad_idx += idx[j] == idx[i];
    }
    printf("poisoned rows %ld: with a finite output element %ld; clean rows with a non-finite one %ld\n"
           "idx out of range or repeated %ld\n", npoison, poison_finite, clean_nonfinite, bad_idx);
    if (!bad_idx) {   // the permutation of the forward's own top-k
        std::vector<int32_t> oc((size_t)E), oo((size_t)E + 1), op((size_t)T * k), oi((size_t)T * k);
        xo_permute(idx, T, E, k, oc.data(), oo.data(), op.data(), oi.data());
        long b = 0;
        for (int e = 0; e < E; ++e) b += oc[e] != counts[e];
        for (int e = 0; e <= E; ++e) b += oo[e] != offsets[e];
        for (size_t i = 0; i < (size_t)T * k; ++i) b += (op[i] != perm[i]) + (oi[i] != inv[i]);
        printf("own permutation mismatches %ld\n", b);
    }
    printf("idx mismatches %ld\nw mismatches %ld\ncounts mismatches %ld\noffsets mismatches %ld\n"
           "perm mismatches %ld\ninv mismatches %ld\nref idx mismatches %ld\nlogit mismatches %ld\n",
           b_idx, b_w, b_c, b_o, b_p, b_i, b_xidx, b_lg);
    uint64_t hsh = 1469598103934665603ull;   // FNV-1a of the output bytes
    for (size_t i = 0; i < (size_t)T * H * el; ++i) hsh = (hsh ^ ((const uint8_t *)out)[i]) * 1099511628211ull;
    printf("out hash %016llx\n", (unsigned long long)hsh);
    // EMU_NOALLOC_SEQ=T2: the layer at T and then at T2 (the first T2 tokens)
    // through the workspace forward and through the no-allocation forward on
    // the shared static scratch, which keeps the previous call's contents:
    // the outputs must agree bit for bit (every counter re-armed per call)
    if (const char *sq = getenv("EMU_NOALLOC_SEQ")) {
        const int64_t T2 = atoi(sq);
        long bad = 0, zero = 0;
        for (int64_t TT : {(int64_t)T, T2}) {
            xs_moe_params q = p;
            q.T = TT;
            xs_moe_tensors tt = t;
            tt.logits = nullptr; tt.topk_idx = nullptr; tt.topk_w = nullptr; tt.counts = nullptr;
            tt.offsets = nullptr; tt.perm = nullptr; tt.inv = nullptr;
            uint8_t *oa = (uint8_t *)emu_alloc((size_t)TT * H * el, "seq out a");
            uint8_t *ob = (uint8_t *)emu_alloc((size_t)TT * H * el, "seq out b");
            const size_t wsq = xs_moe_workspace_size(&q);
            void *wq = emu_alloc(wsq, "seq workspace");
            tt.out = oa;
            bad += xs_moe_forward(&q, &tt, wq, wsq, nullptr) != 0;
            tt.out = ob;
            if (xs_moe_forward_noalloc(&q, &tt, nullptr)) {
                printf("noalloc sequence: %s\n", xs_last_error());
                ++bad;
            }
            bad += memcmp(oa, ob, (size_t)TT * H * el) != 0;
            bool allz = true;
            for (size_t i = 0; i < (size_t)TT * H * el; ++i) allz &= oa[i] == 0;
            zero += allz;
        }
        printf("noalloc sequence mismatches %ld\n", bad + zero);
    }
    printf("max-abs-rel %.4g\nerrors %ld\n", dmax / (amax > 0 ? amax : 1), (long)g_errors);
    return 0;
}
