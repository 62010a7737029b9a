// Host emulation of the stage entry points of the C ABI (xs_quant_act_fp8,
// xs_quant_act_mxfp8, xs_quant_weight_fp8_block, xs_quant_weight_mxfp4,
// xs_rmsnorm with its fused quant, xs_moe_route, xs_moe_permute and
// xs_moe_router_logits with the chain router, xs_gemm_fp8_blockscale), every kernel run from its
// source on the CPU (gen_fwd.py, hip_emu.hpp), against the CPU oracle.
// usage: stages_emu seed
// Prints "<stage> mismatches N" (each must be 0), "permute errors ok|BAD"
// and "errors N".
#include "hip_emu.hpp"
#include <cmath>
#include <random>

#include "moe_oracle.h"
#include "xs_moe.h"

static std::mt19937 rng;

// values that exercise the codecs: normals over many binades, exact zeros,
// whole zero groups, ties at e4m3 / e2m1 midpoints after scaling, a few huge
static void fill(float *v, size_t n, int group)
{
    std::normal_distribution<float> nd(0.f, 1.f);
    std::uniform_int_distribution<int> pick(0, 99), bin(-30, 10);
    for (size_t g0 = 0; g0 < n; g0 += group) {
        const int kind = pick(rng);
        const float mag = std::ldexp(1.f, bin(rng));
        for (size_t i = g0; i < g0 + group && i < n; ++i) {
            float x = nd(rng) * mag;
            if (kind < 5) x = 0.f;                                          // zero group
            else if (kind < 15) x = std::ldexp((float)(2 * (pick(rng) % 16) + 1), bin(rng) - 4);   // odd multiples: ties
            else if (kind < 17 && i == g0) x = 3.0e38f;                     // huge
            if (pick(rng) < 3) x = 0.f;
            v[i] = x;
        }
    }
}
static void to_bf16(const float *v, uint16_t *b, size_t n)
{
    for (size_t i = 0; i < n; ++i) b[i] = xo_bf16_from_f32(v[i]);
}
template <typename T>
static long diff(const T *a, const T *b, size_t n)
{
    long d = 0;
    for (size_t i = 0; i < n; ++i) d += memcmp(&a[i], &b[i], sizeof(T)) != 0;
    return d;
}

int main(int argc, char **argv)
{
    const int seed = argc > 1 ? atoi(argv[1]) : 1;
    rng.seed(seed);
    g_math = true;
    if (getenv("EMU_EARLY")) g_mode = MODE_EARLY;   // DMAs land at issue instead of at their wait
    long bad;

    // ---- activation quant, both dtypes
    for (int bf = 0; bf < 2; ++bf) {
        const int64_t rows = 37, cols = 1024;
        std::vector<float> x((size_t)rows * cols);
        fill(x.data(), x.size(), 128);
        void *xd = emu_alloc(x.size() * (bf ? 2 : 4), "x");
        if (bf) to_bf16(x.data(), (uint16_t *)xd, x.size());
        else memcpy(xd, x.data(), x.size() * 4);
        std::vector<float> xr(x.size());   // what the kernel reads, widened
        for (size_t i = 0; i < x.size(); ++i) xr[i] = bf ? xo_f32_from_bf16(((uint16_t *)xd)[i]) : x[i];
        uint8_t *q = (uint8_t *)emu_alloc(x.size(), "q");
        float *s = (float *)emu_alloc(4 * rows * cols / 128, "s");
        std::vector<uint8_t> rq(x.size());
        std::vector<float> rs(rows * cols / 128);
        bad = xs_quant_act_fp8(xd, bf ? XS_BF16 : XS_F32, rows, cols, q, s, nullptr) != 0;
        xo_quant_act_fp8(xr.data(), rows, cols, rq.data(), rs.data());
        printf("act fp8 %s mismatches %ld\n", bf ? "bf16" : "f32", bad + diff(q, rq.data(), x.size()) + diff(s, rs.data(), rs.size()));
        uint8_t *ms = (uint8_t *)emu_alloc(rows * cols / 32, "ms");
        std::vector<uint8_t> rms(rows * cols / 32);
        bad = xs_quant_act_mxfp8(xd, bf ? XS_BF16 : XS_F32, rows, cols, q, ms, nullptr) != 0;
        xo_quant_act_mxfp8(xr.data(), rows, cols, rq.data(), rms.data());
        printf("act mxfp8 %s mismatches %ld\n", bf ? "bf16" : "f32", bad + diff(q, rq.data(), x.size()) + diff(ms, rms.data(), rms.size()));
    }

    // ---- weight quant (batched), both dtypes
    for (int bf = 0; bf < 2; ++bf) {
        const int64_t batch = 3, n = 256, k = 384;
        const size_t per = (size_t)n * k;
        std::vector<float> w(batch * per);
        fill(w.data(), w.size(), 32);
        void *wd = emu_alloc(w.size() * (bf ? 2 : 4), "w");
        if (bf) to_bf16(w.data(), (uint16_t *)wd, w.size());
        else memcpy(wd, w.data(), w.size() * 4);
        std::vector<float> wr(w.size());
        for (size_t i = 0; i < w.size(); ++i) wr[i] = bf ? xo_f32_from_bf16(((uint16_t *)wd)[i]) : w[i];
        uint8_t *q = (uint8_t *)emu_alloc(w.size(), "wq");
        float *s = (float *)emu_alloc(4 * batch * (n / 128) * (k / 128), "ws");
        std::vector<uint8_t> rq(per);
        std::vector<float> rs((n / 128) * (k / 128));
        long b8 = xs_quant_weight_fp8_block(wd, bf ? XS_BF16 : XS_F32, batch, n, k, q, s, nullptr) != 0;
        for (int64_t b = 0; b < batch; ++b) {
            xo_quant_weight_fp8_block(wr.data() + b * per, n, k, rq.data(), rs.data());
            b8 += diff(q + b * per, rq.data(), per) + diff(s + b * rs.size(), rs.data(), rs.size());
        }
        printf("weight fp8 %s mismatches %ld\n", bf ? "bf16" : "f32", b8);
        uint8_t *q4 = (uint8_t *)emu_alloc(w.size() / 2, "wq4");
        uint8_t *s4 = (uint8_t *)emu_alloc(w.size() / 32, "ws4");
        std::vector<uint8_t> rq4(per / 2), rs4(per / 32);
        long b4 = xs_quant_weight_mxfp4(wd, bf ? XS_BF16 : XS_F32, batch, n, k, q4, s4, nullptr) != 0;
        for (int64_t b = 0; b < batch; ++b) {
            xo_quant_weight_mxfp4(wr.data() + b * per, n, k, rq4.data(), rs4.data());
            b4 += diff(q4 + b * per / 2, rq4.data(), per / 2) + diff(s4 + b * per / 32, rs4.data(), per / 32);
        }
        printf("weight mxfp4 %s mismatches %ld\n", bf ? "bf16" : "f32", b4);
    }

    // ---- RMSNorm with the fused FP8 quant: y within 2 codes of the oracle's
    // sequential-sum norm, q/s equal to the quantization of the kernel's own y
    {
        const int64_t rows = 21, hidden = 1280;
        std::normal_distribution<float> nd(0.f, 1.f);
        std::vector<float> x((size_t)rows * hidden), w(hidden);
        for (auto &v : x) v = nd(rng) * 3.f;
        for (auto &v : w) v = 1.f + 0.1f * nd(rng);
        long bq = 0, over = 0;
        for (int bf = 0; bf < 2; ++bf) {
            const size_t el = bf ? 2 : 4;
            void *xd = emu_alloc(x.size() * el, "nx"), *wd = emu_alloc(w.size() * el, "nw");
            void *y = emu_alloc(x.size() * el, "ny");
            if (bf) { to_bf16(x.data(), (uint16_t *)xd, x.size()); to_bf16(w.data(), (uint16_t *)wd, w.size()); }
            else { memcpy(xd, x.data(), x.size() * 4); memcpy(wd, w.data(), w.size() * 4); }
            uint8_t *q = (uint8_t *)emu_alloc(x.size(), "nq");
            float *s = (float *)emu_alloc(4 * rows * hidden / 128, "ns");
            bq += xs_rmsnorm(xd, wd, bf ? XS_BF16 : XS_F32, rows, hidden, 1e-6f, y, q, s, nullptr) != 0;
            std::vector<uint8_t> ry(x.size() * el);
            xo_rmsnorm(xd, wd, bf, rows, hidden, 1e-6f, ry.data());
            std::vector<float> yf(x.size());
            for (size_t i = 0; i < x.size(); ++i) {
                const long a = bf ? ((int16_t *)y)[i] : ((int32_t *)y)[i];
                const long b = bf ? ((int16_t *)ry.data())[i] : ((int32_t *)ry.data())[i];
                // bf16: 2 codes; f32: the summation-order bound (2H ulps of the sum, a few more for inv and y)
                over += std::labs(a - b) > (bf ? 2 : 2 * hidden + 8);
                yf[i] = bf ? xo_f32_from_bf16(((uint16_t *)y)[i]) : ((float *)y)[i];
            }
            std::vector<uint8_t> rq(x.size());
            std::vector<float> rs(rows * hidden / 128);
            xo_quant_act_fp8(yf.data(), rows, hidden, rq.data(), rs.data());
            bq += diff(q, rq.data(), x.size()) + diff(s, rs.data(), rs.size());
        }
        // every chunk count of the wave kernel (hidden = 512 NC, NC = 1..16,
        // with the fused quant), and the block kernel: hidden above 8192 (with
        // the quant), hidden not a multiple of 8, rows misaligned by one element
        struct N { int64_t rows, hidden; bool quant; int mis; };
        std::vector<N> ns;
        for (int nc = 1; nc <= 16; ++nc) ns.push_back({3, 512 * nc, true, 0});
        ns.push_back({3, 8320, true, 0});
        ns.push_back({4, 1001, false, 0});
        ns.push_back({3, 1024, false, 1});
        for (const N &c : ns)
            for (int bf = 0; bf < 2; ++bf) {
                const size_t el = bf ? 2 : 4, n = (size_t)c.rows * c.hidden;
                uint8_t *xb = (uint8_t *)emu_alloc((n + 8) * el, "sx"), *wb = (uint8_t *)emu_alloc(c.hidden * el, "sw");
                uint8_t *yb = (uint8_t *)emu_alloc((n + 8) * el, "sy");
                void *xd = xb + c.mis * el, *y = yb + c.mis * el;
                for (size_t i = 0; i < n; ++i) {
                    const float v = 2.f * nd(rng);
                    if (bf) ((uint16_t *)xd)[i] = xo_bf16_from_f32(v); else ((float *)xd)[i] = v;
                }
                for (int64_t i = 0; i < c.hidden; ++i) {
                    const float v = 1.f + 0.1f * nd(rng);
                    if (bf) ((uint16_t *)wb)[i] = xo_bf16_from_f32(v); else ((float *)wb)[i] = v;
                }
                uint8_t *q = c.quant ? (uint8_t *)emu_alloc(n, "sq") : nullptr;
                float *sc = c.quant ? (float *)emu_alloc(4 * n / 128, "ss") : nullptr;
                bq += xs_rmsnorm(xd, wb, bf ? XS_BF16 : XS_F32, c.rows, c.hidden, 1e-6f, y, q, sc, nullptr) != 0;
                std::vector<uint8_t> ry(n * el);
                xo_rmsnorm(xd, wb, bf, c.rows, c.hidden, 1e-6f, ry.data());
                std::vector<float> yf(n);
                for (size_t i = 0; i < n; ++i) {
                    const long a = bf ? ((int16_t *)y)[i] : ((int32_t *)y)[i];
                    const long b = bf ? ((int16_t *)ry.data())[i] : ((int32_t *)ry.data())[i];
                    over += std::labs(a - b) > (bf ? 2 : 2 * c.hidden + 8);
                    yf[i] = bf ? xo_f32_from_bf16(((uint16_t *)y)[i]) : ((float *)y)[i];
                }
                if (c.quant) {
                    std::vector<uint8_t> rq(n);
                    std::vector<float> rs(n / 128);
                    xo_quant_act_fp8(yf.data(), c.rows, c.hidden, rq.data(), rs.data());
                    bq += diff(q, rq.data(), n) + diff(sc, rs.data(), rs.size());
                }
            }
        printf("norm quant mismatches %ld\nnorm beyond bound mismatches %ld\n", bq, over);
    }

    // ---- route: plain, ties, group-limited, scaling, no renormalization
    {
        struct R { int64_t T, E, k, ng, tg; int renorm; float scaling; };
        const R cases[] = {{40, 256, 8, 1, 1, 1, 2.5f}, {33, 256, 8, 8, 4, 1, 1.f}, {17, 72, 6, 1, 1, 0, 1.f},
                           {9, 1024, 16, 16, 3, 1, 1.f}, {5, 1, 1, 1, 1, 0, 1.f}, {64, 64, 6, 4, 2, 0, 1.5f}};
        long br = 0;
        std::normal_distribution<float> nd(0.f, 1.f);
        for (const R &c : cases) {
            float *lg = (float *)emu_alloc(4 * c.T * c.E, "lg");
            float *bias = (float *)emu_alloc(4 * c.E, "bias");
            for (int64_t i = 0; i < c.T * c.E; ++i) lg[i] = nd(rng);
            for (int64_t e = 0; e < c.E; ++e) bias[e] = 0.1f * nd(rng);
            if (c.T > 1)   // ties: row 1 repeats its first half, row 0 all equal
                for (int64_t e = 0; e < c.E; ++e) { lg[c.E + e] = lg[c.E + e % ((c.E + 1) / 2)]; lg[e] = 0.25f; }
            int32_t *idx = (int32_t *)emu_alloc(4 * c.T * c.k, "idx");
            float *w = (float *)emu_alloc(4 * c.T * c.k, "w");
            std::vector<int32_t> ri(c.T * c.k);
            std::vector<float> rw(c.T * c.k);
            br += xs_moe_route(lg, bias, c.T, c.E, c.k, c.ng, c.tg, c.renorm, c.scaling, idx, w, nullptr) != 0;
            xo_route(lg, bias, c.T, c.E, c.k, c.ng, c.tg, c.renorm, c.scaling, ri.data(), rw.data());
            br += diff(idx, ri.data(), ri.size()) + diff(w, rw.data(), rw.size());
            // without a bias
            br += xs_moe_route(lg, nullptr, c.T, c.E, c.k, c.ng, c.tg, c.renorm, c.scaling, idx, w, nullptr) != 0;
            xo_route(lg, nullptr, c.T, c.E, c.k, c.ng, c.tg, c.renorm, c.scaling, ri.data(), rw.data());
            br += diff(idx, ri.data(), ri.size()) + diff(w, rw.data(), rw.size());
        }
        printf("route mismatches %ld\n", br);
    }

    // ---- permute, and its rejection of invalid idx
    {
        long bp = 0;
        bool errs_ok = true;
        for (int64_t T : {1, 7, 300, 2000}) {
            const int64_t E = T == 2000 ? 256 : 16, k = T == 1 ? 1 : 6;
            int32_t *idx = (int32_t *)emu_alloc(4 * T * k, "pidx");
            std::vector<int> ex(E);
            for (int64_t t = 0; t < T; ++t) {   // k distinct experts per row, in random order
                for (int64_t e = 0; e < E; ++e) ex[e] = (int)e;
                std::shuffle(ex.begin(), ex.end(), rng);
                for (int64_t j = 0; j < k; ++j) idx[t * k + j] = ex[j];
            }
            int32_t *cnt = (int32_t *)emu_alloc(4 * E, "pc"), *off = (int32_t *)emu_alloc(4 * (E + 1), "po");
            int32_t *perm = (int32_t *)emu_alloc(4 * T * k, "pp"), *inv = (int32_t *)emu_alloc(4 * T * k, "pi");
            const size_t wsb = xs_moe_permute_workspace_size(T, E);
            void *ws = emu_alloc(wsb, "pws");
            bp += xs_moe_permute(idx, T, E, k, cnt, off, perm, inv, ws, wsb, nullptr) != 0;
            std::vector<int32_t> rc(E), ro(E + 1), rp(T * k), ri(T * k);
            xo_permute(idx, T, E, k, rc.data(), ro.data(), rp.data(), ri.data());
            bp += diff(cnt, rc.data(), E) + diff(off, ro.data(), E + 1) + diff(perm, rp.data(), T * k) +
                  diff(inv, ri.data(), T * k);
            if (k > 1) {
                const int32_t keep = idx[k + 1];
                idx[k + 1] = idx[k];   // an expert named twice in row 1
                errs_ok &= xs_moe_permute(idx, T, E, k, cnt, off, perm, inv, ws, wsb, nullptr) == XS_ERR_INVALID &&
                           strstr(xs_last_error(), "named twice") != nullptr;
                idx[k + 1] = (int32_t)E;   // out of range
                errs_ok &= xs_moe_permute(idx, T, E, k, cnt, off, perm, inv, ws, wsb, nullptr) == XS_ERR_INVALID &&
                           strstr(xs_last_error(), "outside") != nullptr;
                idx[k + 1] = keep;
            }
        }
        printf("permute mismatches %ld\npermute errors %s\n", bp, errs_ok ? "ok" : "BAD");
    }

    // ---- router logits, chain router: gemm_cpu bits, bf16 and f32
    {
        const int64_t T = 9, E = 72, H = 640;
        long bl = 0;
        std::normal_distribution<float> nd(0.f, 1.f);
        for (int bf = 0; bf < 2; ++bf) {
            const size_t el = bf ? 2 : 4;
            void *x = emu_alloc(T * H * el, "lx"), *wr = emu_alloc(E * H * el, "lw");
            for (int64_t i = 0; i < T * H; ++i) { const float v = nd(rng); if (bf) ((uint16_t *)x)[i] = xo_bf16_from_f32(v); else ((float *)x)[i] = v; }
            for (int64_t i = 0; i < E * H; ++i) { const float v = 0.02f * nd(rng); if (bf) ((uint16_t *)wr)[i] = xo_bf16_from_f32(v); else ((float *)wr)[i] = v; }
            float *lg = (float *)emu_alloc(4 * T * E, "ll");
            std::vector<float> rl(T * E);
            bl += xs_moe_router_logits(x, wr, bf ? XS_BF16 : XS_F32, T, E, H, 1, lg, nullptr) != 0;
            xo_router_logits(x, wr, bf, T, E, H, rl.data());
            bl += diff(lg, rl.data(), rl.size());
        }
        printf("logits mismatches %ld\n", bl);
    }
    // ---- the single FP8 GEMM (gemm_dense.hip): split-K with the sc1 partial
    // exchange, and whole-K; against float64 on the dequantized operands
    // (the activation quantizer is bit-exact), and the same bits again
    {
        struct G { int64_t M, N, K; };
        // local K steps per block: 3, 1, 4 (split 4 ways), 4 (2 ways), 1 (whole-K,
        // 256 tiles), 7 and 5 (more steps than the 4 ring stages: the ring's
        // refills, row scales included); XS_EMU_FULL adds the bench's
        // 512 x 4096 x 4096 (2 ways, 16 steps)
        std::vector<G> gs = {{40, 256, 384}, {1, 128, 128}, {130, 384, 2048}, {300, 512, 1024},
                             {2048, 2048, 128}, {256, 512, 896}, {100, 384, 1152}};
        if (getenv("XS_EMU_FULL") && !strcmp(getenv("XS_EMU_FULL"), "1")) gs.push_back({512, 4096, 4096});
        long bg = 0;
        double worst = 0;
        std::normal_distribution<float> nd(0.f, 1.f);
        for (const G &c : gs) {
            uint16_t *A = (uint16_t *)emu_alloc(2 * c.M * c.K, "gA");
            std::vector<float> af(c.M * c.K), wf(c.N * c.K);
            for (int64_t i = 0; i < c.M * c.K; ++i) { A[i] = xo_bf16_from_f32(nd(rng)); af[i] = xo_f32_from_bf16(A[i]); }
            for (auto &v : wf) v = 0.02f * nd(rng);
            uint8_t *B = (uint8_t *)emu_alloc(c.N * c.K, "gB");
            float *Bs = (float *)emu_alloc(4 * (c.N / 128) * (c.K / 128), "gBs");
            xo_quant_weight_fp8_block(wf.data(), c.N, c.K, B, Bs);
            uint16_t *C = (uint16_t *)emu_alloc(2 * c.M * c.N, "gC");
            const size_t wsb = xs_gemm_fp8_blockscale_workspace_size(c.M, c.K);
            void *ws = emu_alloc(wsb, "gws");
            bg += xs_gemm_fp8_blockscale(A, B, Bs, c.M, c.N, c.K, C, ws, wsb, nullptr) != 0;
            std::vector<uint16_t> first(C, C + c.M * c.N);
            bg += xs_gemm_fp8_blockscale(A, B, Bs, c.M, c.N, c.K, C, ws, wsb, nullptr) != 0;
            bg += diff(C, first.data(), first.size());
            std::vector<uint8_t> aq(c.M * c.K);
            std::vector<float> as(c.M * c.K / 128);
            xo_quant_act_fp8(af.data(), c.M, c.K, aq.data(), as.data());
            std::vector<double> ad(c.M * c.K), bd(c.N * c.K);
            for (int64_t i = 0; i < c.M * c.K; ++i) ad[i] = (double)xo_e4m3_decode(aq[i]) * as[i / 128];
            for (int64_t n = 0; n < c.N; ++n)
                for (int64_t kk = 0; kk < c.K; ++kk)
                    bd[n * c.K + kk] = (double)xo_e4m3_decode(B[n * c.K + kk]) * Bs[(n / 128) * (c.K / 128) + kk / 128];
            double rmax = 0, dmax = 0;
            for (int64_t m = 0; m < c.M; ++m)
                for (int64_t n = 0; n < c.N; ++n) {
                    double r = 0;
                    for (int64_t kk = 0; kk < c.K; ++kk) r += ad[m * c.K + kk] * bd[n * c.K + kk];
                    rmax = std::max(rmax, std::fabs(r));
                    dmax = std::max(dmax, std::fabs((double)xo_f32_from_bf16(C[m * c.N + n]) - r));
                }
            const double err = dmax / (rmax > 0 ? rmax : 1);
            if (getenv("EMU_VERBOSE")) printf("dense %lld x %lld x %lld: max-abs-rel %.3g\n", (long long)c.M, (long long)c.N, (long long)c.K, err);
            worst = std::max(worst, err);
            bg += !(err < 4e-3);
        }
        printf("dense gemm mismatches %ld\ndense gemm max-abs-rel %.3g\n", bg, worst);
    }
    printf("errors %ld\n", (long)g_errors);
    return 0;
}
