// Host emulation of the router kernels of moe_router.hip (the kernels' own
// source, one fiber per lane): the certified router (MFMA logits with their
// error-bound terms, route MODE 1, the chain kernel over the listed pairs,
// route MODE 2) and the chain router over every logit, against the CPU
// oracle's gemm_cpu-order logits and routing.
// usage: router_emu mode T E k H seed [nsplit] [margin] [bias_std] [zipf] [dup] [n_group topk_group] [path]
//   mode cert: the certified router; prints "idx mismatches N" (must be 0),
//     "w mismatches N" (weights against the oracle's routing of the logits
//     the kernels routed on: 0), "mask mismatches N", and the listed pairs;
//     margin > 1 widens every interval (every token then takes the exact
//     pass, and the patched logits must equal the oracle's bit for bit).
//   dup > 0: router rows E-dup..E-1 (and their biases) copy rows 0..dup-1
//     (exact ties, broken by the lower index), every other copy with one
//     element one bf16 step apart (near ties).
//   path: how the certified routing runs: 0 as the forward does (for
//     T <= 256 one launch with a block per token that routes, runs the exact
//     pass and routes again; else the routing launch, the pair-parallel chain
//     launch and a second routing launch), 1 always the latter, 2 always the
//     former.
//   EMU_CANCEL=C: a quarter of K holds pairs x = C, C / w = a, -a whose
//     products cancel at magnitude 1000 (the bound then carries real weight).
//   EMU_MFMA_MODEL=0..5: the MFMA summation model (router_emu.hpp).
//   mode bf16 [libxsref.so]: the bf16 rounding on every float (device,
//     oracle and, given its path, the reference's own); mode sigmoid
//     [stride]: xs_sigmoid's error on every float, and against the oracle;
//     mode codecs: the software e4m3 / e2m1 encoders on every float.
//   mode chain_bf16 / chain_f32: every logit in gemm_cpu order; prints
//     "logit mismatches N".
#include "router_emu.hpp"
#include <cmath>
#include <random>
#include <thread>
#include <dlfcn.h>

#include "router_emu.inc"
#include "moe_oracle.h"

using namespace xs;

static uint16_t bf(float f) { return xo_bf16_from_f32(f); }

int main(int argc, char **argv)
{
    const std::string mode = argc > 1 ? argv[1] : "cert";
    const int T = argc > 2 ? atoi(argv[2]) : 16, E = argc > 3 ? atoi(argv[3]) : 64, k = argc > 4 ? atoi(argv[4]) : 6;
    const int H = argc > 5 ? atoi(argv[5]) : 1024, seed = argc > 6 ? atoi(argv[6]) : 1;
    int nsplit = argc > 7 ? atoi(argv[7]) : 1;
    const float margin = argc > 8 ? (float)atof(argv[8]) : 1.0f;
    const double bias_std = argc > 9 ? atof(argv[9]) : 0.1;
    const double zipf = argc > 10 ? atof(argv[10]) : 0.0;
    const int dup = argc > 11 ? atoi(argv[11]) : 0;
    const int n_group = argc > 12 ? atoi(argv[12]) : 1, topk_group = argc > 13 ? atoi(argv[13]) : 1;
    const int path = argc > 14 ? atoi(argv[14]) : 0;
    if (getenv("EMU_MFMA_MODEL")) g_mfma_model = atoi(getenv("EMU_MFMA_MODEL"));
    if (mode == "sigmoid") {
        // xs_sigmoid (the route kernel's) against the sigmoid in double and
        // against the oracle's xo_sigmoid (bit for bit; on every ostride-th
        // pattern, argument 2, default 1) on every float but NaN
        // (2^32 - 2^24 bit patterns, both signs, infinities), over 8 host
        // threads; prints the largest absolute error in units of 2^-22, where
        // it occurs, and the number of floats where the two differ
        const int nth = 8;
        const uint64_t ostride = argc > 2 ? (uint64_t)std::max(1, atoi(argv[2])) : 1;   // oracle comparison stride
        std::vector<double> worst(nth, 0.0);
        std::vector<float> at(nth, 0.0f);
        std::vector<long> differ(nth, 0);
        std::vector<std::thread> th;
        for (int q = 0; q < nth; ++q)
            th.emplace_back([&, q] {
                const uint64_t lo = ((uint64_t)1 << 32) * q / nth, hi = ((uint64_t)1 << 32) * (q + 1) / nth;
                for (uint64_t v = lo; v < hi; ++v) {
                    const uint32_t u = (uint32_t)v;
                    if ((u & 0x7fffffffu) > 0x7f800000u) continue;   // NaN
                    float x;
                    memcpy(&x, &u, 4);
                    const double r = 1.0 / (1.0 + std::exp(-(double)x));
                    const float g = xs_sigmoid(x);
                    const double err = std::fabs((double)g - r);
                    if (err > worst[q]) { worst[q] = err; at[q] = x; }
                    if (v % ostride == 0) {
                        const float o = xo_sigmoid(x);
                        differ[q] += memcmp(&g, &o, 4) != 0;
                    }
                }
            });
        for (auto &t : th) t.join();
        const int b = (int)(std::max_element(worst.begin(), worst.end()) - worst.begin());
        long nd = 0;
        for (long d : differ) nd += d;
        printf("sigmoid max error %.4f x 2^-22 at %.9g\nsigmoid oracle mismatches %ld\nerrors %ld\n",
               worst[b] * 4194304.0, at[b], nd, (long)g_errors);
        return 0;
    }
    if (mode == "bf16") {
        // xs::bf16_from_f32 (every kernel's bf16 rounding, from xs_device.hpp
        // as written; not the emulator's stand-in of the same name) against the
        // oracle's xo_bf16_from_f32, and the oracle against the reference's
        // own bfloat16(float) (xstar_cpp/src/bfloat16.cpp, compiled into
        // oracle/_ref, argument 2: its path, when built; argument 3: compare
        // with it on every n-th chunk of 65536 floats), on every float
        // including NaN and infinities, over 8 host threads
        typedef void (*RefFn)(const float *, uint16_t *, int64_t);
        RefFn ref = nullptr;
        if (argc > 2) {
            if (void *h = dlopen(argv[2], RTLD_NOW)) ref = (RefFn)dlsym(h, "xsref_bf16_from_f32");
            if (!ref) { printf("cannot load the reference conversion from %s\n", argv[2]); return 1; }
        }
        const int nth = 8;
        const uint64_t rstride = argc > 3 ? (uint64_t)std::max(1, atoi(argv[3])) : 1;   // reference: every rstride-th chunk
        std::vector<long> dev(nth, 0), rdiff(nth, 0);
        std::vector<std::thread> th;
        for (int q = 0; q < nth; ++q)
            th.emplace_back([&, q] {
                const uint64_t lo = ((uint64_t)1 << 32) * q / nth, hi = ((uint64_t)1 << 32) * (q + 1) / nth;
                const size_t chunk = 1 << 16;
                std::vector<float> xs(chunk);
                std::vector<uint16_t> rs(chunk);
                for (uint64_t c0 = lo; c0 < hi; c0 += chunk) {
                    const size_t n = (size_t)std::min<uint64_t>(chunk, hi - c0);
                    for (size_t i = 0; i < n; ++i) {
                        const uint32_t u = (uint32_t)(c0 + i);
                        memcpy(&xs[i], &u, 4);
                    }
                    const bool withref = ref && (c0 / chunk) % rstride == 0;
                    if (withref) ref(xs.data(), rs.data(), (int64_t)n);
                    for (size_t i = 0; i < n; ++i) {
                        const uint16_t o = xo_bf16_from_f32(xs[i]);
                        dev[q] += xs::bf16_from_f32(xs[i]) != o;
                        if (withref) rdiff[q] += rs[i] != o;
                    }
                }
            });
        for (auto &t : th) t.join();
        long nd_ = 0, nr = 0;
        for (int q = 0; q < nth; ++q) { nd_ += dev[q]; nr += rdiff[q]; }
        printf("bf16 device mismatches %ld\n", nd_);
        if (ref) printf("bf16 reference mismatches %ld\n", nr);
        printf("errors %ld\n", (long)g_errors);
        return 0;
    }
    if (mode == "codecs") {
        // the kernels' software encoders (xs_device.hpp: e4m3_encode_sw for
        // MXFP8 activations and FP8 weights, e2m1_encode_sw for MXFP4
        // weights) against the oracle's on every float (every stride-th bit
        // pattern, argument 2, default 1), NaN and infinities included, over 8
        // host threads
        const int nth = 8;
        const uint64_t stride = argc > 2 ? (uint64_t)std::max(1, atoi(argv[2])) : 1;   // every stride-th pattern
        std::vector<long> d8(nth, 0), d4(nth, 0);
        std::vector<std::thread> th;
        for (int q = 0; q < nth; ++q)
            th.emplace_back([&, q] {
                const uint64_t lo = ((uint64_t)1 << 32) * q / nth, hi = ((uint64_t)1 << 32) * (q + 1) / nth;
                for (uint64_t v = lo + (stride - lo % stride) % stride; v < hi; v += stride) {
                    const uint32_t u = (uint32_t)v;
                    float x;
                    memcpy(&x, &u, 4);
                    d8[q] += xs::e4m3_encode_sw(x) != (uint32_t)xo_e4m3_encode(x);
                    d4[q] += xs::e2m1_encode_sw(x) != (uint32_t)xo_e2m1_encode(x);
                }
            });
        for (auto &t : th) t.join();
        long a = 0, b = 0;
        for (int q = 0; q < nth; ++q) { a += d8[q]; b += d4[q]; }
        printf("e4m3 encode mismatches %ld\ne2m1 encode mismatches %ld\nerrors %ld\n", a, b, (long)g_errors);
        return 0;
    }
    std::mt19937 rng(seed);
    std::normal_distribution<float> nd(0.f, 1.f);
    const bool f32 = mode == "chain_f32";
    const size_t el = f32 ? 4 : 2;
    uint8_t *x = (uint8_t *)emu_alloc((size_t)T * H * el, "x");
    uint8_t *wr = (uint8_t *)emu_alloc((size_t)E * H * el, "router_w");
    float *bias = (float *)emu_alloc(4 * (size_t)E, "bias");
    for (size_t i = 0; i < (size_t)T * H; ++i) {
        const float v = nd(rng);
        if (f32) ((float *)x)[i] = v; else ((uint16_t *)x)[i] = bf(v);
    }
    for (size_t i = 0; i < (size_t)E * H; ++i) {
        const float v = 0.02f * nd(rng);
        if (f32) ((float *)wr)[i] = v; else ((uint16_t *)wr)[i] = bf(v);
    }
    // bias ~ N(0, bias_std), plus log p_e of a Zipf profile when zipf > 0
    for (int e = 0; e < E; ++e)
        bias[e] = (float)(bias_std * nd(rng) + (zipf > 0 ? -zipf * std::log(1.0 + (e * 7919) % E) * 0.05 : 0.0));
    for (int d = 0; d < dup && !f32; ++d) {
        uint16_t *dst = (uint16_t *)wr + (size_t)(E - dup + d) * H, *src = (uint16_t *)wr + (size_t)d * H;
        memcpy(dst, src, 2 * (size_t)H);
        if (d & 1) dst[d % H] ^= 1;   // one step of the last mantissa bit
        bias[E - dup + d] = bias[d];
    }
    // EMU_CANCEL=C: a quarter of the K columns hold pairs with x = C, C and
    // w = a, -a (|C a| about 1000): they cancel in exact arithmetic, but every
    // sum of them rounds at that magnitude, so the MFMA logits and the
    // gemm_cpu logits differ by far more than the margins' fixed terms cover
    // and only the proven bound keeps the routing exact
    if (const char *cz = getenv("EMU_CANCEL"); cz && !f32) {
        const float C = (float)atof(cz);
        for (int t = 0; t < T; ++t)
            for (int i = 0; i < H / 4; i += 2) {
                ((uint16_t *)x)[(size_t)t * H + i] = bf(C);
                ((uint16_t *)x)[(size_t)t * H + i + 1] = bf(C);
            }
        for (int e = 0; e < E; ++e)
            for (int i = 0; i < H / 4; i += 2) {
                const uint16_t a = bf(1000.0f / C * nd(rng));
                ((uint16_t *)wr)[(size_t)e * H + i] = a;
                ((uint16_t *)wr)[(size_t)e * H + i + 1] = a ^ 0x8000;
            }
    }
    std::vector<float> ref((size_t)T * E);
    xo_router_logits(x, wr, f32 ? 0 : 1, T, E, H, ref.data());

    if (mode != "cert") {
        float *out = (float *)emu_alloc(4 * (size_t)T * E, "logits");
        const int64_t groups = ((int64_t)T * E + 63) / 64;
        const unsigned grid = (unsigned)std::min<int64_t>(groups, 3);   // blocks loop over the groups
        if (f32)
            emu_launch3([&] { router_chain_kernel<float>((const float *)x, (const float *)wr, E, H, nullptr, nullptr,
                                                         (int64_t)T * E, out, nullptr, 0); },
                        grid, 1, 1, kChainThreads, sizeof(float) * 2 * 64 * kCR, 3);
        else
            emu_launch3([&] { router_chain_kernel<uint16_t>((const uint16_t *)x, (const uint16_t *)wr, E, H, nullptr,
                                                            nullptr, (int64_t)T * E, out, nullptr, 0); },
                        grid, 1, 1, kChainThreads, sizeof(float) * 2 * 64 * kCR, 3);
        long bad = 0;
        for (size_t i = 0; i < (size_t)T * E; ++i) bad += memcmp(&out[i], &ref[i], 4) != 0;
        printf("logit mismatches %ld of %zu\nerrors %ld\n", bad, (size_t)T * E, (long)g_errors);
        return 0;
    }

    g_math = true;
    const size_t TE = (size_t)T * E;
    float *part = (float *)emu_alloc(4 * TE * nsplit, "logit slices");
    float *dpart = (float *)emu_alloc(4 * TE * nsplit, "bound slices");
    float *flog = (float *)emu_alloc(4 * TE, "flog");
    int32_t *pairs = (int32_t *)emu_alloc(8 * TE, "pairs");
    int32_t *cnt = (int32_t *)emu_alloc(8, "counters");
    int32_t *flagged = (int32_t *)emu_alloc(4 * (size_t)T, "flagged");
    int32_t *fbase = (int32_t *)emu_alloc(4 * (size_t)T, "flagged pair base");
    int32_t *fcnt = (int32_t *)emu_alloc(4 * (size_t)T, "flagged pair count");
    int32_t *idx = (int32_t *)emu_alloc(4 * (size_t)T * k, "idx");
    float *w = (float *)emu_alloc(4 * (size_t)T * k, "w");
    const int Wd = (T + 31) / 32;
    uint32_t *mask = (uint32_t *)emu_alloc(4 * (size_t)Wd * E, "mask");
    float *lout = (float *)emu_alloc(4 * TE, "logits_out");
    cnt[0] = cnt[1] = 12345;    // the logits launch zeroes them
    memset(mask, 0xff, 4 * (size_t)Wd * E);
    CertState cs{dpart, H / nsplit / 32, flog, pairs, cnt, flagged, fbase, fcnt, margin};
    CertArgs ca{dpart, cs.kblocks, flog, pairs, cnt, flagged, fbase, fcnt, margin};
    const uint16_t *xb = (const uint16_t *)x, *wb = (const uint16_t *)wr;
    if (T <= 256) {
        emu_launch3([&] { router_logits_mfma_kernel<1, 2, true>(xb, wb, T, E, H, H / nsplit, part, mask,
                                                                (int64_t)Wd * E, nullptr, nullptr, dpart, cnt, 2); },
                    (E + 63) / 64, (T + 31) / 32, nsplit, 256, 0, 4);
    } else {
        emu_launch3([&] { router_logits_tile_kernel<true>(xb, wb, T, E, H, H / nsplit, part, mask, (int64_t)Wd * E,
                                                          dpart, cnt, 2); },
                    (E + kRtBE - 1) / kRtBE, (T + kRtBT - 1) / kRtBT, nsplit, 256, kRtNST * kRtStage, 4);
    }
    const int nv = (E + 63) / 64;
    auto route = [&](int m) {
        const unsigned g = m == 2 ? (unsigned)std::min((T + 3) / 4, 2) : (unsigned)((T + 3) / 4);
        auto body = [&] {
            const int nsp = m == 2 ? 1 : nsplit;
            switch (nv) {
            case 1: m == 1 ? route_kernel<1, 1>(part, bias, T, E, k, n_group, topk_group, 1, 1.f, idx, w, mask, Wd, nsp, lout, ca)
                           : route_kernel<1, 2>(part, bias, T, E, k, n_group, topk_group, 1, 1.f, idx, w, mask, Wd, nsp, lout, ca); break;
            case 2: m == 1 ? route_kernel<2, 1>(part, bias, T, E, k, n_group, topk_group, 1, 1.f, idx, w, mask, Wd, nsp, lout, ca)
                           : route_kernel<2, 2>(part, bias, T, E, k, n_group, topk_group, 1, 1.f, idx, w, mask, Wd, nsp, lout, ca); break;
            case 3: case 4: m == 1 ? route_kernel<4, 1>(part, bias, T, E, k, n_group, topk_group, 1, 1.f, idx, w, mask, Wd, nsp, lout, ca)
                            : route_kernel<4, 2>(part, bias, T, E, k, n_group, topk_group, 1, 1.f, idx, w, mask, Wd, nsp, lout, ca); break;
            case 5: case 6: case 7: case 8: m == 1 ? route_kernel<8, 1>(part, bias, T, E, k, n_group, topk_group, 1, 1.f, idx, w, mask, Wd, nsp, lout, ca)
                            : route_kernel<8, 2>(part, bias, T, E, k, n_group, topk_group, 1, 1.f, idx, w, mask, Wd, nsp, lout, ca); break;
            default: m == 1 ? route_kernel<16, 1>(part, bias, T, E, k, n_group, topk_group, 1, 1.f, idx, w, mask, Wd, nsp, lout, ca)
                            : route_kernel<16, 2>(part, bias, T, E, k, n_group, topk_group, 1, 1.f, idx, w, mask, Wd, nsp, lout, ca);
            }
        };
        emu_launch3(body, g, 1, 1, 256, 0, 8);
    };
    if (path == 2 || (path == 0 && T <= 256)) {
        // one launch: a block per token routes it, runs the exact pass of its
        // undecided pairs and routes it again
        auto body = [&] {
            switch (nv) {
            case 1: route_block_kernel<uint16_t, 1>(xb, wb, part, bias, T, E, H, k, n_group, topk_group, 1, 1.f, idx, w, mask, Wd, nsplit, lout, ca); break;
            case 2: route_block_kernel<uint16_t, 2>(xb, wb, part, bias, T, E, H, k, n_group, topk_group, 1, 1.f, idx, w, mask, Wd, nsplit, lout, ca); break;
            case 3: case 4: route_block_kernel<uint16_t, 4>(xb, wb, part, bias, T, E, H, k, n_group, topk_group, 1, 1.f, idx, w, mask, Wd, nsplit, lout, ca); break;
            case 5: case 6: case 7: case 8: route_block_kernel<uint16_t, 8>(xb, wb, part, bias, T, E, H, k, n_group, topk_group, 1, 1.f, idx, w, mask, Wd, nsplit, lout, ca); break;
            default: route_block_kernel<uint16_t, 16>(xb, wb, part, bias, T, E, H, k, n_group, topk_group, 1, 1.f, idx, w, mask, Wd, nsplit, lout, ca);
            }
        };
        emu_launch3(body, T, 1, 1, kChainThreads, sizeof(float) * 2 * 64 * kCR, 3);
    } else {
        route(1);
        const int64_t groups = (TE + 63) / 64;
        const unsigned grid = (unsigned)std::min<int64_t>(groups, 3);
        emu_launch3([&] { router_chain_kernel<uint16_t>(xb, wb, E, H, pairs, cnt, (int64_t)TE, flog, nullptr, 0); },
                    grid, 1, 1, kChainThreads, sizeof(float) * 2 * 64 * kCR, 3);
        route(2);
    }
    const int npairs = cnt[0], nflag = cnt[1];
    // the oracle's routing of the reference logits, and of the logits routed on
    std::vector<int32_t> ridx((size_t)T * k), midx((size_t)T * k);
    std::vector<float> rw((size_t)T * k), mw((size_t)T * k);
    xo_route(ref.data(), bias, T, E, k, n_group, topk_group, 1, 1.f, ridx.data(), rw.data());
    xo_route(lout, bias, T, E, k, n_group, topk_group, 1, 1.f, midx.data(), mw.data());
    long bad_idx = 0, bad_w = 0, bad_mask = 0, bad_pair = 0, bad_exact = 0;
    for (size_t i = 0; i < (size_t)T * k; ++i) {
        bad_idx += idx[i] != ridx[i];
        bad_w += memcmp(&w[i], &mw[i], 4) != 0 || midx[i] != idx[i];
    }
    for (int e = 0; e < E; ++e)
        for (int t = 0; t < T; ++t) {
            bool want = false;
            for (int j = 0; j < k; ++j) want |= ridx[(size_t)t * k + j] == e;
            bad_mask += (bool)((mask[(size_t)e * Wd + t / 32] >> (t % 32)) & 1) != want;
        }
    for (int p = 0; p < npairs; ++p) {
        const int t = pairs[2 * p], e = pairs[2 * p + 1];
        bad_pair += memcmp(&flog[(size_t)t * E + e], &ref[(size_t)t * E + e], 4) != 0;
    }
    if (margin > 1e6f)
        for (size_t i = 0; i < TE; ++i)
            if (memcmp(&lout[i], &ref[i], 4) != 0 && bad_exact++ < 5)
                printf("logit (%zu, %zu): %.9g, flog %.9g, reference %.9g\n", i / E, i % E, lout[i], flog[i], ref[i]);
    double maxerr = 0, maxdelta = 0;
    for (size_t i = 0; i < TE; ++i) {
        float lg = part[i];
        for (int s = 1; s < nsplit; ++s) lg += part[s * TE + i];
        maxerr = std::max(maxerr, (double)std::fabs(lg - ref[i]));
        maxdelta = std::max(maxdelta, (double)dpart[i]);
    }
    printf("pairs %d flagged %d of %d tokens\n", npairs, nflag, T);
    printf("idx mismatches %ld\nw mismatches %ld\nmask mismatches %ld\npair mismatches %ld\nexact mismatches %ld\n",
           bad_idx, bad_w, bad_mask, bad_pair, bad_exact);
    printf("max |mfma - ref| %.3g, max D %.3g\nerrors %ld\n", maxerr, maxdelta, (long)g_errors);
    return 0;
}
