// Host emulation of the weight-direct decode GEMMs (moe_gemm_wdd.hip): a MoE
// layer's gate_up (SwiGLU, FP8 requantised) and down GEMMs on 16-row tiles
// run from the kernel's own source, then both are checked against a float64
// recomputation from the same FP8 inputs.
// usage: wdd_emu T E k zipf seed H I conc mode(0 late,1 early) math(0/1) shared(0/1)
// (H and I in {512, 1024, 2048, 4096}); EMU_CMP_TILED=1 also runs the tiled
// kernel of moe_gemm.hip on the same inputs and compares the bytes
// EMU_HAZARD=1|2|3, EMU_HAZARD_P, EMU_HAZARD_SEED: the wait-state hazard model of emu.hpp
#include "emu.hpp"
#include <algorithm>
#include <numeric>
#include <random>

#include "wdd_emu.inc"
#include "tiled_emu.inc"

using namespace xs;
using I4 = int4;

static void pack_frag(const uint8_t *w, uint8_t *out, int batch, int n, int k)
{
    const int KB = k / 128;
    const size_t chunks = (size_t)batch * n * k / 16;
    for (size_t c = 0; c < chunks; ++c) {
        const int l = (int)(c & 63), h = (int)((c >> 6) & 1);
        const size_t blk = c >> 7;
        const int kb = (int)(blk % KB);
        const size_t bt = blk / KB;
        const size_t b = bt / (n / 16), t = bt % (n / 16);
        memcpy(out + c * 16, w + (b * n + 16 * t + (l & 15)) * (size_t)k + 128 * kb + 64 * h + 16 * (l >> 4), 16);
    }
}

int main(int argc, char **argv)
{
    int T = argc > 1 ? atoi(argv[1]) : 300, E = argc > 2 ? atoi(argv[2]) : 8, k = argc > 3 ? atoi(argv[3]) : 4;
    double zipf = argc > 4 ? atof(argv[4]) : 1.1;
    int seed = argc > 5 ? atoi(argv[5]) : 21;
    int H = argc > 6 ? atoi(argv[6]) : 1024, I = argc > 7 ? atoi(argv[7]) : 512;
    int conc = argc > 8 ? atoi(argv[8]) : 2;
    g_mode = argc > 9 ? atoi(argv[9]) : 0;
    g_math = argc > 10 ? atoi(argv[10]) : 1;
    int shared = argc > 11 ? atoi(argv[11]) : 1;
    if (getenv("EMU_HAZARD")) g_hazard = atoi(getenv("EMU_HAZARD"));
    if (getenv("EMU_HAZARD_P")) g_hazard_p = atof(getenv("EMU_HAZARD_P"));
    if (getenv("EMU_HAZARD_SEED")) g_hazard_seed = atoi(getenv("EMU_HAZARD_SEED"));
    const int BM = 16;
    std::mt19937 rng(seed);

    const int S = T * k;
    std::vector<double> wgt(E);
    for (int e = 0; e < E; ++e) wgt[e] = zipf > 0 ? 1.0 / std::pow(e + 1.0, zipf) : 1.0;
    std::shuffle(wgt.begin(), wgt.end(), rng);
    double ws = std::accumulate(wgt.begin(), wgt.end(), 0.0);
    std::vector<int> cnt(E);
    int left = S;
    for (int e = 0; e < E; ++e) { cnt[e] = std::min(T, (int)(S * wgt[e] / ws)); left -= cnt[e]; }
    for (int e = 0; left > 0; e = (e + 1) % E)
        if (cnt[e] < T) { ++cnt[e]; --left; }
    const int SH = shared ? T : 0, R = S + SH;
    int32_t *offsets = (int32_t *)emu_alloc(4 * (E + 2), "offsets");
    offsets[0] = 0;
    for (int e = 0; e < E; ++e) offsets[e + 1] = offsets[e] + cnt[e];
    offsets[E + 1] = S + SH;
    int32_t *row_token = (int32_t *)emu_alloc(4 * (size_t)R, "row_token");
    std::vector<int> toks(T);
    std::iota(toks.begin(), toks.end(), 0);
    for (int e = 0; e < E; ++e) {
        std::shuffle(toks.begin(), toks.end(), rng);
        std::vector<int> s(toks.begin(), toks.begin() + cnt[e]);
        std::sort(s.begin(), s.end());
        for (int i = 0; i < cnt[e]; ++i) row_token[offsets[e] + i] = s[i];
    }
    for (int t = 0; t < SH; ++t) row_token[S + t] = t;
    const int nsh = (SH + BM - 1) / BM;
    int tt = 0;
    for (int e = 0; e < E; ++e) tt += (cnt[e] + BM - 1) / BM;
    I4 *tab = (I4 *)emu_alloc(16 * (size_t)(1 + tt + nsh), "tile_tab");
    tab[0] = {tt + nsh, nsh, 0, 0};
    for (int t = 0; t < nsh; ++t) tab[1 + t] = {E, S + t * BM, std::min(BM, SH - t * BM), t | (std::min(nsh, 0x7fff) << 16)};
    for (int e = 0, toff = 0; e < E; ++e) {
        const int nt = (cnt[e] + BM - 1) / BM;
        for (int t = 0; t < nt; ++t)
            tab[1 + nsh + toff + t] = {e, offsets[e] + t * BM, std::min(BM, cnt[e] - t * BM), t | (std::min(nt, 0x7fff) << 16)};
        toff += nt;
    }
    printf("T=%d E=%d k=%d S=%d shared=%d tiles=%d (+%d shared) counts:", T, E, k, S, SH, tt, nsh);
    for (int e = 0; e < E; ++e) printf(" %d", cnt[e]);
    printf("\n");

    auto fp8buf = [&](size_t n, const char *name) {
        uint8_t *p = (uint8_t *)emu_alloc(n, name);
        for (size_t i = 0; i < n; ++i) { uint8_t b = rng() & 0x3f; p[i] = (rng() & 1 ? 0x80 : 0) | (b < 0x38 ? b + 0x08 : b - 0x20); }
        return p;
    };
    auto f32buf = [&](size_t n, const char *name, float lo, float hi) {
        float *p = (float *)emu_alloc(4 * n, name);
        std::uniform_real_distribution<float> d(lo, hi);
        for (size_t i = 0; i < n; ++i) p[i] = d(rng);
        return p;
    };
    auto packed = [&](const uint8_t *w, int batch, int n, int kk, const char *name) {
        uint8_t *p = (uint8_t *)emu_alloc((size_t)batch * n * kk, name);
        pack_frag(w, p, batch, n, kk);
        return p;
    };
    uint8_t *xq = fp8buf((size_t)T * H, "xq");
    float *xs_ = f32buf((size_t)T * (H / 128), "xs", 0.5f, 1.f);
    uint8_t *w13 = fp8buf((size_t)E * 2 * I * H, "w13");
    float *w13s = f32buf((size_t)E * (2 * I / 128) * (H / 128), "w13s", 0.001f, 0.002f);
    uint8_t *sw13 = fp8buf((size_t)2 * I * H, "sw13");
    float *sw13s = f32buf((size_t)(2 * I / 128) * (H / 128), "sw13s", 0.001f, 0.002f);
    uint8_t *w2 = fp8buf((size_t)E * H * I, "w2");
    float *w2s = f32buf((size_t)E * (H / 128) * (I / 128), "w2s", 0.001f, 0.002f);
    uint8_t *sw2 = fp8buf((size_t)H * I, "sw2");
    float *sw2s = f32buf((size_t)(H / 128) * (I / 128), "sw2s", 0.001f, 0.002f);
    uint8_t *w13p = packed(w13, E, 2 * I, H, "w13p"), *sw13p = packed(sw13, 1, 2 * I, H, "sw13p");
    uint8_t *w2p = packed(w2, E, H, I, "w2p"), *sw2p = packed(sw2, 1, H, I, "sw2p");
    uint8_t *actq = (uint8_t *)emu_alloc((size_t)R * I, "actq");
    float *acts = (float *)emu_alloc(4 * (size_t)R * (I / 128), "acts");
    float *y = (float *)emu_alloc(4 * (size_t)R * H, "y");

    GemmArgs g1 = {};
    g1.A = xq; g1.As = xs_; g1.row_token = row_token; g1.B = w13; g1.Bs = w13s; g1.Bsh = sw13; g1.Bssh = sw13s;
    g1.Bp = w13p; g1.Bshp = sw13p;
    g1.offsets = offsets; g1.tile_tab = (const int32_t *)tab; g1.E = E; g1.K = H; g1.N = I; g1.bm = BM; g1.e_lo = 0; g1.e_hi = E + (shared ? 1 : 0);
    g1.Cq = actq; g1.Cs = acts;
    GemmArgs g2 = {};
    g2.A = actq; g2.As = acts; g2.row_token = nullptr; g2.B = w2; g2.Bs = w2s; g2.Bsh = sw2; g2.Bssh = sw2s;
    g2.Bp = w2p; g2.Bshp = sw2p;
    g2.offsets = offsets; g2.tile_tab = (const int32_t *)tab; g2.E = E; g2.K = I; g2.N = H; g2.bm = BM; g2.e_lo = 0; g2.e_hi = E + (shared ? 1 : 0);
    g2.Cf = y; g2.ldc = H;

    auto run = [&](const GemmArgs &a, bool gateup) {
        const unsigned gx = (unsigned)(a.N / kBN), gy = (unsigned)(tt + nsh);
        const size_t smem = 16 * 1024;   // static arrays only
        printf("pass %s: K=%d grid %ux%u\n", gateup ? "gate_up" : "down", a.K, gx, gy);
        fflush(stdout);
        // the launcher's prefetch depth (8 for gate_up and for launches of
        // fewer than 512 blocks, else 4); EMU_WDD_PD=4|8 forces one
        const char *pf = getenv("EMU_WDD_PD");
        const bool deep = pf ? atoi(pf) == 8 : (gateup || (int64_t)gx * gy < 512);
#define XS_EMU_KB(KBV)                                                                                   \
        if (a.K == 128 * KBV) {                                                                          \
            constexpr int P4 = KBV < 4 ? KBV : 4, P8 = KBV < 8 ? KBV : 8;                                \
            if (gateup && deep) emu_launch([&] { moe_gemm_wdd_kernel<true, KBV, P8>(a); }, gx, gy, kNT, smem, conc); \
            else if (gateup) emu_launch([&] { moe_gemm_wdd_kernel<true, KBV, P4>(a); }, gx, gy, kNT, smem, conc); \
            else if (deep) emu_launch([&] { moe_gemm_wdd_kernel<false, KBV, P8>(a); }, gx, gy, kNT, smem, conc); \
            else emu_launch([&] { moe_gemm_wdd_kernel<false, KBV, P4>(a); }, gx, gy, kNT, smem, conc);   \
            return;                                                                                      \
        }
        XS_EMU_KB(4) XS_EMU_KB(8) XS_EMU_KB(16) XS_EMU_KB(32)
#undef XS_EMU_KB
        fprintf(stderr, "unsupported K=%d\n", a.K);
        exit(2);
    };
    run(g1, true);
    printf("gate_up done, errors %ld\n", g_errors.load());
    run(g2, false);
    printf("down done, errors %ld\n", g_errors.load());

    if (getenv("EMU_CMP_TILED")) {
        // the reference kernel on the same inputs (row-major weights): every
        // output byte must match
        std::vector<uint8_t> q0(actq, actq + (size_t)R * I);
        std::vector<float> s0(acts, acts + (size_t)R * (I / 128)), y0(y, y + (size_t)R * H);
        memset(actq, 0, (size_t)R * I);
        memset(acts, 0, 4 * (size_t)R * (I / 128));
        memset(y, 0, 4 * (size_t)R * H);
        GemmArgs t1 = g1, t2 = g2;
        t1.Bp = t1.Bshp = t2.Bp = t2.Bshp = nullptr;
        using namespace xs::tiled;
        const size_t sm1 = gemm_smem_bytes<16, true, false>(H), sm2 = gemm_smem_bytes<16, false, false>(I);
        emu_launch([&] { moe_gemm_kernel<16, true, false>(t1); }, I / 128, tt + nsh, Cfg<16, false>::NT, sm1, conc);
        emu_launch([&] { moe_gemm_kernel<16, false, false>(t2); }, (H + 255) / 256, tt + nsh, Cfg<16, false>::NT, sm2, conc);
        const bool same = !memcmp(q0.data(), actq, q0.size()) && !memcmp(s0.data(), acts, 4 * s0.size()) &&
                          !memcmp(y0.data(), y, 4 * y0.size());
        printf("tiled kernel: errors %ld, identical bytes: %s\n", g_errors.load(), same ? "yes" : "NO");
        if (!same) g_errors++;
    }

    if (g_math) {
        double maxerr = 0, maxref = 0;
        std::vector<float> act(I);
        for (int p = 0; p < R; ++p) {
            const int e = p < S ? (int)(std::upper_bound(offsets, offsets + E + 1, p) - offsets - 1) : E;
            const int tok = row_token[p];
            const uint8_t *W = e == E ? sw13 : w13 + (size_t)e * 2 * I * H;
            const float *Ws = e == E ? sw13s : w13s + (size_t)e * (2 * I / 128) * (H / 128);
            for (int n = 0; n < I; ++n) {
                double gsum = 0, usum = 0;
                for (int kb = 0; kb < H / 128; ++kb) {
                    float gp = 0, up = 0;
                    for (int kk = 0; kk < 128; ++kk) {
                        const float x = e4m3_dec(xq[(size_t)tok * H + kb * 128 + kk]);
                        gp += x * e4m3_dec(W[(size_t)n * H + kb * 128 + kk]);
                        up += x * e4m3_dec(W[(size_t)(I + n) * H + kb * 128 + kk]);
                    }
                    const float sa = xs_[(size_t)tok * (H / 128) + kb];
                    gsum += gp * sa * Ws[(size_t)(n / 128) * (H / 128) + kb];
                    usum += up * sa * Ws[(size_t)((I + n) / 128) * (H / 128) + kb];
                }
                act[n] = (float)(gsum / (1 + std::exp(-gsum)) * usum);
            }
            for (int n = 0; n < I; ++n) {
                const float got = e4m3_dec(actq[(size_t)p * I + n]) * acts[(size_t)p * (I / 128) + n / 128];
                maxerr = std::max(maxerr, (double)std::fabs(got - act[n]));
                maxref = std::max(maxref, (double)std::fabs(act[n]));
            }
        }
        printf("gate_up act: max abs err %.4g, max |ref| %.4g, rel %.4g\n", maxerr, maxref, maxerr / maxref);
        maxerr = maxref = 0;
        for (int p = 0; p < R; ++p) {
            const int e = p < S ? (int)(std::upper_bound(offsets, offsets + E + 1, p) - offsets - 1) : E;
            const uint8_t *W = e == E ? sw2 : w2 + (size_t)e * H * I;
            const float *Ws = e == E ? sw2s : w2s + (size_t)e * (H / 128) * (I / 128);
            for (int n = 0; n < H; ++n) {
                double s = 0;
                for (int kb = 0; kb < I / 128; ++kb) {
                    float d = 0;
                    for (int kk = 0; kk < 128; ++kk)
                        d += e4m3_dec(actq[(size_t)p * I + kb * 128 + kk]) * e4m3_dec(W[(size_t)n * I + kb * 128 + kk]);
                    s += d * acts[(size_t)p * (I / 128) + kb] * Ws[(size_t)(n / 128) * (I / 128) + kb];
                }
                const float got = y[(size_t)p * H + n];
                maxerr = std::max(maxerr, std::fabs(got - s));
                maxref = std::max(maxref, std::fabs(s));
            }
        }
        printf("down y: max abs err %.4g, max |ref| %.4g, rel %.4g\n", maxerr, maxref, maxerr / maxref);
    }
    if (g_hazard) printf("hazard hits %ld\n", g_hazard_hits.load());
    printf("errors %ld\n", g_errors.load());
    return g_errors.load() ? 1 : 0;
}
