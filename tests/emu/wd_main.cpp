// Host emulation of the weight-direct tall-tile GEMMs (moe_gemm_wd.hip): a
// skewed MoE layer's gate_up (SwiGLU, FP8 requantised) and down GEMMs run from
// the kernel's own source, then both are checked against a float64
// recomputation from the same FP8 inputs.
// usage: wd_emu T E k zipf seed H I conc mode(0 late,1 early) math(0/1) shared(0/1)
// EMU_HAZARD=1|2|3, EMU_HAZARD_P, EMU_HAZARD_SEED: the wait-state hazard model of emu.hpp
// EMU_CMP_WIDE=1 also runs the tall-tile LDS-ring kernel of moe_gemm_wide.hip
// (192-row tiles) on the same inputs and compares the bytes
#include "emu.hpp"
#include <algorithm>
#include <numeric>
#include <random>

#include "wd_emu.inc"
#include "wide_emu.inc"

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
    const int BM = kBM;
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
    g1.offsets = offsets; g1.tile_tab = (const int32_t *)tab; g1.E = E; g1.K = H; g1.N = I; g1.bm = BM;
    g1.Cq = actq; g1.Cs = acts;
    GemmArgs g2 = {};
    g2.A = actq; g2.As = acts; g2.row_token = nullptr; g2.B = w2; g2.Bs = w2s; g2.Bsh = sw2; g2.Bssh = sw2s;
    g2.Bp = w2p; g2.Bshp = sw2p;
    g2.offsets = offsets; g2.tile_tab = (const int32_t *)tab; g2.E = E; g2.K = I; g2.N = H; g2.bm = BM;
    g2.Cf = y; g2.ldc = H;
    // every tile of the table: the shared segment (when present) and the routed experts
    g1.e_lo = g2.e_lo = 0;
    g1.e_hi = g2.e_hi = E + 1;

    for (int pass = 0; pass < 2; ++pass) {
        const GemmArgs &a = pass ? g2 : g1;
        const int KB = a.K / 128;
        const size_t smem = (size_t)kNSA * kStage + 8 * (size_t)KB + 4 * kNW * kBM + 256;
        const int gx = pass ? a.N / 256 : a.N / 128;
        const int gy = tt + nsh;
        const unsigned nb = (unsigned)(((gy + 7) / 8 * (gx / 4) + 7) / 8 * 256);
        printf("pass %d: smem %zu, blocks %u\n", pass, smem, nb);
        // the launcher's choice: unrolled kernels for 4, 8, 16 and 32 K steps
#define XS_EMU_KB(KBV)                                                                                  \
        if (KB == KBV || KBV == 0) {                                                                    \
            if (pass == 0) emu_launch([&] { moe_gemm_wd_kernel<true, KBV>(a); }, nb, 1, kNT, smem, conc); \
            else emu_launch([&] { moe_gemm_wd_kernel<false, KBV>(a); }, nb, 1, kNT, smem, conc);          \
        } else
        XS_EMU_KB(4) XS_EMU_KB(8) XS_EMU_KB(16) XS_EMU_KB(32) XS_EMU_KB(0) {}
#undef XS_EMU_KB
        printf("pass %d done, errors %ld\n", pass, g_errors.load());
    }

    if (getenv("EMU_CMP_SHARED") && SH > 0) {
        // the shared segment alone, in 128-row tiles the kernel computes
        // itself (no tile table): the same bytes in the shared rows
        std::vector<uint8_t> q0(actq + (size_t)S * I, actq + (size_t)R * I);
        std::vector<float> s0(acts + (size_t)S * (I / 128), acts + (size_t)R * (I / 128));
        std::vector<float> y0(y + (size_t)S * H, y + (size_t)R * H);
        std::vector<uint8_t> qa(actq, actq + (size_t)R * I);   // restored afterwards
        std::vector<float> sa(acts, acts + (size_t)R * (I / 128)), ya(y, y + (size_t)R * H);
        memset(actq, 0, (size_t)R * I);
        memset(acts, 0, 4 * (size_t)R * (I / 128));
        memset(y, 0, 4 * (size_t)R * H);
        GemmArgs h1 = g1, h2 = g2;
        h1.tile_tab = h2.tile_tab = nullptr;
        h1.Bp = h2.Bp = nullptr;
        h1.sh_rows = h2.sh_rows = SH;
        h1.shared_base = h2.shared_base = S;
        h1.e_lo = h2.e_lo = E;
        h1.e_hi = h2.e_hi = E + 1;
        const int st = (SH + kBM - 1) / kBM;
        for (int pass = 0; pass < 2; ++pass) {
            const GemmArgs &a = pass ? h2 : h1;
            const int KB = a.K / 128;
            const size_t smem = (size_t)kNSA * kStage + 8 * (size_t)KB + 4 * kNW * kBM + 256;
            const int gx = pass ? a.N / 256 : a.N / 128;
            const unsigned nb = (unsigned)(((st + 7) / 8 * (gx / 4) + 7) / 8 * 256);
            if (pass == 0) emu_launch([&] { moe_gemm_wd_kernel<true, 0>(a); }, nb, 1, kNT, smem, conc);
            else emu_launch([&] { moe_gemm_wd_kernel<false, 0>(a); }, nb, 1, kNT, smem, conc);
        }
        bool same = !memcmp(q0.data(), actq + (size_t)S * I, q0.size()) &&
                    !memcmp(s0.data(), acts + (size_t)S * (I / 128), 4 * s0.size()) &&
                    !memcmp(y0.data(), y + (size_t)S * H, 4 * y0.size());
        for (size_t i = 0; same && i < (size_t)S * I; ++i) same = actq[i] == 0;   // routed rows untouched
        printf("shared segment alone: errors %ld, identical bytes: %s\n", g_errors.load(), same ? "yes" : "NO");
        if (!same) g_errors++;
        memcpy(actq, qa.data(), qa.size());
        memcpy(acts, sa.data(), 4 * sa.size());
        memcpy(y, ya.data(), 4 * ya.size());
    }

    if (getenv("EMU_CMP_WIDE")) {
        // the LDS-ring kernel on its own 192-row tile table: every output byte
        // must match (the same per-row arithmetic in the same order)
        const int WB = 192;
        const int wsh = (SH + WB - 1) / WB;
        int wt = 0;
        for (int e = 0; e < E; ++e) wt += (cnt[e] + WB - 1) / WB;
        I4 *wtab = (I4 *)emu_alloc(16 * (size_t)(1 + wt + wsh), "wide_tile_tab");
        wtab[0] = {wt + wsh, wsh, 0, 0};
        for (int t = 0; t < wsh; ++t) wtab[1 + t] = {E, S + t * WB, std::min(WB, SH - t * WB), t | (std::min(wsh, 0x7fff) << 16)};
        for (int e = 0, toff = 0; e < E; ++e) {
            const int nt = (cnt[e] + WB - 1) / WB;
            for (int t = 0; t < nt; ++t)
                wtab[1 + wsh + toff + t] = {e, offsets[e] + t * WB, std::min(WB, cnt[e] - t * WB), t | (std::min(nt, 0x7fff) << 16)};
            toff += nt;
        }
        std::vector<uint8_t> q0(actq, actq + (size_t)R * I);
        std::vector<float> s0(acts, acts + (size_t)R * (I / 128)), y0(y, y + (size_t)R * H);
        memset(actq, 0, (size_t)R * I);
        memset(acts, 0, 4 * (size_t)R * (I / 128));
        memset(y, 0, 4 * (size_t)R * H);
        GemmArgs w1 = g1, w2a = g2;
        w1.Bp = w1.Bshp = w2a.Bp = w2a.Bshp = nullptr;
        w1.tile_tab = w2a.tile_tab = (const int32_t *)wtab;
        w1.bm = w2a.bm = WB;
        w1.xcd_order = w2a.xcd_order = 1;
        w1.short_deep = w2a.short_deep = 1;
        for (int pass = 0; pass < 2; ++pass) {
            const GemmArgs &a = pass ? w2a : w1;
            const size_t smem = (size_t)xs::wide::kRing + xs::wide::kTrash + 8 * (size_t)(a.K / 128) + 4 * 4 * WB;
            const int gx = pass ? a.N / 256 : a.N / 128;
            const unsigned nb = (unsigned)(((wt + wsh + 7) / 8 * (gx / 4) + 7) / 8 * 256);
            if (pass == 0) emu_launch([&] { xs::wide::moe_gemm_wide_kernel<192, true, 8>(a); }, nb, 1, 512, smem, conc);
            else emu_launch([&] { xs::wide::moe_gemm_wide_kernel<192, false, 8>(a); }, nb, 1, 512, smem, conc);
        }
        const bool same = !memcmp(q0.data(), actq, q0.size()) && !memcmp(s0.data(), acts, 4 * s0.size()) &&
                          !memcmp(y0.data(), y, 4 * y0.size());
        printf("tall-tile kernel: errors %ld, identical bytes: %s\n", g_errors.load(), same ? "yes" : "NO");
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
