// Host emulation of the weight-direct MXFP4 GEMMs (moe_gemm_wd4.hip): the
// routed experts' gate_up (SwiGLU, MXFP8 requantised) and down GEMMs on
// BM-row tiles run from the kernel's own source, then both are checked
// against a float64 recomputation from the same MXFP4 / MXFP8 inputs.
// usage: wd4_emu T E k zipf seed H I conc mode(0 late,1 early) math(0/1) BM(64|128)
// EMU_CMP_TILED=1 also runs the tiled MXFP4 kernel of moe_gemm.hip on the same
// inputs and compares the bytes of the routed rows
#include "emu.hpp"
#include <algorithm>
#include <numeric>
#include <random>

#include "wd4_emu.inc"
#include "tiled_emu.inc"

using namespace xs;
using I4 = int4;

// [batch, n, k/2] + [batch, n, k/32] -> fragment order (xs_pack_weight_mxfp4_frag)
static void pack4(const uint8_t *w, const uint8_t *s, uint8_t *ow, uint8_t *os, int batch, int n, int k)
{
    const int KS = k / 128;
    const size_t chunks = (size_t)batch * (n / 16) * KS * 64;
    for (size_t c = 0; c < chunks; ++c) {
        const int l = (int)(c & 63);
        const size_t blk = c >> 6;
        const int ks = (int)(blk % KS);
        const size_t bt = blk / KS;
        const size_t b = bt / (n / 16), t = bt % (n / 16);
        const size_t row = b * n + 16 * t + (l & 15);
        memcpy(ow + c * 16, w + row * (k / 2) + 64 * ks + 16 * (l >> 4), 16);
        os[c] = s[row * (k / 32) + 4 * ks + (l >> 4)];
    }
}
static float fp4_at(const uint8_t *row, int kk) { const uint8_t b = row[kk / 2]; return e2m1_dec((kk & 1) ? b >> 4 : b & 15); }
static double e8(uint8_t s) { return std::ldexp(1.0, (int)s - 127); }

int main(int argc, char **argv)
{
    int T = argc > 1 ? atoi(argv[1]) : 64, E = argc > 2 ? atoi(argv[2]) : 4, k = argc > 3 ? atoi(argv[3]) : 2;
    double zipf = argc > 4 ? atof(argv[4]) : 1.1;
    int seed = argc > 5 ? atoi(argv[5]) : 21;
    int H = argc > 6 ? atoi(argv[6]) : 1024, I = argc > 7 ? atoi(argv[7]) : 512;
    int conc = argc > 8 ? atoi(argv[8]) : 4;
    g_mode = argc > 9 ? atoi(argv[9]) : 0;
    g_math = argc > 10 ? atoi(argv[10]) : 1;
    const int BM = argc > 11 ? atoi(argv[11]) : 64;
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
    const int SH = T, R = S + SH;   // a shared segment in the table (FP8: not this kernel's)
    int32_t *offsets = (int32_t *)emu_alloc(4 * (E + 2), "offsets");
    offsets[0] = 0;
    for (int e = 0; e < E; ++e) offsets[e + 1] = offsets[e] + cnt[e];
    offsets[E + 1] = S + SH;
    int32_t *row_token = (int32_t *)emu_alloc(4 * (size_t)R, "row_token");
    std::vector<int> toks(T);
    std::iota(toks.begin(), toks.end(), 0);
    for (int e = 0; e < E; ++e) {
        std::shuffle(toks.begin(), toks.end(), rng);
        std::vector<int> sv(toks.begin(), toks.begin() + cnt[e]);
        std::sort(sv.begin(), sv.end());
        for (int i = 0; i < cnt[e]; ++i) row_token[offsets[e] + i] = sv[i];
    }
    for (int t = 0; t < SH; ++t) row_token[S + t] = t;
    const int nsh = (SH + BM - 1) / BM;
    int tt = 0;
    for (int e = 0; e < E; ++e) tt += (cnt[e] + BM - 1) / BM;
    I4 *tab = (I4 *)emu_alloc(16 * (size_t)(1 + tt + nsh), "tile_tab");
    tab[0] = {tt + nsh, nsh, 0, 0};
    for (int t = 0; t < nsh; ++t) tab[1 + t] = {E, S + t * BM, std::min(BM, SH - t * BM), 0};
    for (int e = 0, toff = 0; e < E; ++e) {
        const int nt = (cnt[e] + BM - 1) / BM;
        for (int t = 0; t < nt; ++t) tab[1 + nsh + toff + t] = {e, offsets[e] + t * BM, std::min(BM, cnt[e] - t * BM), 0};
        toff += nt;
    }
    printf("T=%d E=%d k=%d S=%d BM=%d routed tiles=%d counts:", T, E, k, S, BM, tt);
    for (int e = 0; e < E; ++e) printf(" %d", cnt[e]);
    printf("\n");

    auto bytes = [&](size_t n, const char *name, int lo, int hi) {
        uint8_t *p = (uint8_t *)emu_alloc(n, name);
        std::uniform_int_distribution<int> d(lo, hi);
        for (size_t i = 0; i < n; ++i) p[i] = (uint8_t)d(rng);
        return p;
    };
    auto fp8buf = [&](size_t n, const char *name) {
        uint8_t *p = (uint8_t *)emu_alloc(n, name);
        for (size_t i = 0; i < n; ++i) { uint8_t b = rng() & 0x3f; p[i] = (rng() & 1 ? 0x80 : 0) | (b < 0x38 ? b + 0x08 : b - 0x20); }
        return p;
    };
    uint8_t *xq = fp8buf((size_t)T * H, "xq");
    uint8_t *xs_ = bytes((size_t)T * (H / 32), "xs", 122, 128);
    uint8_t *w13 = bytes((size_t)E * 2 * I * H / 2, "w13", 0, 255);
    uint8_t *s13 = bytes((size_t)E * 2 * I * (H / 32), "s13", 118, 124);
    uint8_t *w2 = bytes((size_t)E * H * I / 2, "w2", 0, 255);
    uint8_t *s2 = bytes((size_t)E * H * (I / 32), "s2", 118, 124);
    uint8_t *w13p = (uint8_t *)emu_alloc((size_t)E * 2 * I * H / 2, "w13p");
    uint8_t *s13p = (uint8_t *)emu_alloc((size_t)E * 2 * I * (H / 32), "s13p");
    uint8_t *w2p = (uint8_t *)emu_alloc((size_t)E * H * I / 2, "w2p");
    uint8_t *s2p = (uint8_t *)emu_alloc((size_t)E * H * (I / 32), "s2p");
    pack4(w13, s13, w13p, s13p, E, 2 * I, H);
    pack4(w2, s2, w2p, s2p, E, H, I);
    uint8_t *actq = (uint8_t *)emu_alloc((size_t)R * I, "actq");
    uint8_t *acts = (uint8_t *)emu_alloc((size_t)R * (I / 32), "acts");
    float *y = (float *)emu_alloc(4 * (size_t)R * H, "y");

    GemmArgs g1 = {};
    g1.A = xq; g1.As = xs_; g1.row_token = row_token; g1.Bp = w13p; g1.Bsp = s13p;
    g1.offsets = offsets; g1.tile_tab = (const int32_t *)tab; g1.E = E; g1.K = H; g1.N = I; g1.bm = BM;
    g1.Cq = actq; g1.Cs = acts;
    GemmArgs g2 = {};
    g2.A = actq; g2.As = acts; g2.row_token = nullptr; g2.Bp = w2p; g2.Bsp = s2p;
    g2.offsets = offsets; g2.tile_tab = (const int32_t *)tab; g2.E = E; g2.K = I; g2.N = H; g2.bm = BM;
    g2.Cf = y; g2.ldc = H;

    for (int pass = 0; pass < 2; ++pass) {
        const GemmArgs &a = pass ? g2 : g1;
        const int KB = a.K / 128;
        const size_t stage = (size_t)BM * 128 + BM * 4;
        const size_t smem = 5 * stage + 4 * 8 * (size_t)BM + 256;
        const int gx = pass ? a.N / 256 : a.N / 128;
        const unsigned nb = (unsigned)(((tt + 7) / 8 * (gx / 4) + 7) / 8 * 256);
        printf("pass %d: K=%d smem %zu, blocks %u\n", pass, a.K, smem, nb);
        // the launcher's choice: 64-row tiles unrolled for 16 and 32 slices
#define XS_EMU(BMV, KBV)                                                                                       \
        if (BM == BMV && (KB == KBV || KBV == 0)) {                                                            \
            if (pass == 0) emu_launch([&] { moe_gemm_wd4_kernel<true, KBV, BMV>(a); }, nb, 1, kNT, smem, conc); \
            else emu_launch([&] { moe_gemm_wd4_kernel<false, KBV, BMV>(a); }, nb, 1, kNT, smem, conc);         \
        } else
        XS_EMU(64, 16) XS_EMU(64, 32) XS_EMU(64, 0) XS_EMU(128, 0) { fprintf(stderr, "unsupported\n"); return 2; }
#undef XS_EMU
        printf("pass %d done, errors %ld\n", pass, g_errors.load());
    }

    if (getenv("EMU_CMP_TILED")) {
        std::vector<uint8_t> q0(actq, actq + (size_t)S * I), s0(acts, acts + (size_t)S * (I / 32));
        std::vector<float> y0(y, y + (size_t)S * H);
        memset(actq, 0, (size_t)R * I);
        memset(acts, 0, (size_t)R * (I / 32));
        memset(y, 0, 4 * (size_t)R * H);
        GemmArgs t1 = g1, t2 = g2;
        t1.B = w13; t1.Bs = s13; t2.B = w2; t2.Bs = s2;
        t1.Bp = t2.Bp = t1.Bsp = t2.Bsp = nullptr;
        t1.e_lo = t2.e_lo = 0;
        t1.e_hi = t2.e_hi = E;   // routed tiles only
        using namespace xs::tiled;
#define XS_EMU_T(BMV)                                                                                         \
        if (BM == BMV) {                                                                                      \
            emu_launch([&] { moe_gemm_kernel<BMV, true, true>(t1); }, I / 128, tt, Cfg<BMV, true>::NT,         \
                       gemm_smem_bytes<BMV, true, true>(H), conc);                                            \
            emu_launch([&] { moe_gemm_kernel<BMV, false, true>(t2); }, (H + 255) / 256, tt, Cfg<BMV, true>::NT, \
                       gemm_smem_bytes<BMV, false, true>(I), conc);                                           \
        }
        XS_EMU_T(64) XS_EMU_T(128)
#undef XS_EMU_T
        const bool same = !memcmp(q0.data(), actq, q0.size()) && !memcmp(s0.data(), acts, s0.size()) &&
                          !memcmp(y0.data(), y, 4 * y0.size());
        printf("tiled kernel: errors %ld, identical bytes: %s\n", g_errors.load(), same ? "yes" : "NO");
        if (!same) g_errors++;
    }

    if (g_math) {
        double maxerr = 0, maxref = 0;
        long viol = 0;
        std::vector<double> act(I), acc_slack(I);
        for (int p = 0; p < S; ++p) {
            const int e = (int)(std::upper_bound(offsets, offsets + E + 1, p) - offsets - 1);
            const int tok = row_token[p];
            for (int n = 0; n < I; ++n) {
                double gs = 0, us = 0, ga = 0, ua = 0;
                const uint8_t *gr = w13 + ((size_t)e * 2 * I + n) * (H / 2), *ur = w13 + ((size_t)e * 2 * I + I + n) * (H / 2);
                const uint8_t *gsr = s13 + ((size_t)e * 2 * I + n) * (H / 32), *usr = s13 + ((size_t)e * 2 * I + I + n) * (H / 32);
                for (int kk = 0; kk < H; ++kk) {
                    const double x = e4m3_dec(xq[(size_t)tok * H + kk]) * e8(xs_[(size_t)tok * (H / 32) + kk / 32]);
                    gs += x * fp4_at(gr, kk) * e8(gsr[kk / 32]);
                    us += x * fp4_at(ur, kk) * e8(usr[kk / 32]);
                    ga += std::fabs(x * fp4_at(gr, kk) * e8(gsr[kk / 32]));
                    ua += std::fabs(x * fp4_at(ur, kk) * e8(usr[kk / 32]));
                }
                act[n] = gs / (1 + std::exp(-gs)) * us;
                // the kernel's f32 sums of H products are off by up to about
                // 16 f32 ulps of the sum of |products|, which moves SwiGLU by
                // |silu'(g) u| dg + |silu(g)| du
                const double sg = 1 / (1 + std::exp(-gs));
                acc_slack[n] = 1e-6 * (std::fabs(sg * (1 + gs * (1 - sg)) * us) * ga + std::fabs(gs * sg) * ua);
            }
            for (int n = 0; n < I; ++n) {
                const uint8_t sc = acts[(size_t)p * (I / 32) + n / 32];
                const double got = e4m3_dec(actq[(size_t)p * I + n]) * e8(sc);
                const double err = std::fabs(got - act[n]), a = std::fabs(act[n]);
                maxerr = std::max(maxerr, err);
                maxref = std::max(maxref, a);
                // given the block's scale 2^se: the clamp at 448 2^se, else half
                // an e4m3 step (2^-4 relative; 2^-10 2^se below the normals), plus
                // the f32 accumulation's rounding (a value within that of a
                // rounding tie may land on either side of it)
                const double lim = std::max({a - 448 * e8(sc), a / 16, e8(sc) / 1024}) + acc_slack[n] + 1e-30;
                if (err > lim && ++viol <= 4)
                    printf("  act[%d][%d]: ref %.9g got %.9g err %.4g lim %.4g scale 2^%d\n", p, n, act[n], got, err, lim, (int)sc - 127);
            }
        }
        printf("gate_up act: max abs err %.4g, max |ref| %.4g, rel %.4g, outside the MXFP8 bound %ld\n", maxerr, maxref,
               maxerr / maxref, viol);
        maxerr = maxref = 0;
        for (int p = 0; p < S; ++p) {
            const int e = (int)(std::upper_bound(offsets, offsets + E + 1, p) - offsets - 1);
            for (int n = 0; n < H; ++n) {
                const uint8_t *wr = w2 + ((size_t)e * H + n) * (I / 2), *sr = s2 + ((size_t)e * H + n) * (I / 32);
                double sum = 0;
                for (int kk = 0; kk < I; ++kk)
                    sum += e4m3_dec(actq[(size_t)p * I + kk]) * e8(acts[(size_t)p * (I / 32) + kk / 32]) * fp4_at(wr, kk) *
                           e8(sr[kk / 32]);
                maxerr = std::max(maxerr, std::fabs(y[(size_t)p * H + n] - sum));
                maxref = std::max(maxref, std::fabs(sum));
            }
        }
        printf("down y: max abs err %.4g, max |ref| %.4g, rel %.4g\n", maxerr, maxref, maxerr / maxref);
    }
    printf("errors %ld\n", g_errors.load());
    return g_errors.load() ? 1 : 0;
}
