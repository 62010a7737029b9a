// Host emulation of the single FP8 GEMM from fragment-packed B
// (gemm_wd_dense_kernel of moe_gemm_wd.hip): the kernel's own source runs on
// the CPU, and its bf16 output is compared bit for bit with the same
// arithmetic done directly: per 128-wide K block the MFMA's sum of exact FP8
// products (the emulated MFMA's order), folded into f32 as
// fma(block sum, row scale x block scale, acc) in K order, one bf16 rounding.
// usage: wdense_emu M N K conc mode(0 late, 1 early)
// EMU_HAZARD=1|2|3, EMU_HAZARD_P, EMU_HAZARD_SEED: the wait-state hazard model of emu.hpp
#include "emu.hpp"
#include <random>

#include "wd_emu.inc"

using namespace xs;

static void pack_frag(const uint8_t *w, uint8_t *out, int n, int k)
{
    const int KB = k / 128;
    const size_t chunks = (size_t)n * k / 16;
    for (size_t c = 0; c < chunks; ++c) {
        const int l = (int)(c & 63), h = (int)((c >> 6) & 1);
        const size_t blk = c >> 7;
        const int kb = (int)(blk % KB);
        const size_t t = blk / KB;
        memcpy(out + c * 16, w + (16 * t + (l & 15)) * (size_t)k + 128 * kb + 64 * h + 16 * (l >> 4), 16);
    }
}

int main(int argc, char **argv)
{
    const int M = argc > 1 ? atoi(argv[1]) : 100, N = argc > 2 ? atoi(argv[2]) : 512, K = argc > 3 ? atoi(argv[3]) : 1024;
    const int conc = argc > 4 ? atoi(argv[4]) : 4;
    g_mode = argc > 5 ? atoi(argv[5]) : 0;
    g_math = true;
    if (getenv("EMU_HAZARD")) g_hazard = atoi(getenv("EMU_HAZARD"));
    if (getenv("EMU_HAZARD_P")) g_hazard_p = atof(getenv("EMU_HAZARD_P"));
    if (getenv("EMU_HAZARD_SEED")) g_hazard_seed = atoi(getenv("EMU_HAZARD_SEED"));
    std::mt19937 rng(M * 131 + N * 7 + K);
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
    const int KB = K / 128;
    uint8_t *A = fp8buf((size_t)M * K, "A");
    float *As = f32buf((size_t)M * KB, "As", 0.5f, 1.f);
    uint8_t *B = fp8buf((size_t)N * K, "B");
    float *Bs = f32buf((size_t)(N / 128) * KB, "Bs", 0.001f, 0.002f);
    uint8_t *Bp = (uint8_t *)emu_alloc((size_t)N * K, "Bp");
    pack_frag(B, Bp, N, K);
    uint16_t *C = (uint16_t *)emu_alloc(2 * (size_t)M * N, "C");
    for (size_t i = 0; i < (size_t)M * N; ++i) C[i] = 0xFFFF;   // a NaN no kernel writes

    GemmArgs a = {};
    a.A = A; a.As = As; a.Bshp = Bp; a.Bssh = Bs; a.E = 0; a.K = K; a.N = N; a.bm = kDenseBM;
    a.Cy = C; a.ldc = N; a.sh_rows = M;
    const size_t smem = (size_t)kNSA * ((size_t)kDenseBM * 128 + kDenseBM * 4) + 8 * (size_t)KB + 4 * kNW * kDenseBM + 256;
    const int64_t total = (M + kDenseBM - 1) / kDenseBM * (N / 256);
    const unsigned nb = (unsigned)(8 * ((total + 7) / 8));
    printf("M=%d N=%d K=%d: %lld tiles, %u blocks, smem %zu\n", M, N, K, (long long)total, nb, smem);
    // the launcher's choice: unrolled kernels for 4, 8, 16 and 32 K steps
#define XS_EMU_KB(KBV)                                                                  \
    if (KB == KBV || KBV == 0) {                                                        \
        emu_launch([&] { gemm_wd_dense_kernel<KBV>(a); }, nb, 1, kNT, smem, conc);      \
    } else
    XS_EMU_KB(4) XS_EMU_KB(8) XS_EMU_KB(16) XS_EMU_KB(32) XS_EMU_KB(0) {}
#undef XS_EMU_KB
    printf("kernel done, errors %ld\n", g_errors.load());

    long diff = 0;
    for (int m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n) {
            float acc = 0.f;
            for (int kb = 0; kb < KB; ++kb) {
                float s = 0;
                for (int k = 0; k < 128; ++k)
                    s += e4m3_dec(B[(size_t)n * K + kb * 128 + k]) * 1.f * e4m3_dec(A[(size_t)m * K + kb * 128 + k]) * 1.f;
                s = 0.f + s;
                const float c = As[(size_t)m * KB + kb] * Bs[(size_t)(n / 128) * KB + kb];
                acc = std::fma(s, c, acc);
            }
            const uint16_t want = bf16_from_f32(acc);
            if (C[(size_t)m * N + n] != want && diff++ < 10)
                fprintf(stderr, "C[%d][%d] = %04x, want %04x\n", m, n, C[(size_t)m * N + n], want);
        }
    printf("bf16 outputs differing from the direct computation: %ld of %lld\n", diff, (long long)M * N);
    if (diff) g_errors++;
    if (g_hazard) printf("hazard hits %ld\n", g_hazard_hits.load());
    printf("errors %ld\n", g_errors.load());
    return g_errors.load() ? 1 : 0;
}
