// Additions to emu.hpp for the router kernels of moe_router.hip: the wave
// exchanges they use (shuffles of ints, shfl_up, readlane, DPP row patterns,
// __any), device atomics, the bf16 16x16x32 MFMA (exact products, the sum
// rounded once to f32), and a launcher with a z grid dimension.
#pragma once
#include "emu.hpp"

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

inline float __fadd_rn(float a, float b) { return a + b; }
inline float __fmul_rn(float a, float b) { return a * b; }
inline float __int_as_float(int i) { float f; memcpy(&f, &i, 4); return f; }
inline int atomicOr(uint32_t *p, uint32_t v) { return (int)__atomic_fetch_or(p, v, __ATOMIC_RELAXED); }

// every lane posts v; returns the value lane src posted
inline uint64_t emu_xchg(uint64_t v, int src)
{
    const int w = wave_id(), l = lane_id();
    tb->xch[w][l] = v;
    emu_xpost(w, l, 5);
    tb->wbar[w]->arrive_and_wait();
    emu_xcheck(w, l);
    const uint64_t r = tb->xch[w][src & 63];
    tb->wbar[w]->arrive_and_wait();
    return r;
}
inline int __shfl_xor(int v, int m, int) { return (int)(uint32_t)emu_xchg((uint32_t)v, lane_id() ^ m); }
inline int __shfl_up(int v, int d, int)
{
    const int l = lane_id();
    return (int)(uint32_t)emu_xchg((uint32_t)v, l >= d ? l - d : l);
}
inline int emu_readlane(int v, int src) { return (int)(uint32_t)emu_xchg((uint32_t)v, src); }
#define __builtin_amdgcn_readlane(v, l) emu_readlane((v), (l))
inline int __any(int pred)
{
    const int w = wave_id(), l = lane_id();
    tb->xch[w][l] = pred != 0;
    emu_xpost(w, l, 6);
    tb->wbar[w]->arrive_and_wait();
    emu_xcheck(w, l);
    int r = 0;
    for (int i = 0; i < 64; ++i) r |= (int)tb->xch[w][i];
    tb->wbar[w]->arrive_and_wait();
    return r;
}
// DPP row patterns used by the route kernel: quad_perm (0x00-0xff),
// row_mirror (0x140), row_half_mirror (0x141); all rows and banks enabled
inline int emu_dpp(int old, int src, int ctrl, int, int, bool)
{
    (void)old;
    const int l = lane_id();
    int from;
    if (ctrl < 0x100) from = (l & ~3) + ((ctrl >> (2 * (l & 3))) & 3);
    else if (ctrl == 0x140) from = (l & ~15) + 15 - (l & 15);
    else if (ctrl == 0x141) from = (l & ~7) + 7 - (l & 7);
    else { EMU_ERR("DPP control %#x not modelled", ctrl); from = l; }
    return (int)(uint32_t)emu_xchg((uint32_t)src, from);
}
#define __builtin_amdgcn_update_dpp(o, s, c, r, b, bc) emu_dpp((o), (s), (c), (r), (b), (bc))

// bf16 16x16x32: lane 16g + r gives row r, K elements [8g, 8g + 8) of A and
// B; lane 16g + r receives C[4g + v][r] += sum_k A[4g + v][k] B[r][k].  The
// hardware's internal order and rounding are not specified, so the model is
// selectable (EMU_MFMA_MODEL): 0 the exact products summed in double and
// rounded once with C; 1 C plus the products in k order, each add rounded to
// f32; 2 the same with every add truncated toward zero (the coarsest
// behaviour the certified router's bound allows for); 3 and 4 C and the 32
// products added in a random order (a fresh one per output), rounded (3) or
// truncated (4); 5 a pairwise tree over the products, rounded, then C.
// Every bf16 x bf16 product is exact in f32.
inline int g_mfma_model = 0;
// a + b truncated toward zero, exactly: s = RNE(a + b) and its error e
// (Knuth's two-sum, exact in f32); the truncated sum is s unless e points
// toward zero from s, then the next float toward zero
inline float emu_add_rz(float a, float b)
{
    const float s = a + b;
    const float bb = s - a, e = (a - (s - bb)) + (b - bb);
    if (e == 0.0f || !std::isfinite(s)) return s;
    return (e > 0.0f) == (s > 0.0f) ? s : std::nextafter(s, 0.0f);
}
inline float bf16v(__bf16 b) { uint16_t u; memcpy(&u, &b, 2); return __uint_as_float((uint32_t)u << 16); }
inline v4f emu_mfma_bf16(v8bf a, v8bf b, v4f c, int, int, int)
{
    const int w = wave_id(), l = lane_id();
    memcpy(tb->wx[w][l], &a, 16);
    memcpy(tb->wx[w][l] + 16, &b, 16);
    emu_xpost(w, l, 3);
    tb->wbar[w]->arrive_and_wait();
    emu_xcheck(w, l);
    const int r = l & 15, g = l >> 4;
    v4f out;
    auto el = [&](int row, int k, int off) {
        __bf16 v;
        memcpy(&v, tb->wx[w][16 * (k / 8) + row] + off + 2 * (k % 8), 2);
        return (double)bf16v(v);
    };
    for (int v = 0; v < 4; ++v) {
        float p[33];
        for (int k = 0; k < 32; ++k) p[k] = (float)(el(4 * g + v, k, 0) * el(r, k, 16));
        if (g_mfma_model == 0) {
            double s = c[v];
            for (int k = 0; k < 32; ++k) s += p[k];
            out[v] = (float)s;
        } else if (g_mfma_model <= 2) {
            float s = c[v];
            for (int k = 0; k < 32; ++k) s = g_mfma_model == 1 ? s + p[k] : emu_add_rz(s, p[k]);
            out[v] = s;
        } else if (g_mfma_model <= 4) {
            p[32] = c[v];
            uint64_t z = ((uint64_t)blockIdx.x << 40) ^ ((uint64_t)blockIdx.y << 20) ^ ((uint64_t)threadIdx.x << 8) ^
                         (t_xseq << 2) ^ (uint64_t)v;   // t_xseq: this lane's exchange count
            for (int i = 32; i > 0; --i) {   // Fisher-Yates with splitmix64
                z += 0x9e3779b97f4a7c15ull;
                uint64_t y = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
                y = (y ^ (y >> 27)) * 0x94d049bb133111ebull;
                std::swap(p[i], p[(y ^ (y >> 31)) % (uint64_t)(i + 1)]);
            }
            float s = p[0];
            for (int i = 1; i < 33; ++i) s = g_mfma_model == 3 ? s + p[i] : emu_add_rz(s, p[i]);
            out[v] = s;
        } else {
            for (int n = 32; n > 1; n /= 2)
                for (int i = 0; i < n / 2; ++i) p[i] = p[2 * i] + p[2 * i + 1];
            out[v] = c[v] + p[0];
        }
    }
    tb->wbar[w]->arrive_and_wait();
    return out;
}
#define __builtin_amdgcn_mfma_f32_16x16x32_bf16 emu_mfma_bf16

// the tile kernel's DMA: a per-lane source, a wave-uniform LDS base
inline void dma16x(const void *g, uint32_t lds)
{
    lds = (uint32_t)wave_first(lds, "rt_dma16 lds");
    dma_lane((const uint8_t *)g, lds, 16, "rt_dma16");
}

template <typename F>
inline void emu_launch3(F fn, unsigned gx, unsigned gy, unsigned gz, unsigned nt, size_t smem, unsigned /*conc*/)
{
    emu_run_grid(fn, {gx, gy, gz}, nt, smem ? smem : 16, 0);
}
