// moe_gemm_wd4.hip -- grouped MXFP4 expert GEMMs with the weights loaded
// straight into VGPRs (gfx950), when the layer holds a fragment-packed copy of
// its MXFP4 weights and scales.
//
// Nearest reference code: gemm_silu_and_mul_kernel (xstar_cpp/src/ops/mlp.cu:52-200)
// and gemm_kernel (xstar_cpp/src/ops/gemm.cu:41-210).  Numerics are those of
// the MXFP4 tiles of moe_gemm.hip, step for step: weights e2m1 (operand A) and
// activations MXFP8 e4m3 (operand B), each with e8m0 scales per 32 K applied
// by v_mfma_scale_f32_16x16x128_f8f6f4, accumulated across K in K order;
// SwiGLU in f32, then MXFP8 1x32 requantisation for the down GEMM.  The two
// kernels give the same bits.
//
// As in moe_gemm_wd.hip (the FP8 form), a wave's weight fragments go from HBM
// straight into the registers the MFMA reads, and only the gathered
// activation rows use the LDS ring:
//   * weights packed per 16-row tile and 128-K slice ([rows/16][K/128][64
//     lanes][16 B], xs_pack_weight_mxfp4_frag): lane 16 g + r holds row r's
//     K = [32 g, 32 g + 32), one coalesced 1 KB load per tile and slice; the
//     e8m0 scale of (row r, 32-block g) is the lane's byte of a 64-byte
//     array per tile and slice;
//   * BM-row tiles (64 or 128: the tile table's height), 8 waves, each owning
//     2 weight tiles (gate_up: 16 gate rows and the matching 16 up rows; down:
//     32 rows), PD slices of loads in flight;
//   * the activation ring is the FP8 kernel's: MXFP8 rows are 128 bytes per
//     slice and their e8m0 scales 4 bytes per row and slice, the strides of
//     the FP8 rows and their f32 scales.
#include "moe_gemm.hpp"

namespace xs {
namespace {

constexpr int kNW = 8, kNT = 64 * kNW;       // waves (two per SIMD), threads
constexpr int kWT = 2;                       // 16-row weight tiles per wave
constexpr int kPD = 4;                       // slices in flight (weights and activations)
constexpr int kNSA = 5;                      // activation ring stages (>= kPD + 1)

template <int BM>
struct W4 {
    static constexpr int MI = BM / 16;        // 16-row subtiles
    static constexpr int AB = BM * 128;       // activation rows of one slice
    static constexpr int SB = BM * 4;         // their scale words
    static constexpr int STAGE = AB + SB;
    static constexpr int NA = BM / 8 / kNW;   // 1 KB activation DMAs per wave and slice
    static constexpr int NSW = SB / 256;      // waves that load the scale words
    static_assert(kNSA * STAGE + 8 * 1024 <= 160 * 1024 && NA >= 1 && NSW >= 1 && NSW <= kNW, "ring");
};

__device__ __forceinline__ int swz8(int r, int c) { return c ^ ((r >> 1) & 7); }
__device__ __forceinline__ v8i cat(v4i a, v4i b) { return v8i{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]}; }
typedef const __attribute__((address_space(1))) v4i gv4i;
typedef const __attribute__((address_space(1))) uint8_t gu8;

__device__ __forceinline__ uint32_t lds_addr(const void *p)
{
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}
// Wave-wide LDS DMA: lane i's 16 (4) bytes from sbase + voff land at lds + 16 i
// (4 i).  Issued from asm, out of the compiler's sight (a compiler-visible DMA
// makes every later read of the ring wait for all of them); the wait states
// after the M0 write and the scalar base are in the asm, the counter waits
// are explicit.
__device__ __forceinline__ void dma16(const uint8_t *sbase, uint32_t voff, uint32_t lds)
{
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 4\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(lds) : "memory");
}
__device__ __forceinline__ void dma4(const uint8_t *sbase, uint32_t voff, uint32_t lds)
{
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 4\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(sbase), "s"(lds) : "memory");
}
__device__ __forceinline__ const uint8_t *uniform(const uint8_t *p)
{
    const uint64_t u = (uint64_t)(uintptr_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)u), hi = __builtin_amdgcn_readfirstlane((uint32_t)(u >> 32));
    return reinterpret_cast<const uint8_t *>((uintptr_t)(((uint64_t)hi << 32) | lo));
}
template <int N>
__device__ __forceinline__ void wait_vm()
{
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ __forceinline__ void barrier_lds()
{
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// KBT > 0: K / 128 at compile time (the slice loop unrolled in full); 0: any K.
// Every tile runs all MI subtiles (rows past the tile repeat its last row and
// are not stored).
template <bool GATEUP, int KBT, int BM>
__device__ __forceinline__ void run_tile_wd4(const GemmArgs &a, int e, int pos0, int rows, int slab, uint8_t *smem)
{
    using C = W4<BM>;
    constexpr int MI = C::MI;
    const int KB = KBT ? KBT : a.K / 128;   // slices; a multiple of kPD (checked at launch)
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r16 = lane & 15, g = lane >> 4;
    const int n0 = slab * (GATEUP ? 128 : 256);
    const int Nrows = GATEUP ? 2 * a.N : a.N;
    constexpr int RW = 16 * kWT;                 // weight rows per wave
    auto wrow = [&](int j) -> int {
        return GATEUP ? (j == 0 ? n0 + 16 * wave : a.N + n0 + 16 * wave) : n0 + RW * wave + 16 * j;
    };
    // packed weights: [E][Nrows/16][KB][64][16 B]; packed scales [E][Nrows/16][KB][64]
    const uint8_t *Wexp = a.Bp + (size_t)e * Nrows * (a.K / 2);
    const uint8_t *Sexp = a.Bsp + (size_t)e * Nrows * (a.K / 32);

    float *red = reinterpret_cast<float *>(smem + kNSA * C::STAGE);     // [kNW][BM] epilogue amax
    uint8_t *trash = reinterpret_cast<uint8_t *>(red + kNW * BM);       // [256] scale DMAs of the other waves

    auto token_of = [&](int row) -> int {
        const int p = pos0 + min(row, rows - 1);
        return a.row_token ? a.row_token[p] : p;
    };
    uint32_t oA[C::NA];
#pragma unroll
    for (int u = 0; u < C::NA; ++u) {
        const int row = 8 * (wave + kNW * u) + (lane >> 3);
        oA[u] = (uint32_t)token_of(row) * (uint32_t)a.K + (uint32_t)(swz8(row, lane & 7) * 16);
    }
    const bool sw = wave < C::NSW;
    const uint32_t oS = (uint32_t)token_of(sw ? 64 * wave + lane : 0) * (uint32_t)(KB * 4);
    const bool stream_w = a.offsets[e + 1] - a.offsets[e] <= BM;

    const uint8_t *Wb0 = Wexp + (size_t)(wrow(0) / 16) * KB * 1024;
    const uint8_t *Wb1 = Wexp + (size_t)(wrow(1) / 16) * KB * 1024;
    const uint8_t *Sb0 = Sexp + (size_t)(wrow(0) / 16) * KB * 64;
    const uint8_t *Sb1 = Sexp + (size_t)(wrow(1) / 16) * KB * 64;
    const uint8_t *As = reinterpret_cast<const uint8_t *>(a.As);
    const uint32_t ring = lds_addr(smem), trash_lds = lds_addr(trash);
    auto adma = [&](int k2) __attribute__((always_inline)) {
        const int kk = min(k2, KB - 1);
        const uint32_t sl = ring + (uint32_t)((k2 % kNSA) * C::STAGE);
#pragma unroll
        for (int u = 0; u < C::NA; ++u) dma16(uniform(a.A + (size_t)kk * 128), oA[u], sl + 1024 * (wave + kNW * u));
        // every wave issues the scale DMA (the waves past the scales into the
        // trash line), so every wave's counter sees the same loads
        dma4(uniform(As + (size_t)kk * 4), oS, sw ? sl + C::AB + 256 * wave : trash_lds);
    };
    // the fragment's 16 bytes into the low half of the MFMA operand, the
    // scale byte zero-extended into a register
    auto wload = [&](int k2, v4i (&w)[2], uint32_t (&s)[2]) __attribute__((always_inline)) {
        const int kk = min(k2, KB - 1);
        const uint8_t *p0 = uniform(Wb0 + (size_t)kk * 1024), *p1 = uniform(Wb1 + (size_t)kk * 1024);
        const uint8_t *q0 = uniform(Sb0 + (size_t)kk * 64), *q1 = uniform(Sb1 + (size_t)kk * 64);
        if (stream_w) {
            w[0] = __builtin_nontemporal_load((gv4i *)(p0 + 16 * lane));
            w[1] = __builtin_nontemporal_load((gv4i *)(p1 + 16 * lane));
        } else {
            w[0] = *(gv4i *)(p0 + 16 * lane);
            w[1] = *(gv4i *)(p1 + 16 * lane);
        }
        s[0] = *(gu8 *)(q0 + lane);
        s[1] = *(gu8 *)(q1 + lane);
    };
    // loads per wave per slice, in issue order: activation DMAs and the scale
    // DMA after the slice's barrier, then 2 weight and 2 scale loads after its
    // last MFMA
    constexpr int P = C::NA + 1 + 4;

    v4f acc[MI][2];
#pragma unroll
    for (int i = 0; i < MI; ++i) acc[i][0] = acc[i][1] = v4f{0.f, 0.f, 0.f, 0.f};
    v4i wr[kPD][2];
    uint32_t ws[kPD][2];
    __syncthreads();   // the ring is free
#pragma unroll
    for (int k = 0; k < kPD; ++k) {
        adma(k);
        wload(k, wr[k], ws[k]);
    }
#pragma unroll
    for (int k0 = 0; k0 < KB; k0 += kPD) {
#pragma unroll
        for (int p = 0; p < kPD; ++p) {
            const int k = k0 + p;
            if (k >= KB) break;
            wait_vm<(kPD - 1) * P>();   // slice k (activations and weights) has landed
            barrier_lds();              // ... in every wave; slot (k-1) % kNSA is free
            adma(k + kPD);
            const uint8_t *sA = smem + (k % kNSA) * C::STAGE;
            const uint32_t *sS = reinterpret_cast<const uint32_t *>(sA + C::AB);
            const v8i w0 = v8i{wr[p][0][0], wr[p][0][1], wr[p][0][2], wr[p][0][3], 0, 0, 0, 0};
            const v8i w1 = v8i{wr[p][1][0], wr[p][1][1], wr[p][1][2], wr[p][1][3], 0, 0, 0, 0};
            const int s0 = (int)ws[p][0], s1 = (int)ws[p][1];
#pragma unroll
            for (int i = 0; i < MI; ++i) {
                const int row = 16 * i + r16;
                const uint8_t *rp = sA + row * 128;
                const v8i bx = cat(*reinterpret_cast<const v4i *>(rp + swz8(row, g) * 16),
                                   *reinterpret_cast<const v4i *>(rp + swz8(row, g + 4) * 16));
                const int sx = (int)((sS[row] >> (8 * g)) & 0xffu);
                acc[i][0] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(w0, bx, acc[i][0], 4, 0, 0, s0, 0, sx);
                acc[i][1] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(w1, bx, acc[i][1], 4, 0, 0, s1, 0, sx);
            }
            wload(k + kPD, wr[p], ws[p]);
        }
    }
    wait_vm<0>();   // the clamped loads past the last slice land before the ring is reused
    __syncthreads();

    // ------------------------------------------------------------ epilogue
    // acc[i][j][v]: token row 16 i + r16; gate_up: j = 0 gate, 1 up, act column
    // (of the block's 128) 16 wave + 4 g + v; down: output column n0 + RW wave +
    // 16 j + 4 g + v.
    if (GATEUP) {
        float act[MI][4];
#pragma unroll
        for (int i = 0; i < MI; ++i) {
            float m = 0.f;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const float gt = acc[i][0][v], up = acc[i][1][v];
                act[i][v] = gt * fast_sigmoid(gt) * up;
                m = fmaxf(m, __builtin_fabsf(act[i][v]));
            }
            m = fmaxf(m, __shfl_xor(m, 16, WAVE));
            m = fmaxf(m, __shfl_xor(m, 32, WAVE));
            if (g == 0) red[wave * BM + 16 * i + r16] = m;
        }
        __syncthreads();
        // MXFP8 1x32: a 32-column block is the 16 columns of waves 2q and 2q + 1;
        // the tile is staged in the ring (rows padded to 144 B) and stored as
        // whole 128-byte rows
        constexpr int QS = 144;
        uint8_t *qs = smem;
        uint8_t *Cs8 = reinterpret_cast<uint8_t *>(a.Cs);
        const int nsc = a.N / 32;
        const int w2 = wave & ~1;
#pragma unroll
        for (int i = 0; i < MI; ++i) {
            const int row = 16 * i + r16;
            const float amax = fmaxf(red[w2 * BM + row], red[(w2 + 1) * BM + row]);
            const int se = mx_exponent(amax, 8);
            float x[4];
#pragma unroll
            for (int v = 0; v < 4; ++v) x[v] = fminf(fmaxf(__builtin_ldexpf(act[i][v], -se), -448.f), 448.f);
            *reinterpret_cast<uint32_t *>(qs + row * QS + 16 * wave + 4 * g) =
                e4m3_pack2_hw(x[0], x[1]) | (e4m3_pack2_hw(x[2], x[3]) << 16);
            if ((wave & 1) == 0 && g == 0 && row < rows)
                Cs8[(size_t)(pos0 + row) * nsc + (n0 + 16 * wave) / 32] = (uint8_t)(se + 127);
        }
        __syncthreads();
#pragma unroll
        for (int pass = 0; pass < BM / (kNT / 8); ++pass) {
            const int row = (kNT / 8) * pass + (tid >> 3), c = tid & 7;
            if (row < rows)
                *reinterpret_cast<v4i *>(a.Cq + (size_t)(pos0 + row) * a.N + n0 + 16 * c) =
                    *reinterpret_cast<const v4i *>(qs + row * QS + 16 * c);
        }
    } else {
        // f32 rows, staged in two halves (padded to 1040 B) and stored as whole
        // 1 KB rows
        constexpr int HR = BM / 2, FS = 260;
        static_assert(HR * FS * 4 <= kNSA * C::STAGE, "staging tile");
        float *fs = reinterpret_cast<float *>(smem);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int i = h * (MI / 2); i < (h + 1) * (MI / 2); ++i) {
                const int rl = 16 * i + r16 - h * HR;
#pragma unroll
                for (int j = 0; j < kWT; ++j) *reinterpret_cast<v4f *>(fs + rl * FS + RW * wave + 16 * j + 4 * g) = acc[i][j];
            }
            __syncthreads();
#pragma unroll 4
            for (int pass = 0; pass < HR / (kNT / 64); ++pass) {
                const int rl = (kNT / 64) * pass + (tid >> 6), c = 4 * (tid & 63), row = h * HR + rl;
                if (row < rows)
                    *reinterpret_cast<v4f *>(a.Cf + (size_t)(pos0 + row) * a.ldc + n0 + c) =
                        *reinterpret_cast<const v4f *>(fs + rl * FS + c);
            }
            __syncthreads();
        }
    }
}

template <bool GATEUP, int KBT, int BM>
__global__ __launch_bounds__(kNT) void moe_gemm_wd4_kernel(GemmArgs a)
{
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int4 *tab = reinterpret_cast<const int4 *>(a.tile_tab);
    // routed tiles only (the shared expert is FP8): entries after the shared ones
    const int h0 = tab[0].y, tiles = tab[0].x - h0;
    // 1-D grid, work grouped per XCD as in the tall-tile kernels: groups of 8
    // tiles x 4 slabs, XCD x (linear id L, L % 8 == x) takes groups x, x + 8, ...
    const int gx = GATEUP ? a.N / 128 : a.N / 256, nq = gx / 4;
    const int L = (int)blockIdx.x, j = L >> 3;
    const int sg = (L & 7) + 8 * (j >> 5), i = j & 31;
    const int g = sg / nq, qq = sg - g * nq;
    const int tile = 8 * g + (i >> 2);
    const int slab = 4 * qq + (i & 3);
    if (tile >= tiles) return;
    const int4 d = tab[1 + h0 + tile];   // {expert, first position, rows}
    if (d.z <= 0) return;
    run_tile_wd4<GATEUP, KBT, BM>(a, d.x, d.y, min(d.z, BM), slab, smem);
}

template <bool GATEUP, int BM>
int launch_wd4(const GemmArgs &a, int grid_y, hipStream_t st)
{
    using C = W4<BM>;
    const int gx = GATEUP ? a.N / 128 : a.N / 256;
    const size_t smem = (size_t)kNSA * C::STAGE + 4 * (size_t)kNW * BM + 256;
    // 64-row tiles: the slice loop unrolled for 16 and 32 slices; 128-row
    // tiles keep the loop (unrolled, their 16 accumulator tiles spill)
    const int KB = a.K / 128;
    const int ki = BM == 128 ? 0 : KB == 16 ? 1 : KB == 32 ? 2 : 0;
    void (*const fns[3])(GemmArgs) = {moe_gemm_wd4_kernel<GATEUP, 0, BM>,
                                      moe_gemm_wd4_kernel<GATEUP, BM == 128 ? 0 : 16, BM>,
                                      moe_gemm_wd4_kernel<GATEUP, BM == 128 ? 0 : 32, BM>};
    auto fn = fns[ki];
    static bool attr_set[3] = {};
    if (!attr_set[ki]) {
        XS_HIP(hipFuncSetAttribute((const void *)fn, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
        attr_set[ki] = true;
    }
    const int64_t groups = (grid_y + 7) / 8 * (gx / 4);   // 8-tile x 4-slab groups
    fn<<<dim3((unsigned)((groups + 7) / 8 * 256)), dim3(kNT), smem, st>>>(a);
    XS_LAUNCH_CHECK();
    return XS_OK;
}

}  // namespace

bool wd4_supported(int64_t H, int64_t I)
{
    return H % (128 * kPD) == 0 && I % (128 * kPD) == 0 && (I / 128) % 4 == 0 && (H / 256) % 4 == 0;
}

int launch_gemm_wd4(const GemmArgs &a, bool gateup, int grid_y, hipStream_t st)
{
    if (grid_y <= 0) return XS_OK;
    const int gx = gateup ? a.N / 128 : a.N / 256;
    if ((a.bm != 64 && a.bm != 128) || a.K % (128 * kPD) || gx % 4 || !a.tile_tab || !a.Bp || !a.Bsp ||
        (!gateup && !a.Cf))
        return set_error(XS_ERR_UNSUPPORTED, "weight-direct MXFP4 GEMM shape K=%d N=%d bm=%d", a.K, a.N, a.bm);
    if (a.bm == 64) return gateup ? launch_wd4<true, 64>(a, grid_y, st) : launch_wd4<false, 64>(a, grid_y, st);
    return gateup ? launch_wd4<true, 128>(a, grid_y, st) : launch_wd4<false, 128>(a, grid_y, st);
}

// ------------------------------------------------- fragment packing of MXFP4 weights
// w [batch, n, k/2] (e2m1 pairs) -> [batch][n/16][k/128][64][16 B]: chunk
// (b, t, ks, l) is w[b][16 t + l % 16][64 ks + 16 (l / 16) ...]; s [batch, n,
// k/32] (e8m0) -> [batch][n/16][k/128][64]: byte (b, t, ks, l) is
// s[b][16 t + l % 16][4 ks + l / 16].
__global__ __launch_bounds__(256) void pack_frag4_kernel(const uint8_t *__restrict__ w, const uint8_t *__restrict__ s,
                                                         uint8_t *__restrict__ ow, uint8_t *__restrict__ os,
                                                         int64_t chunks, int n, int k)
{
    const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (c >= chunks) return;
    const int KS = k / 128;
    const int l = (int)(c & 63);
    const int64_t blk = c >> 6;                // (b, t, ks)
    const int ks = (int)(blk % KS);
    const int64_t bt = blk / KS;               // b * n/16 + t
    const int64_t b = bt / (n / 16), t = bt % (n / 16);
    const int64_t row = b * n + 16 * t + (l & 15);
    *reinterpret_cast<v4i *>(ow + c * 16) =
        *reinterpret_cast<const v4i *>(w + row * (int64_t)(k / 2) + 64 * ks + 16 * (l >> 4));
    os[c] = s[row * (int64_t)(k / 32) + 4 * ks + (l >> 4)];
}

}  // namespace xs

extern "C" int xs_pack_weight_mxfp4_frag(const uint8_t *w, const uint8_t *s, int64_t batch, int64_t n, int64_t k,
                                         uint8_t *out_w, uint8_t *out_s, void *stream)
{
    using namespace xs;
    XS_REQUIRE(w && s && out_w && out_s, "null pointer");
    XS_REQUIRE(batch >= 1 && n > 0 && k > 0 && n % 16 == 0 && k % 128 == 0,
               "shape mismatch: n must be a multiple of 16 and k of 128");
    XS_REQUIRE(((uintptr_t)w & 15) == 0 && ((uintptr_t)out_w & 15) == 0,
               "misaligned operand: w and out_w need 16-byte alignment");
    const int64_t wb = batch * n * k / 2, sb = batch * n * k / 32;
    XS_REQUIRE(w + wb <= out_w || out_w + wb <= w, "out_w must not overlap w");
    XS_REQUIRE(s + sb <= out_s || out_s + sb <= s, "out_s must not overlap s");
    const int64_t chunks = batch * (n / 16) * (k / 128) * 64;   // one per (b, 16-row tile, 128-K slice, lane)
    pack_frag4_kernel<<<dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, (hipStream_t)stream>>>(
        w, s, out_w, out_s, chunks, (int)n, (int)k);
    XS_LAUNCH_CHECK();
    return XS_OK;
}
