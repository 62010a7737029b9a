// moe_gemm_wd.hip -- grouped FP8 block-scaled expert GEMMs with the weights
// loaded straight into VGPRs (gfx950): the prefill tall-tile path when the
// layer holds a fragment-packed copy of its FP8 weights.  The same tile
// routine, at 64-row tiles with a bf16 output, is the single FP8 GEMM from a
// packed B (gemm_wd_dense_kernel, xs_gemm_fp8_blockscale_packed).
//
// Nearest reference code: gemm_silu_and_mul_kernel (xstar_cpp/src/ops/mlp.cu:52-200)
// and gemm_kernel (xstar_cpp/src/ops/gemm.cu:41-210).  Numerics are those of the
// tall-tile kernels in moe_gemm_wide.hip, step for step (each 128-K block
// accumulated by the MFMA, folded into f32 with row scale x block scale in K
// order; the same SwiGLU and 1x128 requantization), so the two give the same
// bits.
//
// Why a second form: in the tall-tile kernels both operands stream through the
// LDS ring, which caps the bytes a CU keeps in flight (about two steps), and
// every weight fragment is read from LDS by two waves.  Here:
//   * weights are packed once in MFMA fragment order ([rows/16][K/128][2][64
//     lanes][16 B], xs_pack_weight_fp8_frag): a wave's load of one fragment
//     half is one coalesced 1 KB instruction, and no LDS is involved;
//   * 128-row tiles; each of the 8 waves (two per SIMD) owns two 16-row weight
//     tiles (gate_up: 16 gate rows and the matching 16 up rows; down: 32 rows)
//     over all of the tile's tokens, so every weight byte is loaded once per
//     block, 4 steps ahead into registers (the loop keeps the products of one
//     subtile at a time, folded while the next subtile's MFMAs run; 183-190
//     VGPRs with the K loop unrolled for 4-32 steps, 205-209 for other K);
//   * activations (gathered token rows) alone use the LDS ring;
//   * the weight loads are plain loads, so the compiler tracks their registers
//     and waits itself; the activation DMAs (which write no register) are
//     issued from asm and waited for explicitly, and the block barrier
//     carries no memory fence.
#include "moe_gemm.hpp"

namespace xs {
namespace {

constexpr int kBM = 128;                     // token rows per tile
constexpr int kMI = kBM / 16;                // 16-row subtiles
constexpr int kNW = 8, kNT = 64 * kNW;       // waves (two per SIMD), threads
constexpr int kWT = 256 / 16 / kNW;          // 16-row weight tiles per wave
constexpr int kPD = 4;                       // steps in flight (weights and activations)
constexpr int kNSA = 5;                      // activation ring stages (>= kPD + 1)
constexpr int kAB = kBM * 128;               // activation rows of one step
constexpr int kSB = kBM * 4;                 // their row scales
constexpr int kStage = kAB + kSB;
constexpr int kNSW = kSB / 256;              // waves that load the row scales
static_assert(kNSA >= kPD + 1 && kNSA * kStage + 8 * 1024 <= 160 * 1024 && kNSW <= kNW && kWT == 2 && kMI % 2 == 0,
              "ring");

__device__ __forceinline__ int swz8(int r, int c) { return c ^ ((r >> 1) & 7); }
__device__ __forceinline__ v8i cat(v4i a, v4i b) { return v8i{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]}; }
typedef const __attribute__((address_space(1))) v4i gv4i;

__device__ __forceinline__ uint32_t lds_addr(const void *p)
{
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}
// Wave-wide LDS DMA: lane i's 16 (4) bytes from sbase + voff land at lds + 16 i
// (4 i).  Issued from asm, out of the compiler's sight: it writes no register,
// and a compiler-visible DMA makes every later LDS read of the ring wait for
// all of them (the ring's slots are one LDS object to its alias analysis), the
// prefetch just issued included.  The wait states after the M0 write and the
// scalar base are in the asm (s_nop 4); the counter waits are explicit.
__device__ __forceinline__ void dma16(const uint8_t *sbase, uint32_t voff, uint32_t lds)
{
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 4\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(lds) : "memory");
}
__device__ __forceinline__ void dma4(const uint8_t *sbase, uint32_t voff, uint32_t lds)
{
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 4\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(sbase), "s"(lds) : "memory");
}
// a wave-uniform pointer, made visibly uniform (SGPRs): the DMA then takes the
// scalar-base form with a 32-bit lane offset instead of a 64-bit lane address
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
// block barrier without a memory-model fence (the compiler adds no counter
// waits for it); this wave's LDS reads have completed before it
__device__ __forceinline__ void barrier_lds()
{
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Every tile runs all kMI subtiles: rows past the tile repeat its last row
// (loaded and multiplied, never stored).  A tile short enough for that to
// matter streams its expert's weights from HBM, which bounds it anyway, and a
// single path keeps the register budget of one loop.
// KBT > 0: K / 128, known at compile time (the K loop is unrolled in full, so the
// compiler's waits for the weight registers are exact at every step); 0: any K.
template <bool GATEUP, int KBT, int BM = kBM, bool DENSE = false>
__device__ __forceinline__ void run_tile_wd(const GemmArgs &a, int e, int pos0, int rows, int slab, uint8_t *smem)
{
    // sizes that follow the tile height (BM = kBM for the expert GEMMs)
    constexpr int MI = BM / 16, AB = BM * 128, SB = BM * 4, STG = AB + SB;
    constexpr int NA = BM / 8 / kNW, NSW = SB / 256;
    static_assert(NA >= 1 && NSW >= 1 && NSW <= kNW && MI % 2 == 0 && kNSA * STG + 8 * 1024 <= 160 * 1024, "tile");
    const int KB = KBT ? KBT : a.K / 128;   // a multiple of kPD (checked at launch)
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r16 = lane & 15, g = lane >> 4;
    const int n0 = slab * (GATEUP ? 128 : 256);
    const bool shared = e == a.E;
    const int Nrows = GATEUP ? 2 * a.N : a.N;
    // The wave's two 16-row weight tiles: gate_up, tile 0 the gate rows
    // n0 + 16 wave and tile 1 the matching up rows; down, rows n0 + 32 wave + 16 j.
    constexpr int RW = 16 * kWT;                 // weight rows per wave
    auto wrow = [&](int j) -> int {
        return GATEUP ? (j < kWT / 2 ? n0 + (RW / 2) * wave + 16 * j : a.N + n0 + (RW / 2) * wave + 16 * (j - kWT / 2))
                      : n0 + RW * wave + 16 * j;
    };
    const uint8_t *Wexp = shared ? a.Bshp : a.Bp + (size_t)e * Nrows * a.K;

    float *sB = reinterpret_cast<float *>(smem + kNSA * STG);          // [2][KB] block scales
    float *red = sB + 2 * KB;                                            // [kNW][BM] epilogue amax
    uint8_t *trash = reinterpret_cast<uint8_t *>(red + kNW * BM);       // [256] scale DMAs of the other waves
    {
        const float *Bsf = shared ? a.Bssh : reinterpret_cast<const float *>(a.Bs) + (size_t)e * (Nrows / 128) * KB;
        for (int q = tid; q < 2 * KB; q += kNT) {
            const int b = q / KB, kb = q % KB;
            const int nb = GATEUP ? (b ? a.N + n0 : n0) / 128 : n0 / 128 + b;
            sB[q] = Bsf[(size_t)nb * KB + kb];
        }
    }
    // fold factor block of tile j: gate_up gate 0 / up 1; down (RW wave) / 128
    auto sbl = [&](int j) -> int { return GATEUP ? (j < kWT / 2 ? 0 : 1) : (RW * wave) / 128; };

    auto token_of = [&](int row) -> int {
        const int p = pos0 + min(row, rows - 1);
        return a.row_token ? a.row_token[p] : p;
    };
    uint32_t oA[NA];
#pragma unroll
    for (int u = 0; u < NA; ++u) {
        const int row = 8 * (wave + kNW * u) + (lane >> 3);
        oA[u] = (uint32_t)token_of(row) * (uint32_t)a.K + (uint32_t)(swz8(row, lane & 7) * 16);
    }
    const bool sw = wave < NSW;
    const uint32_t oS = (uint32_t)token_of(sw ? 64 * wave + lane : 0) * (uint32_t)(KB * 4);
    // an expert whose rows fit one tile reads its weights once: stream them
    const bool stream_w = !DENSE && a.offsets[e + 1] - a.offsets[e] <= BM;

    // loads of step k2 (clamped to the last step: every iteration issues the
    // same loads): activations into ring slot k2 % kNSA, the wave's two weight
    // fragments into w (a wave-uniform tile base in SGPRs + the lane's 16 bytes)
    const uint8_t *Wb0 = Wexp + (size_t)(wrow(0) / 16) * KB * 2048;
    const uint8_t *Wb1 = Wexp + (size_t)(wrow(1) / 16) * KB * 2048;
    const uint8_t *Sb = reinterpret_cast<const uint8_t *>(a.As);
    const uint32_t ring = lds_addr(smem), trash_lds = lds_addr(trash);
    auto adma = [&](int k2) __attribute__((always_inline)) {
        const int kk = min(k2, KB - 1);
        const uint32_t sl = ring + (uint32_t)((k2 % kNSA) * STG);
#pragma unroll
        for (int u = 0; u < NA; ++u) dma16(uniform(a.A + (size_t)kk * 128), oA[u], sl + 1024 * (wave + kNW * u));
        // every wave issues the scale DMA (the waves past the scales into the
        // trash line), so every wave's counter sees the same loads
        dma4(uniform(Sb + (size_t)kk * 4), oS, sw ? sl + AB + 256 * wave : trash_lds);
    };
    // each fragment is loaded straight into the 8 registers its MFMA reads
    auto wload = [&](int k2, v8i (&w)[2]) __attribute__((always_inline)) {
        const int kk = min(k2, KB - 1);
        const uint8_t *p0 = uniform(Wb0 + (size_t)kk * 2048), *p1 = uniform(Wb1 + (size_t)kk * 2048);
        if (stream_w) {
            w[0] = cat(__builtin_nontemporal_load((gv4i *)(p0 + 16 * lane)),
                       __builtin_nontemporal_load((gv4i *)(p0 + 16 * lane + 1024)));
            w[1] = cat(__builtin_nontemporal_load((gv4i *)(p1 + 16 * lane)),
                       __builtin_nontemporal_load((gv4i *)(p1 + 16 * lane + 1024)));
        } else {
            w[0] = cat(*(gv4i *)(p0 + 16 * lane), *(gv4i *)(p0 + 16 * lane + 1024));
            w[1] = cat(*(gv4i *)(p1 + 16 * lane), *(gv4i *)(p1 + 16 * lane + 1024));
        }
    };
    // loads per wave per step, in issue order: activation DMAs and the scale
    // DMA after the step's barrier, then the 4 weight loads after its last
    // MFMA (into the registers that MFMA has just read)
    constexpr int P = NA + 1 + 4;

    v4f acc[MI][2];
#pragma unroll
    for (int i = 0; i < MI; ++i) acc[i][0] = acc[i][1] = v4f{0.f, 0.f, 0.f, 0.f};
    v8i wr[kPD][2];
    __syncthreads();   // sB visible; the ring is free
#pragma unroll
    for (int k = 0; k < kPD; ++k) {
        adma(k);
        wload(k, wr[k]);
    }
    const int fb0 = sbl(0), fb1 = sbl(1);   // fold factor blocks of the two tiles
    v4f q[2][2];
    float cl = 0.f, cl1 = 0.f;   // fold factors of the previous subtile (first fold: zeros)
    q[(MI - 1) & 1][0] = q[(MI - 1) & 1][1] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k0 = 0; k0 < KB; k0 += kPD) {
#pragma unroll
        for (int p = 0; p < kPD; ++p) {
            const int k = k0 + p;
            if (k >= KB) break;
            // loads retire in order: step k (activations and weights) has landed
            // when only the later kPD-1 steps' loads are outstanding
            wait_vm<(kPD - 1) * P>();
            barrier_lds();   // step k's activations landed everywhere; slot (k-1) % kNSA is free
            adma(k + kPD);
            const uint8_t *sA = smem + (k % kNSA) * STG;
            const float *sS = reinterpret_cast<const float *>(sA + AB);
            const float sb = sB[fb0 * KB + k], sb1 = sB[fb1 * KB + k];
            v8i bx[2];
            auto rb = [&](int i) __attribute__((always_inline)) {
                const int row = 16 * i + r16;
                const uint8_t *rp = sA + row * 128;
                return cat(*reinterpret_cast<const v4i *>(rp + swz8(row, g) * 16),
                           *reinterpret_cast<const v4i *>(rp + swz8(row, g + 4) * 16));
            };
            // subtile i: read B(i+1), 2 MFMAs on B(i), fold the products of i-1
            // (i = 0: the last subtile of step k-1) while they run
            bx[0] = rb(0);
#pragma unroll
            for (int i = 0; i < MI; ++i) {
                if (i + 1 < MI) bx[(i + 1) & 1] = rb(i + 1);
                const float sa = sS[16 * i + r16];
                const float ci = sa * sb, ci1 = sa * sb1;
                q[i & 1][0] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(wr[p][0], bx[i & 1], v4f{0.f, 0.f, 0.f, 0.f},
                                                                               0, 0, 0, 0, 0, 0);
                q[i & 1][1] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(wr[p][1], bx[i & 1], v4f{0.f, 0.f, 0.f, 0.f},
                                                                               0, 0, 0, 0, 0, 0);
                const int fi = i == 0 ? MI - 1 : i - 1;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    acc[fi][0][e] = __builtin_fmaf(q[fi & 1][0][e], cl, acc[fi][0][e]);
                    acc[fi][1][e] = __builtin_fmaf(q[fi & 1][1][e], cl1, acc[fi][1][e]);
                }
                // fold here: left to itself the compiler sinks the folds of the
                // unrolled steps towards the epilogue and keeps their products live
                asm volatile("" : "+v"(acc[fi][0]), "+v"(acc[fi][1]));
                cl = ci;
                cl1 = ci1;
            }
            wload(k + kPD, wr[p]);
        }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        acc[MI - 1][0][e] = __builtin_fmaf(q[(MI - 1) & 1][0][e], cl, acc[MI - 1][0][e]);
        acc[MI - 1][1][e] = __builtin_fmaf(q[(MI - 1) & 1][1][e], cl1, acc[MI - 1][1][e]);
    }
    wait_vm<0>();   // the clamped loads past the last step land before the ring is reused
    __syncthreads();

    // ------------------------------------------------------------ epilogue
    // acc[i][j][v]: token row 16 i + r16; gate_up: tile j < kWT/2 gate, j +
    // kWT/2 its up, act column (of the block's 128) (RW/2) wave + 16 j + 4 g + v;
    // down: output column n0 + RW wave + 16 j + 4 g + v.
    if (GATEUP) {
        constexpr int JH = kWT / 2;
        float act[MI][JH][4];
#pragma unroll
        for (int i = 0; i < MI; ++i) {
            float m = 0.f;
#pragma unroll
            for (int jj = 0; jj < JH; ++jj)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const float gt = acc[i][jj][v], up = acc[i][jj + JH][v];
                    act[i][jj][v] = gt * fast_sigmoid(gt) * up;
                    m = fmaxf(m, __builtin_fabsf(act[i][jj][v]));
                }
            m = fmaxf(m, __shfl_xor(m, 16, WAVE));
            m = fmaxf(m, __shfl_xor(m, 32, WAVE));
            if (g == 0) red[wave * BM + 16 * i + r16] = m;
        }
        __syncthreads();
        // the FP8 tile is staged in the ring (rows padded to 144 B) and stored
        // as whole 128-byte rows
        constexpr int QS = 144;
        uint8_t *qs = smem;
        float *Cs = reinterpret_cast<float *>(a.Cs);
        const int nsc = a.N / 128;
#pragma unroll
        for (int i = 0; i < MI; ++i) {
            const int row = 16 * i + r16;
            float amax = 0.f;
#pragma unroll
            for (int w = 0; w < kNW; ++w) amax = fmaxf(amax, red[w * BM + row]);
            const float inv = amax == 0.f ? 0.f : __fdiv_rn(448.0f, amax);
#pragma unroll
            for (int jj = 0; jj < JH; ++jj) {
                float x[4];
#pragma unroll
                for (int v = 0; v < 4; ++v) x[v] = fminf(fmaxf(act[i][jj][v] * inv, -448.f), 448.f);
                *reinterpret_cast<uint32_t *>(qs + row * QS + (RW / 2) * wave + 16 * jj + 4 * g) =
                    e4m3_pack2_hw(x[0], x[1]) | (e4m3_pack2_hw(x[2], x[3]) << 16);
            }
            if (wave == 0 && g == 0 && row < rows)
                Cs[(size_t)(pos0 + row) * nsc + n0 / 128] = amax == 0.f ? 1.0f : __fdiv_rn(amax, 448.0f);
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
        static_assert(HR * FS * 4 <= kNSA * STG, "staging tile");
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
                if (row < rows) {
                    const v4f v = *reinterpret_cast<const v4f *>(fs + rl * FS + c);
                    if (DENSE) {   // the single GEMM: bf16 output, one rounding
                        const uint32_t lo = bf16_from_f32(v[0]) | ((uint32_t)bf16_from_f32(v[1]) << 16);
                        const uint32_t hi = bf16_from_f32(v[2]) | ((uint32_t)bf16_from_f32(v[3]) << 16);
                        *reinterpret_cast<v2i *>(a.Cy + (size_t)(pos0 + row) * a.ldc + n0 + c) = v2i{(int)lo, (int)hi};
                    } else {
                        *reinterpret_cast<v4f *>(a.Cf + (size_t)(pos0 + row) * a.ldc + n0 + c) = v;
                    }
                }
            }
            __syncthreads();
        }
    }
}

template <bool GATEUP, int KBT>
__global__ __launch_bounds__(kNT) void moe_gemm_wd_kernel(GemmArgs a)
{
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int4 *tab = reinterpret_cast<const int4 *>(a.tile_tab);   // shared + routed tiles
    const int tiles = a.sh_rows > 0 ? (int)((a.sh_rows + kBM - 1) / kBM) : tab[0].x;
    // 1-D grid, work grouped per XCD as in the tall-tile kernels: groups of 8
    // tiles x 4 slabs, XCD x (linear id L, L % 8 == x) takes groups x, x + 8, ...
    const int gx = GATEUP ? a.N / 128 : a.N / 256, nq = gx / 4;
    const int L = (int)blockIdx.x, j = L >> 3;
    const int sg = (L & 7) + 8 * (j >> 5), i = j & 31;
    const int g = sg / nq, qq = sg - g * nq;
    const int tile = 8 * g + (i >> 2);
    const int slab = 4 * qq + (i & 3);
    if (tile >= tiles) return;
    // {expert, first position, rows}: the table's, or the shared segment's own tiles
    const int4 d = a.sh_rows > 0 ? int4{a.E, (int)(a.shared_base + (int64_t)kBM * tile),
                                        (int)min((int64_t)kBM, a.sh_rows - (int64_t)kBM * tile), 0}
                                 : tab[1 + tile];
    run_tile_wd<GATEUP, KBT>(a, d.x, d.y, min(d.z, kBM), slab, smem);
}

// The single FP8 block-scaled GEMM C = A . B^T (bf16 C) from fragment-packed
// B: 64-row tiles of A x 256-column slabs of B, no K split (at 512 x 4096 x
// 4096 that is 128 blocks of 32 K steps, each at its CU's full MFMA rate,
// with no partial tiles to exchange).  B is the "shared expert" of the tile
// routine (e == a.E): a.Bshp packed weights, a.Bssh their block scales.
// Blocks go to the XCDs in contiguous ranges of (slab, tile) order, tiles
// fastest, so one XCD runs a few B slabs against every A tile and reads each
// slab once.
constexpr int kDenseBM = 64;

template <int KBT>
__global__ __launch_bounds__(kNT) void gemm_wd_dense_kernel(GemmArgs a)
{
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int TM = (int)((a.sh_rows + kDenseBM - 1) / kDenseBM), gx = a.N / 256;
    const int total = TM * gx, per = (total + 7) / 8;
    const int L = (int)blockIdx.x;
    const int v = (L & 7) * per + (L >> 3);
    if (v >= total) return;
    const int slab = v / TM, tile = v - slab * TM;
    const int rows = (int)min((int64_t)kDenseBM, a.sh_rows - (int64_t)kDenseBM * tile);
    run_tile_wd<false, KBT, kDenseBM, true>(a, a.E, kDenseBM * tile, rows, slab, smem);
}

}  // namespace

int wd_tile_rows() { return kBM; }

// gate_up: K = H in whole groups of kPD steps, slabs of 128 act columns in
// groups of 4; down: K = I likewise, slabs of 256 columns in groups of 4
bool wd_supported(int64_t H, int64_t I)
{
    return H % (128 * kPD) == 0 && I % (128 * kPD) == 0 && (I / 128) % 4 == 0 && (H / 256) % 4 == 0;
}

int launch_gemm_wd(const GemmArgs &a, bool gateup, int grid_y, hipStream_t st)
{
    if (grid_y <= 0) return XS_OK;
    const bool sh_only = a.sh_rows > 0;   // the shared segment alone, in tiles of its own
    if (!sh_only && a.bm != kBM) return set_error(XS_ERR_INVALID, "weight-direct GEMM needs %d-row tiles", kBM);
    const int gx = gateup ? a.N / 128 : a.N / 256;
    if (a.K % (128 * kPD) || gx % 4 || (!sh_only && (!a.tile_tab || !a.Bp)) || ((sh_only || a.e_hi > a.E) && !a.Bshp) ||
        (!gateup && !a.Cf))
        return set_error(XS_ERR_UNSUPPORTED, "weight-direct GEMM shape K=%d N=%d", a.K, a.N);
    if (sh_only && grid_y != (int)((a.sh_rows + kBM - 1) / kBM))
        return set_error(XS_ERR_INVALID, "weight-direct GEMM: %d tiles for %lld shared rows", grid_y, (long long)a.sh_rows);
    const size_t smem = (size_t)kNSA * kStage + 8 * (size_t)(a.K / 128) + 4 * kNW * kBM + 256;
    if (smem > 160 * 1024) return set_error(XS_ERR_UNSUPPORTED, "K=%d needs %zu bytes of LDS", a.K, smem);
    // unrolled kernels for 4, 8, 16 and 32 K steps, the loop for other K
    const int KB = a.K / 128;
    const int ki = KB == 4 ? 1 : KB == 8 ? 2 : KB == 16 ? 3 : KB == 32 ? 4 : 0;
    void (*const fns[2][5])(GemmArgs) = {
        {moe_gemm_wd_kernel<false, 0>, moe_gemm_wd_kernel<false, 4>, moe_gemm_wd_kernel<false, 8>,
         moe_gemm_wd_kernel<false, 16>, moe_gemm_wd_kernel<false, 32>},
        {moe_gemm_wd_kernel<true, 0>, moe_gemm_wd_kernel<true, 4>, moe_gemm_wd_kernel<true, 8>,
         moe_gemm_wd_kernel<true, 16>, moe_gemm_wd_kernel<true, 32>}};
    auto fn = fns[gateup][ki];
    static bool attr_set[2][5] = {};
    if (!attr_set[gateup][ki]) {
        XS_HIP(hipFuncSetAttribute((const void *)fn, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
        attr_set[gateup][ki] = true;
    }
    const int64_t groups = (grid_y + 7) / 8 * (gx / 4);   // 8-tile x 4-slab groups
    fn<<<dim3((unsigned)((groups + 7) / 8 * 256)), dim3(kNT), smem, st>>>(a);
    XS_LAUNCH_CHECK();
    return XS_OK;
}

// C [M, N] bf16 = A . B^T: A [M, K] e4m3 with row scales [M, K/128], B packed
// in fragment order ([N/16][K/128][2][64][16 B]) with block scales
// [N/128][K/128].  N a multiple of 256, K of 512.
int launch_gemm_wd_dense(const uint8_t *A, const float *As, const uint8_t *Bp, const float *Bs, uint16_t *C,
                         int64_t M, int64_t N, int64_t K, hipStream_t st)
{
    if (M == 0) return XS_OK;
    if (N % 256 || K % (128 * kPD) || N <= 0 || K <= 0)
        return set_error(XS_ERR_UNSUPPORTED, "packed FP8 GEMM shape N=%lld K=%lld (N a multiple of 256, K of %d)",
                         (long long)N, (long long)K, 128 * kPD);
    const int64_t total = (M + kDenseBM - 1) / kDenseBM * (N / 256);
    if (total >= (1ll << 28)) return set_error(XS_ERR_UNSUPPORTED, "packed FP8 GEMM too large");
    GemmArgs a = {};
    a.A = A;
    a.As = As;
    a.Bshp = Bp;
    a.Bssh = Bs;
    a.E = 0;
    a.K = (int)K;
    a.N = (int)N;
    a.bm = kDenseBM;
    a.Cy = C;
    a.ldc = N;
    a.sh_rows = M;
    constexpr size_t stage = (size_t)kDenseBM * 128 + kDenseBM * 4;
    const size_t smem = (size_t)kNSA * stage + 8 * (size_t)(K / 128) + 4 * kNW * kDenseBM + 256;
    if (smem > 160 * 1024) return set_error(XS_ERR_UNSUPPORTED, "K=%lld needs %zu bytes of LDS", (long long)K, smem);
    const int KB = (int)(K / 128);
    const int ki = KB == 4 ? 1 : KB == 8 ? 2 : KB == 16 ? 3 : KB == 32 ? 4 : 0;
    void (*const fns[5])(GemmArgs) = {gemm_wd_dense_kernel<0>, gemm_wd_dense_kernel<4>, gemm_wd_dense_kernel<8>,
                                      gemm_wd_dense_kernel<16>, gemm_wd_dense_kernel<32>};
    static bool attr_set[5] = {};
    if (!attr_set[ki]) {
        XS_HIP(hipFuncSetAttribute((const void *)fns[ki], hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
        attr_set[ki] = true;
    }
    const int64_t per = (total + 7) / 8;
    fns[ki]<<<dim3((unsigned)(8 * per)), dim3(kNT), smem, st>>>(a);
    XS_LAUNCH_CHECK();
    return XS_OK;
}

// ------------------------------------------------- fragment packing of FP8 weights
// w [batch, n, k] e4m3 -> out [batch][n/16][k/128][2][64][16 B]: the 16-byte
// chunk (b, t, kb, h, l) is w[b][16 t + l % 16][128 kb + 64 h + 16 (l / 16) ...].
__global__ __launch_bounds__(256) void pack_frag_kernel(const uint8_t *__restrict__ w, uint8_t *__restrict__ out,
                                                        int64_t chunks, int n, int k)
{
    const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (c >= chunks) return;
    const int KB = k / 128;
    const int l = (int)(c & 63), h = (int)((c >> 6) & 1);
    const int64_t blk = c >> 7;                // (b, t, kb)
    const int kb = (int)(blk % KB);
    const int64_t bt = blk / KB;               // b * n/16 + t
    const int64_t b = bt / (n / 16), t = bt % (n / 16);
    const uint8_t *src = w + (b * n + 16 * t + (l & 15)) * (int64_t)k + 128 * kb + 64 * h + 16 * (l >> 4);
    *reinterpret_cast<v4i *>(out + c * 16) = *reinterpret_cast<const v4i *>(src);
}

}  // namespace xs

extern "C" int xs_pack_weight_fp8_frag(const uint8_t *w, int64_t batch, int64_t n, int64_t k, uint8_t *out,
                                       void *stream)
{
    using namespace xs;
    XS_REQUIRE(w && out, "null pointer");
    XS_REQUIRE(batch >= 1 && n > 0 && k > 0 && n % 16 == 0 && k % 128 == 0,
               "shape mismatch: n must be a multiple of 16 and k of 128");
    XS_REQUIRE(((uintptr_t)w & 15) == 0 && ((uintptr_t)out & 15) == 0,
               "misaligned operand: w and out need 16-byte alignment");
    XS_REQUIRE(w + batch * n * k <= out || out + batch * n * k <= w, "out must not overlap w");
    const int64_t chunks = batch * n * k / 16;
    pack_frag_kernel<<<dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, (hipStream_t)stream>>>(
        w, out, chunks, (int)n, (int)k);
    XS_LAUNCH_CHECK();
    return XS_OK;
}
