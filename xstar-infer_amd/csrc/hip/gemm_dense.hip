// gemm_dense.hip -- dense FP8 block-scaled GEMM C = A . B^T (gfx950), the
// kernel behind xs_gemm_fp8_blockscale.
//
// Nearest reference code: gemm_launch / gemm_kernel (xstar_cpp/include/ops/gemm.h:165-176,
// xstar_cpp/src/ops/gemm.cu:41-210).  Numerics as the expert GEMMs: each 128-wide
// K block is accumulated exactly by the MFMA from the e4m3 operands, then added
// to the f32 accumulator times (row scale of A) x (128x128 block scale of B).
//
// Structure, sized by a CU's budgets (vector memory path ~64 B/clk, one
// 16x16x128 FP8 MFMA per 32 clk per SIMD, LDS reads ~256 B/clk):
//   * a block owns a 128 x 128 output tile (128 rows of A, 128 rows of B: one
//     B scale block), so a K step loads 32 KB for 4.2 MFLOP and the loads and
//     the MFMAs ask for about the same 512 clk;
//   * when the tiles do not fill the chip the K range is split over S blocks;
//     each writes its f32 partial tile, and the last to arrive (per-tile
//     counter) sums all S partials in split order, so the result does not
//     depend on which block finishes last;
//   * operands move global -> LDS by DMA (global_load_lds_dwordx4, 8 lanes per
//     128-byte row, XOR-swizzled chunks) into a 4-stage ring;
//   * 8 waves, 2 per SIMD, as 2 (64 B rows each) x 4 (32 A rows each): a wave
//     runs 8 MFMAs per step with B as operand A and A as operand B, so a lane's
//     4 results share one A row (one row scale) and are 4 consecutive columns;
//   * the loop is software-pipelined: a step's MFMAs use fragments read from
//     LDS during the previous step, its products are folded one subtile
//     later, and its DMAs go out one at a time between MFMAs (a DMA
//     instruction holds its wave until the memory path takes it);
//   * blocks are dealt to the 8 XCDs in contiguous ranges of (tile group,
//     split) order, so the blocks running on one XCD share A and B tiles in
//     its L2 (measured 87% L2 hits at 4096^3).
#include "moe_internal.hpp"
#include "xs_device.hpp"

#include <algorithm>

namespace xs {
namespace {

constexpr int kNS = 4;                           // ring stages
constexpr int kA = 128 * 128;                    // A rows of one K step
constexpr int kS = 128 * 4;                      // their row scales
constexpr int kB = 128 * 128;                    // B rows of one K step
constexpr int kStage = kA + kS + kB;
constexpr int kLds = 159 * 1024;                // dynamic LDS cap (the rest: static)
constexpr int kDenseWaves = 8;                 // waves per block (4 or 8)

struct DenseArgs {
    const uint8_t *A;   // [M, K] e4m3
    const float *As;    // [M, K/128]
    const uint8_t *B;   // [N, K] e4m3
    const float *Bs;    // [N/128, K/128]
    uint16_t *C;        // [M, N] bf16
    float *part;        // [tiles][S][128 x 128] f32 partial tiles (S > 1)
    int32_t *cnt;       // [tiles] arrival counters, zero on entry (S > 1)
    int M, N, K;
    int TM, TN;         // tiles along M and N
    int S, KBs;         // K splits, K steps per split
    int total;          // TM * TN * S
};

__device__ __forceinline__ int swz8(int r, int c) { return c ^ ((r >> 1) & 7); }

__device__ __forceinline__ uint32_t lds_addr(const void *p)
{
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

__device__ __forceinline__ v8i cat(v4i a, v4i b) { return v8i{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]}; }

// Wave-wide DMA global -> LDS: lane i's 16 (4) bytes, read from sbase + voff,
// land at lds + 16 i (4 i).  M0 carries the LDS base; the s_nop 4 covers the
// wait states the asm hides from the compiler (SALU M0 write -> LDS DMA, and
// a VALU-written SGPR base -> VMEM).
__device__ __forceinline__ void dma16(const uint8_t *sbase, uint32_t voff, uint32_t lds)
{
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 4\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(lds) : "memory");
}
__device__ __forceinline__ void dma4(const uint8_t *sbase, uint32_t voff, uint32_t lds)
{
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 4\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(sbase), "s"(lds) : "memory");
}
// a wave-uniform pointer in SGPRs (the DMA's scalar base operand)
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

// 16-byte store and load with the sc1 cache policy, the one agent-scope
// atomics carry: the store writes through this XCD's L2 and the load misses
// in the reader's, so partial tiles pass between XCDs without a cache-wide
// write-back or invalidation.  The load is the compiler's own buffer load
// (cache-policy operand 16 = sc1), so the compiler tracks its destination
// registers and places the vmcnt wait before their first use.  The resource
// is raw (stride 0): num_records bounds the byte offset; word 3 is gfx9's
// 32-bit data format, which untyped buffer loads need.
__device__ __forceinline__ void store16_coh(float *p, v4f v)
{
    asm volatile("global_store_dwordx4 %0, %1, off sc1" ::"v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ v4f load16_coh(const float *base, uint32_t byte_off)
{
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(base), (short)0, 0x7fffffff, 0x00020000);
    return __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 16));
}

// NW waves: NW/2 along the A rows (MI 16-row subtiles each) x 2 along the
// B rows (64 each).  8 waves: 32 x 64 per wave, 2 per SIMD; 4 waves: 64 x 64
// per wave (a third fewer LDS bytes per MFMA), 1 per SIMD.
template <int NW>
__global__ __launch_bounds__(64 * NW) void gemm_dense_fp8_kernel(DenseArgs a)
{
    constexpr int NT = 64 * NW;
    constexpr int MI = 16 / NW;                 // A subtiles per wave
    constexpr int NU = 16 / NW;                 // 1 KB DMAs per wave per step and operand
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    __shared__ int last_flag;
    // XCD x (linear block id L, L % 8 == x) runs the contiguous range
    // [x per, (x + 1) per) of the (tile group, split) order.
    const int per = (a.total + 7) / 8;
    const int L = (int)blockIdx.x;
    const int v = (L & 7) * per + (L >> 3);
    if (v >= a.total) return;
    // tiles in groups of up to 8 A tiles x all B tiles, A tile fastest: the 32
    // blocks an XCD runs at once cover 8 A tiles x 4 B tiles
    const int s = v % a.S, t = v / a.S;
    const int gm0 = t / (8 * a.TN) * 8, gm = min(a.TM - gm0, 8);
    const int tm = gm0 + t % gm, tn = t % (8 * a.TN) / gm;
    const int KB = a.K / 128;
    const int kb0 = s * a.KBs;
    const int nk = min(a.KBs, KB - kb0);   // >= 1 (the host picks S so)
    const int m0 = 128 * tm, n0 = 128 * tn;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wn = wave & 1, wt = wave >> 1;
    const int r16 = lane & 15, g = lane >> 4;

    float *sB = reinterpret_cast<float *>(smem + kNS * kStage);   // [nk] B block scales
    for (int q = tid; q < nk; q += NT) sB[q] = a.Bs[(size_t)tn * KB + kb0 + q];

    // DMA sources: rows past M repeat row M-1 (loaded, never stored)
    const uint8_t *Ab = a.A + (size_t)m0 * a.K;
    const uint8_t *Bb = a.B + (size_t)n0 * a.K;
    const uint8_t *Sb = reinterpret_cast<const uint8_t *>(a.As + (size_t)m0 * KB);
    uint32_t oA[NU], oB[NU];
#pragma unroll
    for (int u = 0; u < NU; ++u) {
        const int row = 8 * (wave + NW * u) + (lane >> 3);
        const int ar = min(m0 + row, a.M - 1) - m0;
        oA[u] = (uint32_t)ar * (uint32_t)a.K + (uint32_t)(swz8(row, lane & 7) * 16);
        oB[u] = (uint32_t)row * (uint32_t)a.K + (uint32_t)(swz8(row, lane & 7) * 16);
    }
    const bool sw = wave < 2;   // waves 0, 1 load the 128 row scales
    const uint32_t oS = (uint32_t)(min(m0 + 64 * wave + lane, a.M - 1) - m0) * (uint32_t)(KB * 4);
    const uint32_t ring = lds_addr(smem);
    // the loads of local step k2 into slot k2 % kNS; steps past the split
    // reload its last step (into a slot nothing reads again), so every
    // iteration issues the same number of loads
    auto issue = [&](int k2) __attribute__((always_inline)) {
        const int kk = kb0 + min(k2, nk - 1);
        const uint32_t sl = ring + (uint32_t)((k2 % kNS) * kStage);
#pragma unroll
        for (int u = 0; u < NU; ++u) dma16(Ab + (size_t)kk * 128, oA[u], sl + 1024 * (wave + NW * u));
#pragma unroll
        for (int u = 0; u < NU; ++u) dma16(Bb + (size_t)kk * 128, oB[u], sl + kA + kS + 1024 * (wave + NW * u));
        if (sw) dma4(uniform(Sb + (size_t)kk * 4), oS, sl + kA + 256 * wave);
    };
    constexpr int P = 2 * NU;   // loads per wave per step (+1 on the scale waves)
    // load d of local step k2 (A rows, then B rows, then the row scales)
    auto issue_one = [&](int k2, int d) __attribute__((always_inline)) {
        const int kk = kb0 + min(k2, nk - 1);
        const uint32_t sl = ring + (uint32_t)((k2 % kNS) * kStage);
        if (d < NU) dma16(Ab + (size_t)kk * 128, oA[d], sl + 1024 * (wave + NW * d));
        else if (d < 2 * NU) dma16(Bb + (size_t)kk * 128, oB[d - NU], sl + kA + kS + 1024 * (wave + NW * (d - NU)));
        else if (sw) dma4(uniform(Sb + (size_t)kk * 4), oS, sl + kA + 256 * wave);
    };

    v4f acc[MI][4];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

    // Fragments of one step: B rows (operand A) and A rows (operand B) with the
    // step's fold factors (row scale x block scale).
    struct Frag {
        v8i wf[4], bx[MI];
        float c[MI];
    };
    // operand layout of v_mfma_f32_16x16x128_f8f6f4: lane 16g + r holds row r,
    // K bytes [16g, 16g+16) and [64+16g, 64+16g+16): LDS chunks g and g+4
    auto read_frag = [&](int k, Frag &f) __attribute__((always_inline)) {
        const uint8_t *sA = smem + (k % kNS) * kStage;
        const float *sS = reinterpret_cast<const float *>(sA + kA);
        const uint8_t *sW = sA + kA + kS;
        const float sb = sB[min(k, nk - 1)];
#pragma unroll
        for (int i = 0; i < MI; ++i) f.c[i] = sS[16 * (MI * wt + i) + r16] * sb;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int row = 64 * wn + 16 * j + r16;
            const uint8_t *rp = sW + row * 128;
            f.wf[j] = cat(*reinterpret_cast<const v4i *>(rp + swz8(row, g) * 16),
                          *reinterpret_cast<const v4i *>(rp + swz8(row, g + 4) * 16));
        }
#pragma unroll
        for (int i = 0; i < MI; ++i) {
            const int row = 16 * (MI * wt + i) + r16;
            const uint8_t *rp = sA + row * 128;
            f.bx[i] = cat(*reinterpret_cast<const v4i *>(rp + swz8(row, g) * 16),
                          *reinterpret_cast<const v4i *>(rp + swz8(row, g + 4) * 16));
        }
    };
    // One step, software-pipelined: the MFMAs of step k (fragments fc, read
    // during step k-1) run while the fragments of step k+1 come in from LDS
    // (fn).  Products fold one A subtile later (the last subtile of step k-1,
    // factor cl, during subtile 0 of step k).
    v4f q[2][4];
    auto fold = [&](int i, int b, float c) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[i][j][e] = __builtin_fmaf(q[b][j][e], c, acc[i][j][e]);
    };
    auto step = [&](int k, const Frag &fc, Frag &fn, float &cl) __attribute__((always_inline)) {
        // Each MFMA slot m of the step, in this order (a scheduling barrier
        // closes each): the MFMA, a quarter of the fold of the previous
        // subtile, and from the second subtile on, which follows the wait and
        // the block barrier, the fragments (and fold factors) of step k+1 and
        // a share of the P + 1 loads of step k+kNS: slot s after the barrier
        // issues loads [ceil(s (P+1) / NS_), ceil((s+1) (P+1) / NS_)), so
        // every load of the step goes out (the row-scale load, the last, on
        // the scale waves), as the waits count them.  Subtile 0 needs only
        // registers, so the matrix core has work queued across the barrier; a
        // DMA instruction holds its wave until the CU's ~64 B/clk memory path
        // takes it, so the DMAs go out a few at a time between MFMAs.
        constexpr int M0 = 4;                         // slots before the barrier
        constexpr int NR = 4 + 2 * MI;                // fragment and factor reads
        constexpr int NS_ = 4 * MI - M0;              // slots after the barrier
        constexpr int RG = (NR + NS_ - 1) / NS_;      // reads per slot
        const uint8_t *nA = smem + ((k + 1) % kNS) * kStage;
        const float *nS = reinterpret_cast<const float *>(nA + kA);
        const uint8_t *nW = nA + kA + kS;
        const float nsb = sB[min(k + 1, nk - 1)];
        auto read_item = [&](int r) __attribute__((always_inline)) {
            if (r < 4) {
                const int row = 64 * wn + 16 * r + r16;
                const uint8_t *rp = nW + row * 128;
                fn.wf[r] = cat(*reinterpret_cast<const v4i *>(rp + swz8(row, g) * 16),
                               *reinterpret_cast<const v4i *>(rp + swz8(row, g + 4) * 16));
            } else if (r < 4 + MI) {
                const int row = 16 * (MI * wt + r - 4) + r16;
                const uint8_t *rp = nA + row * 128;
                fn.bx[r - 4] = cat(*reinterpret_cast<const v4i *>(rp + swz8(row, g) * 16),
                                   *reinterpret_cast<const v4i *>(rp + swz8(row, g + 4) * 16));
            } else if (r < NR) {
                fn.c[r - 4 - MI] = nS[16 * (MI * wt + r - 4 - MI) + r16] * nsb;
            }
        };
#pragma unroll
        for (int i = 0; i < MI; ++i) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int m = 4 * i + j;
                if (m == M0) {
                    // loads retire in order: step k+1 has landed when at most the
                    // loads of steps k+2 .. k+kNS-1 are outstanding
                    if (sw) wait_vm<(kNS - 2) * (P + 1)>();
                    else wait_vm<(kNS - 2) * P>();
                    __syncthreads();   // step k+1 landed everywhere; slot k % kNS is free
                }
                if (m >= M0) {
                    const int d0 = ((m - M0) * (P + 1) + NS_ - 1) / NS_, d1 = ((m - M0 + 1) * (P + 1) + NS_ - 1) / NS_;
#pragma unroll
                    for (int d = d0; d < d1; ++d) issue_one(k + kNS, d);
                }
                q[i & 1][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(fc.wf[j], fc.bx[i], v4f{0.f, 0.f, 0.f, 0.f},
                                                                               0, 0, 0, 0, 0, 0);
                if (m >= M0)
#pragma unroll
                    for (int r = 0; r < RG; ++r) read_item((m - M0) * RG + r);
                // fold of the previous subtile, tile j
                const int fi = i == 0 ? MI - 1 : i - 1;
                const float c = i == 0 ? cl : fc.c[i - 1];
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[fi][j][e] = __builtin_fmaf(q[fi & 1][j][e], c, acc[fi][j][e]);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        cl = fc.c[MI - 1];
    };

    __syncthreads();   // sB visible
#pragma unroll
    for (int k = 0; k < kNS; ++k) issue(k);
    if (sw) wait_vm<(kNS - 1) * (P + 1)>();
    else wait_vm<(kNS - 1) * P>();
    __syncthreads();   // step 0 landed everywhere
    Frag f0, f1;
    read_frag(0, f0);
    float cl = 0.f;    // the first fold is of zero products
#pragma unroll
    for (int j = 0; j < 4; ++j) q[(MI - 1) & 1][j] = v4f{0.f, 0.f, 0.f, 0.f};
    for (int k = 0; k < nk; k += 2) {
        step(k, f0, f1, cl);
        if (k + 1 < nk) step(k + 1, f1, f0, cl);
    }
    fold(MI - 1, (MI - 1) & 1, cl);
    wait_vm<0>();   // the reloads past the split land before the block ends

    if (a.S > 1) {
        // Partial tiles go out and come back with the sc1 policy (coherent
        // across the XCDs' L2s); the stores have completed (s_waitcnt) before
        // the counter's atomic.
        float *mine = a.part + ((size_t)t * a.S + s) * (128 * 128);
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) store16_coh(mine + ((i * 4 + j) * NT + tid) * 4, acc[i][j]);
        wait_vm<0>();
        __syncthreads();
        if (tid == 0) {
            const int old = __hip_atomic_fetch_add(a.cnt + t, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            last_flag = old == a.S - 1;
        }
        __syncthreads();
        if (!last_flag) return;
        v4f tot[MI][4];
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) tot[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
        for (int ss = 0; ss < a.S; ++ss) {
            const float *pp = a.part + ((size_t)t * a.S + ss) * (128 * 128);
            if (ss == s) {
#pragma unroll
                for (int i = 0; i < MI; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j) tot[i][j] += acc[i][j];
            } else {
                v4f o[MI][4];
#pragma unroll
                for (int i = 0; i < MI; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j) o[i][j] = load16_coh(pp, (uint32_t)(((i * 4 + j) * NT + tid) * 16));
#pragma unroll
                for (int i = 0; i < MI; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j) tot[i][j] += o[i][j];
            }
        }
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = tot[i][j];
    }

    // acc[i][j][e]: row m0 + 16 (MI wt + i) + r16, column n0 + 64 wn + 16 j + 4 g + e
#pragma unroll
    for (int i = 0; i < MI; ++i) {
        const int row = m0 + 16 * (MI * wt + i) + r16;
        if (row >= a.M) continue;
        uint16_t *cr = a.C + (size_t)row * a.N + n0 + 64 * wn + 4 * g;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t lo = bf16_from_f32(acc[i][j][0]) | ((uint32_t)bf16_from_f32(acc[i][j][1]) << 16);
            const uint32_t hi = bf16_from_f32(acc[i][j][2]) | ((uint32_t)bf16_from_f32(acc[i][j][3]) << 16);
            *reinterpret_cast<v2i *>(cr + 16 * j) = v2i{(int)lo, (int)hi};
        }
    }
}

}  // namespace

// Split count: the tiles alone when they fill the 256 CUs, else up to
// 256 / tiles splits of at least 4 K steps each.
static void dense_plan(int64_t M, int64_t N, int64_t K, int *S, int *KBs)
{
    const int64_t tiles = ((M + 127) / 128) * (N / 128);
    const int KB = (int)(K / 128);
    int s = tiles >= 256 ? 1 : (int)(256 / tiles);
    s = std::max(1, std::min(s, KB / 4));
    const int kbs = (KB + s - 1) / s;
    *KBs = kbs;
    *S = (KB + kbs - 1) / kbs;   // every split gets at least one step
}

size_t dense_part_bytes(int64_t M)
{
    // split only when the tiles are fewer than 256, so tiles x S <= 256
    return (M + 127) / 128 >= 256 ? 0 : (size_t)256 * 128 * 128 * 4 + 1024;
}

int launch_gemm_dense(const uint8_t *A, const float *As, const uint8_t *B, const float *Bs, uint16_t *C,
                      int64_t M, int64_t N, int64_t K, float *part, int32_t *cnt, hipStream_t st)
{
    if (M == 0) return XS_OK;
    DenseArgs a = {};
    a.A = A;
    a.As = As;
    a.B = B;
    a.Bs = Bs;
    a.C = C;
    a.part = part;
    a.cnt = cnt;
    a.M = (int)M;
    a.N = (int)N;
    a.K = (int)K;
    a.TM = (int)((M + 127) / 128);
    a.TN = (int)(N / 128);
    dense_plan(M, N, K, &a.S, &a.KBs);
    if (a.S > 1 && (!part || !cnt || (int64_t)a.TM * a.TN * a.S > 256))
        return set_error(XS_ERR_WORKSPACE, "dense GEMM split without its partial buffer");
    if ((int64_t)a.TM * a.TN * a.S >= (1ll << 31)) return set_error(XS_ERR_UNSUPPORTED, "dense GEMM too large");
    if ((uint64_t)128 * (uint64_t)K > 0xffffffffull) return set_error(XS_ERR_UNSUPPORTED, "K too large");
    a.total = a.TM * a.TN * a.S;
    const size_t smem = (size_t)kNS * kStage + 4 * (size_t)a.KBs;
    if (smem > (size_t)kLds) return set_error(XS_ERR_UNSUPPORTED, "K=%lld needs %zu bytes of LDS", (long long)K, smem);
    static bool attr_set = false;
    if (!attr_set) {
        XS_HIP(hipFuncSetAttribute((const void *)gemm_dense_fp8_kernel<kDenseWaves>,
                                   hipFuncAttributeMaxDynamicSharedMemorySize, kLds));
        attr_set = true;
    }
    const int per = (a.total + 7) / 8;
    gemm_dense_fp8_kernel<kDenseWaves><<<dim3((unsigned)(8 * per)), dim3(64 * kDenseWaves), smem, st>>>(a);
    XS_LAUNCH_CHECK();
    return XS_OK;
}

int dense_counters(int64_t M, int64_t N)
{
    const int64_t tiles = ((M + 127) / 128) * (N / 128);
    return tiles >= 256 ? 0 : (int)tiles;
}

}  // namespace xs
