// moe_gemm_wide.hip -- grouped FP8 block-scaled expert GEMMs on tall tiles (gfx950),
// the prefill path of the MoE layer.
//
// Nearest reference code: gemm_silu_and_mul_kernel (xstar_cpp/src/ops/mlp.cu:52-200)
// and gemm_kernel (xstar_cpp/src/ops/gemm.cu:41-210); numerics as the FP8 tiles of
// moe_gemm.hip (f32 accumulation of each 128-K block, scaled by the activation row
// scale times the weight block scale; SwiGLU in f32; 1x128 FP8 requantization).
//
// Structure, chosen from measurements of CDNA4's per-CU budgets (a CU's vector
// memory path moves ~16 clk per fully coalesced KB but ~4x that when one
// instruction touches 16+ rows; LDS reads ~256 B/clk; 16x16x128 FP8 MFMA 32
// clk per SIMD):
//   * a block owns BM (128 or 192) rows of one expert and a 256-column weight
//     slab (gate_up: 128 gate + the matching 128 up rows; down: 256 rows of W2);
//   * both operand tiles move global -> LDS by DMA (global_load_lds_dwordx4,
//     8 lanes per 128-byte row, so every load instruction is fully coalesced)
//     into two rings: tiles of up to 128 rows keep activations 2 deep and
//     weights 3 deep (their weights stream from HBM, the longer latency),
//     taller tiles 3 and 2 (their weights are shared with the expert's other
//     tiles through L2, and the gathered activation rows wait longest);
//     16-byte chunks are XOR-swizzled per row so the MFMA fragment reads are
//     bank-conflict free;
//   * 8 waves as 2 (tokens) x 4 (weight columns): a wave owns 64 weight rows
//     (gate_up: 32 gate + the matching 32 up) and the 16-token subtiles of its
//     parity, so a partially filled tile still splits evenly over both halves;
//   * v_mfma_f32_16x16x128_f8f6f4 with weights as operand A and tokens as
//     operand B: a lane's 4 results belong to one token (one activation scale)
//     and a lane holds gate and matching up values, so SwiGLU and the
//     requantization are register epilogues;
//   * per K step each subtile's 4 products are folded into the f32
//     accumulators with (row scale x block scale) one subtile later, while the
//     next subtile's MFMAs run; subtiles past the tile's rows are skipped;
//   * tile descriptors (expert, first row, rows) come from the table the
//     permute builds, so a block starts with one load instead of a search.
#include "moe_gemm.hpp"

#include <cstdlib>

namespace xs {
namespace {

constexpr int kRing = 148 * 1024;    // LDS bytes of the operand ring
constexpr int kTrash = 1024;         // LDS target of padding DMAs

// Ring modes: 0 = 2 activation + 3 weight stages, 1 = 3 + 2, 2 = 2 + 4, 3 = 3 + 3.
// NW waves per block: 4 along the weight rows times NW / 4 along the tokens.
template <int BM, int MODE, int NW, int DMAW = NW>
struct WCfg {
    static constexpr int WM = NW / 4;                      // waves along the tokens
    static constexpr int NS16 = BM / 16;                   // 16-token subtiles per tile
    static constexpr int MI = NS16 / WM;                   // subtiles per wave: s16 = wm + WM i
    static constexpr int A_BYTES = BM * 128;               // activation rows of one K step
    static constexpr int W_BYTES = 256 * 128;              // weight rows of one K step
    static constexpr int S_BYTES = BM * 4;                 // activation row scales
    static constexpr int AS_BYTES = A_BYTES + S_BYTES;     // activation ring stage
    // Two rings: activations (+ row scales) NAR deep, weights NWR deep (prefetch
    // distances NAR-1 and NWR-1 steps).  Tiles of more than 128 rows (experts
    // with several tiles, whose weight slabs the tiles share through L2) wait on
    // their activation rows: 3 + 2 stages.  Shorter tiles stream their weights
    // from HBM: 2 + 3 stages.
    static constexpr int NAR = (MODE == 1 || MODE == 3) ? 3 : 2;
    static constexpr int NWR = MODE == 1 ? 2 : (MODE == 2 ? 4 : 3);
    static constexpr int DA = NAR - 1, DW = NWR - 1;
    // the first DMAW waves issue the loads (DMAW < NW: the other waves only compute)
    static constexpr int NA = BM / 8 / DMAW;               // 1 KB activation DMAs per loading wave and step
    static constexpr int NB = 256 / 8 / DMAW;              // 1 KB weight DMAs per loading wave and step
    static constexpr int NSA = S_BYTES / 256;              // scale DMAs (waves 0 .. NSA-1)
    static constexpr int PER_STEP = NA + NB + 1;           // loads per wave per step
    // Each iteration issues the operand with the shorter prefetch distance first.
    // Loads retire in order: at the top of step kb at most X may be outstanding
    // for both W(kb) and A(kb) to have landed.
    static constexpr bool W_FIRST = DA >= DW;
    static constexpr int XW = W_FIRST ? (NA + 1) + (DW - 1) * PER_STEP : (DW - 1) * PER_STEP;
    static constexpr int XA = W_FIRST ? (DA - 1) * PER_STEP : NB + (DA - 1) * PER_STEP;
    static constexpr int X = XW < XA ? XW : XA;
    static constexpr int PRO = DA > DW ? DA : DW;          // prologue iterations
    static_assert(BM % 64 == 0 && DA >= 1 && DW >= 1 && NAR * AS_BYTES + NWR * W_BYTES <= kRing, "tile");
    static_assert(NA >= 1 && NSA <= DMAW && DMAW <= NW && MI % 2 == 0, "waves");
};

__device__ __forceinline__ int swz8(int r, int c) { return c ^ ((r >> 1) & 7); }

__device__ __forceinline__ uint32_t lds_addr(const void *p)
{
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

__device__ __forceinline__ v8i cat(v4i a, v4i b) { return v8i{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]}; }

// Wave-wide DMA global -> LDS: lane i's 16 (4) bytes, read from sbase + voff,
// land at lds + 16 i (4 i).  M0 carries the wave-uniform LDS base; it is
// written only here.
// Wait states inside the asm (the compiler's hazard checks do not look into
// an asm string): an LDS DMA that reads M0 needs one after the SALU write of
// M0, and a VMEM instruction reading an SGPR that a VALU instruction wrote
// (v_readfirstlane of the base) needs five, hence s_nop 4 where the base is a
// scalar operand and s_nop 0 where the address is a VGPR.
__device__ __forceinline__ void dma16(const uint8_t *sbase, uint32_t voff, uint32_t lds)
{
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 4\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(lds) : "memory");
}
// Non-temporal variant for weights read by a single tile (streamed once).
__device__ __forceinline__ void dma16_nt(const uint8_t *sbase, uint32_t voff, uint32_t lds)
{
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 4\n\tglobal_load_lds_dwordx4 %0, %1 nt" ::"v"(voff), "s"(sbase), "s"(lds) : "memory");
}
__device__ __forceinline__ void dma4(const uint8_t *sbase, uint32_t voff, uint32_t lds)
{
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 4\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(sbase), "s"(lds) : "memory");
}
template <int N>
__device__ __forceinline__ void wait_vm()
{
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// 4 consecutive f32 values, read around the L2 (system scope): rows another
// XCD stored with system-scope stores are seen without an L2 invalidation.
__device__ __forceinline__ v4f load4_sys(const float *p)
{
    uint64_t *q = reinterpret_cast<uint64_t *>(const_cast<float *>(p));
    const uint64_t a = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    const uint64_t b = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    return v4f{__uint_as_float((uint32_t)a), __uint_as_float((uint32_t)(a >> 32)), __uint_as_float((uint32_t)b),
               __uint_as_float((uint32_t)(b >> 32))};
}

// Down epilogue with f32 rows: acc[i][j][v] is token row 16 (wm + 2 i) + r16,
// column n0 + 64 wn + 16 j + 4 g + v.  The tile is staged through the ring in
// two halves (BM/2 rows of 1 KB each, padded to 1040 B) and stored as whole
// rows.  With fuse_combine the rows are stored around the L2 (system scope),
// then every row bumps its (token, slab) counter; a row that completes its
// token (the counter reaches k + shared) puts the token on the block's list,
// and the block sums the listed tokens' rows in the combine's fixed order:
// shared row, then slots 0 .. k-1 as acc + w_j * y_j (each product and sum
// rounded, no FMA), then the residual, and writes the slab of out with the
// one cast.  The sum does not depend on which block finishes a token.
template <int BM, int NW>
__device__ __forceinline__ void store_f32_tile(const GemmArgs &a, const v4f (&acc)[BM / 16 / (NW / 4)][4], int pos0,
                                               int rows, int slab, int wm, int wn, uint8_t *smem, float *red)
{
#pragma clang fp contract(off)
    constexpr int WM = NW / 4, MI = BM / 16 / WM, HR = BM / 2, FS = 260, NT = 64 * NW;
    static_assert(HR * FS * 4 <= kRing, "staging tile");
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r16 = lane & 15, g = lane >> 4;
    const int n0 = slab * 256;
    const bool fuse = a.fuse_combine != 0;
    const bool shcomb = a.shared_combine != 0;
    float *fs = reinterpret_cast<float *>(smem);
    __syncthreads();   // every wave is past its loop: the ring is free for staging
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        // rows [h HR, h HR + HR) are the subtiles i in [h MI/2, h MI/2 + MI/2)
#pragma unroll
        for (int i = h * (MI / 2); i < (h + 1) * (MI / 2); ++i) {
            const int rl = 16 * (wm + WM * i) + r16 - h * HR;
#pragma unroll
            for (int j = 0; j < 4; ++j) *reinterpret_cast<v4f *>(fs + rl * FS + 64 * wn + 16 * j + 4 * g) = acc[i][j];
        }
        __syncthreads();
        if (shcomb) {
            // the combine of the tokens of these shared rows, slab columns
            // n0 .. n0 + 255: acc = the shared row (f32, as it would be
            // stored), then acc + w_j * y_j over the routed slots in order,
            // then the residual, one cast (combine_kernel's arithmetic)
#pragma unroll 2
            for (int pass = 0; pass < HR / (NT / 64); ++pass) {
                const int rl = (NT / 64) * pass + (tid >> 6), c = 4 * (tid & 63), row = h * HR + rl;
                if (row >= rows) continue;
                const int t = (int)(pos0 + row - a.shared_base);
                v4f s = *reinterpret_cast<const v4f *>(fs + rl * FS + c);
                v4f yv[16];
#pragma unroll
                for (int j = 0; j < 16; ++j)
                    if (j < a.topk)
                        yv[j] = *reinterpret_cast<const v4f *>(a.Cf + (size_t)a.inv[(size_t)t * a.topk + j] * a.ldc +
                                                               n0 + c);
#pragma unroll
                for (int j = 0; j < 16; ++j)
                    if (j < a.topk) {
                        const float wt = a.cw[(size_t)t * a.topk + j];
#pragma unroll
                        for (int v = 0; v < 4; ++v) s[v] = s[v] + wt * yv[j][v];   // no contraction (pragma above)
                    }
                const size_t o = (size_t)t * a.N + n0 + c;
                if (a.out_dtype == XS_BF16) {
                    if (a.residual) {
                        const v2i r = *reinterpret_cast<const v2i *>(reinterpret_cast<const uint16_t *>(a.residual) + o);
                        s[0] = __uint_as_float((uint32_t)r[0] << 16) + s[0];
                        s[1] = __uint_as_float((uint32_t)r[0] & 0xFFFF0000u) + s[1];
                        s[2] = __uint_as_float((uint32_t)r[1] << 16) + s[2];
                        s[3] = __uint_as_float((uint32_t)r[1] & 0xFFFF0000u) + s[3];
                    }
                    v2i pk;
                    pk[0] = (int)((uint32_t)bf16_from_f32(s[0]) | ((uint32_t)bf16_from_f32(s[1]) << 16));
                    pk[1] = (int)((uint32_t)bf16_from_f32(s[2]) | ((uint32_t)bf16_from_f32(s[3]) << 16));
                    *reinterpret_cast<v2i *>(reinterpret_cast<uint16_t *>(a.out) + o) = pk;
                } else {
                    if (a.residual) {
                        const v4f r = *reinterpret_cast<const v4f *>(reinterpret_cast<const float *>(a.residual) + o);
#pragma unroll
                        for (int v = 0; v < 4; ++v) s[v] = r[v] + s[v];
                    }
                    *reinterpret_cast<v4f *>(reinterpret_cast<float *>(a.out) + o) = s;
                }
            }
        } else if (fuse) {
#pragma unroll 4
            for (int pass = 0; pass < HR / (NT / 128); ++pass) {
                const int rl = (NT / 128) * pass + (tid >> 7), c = 2 * (tid & 127), row = h * HR + rl;
                if (row < rows)
                    __hip_atomic_store(reinterpret_cast<uint64_t *>(a.Cf + (size_t)(pos0 + row) * a.ldc + n0 + c),
                                       *reinterpret_cast<const uint64_t *>(fs + rl * FS + c), __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_SYSTEM);
            }
        } else {
#pragma unroll 4
            for (int pass = 0; pass < HR / (NT / 64); ++pass) {
                const int rl = (NT / 64) * pass + (tid >> 6), c = 4 * (tid & 63), row = h * HR + rl;
                if (row < rows)
                    *reinterpret_cast<v4f *>(a.Cf + (size_t)(pos0 + row) * a.ldc + n0 + c) =
                        *reinterpret_cast<const v4f *>(fs + rl * FS + c);
            }
        }
        __syncthreads();   // the staging rows are free again
    }
    if (!fuse) return;

    wait_vm<0>();          // this thread's rows have reached memory
    int *lst = reinterpret_cast<int *>(red);   // [0]: count, [1 ..]: tokens this block completes
    if (tid == 0) lst[0] = 0;
    __syncthreads();       // ... every thread's, and the list is empty
    const int nslab = a.N / 256, need = a.topk + a.has_shared;
    if (tid < rows) {
        const int t = a.pos_token[pos0 + tid];
        const int old = __hip_atomic_fetch_add(a.ccnt + (size_t)t * nslab + slab, 1, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
        if (old == need - 1) lst[1 + atomicAdd(&lst[0], 1)] = t;
    }
    __syncthreads();
    const int nl = lst[0];
    const int c = n0 + 4 * lane;
    for (int q = wave; q < nl; q += NW) {
        const int t = lst[1 + q];
        v4f s = a.has_shared ? load4_sys(a.Cf + (size_t)(a.shared_base + t) * a.ldc + c) : v4f{0.f, 0.f, 0.f, 0.f};
        for (int j = 0; j < a.topk; ++j) {
            const int p = a.inv[(size_t)t * a.topk + j];
            const float wt = a.cw[(size_t)t * a.topk + j];
            const v4f y = load4_sys(a.Cf + (size_t)p * a.ldc + c);
#pragma unroll
            for (int v = 0; v < 4; ++v) s[v] = s[v] + wt * y[v];   // no contraction (pragma above)
        }
        const size_t o = (size_t)t * a.N + c;
        if (a.out_dtype == XS_BF16) {
            if (a.residual) {
                const v2i r = *reinterpret_cast<const v2i *>(reinterpret_cast<const uint16_t *>(a.residual) + o);
                s[0] = __uint_as_float((uint32_t)r[0] << 16) + s[0];
                s[1] = __uint_as_float((uint32_t)r[0] & 0xFFFF0000u) + s[1];
                s[2] = __uint_as_float((uint32_t)r[1] << 16) + s[2];
                s[3] = __uint_as_float((uint32_t)r[1] & 0xFFFF0000u) + s[3];
            }
            v2i pk;
            pk[0] = (int)((uint32_t)bf16_from_f32(s[0]) | ((uint32_t)bf16_from_f32(s[1]) << 16));
            pk[1] = (int)((uint32_t)bf16_from_f32(s[2]) | ((uint32_t)bf16_from_f32(s[3]) << 16));
            *reinterpret_cast<v2i *>(reinterpret_cast<uint16_t *>(a.out) + o) = pk;
        } else {
            if (a.residual) {
                const v4f r = *reinterpret_cast<const v4f *>(reinterpret_cast<const float *>(a.residual) + o);
#pragma unroll
                for (int v = 0; v < 4; ++v) s[v] = r[v] + s[v];
            }
            *reinterpret_cast<v4f *>(reinterpret_cast<float *>(a.out) + o) = s;
        }
    }
}

#ifdef XS_WIDE_TRACE
// Development builds only: per-block phase timestamps (100 MHz wall clock).
__device__ uint64_t g_wide_trace[2][16384][6];
#define XS_WTRACE(ev) \
    if (threadIdx.x == 0 && blockIdx.x + gridDim.x * blockIdx.y < 16384) \
        g_wide_trace[GATEUP ? 1 : 0][blockIdx.x + gridDim.x * blockIdx.y][ev] = wall_clock64()
#else
#define XS_WTRACE(ev)
#endif

template <int BM, bool GATEUP, bool FULL, int MODE, int NW, int DMAW = NW>
__device__ __forceinline__ void run_tile(const GemmArgs &a, int e, int pos0, int rows, int slab, uint8_t *smem)
{
    using C = WCfg<BM, MODE, NW, DMAW>;
    constexpr int kNW = DMAW, kNT = 64 * NW;   // kNW: waves that issue DMAs
    const int KB = a.K / 128;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 2, wn = wave & 3;
    const int r16 = lane & 15, g = lane >> 4;
    const int n0 = slab * (GATEUP ? 128 : 256);
    const bool shared = e == a.E;
    const int Nrows = GATEUP ? 2 * a.N : a.N;
    const uint8_t *Bexp = shared ? a.Bsh : a.B + (size_t)e * Nrows * a.K;

    uint8_t *trash = smem + kRing;
    float *sB = reinterpret_cast<float *>(trash + kTrash);                 // [2][KB]
    float *red = sB + 2 * KB;                                              // [4][BM]
    const uint32_t ring_lds = lds_addr(smem), trash_lds = lds_addr(trash);

    // ---- weight block scales of the slab: gate_up [gate blk][KB], [up blk][KB];
    //      down [n0/128][KB], [n0/128 + 1][KB]
    {
        const float *Bsf = shared ? a.Bssh : reinterpret_cast<const float *>(a.Bs) + (size_t)e * (Nrows / 128) * KB;
        for (int q = tid; q < 2 * KB; q += kNT) {
            const int b = q / KB, kb = q % KB;
            const int nb = GATEUP ? (b ? a.N + n0 : n0) / 128 : n0 / 128 + b;
            sB[q] = Bsf[(size_t)nb * KB + kb];
        }
    }

    // ---- per-lane DMA source offsets (the K offset goes into the scalar base) ----
    auto token_of = [&](int row) -> int {
        const int p = pos0 + min(row, rows - 1);
        return a.row_token ? a.row_token[p] : p;
    };
    uint32_t oA[C::NA], oW[C::NB];
#pragma unroll
    for (int u = 0; u < C::NA; ++u) {
        const int row = 8 * (wave + kNW * u) + (lane >> 3);
        oA[u] = (uint32_t)token_of(row) * (uint32_t)a.K + (uint32_t)(swz8(row, lane & 7) * 16);
    }
#pragma unroll
    for (int u = 0; u < C::NB; ++u) {
        const int R = 8 * (wave + kNW * u) + (lane >> 3);        // weight row of the LDS tile
        const int wr = GATEUP ? (R < 128 ? n0 + R : a.N + n0 + R - 128) : n0 + R;
        oW[u] = (uint32_t)wr * (uint32_t)a.K + (uint32_t)(swz8(R, lane & 7) * 16);
    }
    const bool sa_real = wave < C::NSA;
    const uint32_t oS = (uint32_t)token_of(sa_real ? 64 * wave + lane : 0) * (uint32_t)(KB * 4);
    const uint8_t *gS = reinterpret_cast<const uint8_t *>(a.As);
    // an expert whose rows fit one partial tile reads its weights once: stream
    // them (full tiles keep the default policy, so their loop has no branch)
    const bool stream_w = !FULL && a.offsets[e + 1] - a.offsets[e] <= BM;

    const uint32_t wring_lds = ring_lds + (uint32_t)(C::NAR * C::AS_BYTES);
    // operands of step kb into ring slot kb % depth; kb < 0 (prologue padding)
    // goes to the trash line, kb >= KB reloads the last step into a slot that is
    // not read again: every iteration issues the same number of loads
    auto issue_a = [&](int kb) {
        const int kk = kb < 0 ? 0 : (kb < KB ? kb : KB - 1);
        const uint32_t st = ring_lds + (uint32_t)(((kb < 0 ? 0 : kb) % C::NAR) * C::AS_BYTES);
#pragma unroll
        for (int u = 0; u < C::NA; ++u)
            dma16(a.A + (size_t)kk * 128, oA[u], kb < 0 ? trash_lds : st + 1024 * (wave + kNW * u));
        dma4(gS + (size_t)kk * 4, oS, (kb >= 0 && sa_real) ? st + C::A_BYTES + 256 * wave : trash_lds);
    };
    auto issue_w = [&](int kb) {
        const int kk = kb < 0 ? 0 : (kb < KB ? kb : KB - 1);
        const uint32_t st = wring_lds + (uint32_t)(((kb < 0 ? 0 : kb) % C::NWR) * C::W_BYTES);
        if (stream_w) {
#pragma unroll
            for (int u = 0; u < C::NB; ++u)
                dma16_nt(Bexp + (size_t)kk * 128, oW[u], kb < 0 ? trash_lds : st + 1024 * (wave + kNW * u));
        } else {
#pragma unroll
            for (int u = 0; u < C::NB; ++u)
                dma16(Bexp + (size_t)kk * 128, oW[u], kb < 0 ? trash_lds : st + 1024 * (wave + kNW * u));
        }
    };
    // the d-th load of iteration kb in issue order (W rows, then A rows and the
    // row scales when W_FIRST, else A first): one DMA instruction.  Full tiles
    // never stream their weights with the non-temporal hint (their experts have
    // more tiles reading the same slab), so this path has no branch.
    auto issue_one = [&](int kb, int d) {
        const int dw = C::W_FIRST ? d : d - (C::NA + 1);
        const int da = C::W_FIRST ? d - C::NB : d;
        if (dw >= 0 && dw < C::NB) {
            const int k2 = kb + C::DW;
            const int kk = k2 < KB ? k2 : KB - 1;
            dma16(Bexp + (size_t)kk * 128, oW[dw], wring_lds + (uint32_t)((k2 % C::NWR) * C::W_BYTES) + 1024 * (wave + kNW * dw));
        } else if (da >= 0 && da < C::NA) {
            const int k2 = kb + C::DA;
            const int kk = k2 < KB ? k2 : KB - 1;
            dma16(a.A + (size_t)kk * 128, oA[da], ring_lds + (uint32_t)((k2 % C::NAR) * C::AS_BYTES) + 1024 * (wave + kNW * da));
        } else if (da == C::NA) {
            const int k2 = kb + C::DA;
            const int kk = k2 < KB ? k2 : KB - 1;
            dma4(gS + (size_t)kk * 4, oS, sa_real ? ring_lds + (uint32_t)((k2 % C::NAR) * C::AS_BYTES) + C::A_BYTES + 256 * wave : trash_lds);
        }
    };
    auto issue = [&](int kb) {   // the loads of iteration kb: A(kb + DA), W(kb + DW)
        if (C::W_FIRST) {
            issue_w(kb + C::DW);
            issue_a(kb + C::DA);
        } else {
            issue_a(kb + C::DA);
            issue_w(kb + C::DW);
        }
    };

    // the wave's four 16-row A tiles (rows of the LDS weight tile)
    int wrow[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
        wrow[j] = GATEUP ? (j < 2 ? 0 : 128) + 32 * wn + 16 * (j & 1) + r16 : 64 * wn + 16 * j + r16;
    // 16-token subtiles of this wave: s16 = wm + WM i, live when 16 s16 < rows
    int nlive = 0;
#pragma unroll
    for (int i = 0; i < C::MI; ++i) nlive += 16 * (wm + C::WM * i) < rows ? 1 : 0;

    v4f acc[C::MI][4];
#pragma unroll
    for (int i = 0; i < C::MI; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

    const bool dma_wave = wave < DMAW;
    __syncthreads();   // sB visible
    if (dma_wave) {
#pragma unroll
        for (int j = -C::PRO; j < 0; ++j) issue(j);
    }
    XS_WTRACE(1);

    const int sbi = GATEUP ? 0 : (wn >> 1);   // down: the wave's 128-row scale block
    for (int kb = 0; kb < KB; ++kb) {
        if (dma_wave) wait_vm<C::X>();   // this wave's loads of step kb landed
        __syncthreads();          // ... and every wave's; the slots of step kb-1 are free
        // Full tiles spread the step's DMAs over its subtiles (below): a DMA
        // instruction holds the issuing wave until the memory pipeline takes it,
        // so a burst of them after the barrier keeps that wave off its MFMAs.
        if (dma_wave && !FULL) issue(kb);
        const uint8_t *sA = smem + (kb % C::NAR) * C::AS_BYTES;
        const float *sS = reinterpret_cast<const float *>(sA + C::A_BYTES);
        const uint8_t *sW = smem + C::NAR * C::AS_BYTES + (kb % C::NWR) * C::W_BYTES;
        const float sb0 = sB[sbi * KB + kb];
        const float sb1 = GATEUP ? sB[KB + kb] : sb0;

        // The step's activation scales first: LDS reads retire in order, so a
        // scale read queued behind the fragment prefetch would make every fold
        // wait for that prefetch.
        float sav[C::MI];
#pragma unroll
        for (int i = 0; i < C::MI; ++i) sav[i] = (FULL || i < nlive) ? sS[16 * (wm + C::WM * i) + r16] : 0.f;
        // Operand layout of v_mfma_f32_16x16x128_f8f6f4: lane 16g + r holds row r
        // with K bytes [16g, 16g+16) and [64+16g, 64+16g+16): LDS chunks g, g+4.
        v8i wf[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint8_t *rp = sW + wrow[j] * 128;
            wf[j] = cat(*reinterpret_cast<const v4i *>(rp + swz8(wrow[j], g) * 16),
                        *reinterpret_cast<const v4i *>(rp + swz8(wrow[j], g + 4) * 16));
        }
        auto read_b = [&](int i) -> v8i {
            const int row = 16 * (wm + C::WM * i) + r16;
            const uint8_t *rp = sA + row * 128;
            return cat(*reinterpret_cast<const v4i *>(rp + swz8(row, g) * 16),
                       *reinterpret_cast<const v4i *>(rp + swz8(row, g + 4) * 16));
        };
        // Subtile i: read B(i+2), 4 MFMAs on B(i), fold the products of i-1.
        // Full tiles run branch free; partial ones skip the subtiles past rows.
        constexpr int PB = 2;                       // fragment prefetch distance (subtiles)
        v8i bx[PB + 1];
#pragma unroll
        for (int i = 0; i < PB; ++i)
            if (i < C::MI && (FULL || i < nlive)) bx[i] = read_b(i);
        v4f q[2][4];
#pragma unroll
        for (int i = 0; i <= C::MI; ++i) {
            if (FULL && dma_wave && i < C::MI) {
                // DMA d of this step goes out in subtile d * MI / PER_STEP
#pragma unroll
                for (int d = 0; d < C::PER_STEP; ++d)
                    if (d * C::MI / C::PER_STEP == i) issue_one(kb, d);
            }
            if (i < C::MI && (FULL || i < nlive)) {
                if (i + PB < C::MI && (FULL || i + PB < nlive)) bx[(i + PB) % (PB + 1)] = read_b(i + PB);
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    q[i & 1][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                        wf[j], bx[i % (PB + 1)], v4f{0.f, 0.f, 0.f, 0.f}, 0, 0, 0, 0, 0, 0);
            }
            if (i >= 1 && (FULL || i - 1 < nlive)) {
                const int m = i - 1;
                const float c0 = sav[m] * sb0, c1 = sav[m] * sb1;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float c = (GATEUP && j >= 2) ? c1 : c0;
#pragma unroll
                    for (int v = 0; v < 4; ++v) acc[m][j][v] = __builtin_fmaf(q[m & 1][j][v], c, acc[m][j][v]);
                }
            }
            if (FULL && i >= 1 && i < C::MI) {
                // Issue order of the region: the fragment prefetch, then each
                // MFMA of subtile i followed by a share of the fold of i-1, whose
                // products finished during the previous region.  Left to itself
                // the scheduler puts the whole fold first, where it waits on the
                // MFMAs that produced it while the matrix core idles.
                __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);   // DS reads
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // one MFMA
                    __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);   // VALU
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    wait_vm<0>();      // the clamped DMAs past the last step land before the block ends
    XS_WTRACE(2);

    // ------------------------------------------------------------ epilogue
    // acc[i][j][v]: token row 16 (wm + WM i) + r16; A-tile j row 4 g + v.
    if (GATEUP) {
        // act feature (within the block's 128): 32 wn + 16 jj + 4 g + v, jj = 0, 1
        float act[C::MI][2][4];
#pragma unroll
        for (int i = 0; i < C::MI; ++i) {
            float m = 0.f;
#pragma unroll
            for (int jj = 0; jj < 2; ++jj)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const float gt = acc[i][jj][v], up = acc[i][jj + 2][v];
                    act[i][jj][v] = gt * fast_sigmoid(gt) * up;
                    m = fmaxf(m, __builtin_fabsf(act[i][jj][v]));
                }
            m = fmaxf(m, __shfl_xor(m, 16, WAVE));
            m = fmaxf(m, __shfl_xor(m, 32, WAVE));
            if (g == 0) red[wn * BM + 16 * (wm + C::WM * i) + r16] = m;
        }
        __syncthreads();   // every wave is past its loop: the ring is free for staging
        // The FP8 tile is staged in the ring (rows padded to 144 B: a wave's
        // 16-row x 4-lane writes hit 64 distinct banks) and stored as whole
        // 128-byte rows; an instruction that scatters 4 bytes over 16 rows
        // moves about a quarter of the bytes per clock of a row-contiguous one.
        constexpr int QS = 144;
        static_assert(BM * QS <= kRing, "staging tile");
        uint8_t *qs = smem;
        float *Cs = reinterpret_cast<float *>(a.Cs);
        const int nsc = a.N / 128;
#pragma unroll
        for (int i = 0; i < C::MI; ++i) {
            const int row = 16 * (wm + C::WM * i) + r16;
            float amax = 0.f;
#pragma unroll
            for (int w = 0; w < 4; ++w) amax = fmaxf(amax, red[w * BM + row]);
            const float inv = amax == 0.f ? 0.f : __fdiv_rn(448.0f, amax);
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) {
                float x[4];
#pragma unroll
                for (int v = 0; v < 4; ++v) x[v] = fminf(fmaxf(act[i][jj][v] * inv, -448.f), 448.f);
                *reinterpret_cast<uint32_t *>(qs + row * QS + 32 * wn + 16 * jj + 4 * g) =
                    e4m3_pack2_hw(x[0], x[1]) | (e4m3_pack2_hw(x[2], x[3]) << 16);
            }
            if (wn == 0 && g == 0 && row < rows) Cs[(size_t)(pos0 + row) * nsc + n0 / 128] = amax == 0.f ? 1.0f : __fdiv_rn(amax, 448.0f);
        }
        __syncthreads();
#pragma unroll
        for (int pass = 0; pass < BM / (kNT / 8); ++pass) {
            const int row = (kNT / 8) * pass + (tid >> 3), c = tid & 7;
            if (row < rows)
                *reinterpret_cast<v4i *>(a.Cq + (size_t)(pos0 + row) * a.N + n0 + 16 * c) =
                    *reinterpret_cast<const v4i *>(qs + row * QS + 16 * c);
        }
    } else if (a.Cf) {
        store_f32_tile<BM, NW>(a, acc, pos0, rows, slab, wm, wn, smem, red);
    } else {
        // output column n0 + 64 wn + 16 j + 4 g + v.  The bf16 tile is staged in
        // the ring (rows padded to 528 B: a half-wave's 16-row x 2-lane 8-byte
        // writes hit distinct banks) and stored as whole 512-byte rows.
        constexpr int YS = 528;
        static_assert(BM * YS <= kRing, "staging tile");
        uint8_t *ys = smem;
        __syncthreads();   // every wave is past its loop: the ring is free for staging
#pragma unroll
        for (int i = 0; i < C::MI; ++i) {
            const int row = 16 * (wm + C::WM * i) + r16;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                v2i pk;
                pk[0] = (int)((uint32_t)bf16_from_f32(acc[i][j][0]) | ((uint32_t)bf16_from_f32(acc[i][j][1]) << 16));
                pk[1] = (int)((uint32_t)bf16_from_f32(acc[i][j][2]) | ((uint32_t)bf16_from_f32(acc[i][j][3]) << 16));
                *reinterpret_cast<v2i *>(ys + row * YS + 2 * (64 * wn + 16 * j + 4 * g)) = pk;
            }
        }
        __syncthreads();
#pragma unroll
        for (int pass = 0; pass < BM / (kNT / 32); ++pass) {
            const int row = (kNT / 32) * pass + (tid >> 5), c = tid & 31;
            if (row < rows)
                *reinterpret_cast<v4i *>(a.Cy + (size_t)(pos0 + row) * a.ldc + n0 + 8 * c) =
                    *reinterpret_cast<const v4i *>(ys + row * YS + 16 * c);
        }
    }
}

template <int BM, bool GATEUP, int NW>
__global__ __launch_bounds__(64 * NW) void moe_gemm_wide_kernel(GemmArgs a)
{
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int4 *tab = reinterpret_cast<const int4 *>(a.tile_tab);   // shared + routed tiles
    // the launch's range of the table (shared tiles come first): the shared
    // segment alone, the routed experts alone, or both
    int lo = 0, tiles = tab[0].x;
    if (a.e_lo >= a.E) tiles = tab[0].y;
    else if (a.e_hi <= a.E) lo = tab[0].y;
    int tile, slab;
    if (a.xcd_order) {
        // 1-D grid.  Blocks go round-robin to the 8 XCDs (linear id L to XCD
        // L % 8), each with its own L2.  The work is cut into groups of 8
        // tiles x 4 slabs (the 32 blocks an XCD runs at once): a group's tiles
        // share each weight slab and its slabs share each tile's activation
        // rows inside one L2, which per K step and XCD reads 8 x 24 KB of
        // activations and 4 x 32 KB of weights (grid order: 16 tiles x 2
        // slabs, 384 + 64 KB).  XCD x takes groups x, x + 8, ... in order.
        const int gx = GATEUP ? a.N / 128 : a.N / 256, nq = gx / 4;
        const int L = (int)blockIdx.x, j = L >> 3;
        const int sg = (L & 7) + 8 * (j >> 5), i = j & 31;
        const int g = sg / nq, q = sg - g * nq;
        tile = lo + 8 * g + (i >> 2);
        slab = 4 * q + (i & 3);
        if (tile >= tiles) return;
    } else {
        tile = lo + (int)blockIdx.y;
        slab = (int)blockIdx.x;
        if (tile >= tiles) return;
    }
    XS_WTRACE(0);
    const int4 d = tab[1 + tile];   // {expert, first position, rows}
    if constexpr (NW == 8) {
        // 192-row tiles: full tiles 3 + 2 stages, partial ones past 128 rows too
        // the 4 waves of wm = 0 (one per SIMD) issue every DMA, the other 4
        // only compute: after each step's barrier one wave per SIMD goes
        // straight to its MFMAs while the other issues the step's loads
        // (measured 4% faster on the V4-Flash prefill layer than all 8 loading)
        constexpr int DW = NW / 2;
        if (d.z >= BM) run_tile<BM, GATEUP, true, 1, NW, DW>(a, d.x, d.y, BM, slab, smem);
        else if (d.z > 128) run_tile<BM, GATEUP, false, 1, NW, DW>(a, d.x, d.y, d.z, slab, smem);
        else if (d.z > 64 || !a.short_deep) run_tile<BM, GATEUP, false, 0, NW, DW>(a, d.x, d.y, d.z, slab, smem);
        // tiles of up to 64 rows (single-tile experts: a weight stream from HBM)
        // lay out 64-row activation stages, which leaves LDS for 4 weight stages
        else run_tile<64, GATEUP, false, 2, NW, DW>(a, d.x, d.y, d.z, slab, smem);
    } else {
        static_assert(NW == 4, "waves");
        if (d.z >= BM) run_tile<BM, GATEUP, true, 3, NW>(a, d.x, d.y, BM, slab, smem);
        else run_tile<BM, GATEUP, false, 3, NW>(a, d.x, d.y, d.z, slab, smem);
    }
    XS_WTRACE(3);
#ifdef XS_WIDE_TRACE
    if (threadIdx.x == 0 && blockIdx.x + gridDim.x * blockIdx.y < 16384) {
        g_wide_trace[GATEUP ? 1 : 0][blockIdx.x + gridDim.x * blockIdx.y][4] = (uint64_t)d.z;
        g_wide_trace[GATEUP ? 1 : 0][blockIdx.x + gridDim.x * blockIdx.y][5] = (uint64_t)d.x;
    }
#endif
}

template <int BM, bool GATEUP, int NW>
int launch_wide(const GemmArgs &a, int grid_y, hipStream_t st)
{
    if (grid_y <= 0) return XS_OK;
    constexpr int kNT = 64 * NW;
    const size_t smem = (size_t)kRing + kTrash + 8 * (size_t)(a.K / 128) + 4 * 4 * BM;
    if (smem > 160 * 1024) return set_error(XS_ERR_UNSUPPORTED, "K=%d needs %zu bytes of LDS", a.K, smem);
    auto fn = moe_gemm_wide_kernel<BM, GATEUP, NW>;
    static bool attr_set = false;
    if (!attr_set) {
        XS_HIP(hipFuncSetAttribute((const void *)fn, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
        attr_set = true;
    }
    const int grid_x = GATEUP ? a.N / 128 : a.N / 256;
    if (a.xcd_order) {
        const int64_t groups = (grid_y + 7) / 8 * (grid_x / 4);      // 8-tile x 4-slab groups
        fn<<<dim3((unsigned)((groups + 7) / 8 * 256)), dim3(kNT), smem, st>>>(a);
    } else {
        fn<<<dim3((unsigned)grid_x, (unsigned)grid_y), dim3(kNT), smem, st>>>(a);
    }
    XS_LAUNCH_CHECK();
    return XS_OK;
}

}  // namespace

// 192-row tiles on 8 waves (2 per SIMD).  Measured slower on the V4-Flash
// prefill layer: 128-row tiles on 4 waves (one per SIMD, 3 + 3 stages) and
// 128-row tiles on 8 waves with 3 + 3 stages.
constexpr int kWideBM = 192;
int wide_tile_rows() { return kWideBM; }

int launch_gemm_wide(const GemmArgs &a, bool gateup, int grid_y, hipStream_t st)
{
    if (a.bm != wide_tile_rows()) return set_error(XS_ERR_INVALID, "wide GEMM needs %d-row tiles", wide_tile_rows());
    if (a.K % 128 || (gateup ? a.N % 128 : a.N % 256) || !a.tile_tab)
        return set_error(XS_ERR_UNSUPPORTED, "wide GEMM shape K=%d N=%d", a.K, a.N);
    GemmArgs b = a;
    const char *ord = getenv("XS_WIDE_ORDER");
    // XS_WIDE_ORDER=0: one block per (slab, tile) in grid order (measurements)
    b.xcd_order = !(ord && ord[0] == '0') && (gateup ? a.N / 128 : a.N / 256) % 4 == 0;
    const char *sd = getenv("XS_WIDE_SHORT");
    b.short_deep = !(sd && sd[0] == '0');
    return gateup ? launch_wide<kWideBM, true, 8>(b, grid_y, st) : launch_wide<kWideBM, false, 8>(b, grid_y, st);
}

}  // namespace xs

#ifdef XS_WIDE_TRACE
extern "C" int xs_wide_trace_read(void *dst)
{
    return hipMemcpyFromSymbol(dst, HIP_SYMBOL(xs::g_wide_trace), sizeof(xs::g_wide_trace)) == hipSuccess ? 0 : 1;
}
#endif
