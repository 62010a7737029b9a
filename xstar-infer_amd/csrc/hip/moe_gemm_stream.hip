// moe_gemm_stream.hip -- persistent grouped expert GEMMs on gfx950: FP8
// block-scaled experts on 16- or 32-row tiles (decode) and MXFP4 experts on
// 16- to 64-row tiles.
//
// Nearest reference code: gemm_silu_and_mul_kernel (xstar_cpp/src/ops/mlp.cu:52-200)
// and gemm_kernel (xstar_cpp/src/ops/gemm.cu:41-210); numerics as the FP8 tiles of
// moe_gemm.hip (each 128-K block's MFMA product scaled by activation row scale x
// weight block scale into an f32 accumulator; SwiGLU in f32; 1x128 requant).
//
// At decode sizes a layer is a weight stream: every routed expert's W13 / W2
// is read once, and the work is (tiles x weight slabs) items of equal size
// (one 256-row slab of one expert over all of K).  One block per CU walks a
// contiguous range of the flattened (item, K step) sequence, so every CU gets
// the same number of K steps (not whole items) and the LDS ring keeps
// streaming across item boundaries (no per-item fill, no tail of idle CUs):
//   * operand tiles move global -> LDS by DMA (global_load_lds) into a 4-stage
//     ring issued 3 steps ahead; each stage also carries the step's activation
//     row scales and the two weight block scales, so nothing else is read
//     inside the loop;
//   * an item whose K range is split between blocks ("stream-K") is finished
//     by whichever block arrives last: every part writes its f32 partial tile
//     with system-scope stores (through the L2 of its XCD), waits for them,
//     then bumps the item's counter (agent-scope atomic); the last arriver
//     reads the other parts with system-scope loads, sums the parts in block
//     order and runs the epilogue.  No block ever waits for another, so the
//     kernel needs no co-residency, and no L2 is written back or invalidated;
//   * the split is static: CUs stream at rates up to 10-20% apart (whole XCDs
//     differ within a run), and a dynamic share claimed in chunks measured
//     slower overall than this tail;
//   * items are ordered expert by expert, slab by slab, then tile: the tiles
//     of an expert with more rows than one tile read each weight slab back to
//     back, while it is still in L2 (those loads keep the default cache policy;
//     single-tile experts stream their weights with the non-temporal hint).
#include "moe_gemm.hpp"

#include <cstdlib>

namespace xs {
namespace {

constexpr int kNW = 4;                 // waves per block
constexpr int kNT = 64 * kNW;
constexpr int kTrash = 1024;           // LDS target of padding DMAs

// FP8: e4m3 weights with 128x128 f32 block scales, 1x128 FP8 activations, K
// steps of 128 (the products are folded with the scales in VALU).  MXFP4:
// e2m1 weights and MXFP8 activations with e8m0 scales per 32 K, applied by the
// MFMA; K steps of 256, so a weight row is read as whole 128-byte lines.
template <int BM, bool FP4>
struct SCfg {
    static constexpr int MI = BM / 16;             // 16-token subtiles (every wave holds all of them)
    static constexpr int NJ = 4;                   // 16-column subtiles per wave (64 weight rows)
    static constexpr int KSTEP = FP4 ? 256 : 128;
    static constexpr int NST = FP4 ? 3 : 4;    // ring stages (MXFP4: the scale buffers of a pair of steps are
                                               // rewritten 2 steps ahead, which 2 buffers allow)
    static constexpr int MAXIT = FP4 && BM == 64 ? 30 : 40;          // item descriptors a block can hold
    static constexpr int AROW = FP4 ? 256 : 128;                      // activation bytes per row and step
    static constexpr int A_BYTES = BM * AROW;
    static constexpr int B_BYTES = 256 * 128;
    // FP8: 64 row scales and 2 block scales ride in each stage.  MXFP4: the
    // e8m0 scales (8 per row and step) are fetched 16 bytes per row for each
    // pair of steps into a separate double buffer (4-byte gathers from 320
    // rows every step outnumbered all operand requests to the L2).
    static constexpr int SA_BYTES = FP4 ? 0 : 256;
    static constexpr int SB_BYTES = FP4 ? 0 : 256;
    static constexpr int SA_OFF = A_BYTES + B_BYTES;
    static constexpr int SB_OFF = SA_OFF + SA_BYTES;
    static constexpr int STAGE = SB_OFF + SB_BYTES;
    static constexpr int A_INSTR = A_BYTES / 1024;     // wave-wide 1 KB DMAs for A
    static constexpr int NA = A_INSTR > kNW ? A_INSTR / kNW : 1;   // per wave (padding ones target the trash)
    static constexpr int NB = B_BYTES / 1024 / kNW;    // weight DMAs per wave
    static constexpr int NS = FP4 ? 2 : 1;             // scale DMAs per wave
    static constexpr int PER_STAGE = NA + NB + NS;     // loads per wave per stage
    static constexpr int SC_OFF = NST * STAGE + kTrash;    // MXFP4 scale buffers [2][256 + 64 rows][16 B]
    static constexpr int SC_BUF = FP4 ? 320 * 16 : 0;
    static constexpr int RED_OFF = SC_OFF + 2 * SC_BUF;
    static constexpr int META_OFF = RED_OFF + (FP4 ? 0 : 16 * BM);
    static constexpr int RTOK_OFF = META_OFF + 16 * MAXIT;
    static constexpr int SMEM = RTOK_OFF + 2 * BM * MAXIT;   // row tokens as 16-bit (T < 65536)
    static_assert(A_INSTR >= 1 && (A_INSTR <= kNW || A_INSTR % kNW == 0) && BM <= 64, "tile rows");
    static_assert(SMEM <= 160 * 1024, "LDS");
    static_assert(SMEM <= 160 * 1024, "LDS");
};

__device__ __forceinline__ int swz8(int r, int c) { return c ^ ((r >> 1) & 7); }     // 128-byte rows
__device__ __forceinline__ int swz16(int r, int c) { return c ^ (r & 15); }         // 256-byte rows

__device__ __forceinline__ uint32_t lds_addr(const void *p)
{
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

__device__ __forceinline__ v8i cat(v4i a, v4i b) { return v8i{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]}; }

// Wave-wide DMA global -> LDS: lane i's 16 (4) bytes land at lds + 16 i (4 i).
// M0 carries the wave-uniform LDS base; it is written only here.
// Wait states inside the asm (the compiler's hazard checks do not look into
// an asm string): an LDS DMA that reads M0 needs one after the SALU write of
// M0, and a VMEM instruction reading an SGPR that a VALU instruction wrote
// (v_readfirstlane of the base) needs five, hence s_nop 4 where the base is a
// scalar operand and s_nop 0 where the address is a VGPR.
__device__ __forceinline__ void dma16_v(const void *g, uint32_t lds)
{
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(__builtin_amdgcn_readfirstlane(lds))
                 : "memory");
}
__device__ __forceinline__ void dma16_s(const uint8_t *sbase, uint32_t voff, uint32_t lds)
{
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 4\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(lds) : "memory");
}
__device__ __forceinline__ void dma16_s_nt(const uint8_t *sbase, uint32_t voff, uint32_t lds)
{
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 4\n\tglobal_load_lds_dwordx4 %0, %1 nt" ::"v"(voff), "s"(sbase), "s"(lds) : "memory");
}
__device__ __forceinline__ void dma4_v(const void *g, uint32_t lds)
{
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(g), "s"(__builtin_amdgcn_readfirstlane(lds))
                 : "memory");
}
// A pointer the compiler cannot prove wave-uniform (it was read from LDS) made
// scalar, for the saddr form of the DMAs.
__device__ __forceinline__ const uint8_t *uniform_ptr(const uint8_t *p)
{
    const uint64_t v = (uint64_t)(uintptr_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return reinterpret_cast<const uint8_t *>((uintptr_t)(((uint64_t)hi << 32) | lo));
}
template <int N>
__device__ __forceinline__ void wait_vm()
{
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

#ifdef XS_STREAM_TRACE
// Development builds only: per-block phase timestamps (100 MHz wall clock).
__device__ uint64_t g_stream_trace[2][2048][6];
#define XS_TRACE(ev) \
    if (threadIdx.x == 0 && blockIdx.x < 2048) g_stream_trace[GATEUP ? 1 : 0][blockIdx.x][ev] = wall_clock64()
#else
#define XS_TRACE(ev)
#endif

// Number of 256-row weight slabs per tile.
__host__ __device__ __forceinline__ int slabs_of(bool gateup, int N) { return gateup ? N / 128 : (N + 255) / 256; }

template <int BM, bool GATEUP, bool FP4>
__global__ __launch_bounds__(kNT) void moe_gemm_stream_kernel(GemmArgs a)
{
    using C = SCfg<BM, FP4>;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    __shared__ int last_flag;
    float *red = reinterpret_cast<float *>(smem + C::RED_OFF);      // [4][BM]
    int4 *meta = reinterpret_cast<int4 *>(smem + C::META_OFF);      // [MAXIT]
    uint16_t *rtok = reinterpret_cast<uint16_t *>(smem + C::RTOK_OFF);   // [MAXIT][BM]

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l16 = lane & 15, g = lane >> 4;
    const int KB = a.K / C::KSTEP;       // K steps per item
    const int KB128 = a.K / 128;         // FP8 scale blocks along K
    XS_TRACE(0);

    // Counters of the launch that follows (the down GEMM after gate_up).
    if (a.zero_cnt)
        for (int i = blockIdx.x * kNT + tid; i < a.zero_n; i += gridDim.x * kNT) a.zero_cnt[i] = 0;

    // ---- this block's range of the flattened (item, K step) sequence ----
    // (W < 2^31: checked by the host.)  G <= W, so every block of the partition
    // holds at least one step and the blocks holding parts of an item are
    // exactly block_of(first step) .. block_of(last step).
    const int4 *tab = reinterpret_cast<const int4 *>(a.tile_tab);
    const int4 h = tab[0];
    int lo = 0, hi = h.x;
    if (a.e_lo >= a.E) hi = h.y;          // shared segment only
    else if (a.e_hi <= a.E) lo = h.y;     // routed experts only
    const int gx = slabs_of(GATEUP, a.N);
    const int W = (hi - lo) * gx * KB;
    const int G = W < (int)gridDim.x ? W : (int)gridDim.x;
    // Grouped partition (the default; stream-K below when the tiles do not
    // fill the groups or a block would hold more than MAXIT items): whole items only.  Logical
    // block b = 16 g + s (gx = 16 slabs) takes slab s of the tile run
    // [g ntl / NG, (g+1) ntl / NG), and the gx blocks of a group sit on one XCD
    // (blocks go round-robin to the 8 XCDs; logical neighbours are 8 block ids
    // apart), so at any moment the group's CUs read one tile's activation rows
    // together through their L2 instead of each re-reading them from memory,
    // item after item, behind the weight stream.
    const int ntl = hi - lo, NG = G / gx;
    const bool grouped = a.xcd_order && G == (int)gridDim.x && (G & 7) == 0 && ((G >> 3) % gx) == 0 &&
                         ntl >= NG && (ntl + NG - 1) / NG <= C::MAXIT;
    int b = (int)blockIdx.x, s0, s1, it0, it1, gsl = 0, gt0 = 0;
    if (grouped) {
        b = ((int)blockIdx.x & 7) * (G >> 3) + ((int)blockIdx.x >> 3);
        const int grp = b / gx;
        gsl = b - grp * gx;
        gt0 = (int)((int64_t)grp * ntl / NG);
        const int n = (int)((int64_t)(grp + 1) * ntl / NG) - gt0;   // >= 1 (ntl >= NG)
        it0 = gt0 * gx + gsl * n;
        it1 = it0 + n - 1;
        s0 = it0 * KB;
        s1 = (it1 + 1) * KB;
    } else {
        if (b >= G) return;
        s0 = (int)((int64_t)b * W / G);
        s1 = (int)((int64_t)(b + 1) * W / G);
        it0 = s0 / KB;
        it1 = (s1 - 1) / KB;
    }
    const int nit = it1 - it0 + 1;   // <= MAXIT (grid sized by the host)

    // ---- item descriptors: {expert, first position, rows, slab | multi-tile << 30} ----
    // Items run expert by expert, then slab, then tile (tab .w: tile index in
    // the expert's group | tiles in the group << 16); grouped: this block's
    // tile run at slab gsl.
    if (tid < nit) {
        if (grouped) {
            const int4 d = tab[1 + lo + gt0 + tid];
            meta[tid] = int4{d.x, d.y, min(d.z, BM), gsl | ((d.w >> 16) > 1 ? (1 << 30) : 0)};
        } else {
            const int it = it0 + tid;
            const int tm = lo + it / gx;                 // a tile of the item's expert group
            const int4 d = tab[1 + tm];
            const int t = d.w & 0xffff, nt = d.w >> 16, t0 = tm - t;
            const int local = it - (t0 - lo) * gx;
            const int slab = local / nt, tile = t0 + local % nt;
            const int4 dd = tile == tm ? d : tab[1 + tile];
            meta[tid] = int4{d.x, dd.y, min(dd.z, BM), slab | (nt > 1 ? (1 << 30) : 0)};
        }
    }
    __syncthreads();
    for (int q = tid; q < nit * BM; q += kNT) {
        const int4 m = meta[q / BM];
        const int p = m.y + min(q % BM, m.z - 1);
        rtok[q] = (uint16_t)(a.row_token ? a.row_token[p] : p);
    }
    __syncthreads();

    XS_TRACE(1);
    // ---- issue side: DMA sources of the item being loaded ----
    const uint32_t ring = lds_addr(smem), trash = lds_addr(smem + C::NST * C::STAGE);
    const uint32_t sc_base = lds_addr(smem + C::SC_OFF);
    const int Nrows = GATEUP ? 2 * a.N : a.N;
    int cur = -1;
    const uint8_t *gA[C::NA];           // this lane's activation chunks (64-bit: T x K may exceed 4 GB)
    const uint8_t *gS = nullptr;        // this lane's row-scale / block-scale word (FP8), row-scale word (MXFP4)
    const uint8_t *gS2 = nullptr;       // MXFP4: this lane's weight-scale word
    const uint8_t *bW = nullptr;        // wave-uniform weight base of the item
    uint32_t oW[C::NB];                 // this lane's weight chunk offsets in the expert
    bool w_nt = false;

    auto setup = [&](int li) {
        const int4 m = meta[li];
        const int e = m.x, slab = m.w & 0x3fffffff;
        const bool shared = e == a.E;
        const int n0 = slab * (GATEUP ? 128 : 256);
        w_nt = (m.w >> 30) == 0;
        bW = uniform_ptr(shared ? a.Bsh : a.B + (size_t)e * Nrows * (FP4 ? a.K / 2 : a.K));
#pragma unroll
        for (int u = 0; u < C::NA; ++u) {
            const int q = wave + kNW * u, p = 64 * q + lane;
            const int r = FP4 ? p >> 4 : p >> 3, c = FP4 ? swz16(r, p & 15) : swz8(r, p & 7);
            gA[u] = a.A + (size_t)rtok[li * BM + (q < C::A_INSTR ? r : 0)] * a.K + c * 16;
        }
        // weight row of slab row vr (gate_up: 16-row gate / up subtiles interleaved)
        auto brow_of = [&](int vr) -> int {
            if (GATEUP) {
                const int sub = vr >> 4, w = vr & 15, n = n0 + (sub >> 1) * 16 + w;
                return (sub & 1) ? a.N + n : n;
            }
            return min(n0 + vr, a.N - 1);
        };
#pragma unroll
        for (int u = 0; u < C::NB; ++u) {
            const int p = 64 * (wave + kNW * u) + lane;
            const int vr = p >> 3;
            oW[u] = (uint32_t)brow_of(vr) * (uint32_t)(FP4 ? a.K / 2 : a.K) + (uint32_t)(swz8(vr, p & 7) * 16);
        }
        if (FP4)                  // weight scales (e8m0 per 32 K) of slab row 64 * wave + lane
            gS2 = reinterpret_cast<const uint8_t *>(a.Bs) + ((size_t)e * Nrows + brow_of(64 * wave + lane)) * (a.K / 32);
        if (FP4) {                // activation row scales (e8m0 per 32 K), row = lane (clamped)
            gS = reinterpret_cast<const uint8_t *>(a.As) + (size_t)rtok[li * BM + min(lane, BM - 1)] * (a.K / 32);
        } else if (wave == 0) {   // activation row scales, row = lane (clamped)
            gS = reinterpret_cast<const uint8_t *>(a.As) + (size_t)rtok[li * BM + min(lane, BM - 1)] * KB128 * 4;
        } else {                  // wave 1: block scales of the slab's two 128-row blocks
            const float *Bsf = shared ? a.Bssh : reinterpret_cast<const float *>(a.Bs) + (size_t)e * (Nrows / 128) * KB128;
            int nb;
            if (GATEUP) nb = (lane == 1 ? a.N + n0 : n0) / 128;
            else nb = min(n0 / 128 + (lane == 1 ? 1 : 0), a.N / 128 - 1);
            gS = reinterpret_cast<const uint8_t *>(Bsf + (size_t)nb * KB128);
        }
    };
    // Issue side position: item li_i, step kb_i (advanced one step per issue).
    // Issues past the range reload the last step into a stage that is never
    // read, so every wave's load count per step stays uniform.
    int li_i = 0, kb_i = s0 % KB, n_issued = 0;
    const int n_steps = s1 - s0;
    auto issue = [&](int s) {
        if (li_i != cur) {
            setup(li_i);
            cur = li_i;
        }
        const uint32_t st = __builtin_amdgcn_readfirstlane(ring + (uint32_t)((s % C::NST) * C::STAGE));
#pragma unroll
        for (int u = 0; u < C::NA; ++u) {
            const int q = wave + kNW * u;
            dma16_v(gA[u] + (size_t)kb_i * C::AROW, q < C::A_INSTR ? st + 1024 * q : trash);
        }
        const uint8_t *wb = uniform_ptr(bW + (size_t)kb_i * 128);
        const uint32_t d0 = __builtin_amdgcn_readfirstlane(st + C::A_BYTES + (uint32_t)(wave * 1024));
        if (w_nt) {
#pragma unroll
            for (int u = 0; u < C::NB; ++u) dma16_s_nt(wb, oW[u], d0 + (uint32_t)(u * kNW * 1024));
        } else {
#pragma unroll
            for (int u = 0; u < C::NB; ++u) dma16_s(wb, oW[u], d0 + (uint32_t)(u * kNW * 1024));
        }
        if (FP4) {
            // the scales of steps 2p, 2p+1 (16 bytes per row) land in buffer p % 2
            // with step 2p's loads (or with the block's first step); otherwise
            // the same number of loads goes to the trash
            const int gs = s0 + n_issued;
            const bool load = n_issued < n_steps && ((gs & 1) == 0 || n_issued == 0);
            const uint32_t sc = __builtin_amdgcn_readfirstlane(sc_base + (uint32_t)(((gs >> 1) & 1) * C::SC_BUF));
            const int kp = kb_i & ~1;
            dma16_v(gS2 + (size_t)kp * 8, load ? sc + 1024 * wave : trash);
            dma16_v(gS + (size_t)kp * 8, load && wave == 0 ? sc + 4096 : trash);
        } else {
            dma4_v(gS + (size_t)kb_i * 4, wave == 0 ? st + C::SA_OFF : (wave == 1 ? st + C::SB_OFF : trash));
        }
        if (++n_issued < n_steps && ++kb_i == KB) {
            kb_i = 0;
            ++li_i;
        }
    };

    // ---- epilogue of a finished item (acc: full-K sums) ----
    auto epilogue = [&](int li, const v4f (&acc)[C::MI][C::NJ]) {
        const int4 m = meta[li];
        const int pos0 = m.y, rows = m.z, slab = m.w & 0x3fffffff;
        const int wn = wave;
        if (GATEUP && FP4) {
            // MXFP8 1x32 requant: a 32-column block is the wave's two act column
            // subtiles, so the block amax stays within the wave
            const int n0 = slab * 128;
            uint8_t *Cs8 = reinterpret_cast<uint8_t *>(a.Cs);
#pragma unroll
            for (int i = 0; i < C::MI; ++i) {
                const int r = 16 * i + l16;
                float act[2][4];
                float mx = 0.f;
#pragma unroll
                for (int p = 0; p < 2; ++p)
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const float gt = acc[i][2 * p][v], up = acc[i][2 * p + 1][v];
                        act[p][v] = gt * fast_sigmoid(gt) * up;
                        mx = fmaxf(mx, __builtin_fabsf(act[p][v]));
                    }
                mx = fmaxf(mx, __shfl_xor(mx, 16, WAVE));
                mx = fmaxf(mx, __shfl_xor(mx, 32, WAVE));
                const int se = mx_exponent(mx, 8);
                if (r < rows) {
#pragma unroll
                    for (int p = 0; p < 2; ++p) {
                        float q[4];
#pragma unroll
                        for (int v = 0; v < 4; ++v) q[v] = fminf(fmaxf(__builtin_ldexpf(act[p][v], -se), -448.f), 448.f);
                        *reinterpret_cast<uint32_t *>(a.Cq + (size_t)(pos0 + r) * a.N + n0 + (2 * wn + p) * 16 + 4 * g) =
                            e4m3_pack2_hw(q[0], q[1]) | (e4m3_pack2_hw(q[2], q[3]) << 16);
                    }
                    if (g == 0) Cs8[(size_t)(pos0 + r) * (a.N / 32) + (n0 + 32 * wn) / 32] = (uint8_t)(se + 127);
                }
            }
        } else if (GATEUP) {
            const int n0 = slab * 128;
            float act[C::MI][2][4];
#pragma unroll
            for (int i = 0; i < C::MI; ++i)
#pragma unroll
                for (int p = 0; p < 2; ++p)
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const float gt = acc[i][2 * p][v], up = acc[i][2 * p + 1][v];
                        act[i][p][v] = gt * fast_sigmoid(gt) * up;
                    }
            // token amax over the 128 act columns: 8 per lane, the 4 lane groups, the 4 waves
#pragma unroll
            for (int i = 0; i < C::MI; ++i) {
                float mx = 0.f;
#pragma unroll
                for (int p = 0; p < 2; ++p)
#pragma unroll
                    for (int v = 0; v < 4; ++v) mx = fmaxf(mx, __builtin_fabsf(act[i][p][v]));
                mx = fmaxf(mx, __shfl_xor(mx, 16, WAVE));
                mx = fmaxf(mx, __shfl_xor(mx, 32, WAVE));
                if (g == 0) red[wn * BM + 16 * i + l16] = mx;
            }
            __syncthreads();
            float *Cs = reinterpret_cast<float *>(a.Cs);
#pragma unroll
            for (int i = 0; i < C::MI; ++i) {
                const int r = 16 * i + l16;
                const float amax = fmaxf(fmaxf(red[r], red[BM + r]), fmaxf(red[2 * BM + r], red[3 * BM + r]));
                const float inv = amax == 0.f ? 0.f : __fdiv_rn(448.0f, amax);
                if (r < rows) {
#pragma unroll
                    for (int p = 0; p < 2; ++p) {
                        float q[4];
#pragma unroll
                        for (int v = 0; v < 4; ++v) q[v] = fminf(fmaxf(act[i][p][v] * inv, -448.f), 448.f);
                        *reinterpret_cast<uint32_t *>(a.Cq + (size_t)(pos0 + r) * a.N + n0 + (2 * wn + p) * 16 + 4 * g) =
                            e4m3_pack2_hw(q[0], q[1]) | (e4m3_pack2_hw(q[2], q[3]) << 16);
                    }
                    if (wn == 0 && g == 0)
                        Cs[(size_t)(pos0 + r) * (a.N / 128) + n0 / 128] = amax == 0.f ? 1.0f : __fdiv_rn(amax, 448.0f);
                }
            }
        } else {
            const int n0 = slab * 256;
#pragma unroll
            for (int i = 0; i < C::MI; ++i) {
                const int r = 16 * i + l16;
                if (r >= rows) continue;
#pragma unroll
                for (int j = 0; j < C::NJ; ++j) {
                    const int c = n0 + 64 * wn + 16 * j + 4 * g;
                    if (c >= a.N) continue;
                    if (a.Cf) {
                        *reinterpret_cast<v4f *>(a.Cf + (size_t)(pos0 + r) * a.ldc + c) = acc[i][j];
                        continue;
                    }
                    v2i pk;
                    pk[0] = (int)((uint32_t)bf16_from_f32(acc[i][j][0]) | ((uint32_t)bf16_from_f32(acc[i][j][1]) << 16));
                    pk[1] = (int)((uint32_t)bf16_from_f32(acc[i][j][2]) | ((uint32_t)bf16_from_f32(acc[i][j][3]) << 16));
                    *reinterpret_cast<v2i *>(a.Cy + (size_t)(pos0 + r) * a.ldc + c) = pk;
                }
            }
        }
    };

    // ---- stream-K fix-up of an item this block holds only part of ----
    // Partial tiles are written with system-scope stores (through the XCD's
    // L2) and read with system-scope loads (around it), so the item counter's
    // agent-scope atomic is the only synchronization: the L2s of the other
    // XCDs never need a write-back or an invalidation.
    auto block_of = [&](int s) -> int { return (int)(((int64_t)(s + 1) * G - 1) / W); };
    auto slot_of = [&](int bb, int it) -> int {
        return 2 * bb + ((int)((int64_t)bb * W / G) / KB == it ? 0 : 1);
    };
    auto fixup = [&](int it, const v4f (&acc)[C::MI][C::NJ]) {
        constexpr int PF = C::MI * C::NJ * 4;                    // floats per thread
        const int bf = block_of(it * KB), bl = block_of((it + 1) * KB - 1);
        float *mine = a.part + (size_t)slot_of(b, it) * (PF * kNT);
#pragma unroll
        for (int i = 0; i < C::MI; ++i)
#pragma unroll
            for (int j = 0; j < C::NJ; ++j)
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    __hip_atomic_store(mine + ((i * C::NJ + j) * 4 + v) * kNT + tid, acc[i][j][v], __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_SYSTEM);
        wait_vm<0>();             // this thread's partial has reached memory
        __syncthreads();          // ... every thread's
        if (tid == 0) {
            const int old = __hip_atomic_fetch_add(a.cnt + it, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            last_flag = old == bl - bf;
        }
        __syncthreads();
        if (!last_flag) return;
        v4f tot[C::MI][C::NJ];
#pragma unroll
        for (int i = 0; i < C::MI; ++i)
#pragma unroll
            for (int j = 0; j < C::NJ; ++j) tot[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
        for (int bb = bf; bb <= bl; ++bb) {
            const float *pp = a.part + (size_t)slot_of(bb, it) * (PF * kNT);
#pragma unroll
            for (int i = 0; i < C::MI; ++i)
#pragma unroll
                for (int j = 0; j < C::NJ; ++j)
#pragma unroll
                    for (int v = 0; v < 4; ++v)
                        tot[i][j][v] += bb == b ? acc[i][j][v]
                                                : __hip_atomic_load(pp + ((i * C::NJ + j) * 4 + v) * kNT + tid,
                                                                    __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        }
        epilogue(it - it0, tot);
    };

    // ---- main loop ----
    v4f acc[C::MI][C::NJ], accF[C::MI][C::NJ];
#pragma unroll
    for (int i = 0; i < C::MI; ++i)
#pragma unroll
        for (int j = 0; j < C::NJ; ++j) accF[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
    const bool first_split = s0 > it0 * KB || s1 < (it0 + 1) * KB;
    const bool last_split = s1 < (it1 + 1) * KB || s0 > it1 * KB;

#pragma unroll
    for (int j = 0; j < C::NST - 1; ++j) issue(s0 + j);

    int li = 0, kb = s0 % KB;                        // compute side position
    for (int s = s0; s < s1; ++s) {
        wait_vm<(C::NST - 2) * C::PER_STAGE>();  // this wave's loads of step s landed
        __syncthreads();                          // ... and every wave's; stage (s-1) % NST is free
        issue(s + C::NST - 1);
        if (s == s0) XS_TRACE(2);
        if (s == s0 || kb == 0) {
#pragma unroll
            for (int i = 0; i < C::MI; ++i)
#pragma unroll
                for (int j = 0; j < C::NJ; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
        }
        const uint8_t *sA = smem + (s % C::NST) * C::STAGE;
        const uint8_t *sW = sA + C::A_BYTES;
        // Operand layout of v_mfma_*_16x16x128_f8f6f4: an FP8 operand's lane
        // 16g + r holds row r with K bytes [16g, 16g+16) and [64+16g, 64+16g+16)
        // (LDS chunks g, g+4 of a 128-wide slice); an FP4 operand's lane holds K
        // elements [32g, 32g+32), chunk g of the slice's 64 bytes, and the e8m0
        // scale of (row r, 32-wide block b) comes from lane 16b + r.
        // Weights are operand A, tokens operand B: lane 16g + r of the result
        // holds token r and weight rows 4g..4g+3 of the subtile.
        if (FP4) {
            // scale buffer of step s: rows of 16 bytes = [step parity][slice][4 x 32-K block]
            const uint32_t *scw = reinterpret_cast<const uint32_t *>(smem + C::SC_OFF + ((s >> 1) & 1) * C::SC_BUF);
            const int hw = (s & 1) * 2;
#pragma unroll
            for (int u = 0; u < 2; ++u) {      // two 128-wide slices per step
                v8i xf[C::MI];
                int sx[C::MI];
#pragma unroll
                for (int i = 0; i < C::MI; ++i) {
                    const int r = 16 * i + l16;
                    const uint8_t *rp = sA + r * 256;
                    xf[i] = cat(*reinterpret_cast<const v4i *>(rp + swz16(r, 8 * u + g) * 16),
                                *reinterpret_cast<const v4i *>(rp + swz16(r, 8 * u + g + 4) * 16));
                    sx[i] = (int)((scw[4 * (256 + r) + hw + u] >> (8 * g)) & 0xffu);
                }
#pragma unroll
                for (int j = 0; j < C::NJ; ++j) {
                    const int vr = 64 * wave + 16 * j + l16;
                    const v4i b4 = *reinterpret_cast<const v4i *>(sW + vr * 128 + swz8(vr, 4 * u + g) * 16);
                    const v8i wf = v8i{b4[0], b4[1], b4[2], b4[3], 0, 0, 0, 0};
                    const int sw = (int)((scw[4 * vr + hw + u] >> (8 * g)) & 0xffu);
#pragma unroll
                    for (int i = 0; i < C::MI; ++i)
                        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(wf, xf[i], acc[i][j], 4, 0, 0, sw, 0,
                                                                                    sx[i]);
                }
            }
        } else {
            const float *sS = reinterpret_cast<const float *>(sA + C::SA_OFF);
            const float *sBk = reinterpret_cast<const float *>(sA + C::SB_OFF);
            const float sb0 = GATEUP ? sBk[0] : sBk[wave >> 1];
            const float sb1 = GATEUP ? sBk[1] : sb0;
            v8i xf[C::MI];
            float c0[C::MI], c1[C::MI];
#pragma unroll
            for (int i = 0; i < C::MI; ++i) {
                const int r = 16 * i + l16;
                const uint8_t *rp = sA + r * 128;
                xf[i] = cat(*reinterpret_cast<const v4i *>(rp + swz8(r, g) * 16),
                            *reinterpret_cast<const v4i *>(rp + swz8(r, g + 4) * 16));
                const float sx = sS[r];
                c0[i] = sx * sb0;
                c1[i] = sx * sb1;
            }
#pragma unroll
            for (int j = 0; j < C::NJ; ++j) {
                const int vr = 64 * wave + 16 * j + l16;
                const uint8_t *rp = sW + vr * 128;
                const v8i wf = cat(*reinterpret_cast<const v4i *>(rp + swz8(vr, g) * 16),
                                   *reinterpret_cast<const v4i *>(rp + swz8(vr, g + 4) * 16));
#pragma unroll
                for (int i = 0; i < C::MI; ++i) {
                    const v4f pr = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                        wf, xf[i], v4f{0.f, 0.f, 0.f, 0.f}, 0, 0, 0, 0, 0, 0);
                    const float c = (GATEUP && (j & 1)) ? c1[i] : c0[i];
#pragma unroll
                    for (int v = 0; v < 4; ++v) acc[i][j][v] = __builtin_fmaf(pr[v], c, acc[i][j][v]);
                }
            }
        }
        if (kb == KB - 1 || s == s1 - 1) {            // end of this block's part of the item
            const int it = it0 + li;
            if (it * KB >= s0 && (it + 1) * KB <= s1) {
                epilogue(li, acc);
            } else if (it == it0 && it0 != it1) {
#pragma unroll
                for (int i = 0; i < C::MI; ++i)
#pragma unroll
                    for (int j = 0; j < C::NJ; ++j) accF[i][j] = acc[i][j];
            }
        }
        if (++kb == KB) {
            kb = 0;
            ++li;
        }
    }
    XS_TRACE(3);
    wait_vm<0>();
    XS_TRACE(4);
    if (first_split && it0 != it1) fixup(it0, accF);
    if (last_split) fixup(it1, acc);
    XS_TRACE(5);
}

int g_cus = 0;

int cu_count()
{
    if (g_cus == 0) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) == hipSuccess && hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
            g_cus = n;
        else
            g_cus = 256;
    }
    return g_cus;
}

// Blocks: one per CU, more when a block would hold more than MAXIT items.
int stream_grid(int64_t items_max, int maxit)
{
    const int64_t g = cu_count();
    const int64_t need = (items_max + maxit - 3) / (maxit - 2);   // items per block <= maxit
    return (int)(g > need ? g : need);
}

template <int BM, bool GATEUP, bool FP4>
int launch_stream_one(const GemmArgs &a, int64_t items_max, hipStream_t st)
{
    using C = SCfg<BM, FP4>;
    auto fn = moe_gemm_stream_kernel<BM, GATEUP, FP4>;
    static bool attr_set = false;
    if (!attr_set) {
        XS_HIP(hipFuncSetAttribute((const void *)fn, hipFuncAttributeMaxDynamicSharedMemorySize, C::SMEM));
        attr_set = true;
    }
    fn<<<dim3((unsigned)stream_grid(items_max, C::MAXIT)), dim3(kNT), C::SMEM, st>>>(a);
    XS_LAUNCH_CHECK();
    return XS_OK;
}

}  // namespace

int stream_blocks() { return cu_count(); }

// (MXFP4 also needs K % 512 == 0 for both GEMMs: the scale pairs of steps
// must not straddle an item.)
bool stream_fits(int bm, bool fp4, int64_t tiles_max, int64_t rows_max)
{
    const bool bm_ok = fp4 ? (bm == 16 || bm == 32 || bm == 64) : (bm == 16 || bm == 32);
    return bm_ok && tiles_max < 32768 && rows_max < 65536;   // row tokens are kept as 16-bit in LDS
}

int64_t stream_items(bool gateup, int N, int64_t tiles_max) { return tiles_max * slabs_of(gateup, N); }

size_t stream_part_bytes(int64_t items_max, int, int bm)
{
    // two partial tiles per block (its first and last item may be split)
    return (size_t)2 * stream_grid(items_max, 30) * kNT * (bm / 16) * 4 * 16;
}

int launch_gemm_stream(const GemmArgs &a, bool gateup, bool fp4, int tiles_max, int64_t rows_max, hipStream_t st)
{
    XS_REQUIRE(a.K % (fp4 ? 512 : 128) == 0 && a.K >= 128 && a.tile_tab && a.offsets && a.part && a.cnt,
               "stream GEMM: bad arguments");
    XS_REQUIRE(a.N % 128 == 0, "shape mismatch: N must be a multiple of 128");
    XS_REQUIRE((int64_t)(gateup ? 2 * a.N : a.N) * a.K < ((int64_t)1 << 32), "expert weights exceed 4 GB");
    if (tiles_max <= 0) return XS_OK;
    const int64_t items = stream_items(gateup, a.N, tiles_max);
    XS_REQUIRE(items * (a.K / 128) < ((int64_t)1 << 31) && stream_fits(a.bm, fp4, tiles_max, rows_max),
               "stream GEMM: launch exceeds the kernel's tables");
    GemmArgs b = a;
    const char *grp = getenv("XS_STREAM_GROUPED");   // 0: stream-K partition (measurements)
    b.xcd_order = !(grp && grp[0] == '0');
#define XS_S(BMV, FP)                                                                                   \
    return gateup ? launch_stream_one<BMV, true, FP>(b, items, st) : launch_stream_one<BMV, false, FP>(b, items, st)
    if (fp4) {
        if (a.bm == 16) XS_S(16, true);
        if (a.bm == 32) XS_S(32, true);
        XS_S(64, true);
    }
    if (a.bm == 16) XS_S(16, false);
    XS_S(32, false);
#undef XS_S
}

}  // namespace xs

#ifdef XS_STREAM_TRACE
extern "C" int xs_stream_trace_read(void *dst)
{
    return hipMemcpyFromSymbol(dst, HIP_SYMBOL(xs::g_stream_trace), sizeof(xs::g_stream_trace)) == hipSuccess ? 0 : 1;
}
#endif
