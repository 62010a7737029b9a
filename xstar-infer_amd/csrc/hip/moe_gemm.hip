// moe_gemm.hip -- grouped block-scaled GEMMs for the MoE experts on gfx950.
//
// Nearest reference code: gemm_silu_and_mul_kernel (xstar_cpp/src/ops/mlp.cu:52-200;
// paired gate/up tiles sharing one A tile, SwiGLU in f32 with one downcast)
// and gemm_kernel (xstar_cpp/src/ops/gemm.cu:41-210).  Those are SIMT f32
// kernels on 32x32 tiles; here every expert is an FP8 (or MXFP4) MFMA GEMM:
//
//   * rows of one expert are contiguous positions of the permutation; a block
//     owns BM of them and a 256-wide slab of output columns;
//   * K advances 128 at a time (one FP8 scale block).  Operand tiles move
//     global -> LDS with global_load_lds_dwordx4 (no VGPR staging) into a ring
//     of NST stages, issued NST-1 steps ahead of use; 16-byte chunks are
//     XOR-swizzled per row so the MFMA operand reads are bank-conflict free;
//   * FP8: each 16x16x128 MFMA (v_mfma_f32_16x16x128_f8f6f4) yields the
//     partial sum of one 128-K block, folded into the f32 accumulator with the
//     product of the activation row scale and the weight block scale;
//   * MXFP4: v_mfma_scale_f32_16x16x128_f8f6f4 applies the per-32 e8m0 scales
//     of both operands in hardware and accumulates across all of K;
//   * gate_up: the 256 columns are 128 gate rows + the matching 128 up rows of
//     W13 (interleaved per 16-column subtile so one wave holds matching pairs);
//     the epilogue computes silu(g)*u in f32 and re-quantizes the activation
//     for the down GEMM (FP8 1x128, or MXFP8 1x32 for FP4 experts);
//   * down: the epilogue writes bf16 rows (weighted combine runs after).
#include "moe_gemm.hpp"

namespace xs {

template <int BM, bool FP4>
struct Cfg {
    // 8 waves (two per SIMD, so one wave's LDS latency hides behind the other's
    // MFMAs) for tall tiles; 4 for the short decode tiles.
    static constexpr int NW = BM >= 64 ? 8 : 4;
    static constexpr int NT = 64 * NW;          // threads
    static constexpr int WM = NW / 4;
    static constexpr int WN = 4;
    static constexpr int TM = BM / WM;          // wave rows
    static constexpr int TN = 256 / WN;         // wave columns
    static constexpr int MI = TM / 16;
    static constexpr int NJ = TN / 16;
    // A K step is 128 wide for FP8 and 256 wide for MXFP4, so every weight row
    // is read as whole 128-byte lines (a 64-byte half-line step fetched the
    // streamed lines twice).
    static constexpr int KSTEP = FP4 ? 256 : 128;
    static constexpr int NST = FP4 ? (BM <= 16 ? 4 : (BM <= 64 ? 3 : 2)) : (BM <= 32 ? 4 : 3);   // LDS ring stages
    static constexpr int AROW = FP4 ? 256 : 128;                 // A bytes per row per K step (FP8 / MXFP8)
    static constexpr int BROW = 128;                             // B bytes per row per K step
    static constexpr int A_BYTES = BM * AROW;
    static constexpr int B_BYTES = 256 * BROW;
    static constexpr int SA_BYTES = FP4 ? 1024 : 512;            // row scales: 128 f32, or [2][128] x 4 e8m0
    static constexpr int SB_BYTES = FP4 ? 2048 : 0;              // MXFP4 column scales: [2][256] x 4 e8m0
    static constexpr int STAGE = A_BYTES + B_BYTES + SA_BYTES + SB_BYTES;
    static constexpr int A_INSTR = A_BYTES / 1024;               // 1 KB per wave-wide DMA
    static constexpr int NA_W = A_INSTR >= NW ? A_INSTR / NW : 1; // per wave (dummies pad)
    static constexpr int NB_W = B_BYTES / 1024 / NW;
    static constexpr int NS_W = FP4 ? 4 : 1;                     // row-scale (+ column-scale) dwords
    static constexpr int PER_STAGE = NA_W + NB_W + NS_W;         // DMA instructions per wave per stage
    static constexpr int TRASH = 1024;                           // target of padding DMAs
};

// LDS row swizzles: 16-byte chunk c of row r lives at physical chunk c ^ f(r).
__device__ __forceinline__ int swz8(int r, int c) { return c ^ ((r >> 1) & 7); }   // 128-byte rows
__device__ __forceinline__ int swz16(int r, int c) { return c ^ (r & 15); }        // 256-byte rows

__device__ __forceinline__ v8i cat(v4i a, v4i b) { return v8i{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]}; }

__device__ __forceinline__ uint32_t lds_off(const void *p)
{
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

// Wave-wide DMA global -> LDS: lane i's 16 (or 4) bytes land at lds + 16*i (4*i).
// The LDS base goes through M0 and must be wave-uniform.
// M0 is written only inside these statements; compiled kernels here use M0 for
// nothing else.
// Wait state inside the asm (the compiler's hazard checks do not look into an
// asm string): an LDS DMA that reads M0 needs one after the SALU write of M0.
__device__ __forceinline__ void dma16(const void *g, uint32_t lds)
{
    const uint32_t s = __builtin_amdgcn_readfirstlane(lds);
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(s) : "memory");
}
// The same with the non-temporal hint: weights streamed once (decode tiles)
// should not displace reused lines, and the hint raises HBM streaming
// throughput of these DMAs from ~6.3 to ~7 TB/s on MI355X (but lengthens
// latency: launches with fewer blocks than CUs keep the plain loads).
__device__ __forceinline__ void dma16_nt(const void *g, uint32_t lds)
{
    const uint32_t s = __builtin_amdgcn_readfirstlane(lds);
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(g), "s"(s) : "memory");
}
__device__ __forceinline__ void dma4(const void *g, uint32_t lds)
{
    const uint32_t s = __builtin_amdgcn_readfirstlane(lds);
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(g), "s"(s) : "memory");
}
template <int N>
__device__ __forceinline__ void wait_vmcnt()
{
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// The tile of blockIdx.y from the tile table (entry 0: {tiles, shared tiles},
// then {expert, first position, rows}, shared tiles first): a launch over the
// shared segment only, the routed experts only, or both.
__device__ __forceinline__ bool find_tile(const GemmArgs &a, int &e, int &pos0, int &rows)
{
    const int4 *tab = reinterpret_cast<const int4 *>(a.tile_tab);
    const int4 h = tab[0];
    int lo = 0, hi = h.x;
    if (a.e_lo >= a.E) hi = h.y;          // shared segment only
    else if (a.e_hi <= a.E) lo = h.y;     // routed experts only
    const int i = lo + (int)blockIdx.y;
    if (i >= hi) return false;
    const int4 d = tab[1 + i];
    e = d.x;
    pos0 = d.y;
    rows = d.z;
    return rows > 0;
}

template <int BM, bool GATEUP, bool FP4>
__global__ __launch_bounds__(BM >= 64 ? 512 : 256) void moe_gemm_kernel(GemmArgs a)
{
    using S = Cfg<BM, FP4>;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int KB = a.K / 128;
    uint8_t *trash = smem + S::NST * S::STAGE;
    float *sB = reinterpret_cast<float *>(trash + S::TRASH);          // FP8: [2][KB]
    float *red = sB + 2 * KB;                                         // [WN][BM]

    int e, pos0, rows;
    if (!find_tile(a, e, pos0, rows)) return;
    if (rows > BM) rows = BM;
    const bool shared = e == a.E;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / S::WN, wn = wave % S::WN;
    const int l16 = lane & 15, g = lane >> 4;

    const int n0 = blockIdx.x * (GATEUP ? 128 : 256);
    const int Nrows = GATEUP ? 2 * a.N : a.N;                  // rows of B for this expert
    const uint8_t *Bexp = shared ? a.Bsh : a.B + (size_t)e * Nrows * (FP4 ? a.K / 2 : a.K);

    // B row of virtual column vr (0..255)
    auto brow_of = [&](int vr) -> int {
        if (GATEUP) {
            int sub = vr >> 4, w = vr & 15;
            int n = n0 + (sub >> 1) * 16 + w;
            return (sub & 1) ? a.N + n : n;
        }
        return min(n0 + vr, a.N - 1);
    };
    auto arow_of = [&](int r) -> int {
        int p = pos0 + min(r, rows - 1);
        return a.row_token ? a.row_token[p] : p;
    };

    // ---- per-lane DMA sources (fixed across K; the K offset is added per step) ----
    const uint8_t *gA[S::NA_W];
    uint32_t lA[S::NA_W];
#pragma unroll
    for (int u = 0; u < S::NA_W; ++u) {
        const int q = wave + S::NW * u;                    // wave-wide instruction index
        const int p = 64 * q + lane;                   // LDS chunk written by this lane
        const int r = FP4 ? p >> 4 : p >> 3, c = FP4 ? swz16(r, p & 15) : swz8(r, p & 7);
        const bool real = q < S::A_INSTR;
        gA[u] = a.A + (size_t)arow_of(real ? r : 0) * a.K + c * 16;
        lA[u] = real ? (uint32_t)(64 * q * 16) : 0xFFFFFFFFu;
    }
    const uint8_t *gB[S::NB_W];
#pragma unroll
    for (int u = 0; u < S::NB_W; ++u) {
        const int q = wave + S::NW * u;
        const int p = 64 * q + lane;
        if (FP4) {
            const int vr = p >> 3, c = swz8(vr, p & 7);
            gB[u] = Bexp + (size_t)brow_of(vr) * (a.K / 2) + c * 16;
        } else {
            const int vr = p >> 3, c = swz8(vr, p & 7);
            gB[u] = Bexp + (size_t)brow_of(vr) * a.K + c * 16;
        }
    }
    // row scales: waves 0/1 load rows 64w + lane (waves beyond BM target trash)
    const bool sa_real = wave * 64 < BM;
    const bool sb_real = wave < 4;            // MXFP4 column scales: 256 words = 4 waves
    const uint8_t *gSA;
    if (FP4)
        gSA = reinterpret_cast<const uint8_t *>(a.As) + (size_t)arow_of(sa_real ? wave * 64 + lane : 0) * (a.K / 32);
    else
        gSA = reinterpret_cast<const uint8_t *>(a.As) + (size_t)arow_of(sa_real ? wave * 64 + lane : 0) * KB * 4;
    const uint8_t *gSB = nullptr;
    if (FP4)
        gSB = reinterpret_cast<const uint8_t *>(a.Bs) + (size_t)e * Nrows * (a.K / 32) +
              (size_t)brow_of(sb_real ? wave * 64 + lane : 0) * (a.K / 32);

    // ---- FP8 weight block scales for the whole tile ----
    if (!FP4) {
        const float *Bsf = shared ? a.Bssh : reinterpret_cast<const float *>(a.Bs) + (size_t)e * (Nrows / 128) * KB;
        for (int q = tid; q < 2 * KB; q += S::NT) {
            int b = q / KB, kb = q % KB;
            int nb;
            if (GATEUP) nb = (b ? a.N + n0 : n0) / 128;
            else nb = min(n0 / 128 + b, a.N / 128 - 1);
            sB[q] = Bsf[(size_t)nb * KB + kb];
        }
    }

    const uint32_t smem_base = lds_off(smem);
    const uint32_t trash_lds = __builtin_amdgcn_readfirstlane(lds_off(trash));
    // Issue the DMAs of K step kb into ring stage kb % NST.  Steps past the end
    // reload the last step (the stage is never read again): counts stay uniform.
    const int KS = a.K / S::KSTEP;   // K steps
    auto issue = [&](int kb) {
        const int kk = kb < KS ? kb : KS - 1;
        const uint32_t st = __builtin_amdgcn_readfirstlane(smem_base + (uint32_t)((kb % S::NST) * S::STAGE));
#pragma unroll
        for (int u = 0; u < S::NA_W; ++u) {
            const uint32_t dst = lA[u] == 0xFFFFFFFFu ? trash_lds : st + __builtin_amdgcn_readfirstlane(lA[u]);
            dma16(gA[u] + (size_t)kk * S::AROW, dst);
        }
#pragma unroll
        for (int u = 0; u < S::NB_W; ++u)
        {
            const uint32_t d = st + S::A_BYTES + (uint32_t)((wave + S::NW * u) * 1024);
            if (a.stream_w) dma16_nt(gB[u] + (size_t)kk * S::BROW, d);
            else dma16(gB[u] + (size_t)kk * S::BROW, d);
        }
        if (FP4) {         // 8 e8m0 per row per step: two words, halves h of the scale areas
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                dma4(gSA + (size_t)kk * 8 + 4 * h, sa_real ? st + S::A_BYTES + S::B_BYTES + h * 512 + wave * 256 : trash_lds);
                dma4(gSB + (size_t)kk * 8 + 4 * h,
                     sb_real ? st + S::A_BYTES + S::B_BYTES + S::SA_BYTES + h * 1024 + wave * 256 : trash_lds);
            }
        } else {
            dma4(gSA + (size_t)kk * 4, sa_real ? st + S::A_BYTES + S::B_BYTES + wave * 256 : trash_lds);
        }
    };

    v4f acc[S::MI][S::NJ];
#pragma unroll
    for (int i = 0; i < S::MI; ++i)
#pragma unroll
        for (int j = 0; j < S::NJ; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

    __syncthreads();   // sB visible; all address loads done before the DMA stream starts
#pragma unroll
    for (int s = 0; s < S::NST - 1; ++s) issue(s);

    for (int kb = 0; kb < KS; ++kb) {
        wait_vmcnt<(S::NST - 2) * S::PER_STAGE>();   // this wave's DMAs for step kb have landed
        __syncthreads();                             // ... and every other wave's
        issue(kb + S::NST - 1);                      // refills the stage consumed at kb - 1
        const uint8_t *sa_ = smem + (kb % S::NST) * S::STAGE;
        const uint8_t *sb_ = sa_ + S::A_BYTES;
        const uint8_t *ssc = sb_ + S::B_BYTES;

        // Operand layout of v_mfma_*_16x16x128_f8f6f4 (gfx950): for an FP8
        // operand, lane 16g + r holds row r with K = [16g, 16g+16) in bytes 0..15
        // and K = [64+16g, 64+16g+16) in bytes 16..31, i.e. LDS chunks g and g+4
        // of the row; for an FP4 operand, lane 16g + r holds K = [32g, 32g+32)
        // (element 2i in the low nibble), i.e. 16-byte chunk g of the slice's 64 bytes.
        // The e8m0 scale of (row r, 32-wide K block b) is taken from lane 16b + r.
        // Pinned by the FP8 x FP4 parity tests.
        //
        // Weights are the MFMA's A operand and activations its B operand, so the
        // 16x16 result is (weight column n) x (token m): lane 16g + r holds token
        // r and columns 4g..4g+3 -- one activation scale per lane and subtile,
        // and four adjacent output columns per lane for the epilogue stores.
        v8i xfr[S::MI];   // activation fragments, one per 16-token subtile
        if (FP4) {
            // two 128-wide slices u per step: activation chunks 8u+g, 8u+g+4 of a
            // 256-byte row; weight chunk 4u+g of a 128-byte row; scale words [u][row]
            const uint32_t *sAw = reinterpret_cast<const uint32_t *>(ssc);
            const uint32_t *sBw = reinterpret_cast<const uint32_t *>(ssc + S::SA_BYTES);
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                int sx[S::MI];
#pragma unroll
                for (int i = 0; i < S::MI; ++i) {
                    const int r = wm * S::TM + 16 * i + l16;
                    v4i lo = *reinterpret_cast<const v4i *>(sa_ + r * 256 + swz16(r, 8 * u + g) * 16);
                    v4i hi = *reinterpret_cast<const v4i *>(sa_ + r * 256 + swz16(r, 8 * u + g + 4) * 16);
                    xfr[i] = cat(lo, hi);
                    sx[i] = (int)((sAw[128 * u + r] >> (8 * g)) & 0xffu);
                }
#pragma unroll
                for (int j = 0; j < S::NJ; ++j) {
                    const int vr = wn * S::TN + 16 * j + l16;
                    v4i b4 = *reinterpret_cast<const v4i *>(sb_ + vr * 128 + swz8(vr, 4 * u + g) * 16);
                    v8i wfr = v8i{b4[0], b4[1], b4[2], b4[3], 0, 0, 0, 0};
                    const int sw = (int)((sBw[256 * u + vr] >> (8 * g)) & 0xffu);
#pragma unroll
                    for (int i = 0; i < S::MI; ++i)
                        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(wfr, xfr[i], acc[i][j], 4, 0, 0,
                                                                                    sw, 0, sx[i]);
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < S::MI; ++i) {
                int r = wm * S::TM + 16 * i + l16;
                v4i lo = *reinterpret_cast<const v4i *>(sa_ + r * 128 + swz8(r, g) * 16);
                v4i hi = *reinterpret_cast<const v4i *>(sa_ + r * 128 + swz8(r, g + 4) * 16);
                xfr[i] = cat(lo, hi);
            }
            const float *sAk = reinterpret_cast<const float *>(ssc);
            // weight block scales: gate_up uses block 0 (gate) for even subtiles and
            // block 1 (up) for odd ones; down uses the wave's own 128-column block
            const float sb0 = GATEUP ? sB[kb] : sB[((wn * S::TN) >> 7) * KB + kb];
            const float sb1 = GATEUP ? sB[KB + kb] : sb0;
            float c0[S::MI], c1[S::MI];
#pragma unroll
            for (int i = 0; i < S::MI; ++i) {
                const float sx = sAk[wm * S::TM + 16 * i + l16];
                c0[i] = sx * sb0;
                c1[i] = sx * sb1;
            }
            // The partial product of subtile n is folded after MFMA n + PD has
            // been issued; the group barriers below interleave MFMAs with the
            // VALU folds so the matrix pipe and the VALU run concurrently.
            constexpr int NSUB = S::NJ * S::MI, PD = 2;
            v4f pr[PD + 1];
            v8i wfr;
#pragma unroll
            for (int n = 0; n < NSUB + PD; ++n) {
                if (n < NSUB) {
                    const int j = n / S::MI, i = n % S::MI;
                    if (i == 0) {
                        int vr = wn * S::TN + 16 * j + l16;
                        v4i lo = *reinterpret_cast<const v4i *>(sb_ + vr * 128 + swz8(vr, g) * 16);
                        v4i hi = *reinterpret_cast<const v4i *>(sb_ + vr * 128 + swz8(vr, g + 4) * 16);
                        wfr = cat(lo, hi);
                    }
                    pr[n % (PD + 1)] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                        wfr, xfr[i], v4f{0.f, 0.f, 0.f, 0.f}, 0, 0, 0, 0, 0, 0);
                }
                if (n >= PD) {
                    const int m = n - PD, j = m / S::MI, i = m % S::MI;
                    const v4f pp = pr[m % (PD + 1)];
                    const float c = (GATEUP && (j & 1)) ? c1[i] : c0[i];
#pragma unroll
                    for (int v = 0; v < 4; ++v) acc[i][j][v] = __builtin_fmaf(pp[v], c, acc[i][j][v]);
                }
            }
#pragma unroll
            for (int n = 0; n < NSUB; ++n) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // one MFMA
                __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);   // then ~5 VALU
                if ((n & 1) == 0) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // an LDS read
            }
        }
    }
    wait_vmcnt<0>();   // drain the padding DMAs before the stages are reused
    __syncthreads();

    // ------------------------------------------------------------ epilogue
    // acc[i][j][v]: token row wm*TM + 16i + l16, column 16j + 4g + v of the wave.
    if (GATEUP) {
        constexpr int NP = S::NJ / 2;     // gate/up pairs per wave
        constexpr int SROW = 144;         // staging row stride (bytes): conflict-free 4-byte writes
        float act[S::MI][NP][4];
#pragma unroll
        for (int i = 0; i < S::MI; ++i)
#pragma unroll
            for (int p = 0; p < NP; ++p)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    float gt = acc[i][2 * p][v], up = acc[i][2 * p + 1][v];
                    act[i][p][v] = gt * fast_sigmoid(gt) * up;
                }
        uint8_t *stg = smem;   // [BM][SROW] fp8 staging (the ring is free now)
        auto pack4 = [](float x0, float x1, float x2, float x3) -> uint32_t {
            return e4m3_pack2_hw(x0, x1) | (e4m3_pack2_hw(x2, x3) << 16);
        };
        if (!FP4) {
            // FP8 1x128: token amax over the block's 128 act columns (4 column
            // groups of a wave, then the WN waves of the row)
#pragma unroll
            for (int i = 0; i < S::MI; ++i) {
                float m = 0.f;
#pragma unroll
                for (int p = 0; p < NP; ++p)
#pragma unroll
                    for (int v = 0; v < 4; ++v) m = fmaxf(m, __builtin_fabsf(act[i][p][v]));
                m = fmaxf(m, __shfl_xor(m, 16, WAVE));
                m = fmaxf(m, __shfl_xor(m, 32, WAVE));
                if (g == 0) red[wn * BM + wm * S::TM + 16 * i + l16] = m;
            }
            __syncthreads();
#pragma unroll
            for (int i = 0; i < S::MI; ++i) {
                const int r = wm * S::TM + 16 * i + l16;
                float amax = 0.f;
#pragma unroll
                for (int w = 0; w < S::WN; ++w) amax = fmaxf(amax, red[w * BM + r]);
                const float inv = amax == 0.f ? 0.f : __fdiv_rn(448.0f, amax);
#pragma unroll
                for (int p = 0; p < NP; ++p) {
                    float q[4];
#pragma unroll
                    for (int v = 0; v < 4; ++v) q[v] = fminf(fmaxf(act[i][p][v] * inv, -448.f), 448.f);
                    *reinterpret_cast<uint32_t *>(stg + r * SROW + (wn * NP + p) * 16 + 4 * g) =
                        pack4(q[0], q[1], q[2], q[3]);
                }
            }
            __syncthreads();
            float *Cs = reinterpret_cast<float *>(a.Cs);
            for (int r = tid; r < rows; r += S::NT) {
                float amax = 0.f;
#pragma unroll
                for (int w = 0; w < S::WN; ++w) amax = fmaxf(amax, red[w * BM + r]);
                Cs[(size_t)(pos0 + r) * (a.N / 128) + n0 / 128] = amax == 0.f ? 1.0f : __fdiv_rn(amax, 448.0f);
            }
        } else {
            // MXFP8 1x32: a 32-column block is pairs (2q, 2q+1) of one wave
            uint8_t *Cs8 = reinterpret_cast<uint8_t *>(a.Cs);
#pragma unroll
            for (int i = 0; i < S::MI; ++i) {
                const int r = wm * S::TM + 16 * i + l16;
#pragma unroll
                for (int p = 0; p < NP; p += 2) {
                    float m = 0.f;
#pragma unroll
                    for (int v = 0; v < 4; ++v)
                        m = fmaxf(m, fmaxf(__builtin_fabsf(act[i][p][v]), __builtin_fabsf(act[i][p + 1][v])));
                    m = fmaxf(m, __shfl_xor(m, 16, WAVE));
                    m = fmaxf(m, __shfl_xor(m, 32, WAVE));
                    const int se = mx_exponent(m, 8);
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        float q[4];
#pragma unroll
                        for (int v = 0; v < 4; ++v)
                            q[v] = fminf(fmaxf(__builtin_ldexpf(act[i][p + h][v], -se), -448.f), 448.f);
                        *reinterpret_cast<uint32_t *>(stg + r * SROW + (wn * NP + p + h) * 16 + 4 * g) =
                            pack4(q[0], q[1], q[2], q[3]);
                    }
                    if (g == 0 && r < rows)
                        Cs8[(size_t)(pos0 + r) * (a.N / 32) + (n0 + (wn * NP + p) * 16) / 32] = (uint8_t)(se + 127);
                }
            }
            __syncthreads();
        }
        for (int q = tid; q < rows * 8; q += S::NT) {
            int r = q >> 3, c = q & 7;
            *reinterpret_cast<v4i *>(a.Cq + (size_t)(pos0 + r) * a.N + n0 + c * 16) =
                *reinterpret_cast<const v4i *>(stg + r * SROW + c * 16);
        }
    } else if (a.Cf) {
        // f32 rows, straight from the accumulators: a lane's 4 columns are one
        // 16-byte store (these tiles serve small batches; y is small)
#pragma unroll
        for (int i = 0; i < S::MI; ++i)
#pragma unroll
            for (int j = 0; j < S::NJ; ++j) {
                const int r = wm * S::TM + 16 * i + l16;
                const int c = n0 + wn * S::TN + 16 * j + 4 * g;
                if (r < rows && c < a.N) *reinterpret_cast<v4f *>(a.Cf + (size_t)(pos0 + r) * a.ldc + c) = acc[i][j];
            }
    } else {
        constexpr int SROW = 264;         // staging row stride (bf16 elements): conflict-free 8-byte writes
        uint16_t *stg = reinterpret_cast<uint16_t *>(smem);   // [BM][SROW] bf16
#pragma unroll
        for (int i = 0; i < S::MI; ++i)
#pragma unroll
            for (int j = 0; j < S::NJ; ++j) {
                const int r = wm * S::TM + 16 * i + l16;
                const int c = wn * S::TN + 16 * j + 4 * g;
                v2i pk;
                pk[0] = (int)((uint32_t)bf16_from_f32(acc[i][j][0]) | ((uint32_t)bf16_from_f32(acc[i][j][1]) << 16));
                pk[1] = (int)((uint32_t)bf16_from_f32(acc[i][j][2]) | ((uint32_t)bf16_from_f32(acc[i][j][3]) << 16));
                *reinterpret_cast<v2i *>(stg + r * SROW + c) = pk;
            }
        __syncthreads();
        const int ncols = min(256, a.N - n0);
        for (int q = tid; q < rows * 32; q += S::NT) {
            int r = q >> 5, c = q & 31;
            if (c * 8 < ncols)
                *reinterpret_cast<v4i *>(a.Cy + (size_t)(pos0 + r) * a.ldc + n0 + c * 8) =
                    *reinterpret_cast<const v4i *>(stg + r * SROW + c * 8);
        }
    }
}

template <int BM, bool GATEUP, bool FP4>
static size_t gemm_smem_bytes(int K)
{
    using S = Cfg<BM, FP4>;
    const size_t KB = (size_t)K / 128;
    size_t b = (size_t)S::NST * S::STAGE + S::TRASH + 4 * 2 * KB + 4 * (size_t)S::WN * BM;
    size_t epi = GATEUP ? (size_t)BM * 144 : (size_t)BM * 528;
    if (epi > (size_t)S::NST * S::STAGE) b += epi;   // staging reuses the ring when it fits
    return b;
}

template <int BM, bool GATEUP, bool FP4>
static int launch_one(const GemmArgs &a, int grid_y, hipStream_t st)
{
    if (FP4 && a.K % 256 != 0) return set_error(XS_ERR_UNSUPPORTED, "MXFP4 GEMM: K=%d is not a multiple of 256", a.K);
    size_t smem = gemm_smem_bytes<BM, GATEUP, FP4>(a.K);
    if (smem > 160 * 1024) return set_error(XS_ERR_UNSUPPORTED, "K=%d needs %zu bytes of LDS", a.K, smem);
    auto fn = moe_gemm_kernel<BM, GATEUP, FP4>;
    static bool attr_set = false;
    if (!attr_set) {
        XS_HIP(hipFuncSetAttribute((const void *)fn, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
        attr_set = true;
    }
    int grid_x = GATEUP ? a.N / 128 : (a.N + 255) / 256;
    if (grid_y <= 0) return XS_OK;
    GemmArgs b = a;
    b.stream_w = (int64_t)grid_x * grid_y >= 256;
    fn<<<dim3((unsigned)grid_x, (unsigned)grid_y), dim3(Cfg<BM, FP4>::NT), smem, st>>>(b);
    XS_LAUNCH_CHECK();
    return XS_OK;
}

int launch_gemm(const GemmArgs &a, bool gateup, bool fp4, int grid_y, hipStream_t st)
{
#define XS_G(BMV)                                                                           \
    case BMV:                                                                               \
        if (gateup) return fp4 ? launch_one<BMV, true, true>(a, grid_y, st)                 \
                               : launch_one<BMV, true, false>(a, grid_y, st);               \
        return fp4 ? launch_one<BMV, false, true>(a, grid_y, st)                            \
                   : launch_one<BMV, false, false>(a, grid_y, st);
    switch (a.bm) {
        XS_G(16)
        XS_G(32)
        XS_G(64)
        XS_G(128)
    default:
        return set_error(XS_ERR_INVALID, "unsupported tile rows %d", a.bm);
    }
#undef XS_G
}

// --------------------------------------------------------------- combine
// out[t] = [residual[t] +] y_shared[t] + sum_j w[t,j] * y[inv[t*k+j]]
// (f32, slot order, residual added last, one cast)
// One block per token, one pass over the row when H <= 8 * blockDim (the
// launch picks blockDim = H / 8 up to 512), so all k + 1 row loads of a thread
// are in flight together.
// The expert outputs are read exactly once: non-temporal loads (measured at
// C3: combine 105 -> 93 us).
// 8 f32 values read once (the per-slot rows are not read again)
__device__ __forceinline__ void load8_nt(const float *p, float *v)
{
    const v4f a = __builtin_nontemporal_load(reinterpret_cast<const v4f *>(p));
    const v4f b = __builtin_nontemporal_load(reinterpret_cast<const v4f *>(p + 4));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[i] = a[i];
        v[4 + i] = b[i];
    }
}

// One block per token, 8 columns per thread.  The top-k is a template
// argument, so every row's loads are issued before the first add (the gather
// is latency-bound otherwise).  Sum order: shared row, then slots 0 .. k-1 as
// acc + w_j * y_j (each product and sum rounded), then the residual; one cast.
template <typename OutT, int K>
__global__ __launch_bounds__(512) void combine_kernel(const float *__restrict__ y,
                                                      const int32_t *__restrict__ inv,
                                                      const float *__restrict__ w, int H,
                                                      int64_t shared_base, int has_shared,
                                                      const OutT *residual, OutT *out)
{
#pragma clang fp contract(off)
    const int t = blockIdx.x;
    int pos[K];
    float wt[K];
#pragma unroll
    for (int j = 0; j < K; ++j) {
        pos[j] = inv[(size_t)t * K + j];
        wt[j] = w[(size_t)t * K + j];
    }
    for (int c = threadIdx.x * 8; c < H; c += blockDim.x * 8) {
        float acc[8], v[K][8], r[8];
        if (has_shared) load8_nt(y + (size_t)(shared_base + t) * H + c, acc);
        else
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[i] = 0.f;
#pragma unroll
        for (int j = 0; j < K; ++j) load8_nt(y + (size_t)pos[j] * H + c, v[j]);
        if (residual) load8(residual + (size_t)t * H + c, r);   // out may alias residual
#pragma unroll
        for (int j = 0; j < K; ++j)
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[i] = acc[i] + wt[j] * v[j][i];   // no contraction (pragma above)
        if (residual)
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[i] = r[i] + acc[i];
        store8(out + (size_t)t * H + c, acc);
    }
}

template <typename OutT, int K>
static void launch_combine_k(int k, dim3 grid, dim3 block, hipStream_t st, const float *y, const int32_t *inv,
                             const float *w, int H, int64_t shared_base, int has_shared, const void *residual,
                             void *out)
{
    if constexpr (K > 1) {
        if (k < K) {
            launch_combine_k<OutT, K - 1>(k, grid, block, st, y, inv, w, H, shared_base, has_shared, residual, out);
            return;
        }
    }
    combine_kernel<OutT, K><<<grid, block, 0, st>>>(y, inv, w, H, shared_base, has_shared,
                                                    (const OutT *)residual, (OutT *)out);
}

int launch_combine(const float *y, const int32_t *inv, const float *w, int64_t T, int64_t k,
                   int64_t H, int64_t shared_base, int has_shared, void *out, int out_dtype,
                   hipStream_t st, const void *residual)
{
    if (T == 0) return XS_OK;
    if (k < 1 || k > 16) return set_error(XS_ERR_INVALID, "combine: top_k %lld outside [1, 16]", (long long)k);
    const int nt = (int)(H / 8 < 64 ? 64 : (H / 8 > 512 ? 512 : (H / 8 + 63) / 64 * 64));
    if (out_dtype == XS_BF16)
        launch_combine_k<uint16_t, 16>((int)k, dim3((unsigned)T), dim3(nt), st, y, inv, w, (int)H, shared_base,
                                       has_shared, residual, out);
    else
        launch_combine_k<float, 16>((int)k, dim3((unsigned)T), dim3(nt), st, y, inv, w, (int)H, shared_base,
                                    has_shared, residual, out);
    XS_LAUNCH_CHECK();
    return XS_OK;
}

}  // namespace xs
