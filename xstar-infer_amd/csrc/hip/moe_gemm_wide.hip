// moe_gemm_wide.hip -- grouped FP8 block-scaled expert GEMMs on 192 x 256 tiles
// (gfx950), the prefill path of the MoE layer.
//
// Nearest reference code: gemm_silu_and_mul_kernel (xstar_cpp/src/ops/mlp.cu:52-200)
// and gemm_kernel (xstar_cpp/src/ops/gemm.cu:41-210); numerics as the FP8 tiles of
// moe_gemm.hip (f32 accumulation of each 128-K block, scaled by the activation row
// scale times the weight block scale; SwiGLU in f32; 1x128 FP8 requantization).
//
// Structure, chosen for CDNA4's fetch and LDS budgets:
//   * a block owns up to 192 rows of one expert and a 256-column weight slab
//     (gate_up: 128 gate + the matching 128 up rows; down: 256 rows of W2), so
//     each K step moves 56 KB into the CU for 12.6 MFLOP -- 37 B/clk per CU at
//     the MFMA rate, about half of what L2 delivers to a CU (taller tiles would
//     need more than the 256 VGPRs of two waves per SIMD);
//   * 8 waves split the slab: wave w owns 32 weight rows for ALL of the
//     block's tokens.  Its weights are private, so they go global -> VGPR with
//     no LDS round trip; the activation rows, shared by all 8 waves, go
//     global -> LDS by DMA (global_load_lds_dwordx4) into a ring;
//   * v_mfma_f32_32x32x64_f8f6f4 with weights as operand A (rows 0..15 gate,
//     16..31 up for gate_up) and 32 tokens as operand B: a lane's 16 results
//     belong to one token, and its gate and matching up values sit in the same
//     lane, so SwiGLU and the requantization are register epilogues;
//   * the main loop is instantiated per number NS of 32-row token subtiles
//     (1..6), so a short expert segment moves and multiplies only the rows it
//     has, and uses the registers the missing accumulators free for a deeper
//     weight prefetch (the short tiles are bandwidth bound);
//   * every vector-memory load of the loop is issued from inline asm and the
//     waits are explicit s_waitcnt vmcnt(N) with the exact count of loads
//     allowed in flight (the compiler's own accounting would not see the DMAs).
#include "moe_gemm.hpp"

namespace xs {
namespace {

constexpr int kNW = 8;               // waves per block
constexpr int kNT = 64 * kNW;        // threads
constexpr int kBM = 192;             // tile rows (6 subtiles of 32: the register budget of 2 waves/SIMD)
constexpr int kRing = 136 * 1024;    // LDS bytes of the activation ring
constexpr int kTrash = 1024;         // LDS target of padding DMAs

typedef float v16f __attribute__((ext_vector_type(16)));

template <int NS>
struct WCfg {
    static constexpr int A_BYTES = NS * 32 * 128;          // activation rows of one K step
    static constexpr int NSA = (NS + 1) / 2;               // 64-row scale DMAs per step
    static constexpr int S_BYTES = 256 * NSA;
    static constexpr int STAGE = A_BYTES + S_BYTES;
    static constexpr int NST = kRing / STAGE >= 8 ? 8 : kRing / STAGE;   // ring stages
    static constexpr int A_INSTR = 4 * NS;                 // 1 KB DMAs per step
    static constexpr int NA = (A_INSTR + kNW - 1) / kNW;   // per wave (padding DMAs even it out)
    static constexpr int NWB = NS <= 2 ? 8 : 4;            // weight buffers (divide K/128)
    static constexpr int PER_STEP = 4 + NA + 1;            // loads per wave per step: W, A, row scales
    // At the top of step kb this wave needs W(kb) (issued NWB-1 iterations
    // earlier, followed by that iteration's A/scale DMAs) and A(kb) (issued
    // NST-1 iterations earlier).  Loads retire in order, so waiting until at
    // most X are outstanding retires both.
    static constexpr int XW = NA + 1 + (NWB - 2) * PER_STEP;
    static constexpr int XA = (NST - 2) * PER_STEP;
    static constexpr int X = XW < XA ? XW : XA;
    static constexpr int PRO = (NST > NWB ? NST : NWB) - 1; // prologue iterations
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
__device__ __forceinline__ void dma16(const uint8_t *sbase, uint32_t voff, uint32_t lds)
{
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(lds) : "memory");
}
__device__ __forceinline__ void dma4(const uint8_t *sbase, uint32_t voff, uint32_t lds)
{
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(sbase), "s"(lds) : "memory");
}

// The four 16-byte weight chunks of one K step of this lane's row:
// K bytes 16h + {0, 32, 64, 96} (h = lane / 32).  Results arrive
// asynchronously; wait_w() orders their use after the matching s_waitcnt.
__device__ __forceinline__ void load_w(v4i (&w)[4], const uint8_t *sbase, uint32_t voff)
{
    asm volatile(
        "global_load_dwordx4 %0, %4, %5\n\t"
        "global_load_dwordx4 %1, %4, %5 offset:32\n\t"
        "global_load_dwordx4 %2, %4, %5 offset:64\n\t"
        "global_load_dwordx4 %3, %4, %5 offset:96"
        : "+v"(w[0]), "+v"(w[1]), "+v"(w[2]), "+v"(w[3])
        : "v"(voff), "s"(sbase)
        : "memory");
}
template <int N>
__device__ __forceinline__ void wait_w(v4i (&w)[4])
{
    asm volatile("s_waitcnt vmcnt(%4)" : "+v"(w[0]), "+v"(w[1]), "+v"(w[2]), "+v"(w[3]) : "n"(N) : "memory");
}
template <int N>
__device__ __forceinline__ void wait_vm()
{
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

__device__ __forceinline__ bool find_tile(const GemmArgs &a, int &e, int &m0, int &rows)
{
    const int i = a.tile_off[a.e_lo] + (int)blockIdx.y;
    if (i >= a.tile_off[a.e_hi]) return false;
    int lo = a.e_lo, hi = a.e_hi - 1;   // largest e with tile_off[e] <= i
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (a.tile_off[mid] <= i) lo = mid; else hi = mid - 1;
    }
    e = lo;
    m0 = (i - a.tile_off[e]) * kBM;
    rows = a.offsets[e + 1] - a.offsets[e] - m0;
    return rows > 0;
}

struct TileCtx {
    int e, rows, pos0, KB, n0, wave, lane, r, h;
    const uint8_t *Bexp;       // this expert's weight rows
    const float *sB;           // LDS: weight block scales [2][KB]
    uint8_t *smem;
};

template <bool GATEUP, int NS>
__device__ __forceinline__ void run_tile(const GemmArgs &a, const TileCtx &t)
{
    using C = WCfg<NS>;
    const int KB = t.KB, lane = t.lane, wave = t.wave, r = t.r, h = t.h;
    uint8_t *smem = t.smem;
    uint8_t *trash = smem + kRing;
    const uint32_t ring_lds = lds_addr(smem), trash_lds = lds_addr(trash);

    auto token_of = [&](int row) -> int {
        const int p = t.pos0 + min(row, t.rows - 1);
        return a.row_token ? a.row_token[p] : p;
    };

    // ---- per-lane DMA source offsets (the K offset goes into the scalar base) ----
    uint32_t oA[C::NA];
#pragma unroll
    for (int u = 0; u < C::NA; ++u) {
        const int q = wave + kNW * u;                 // 1 KB DMA instruction of the step
        const int row = q < C::A_INSTR ? 8 * q + (lane >> 3) : 0;
        oA[u] = (uint32_t)token_of(row) * (uint32_t)a.K + (uint32_t)(swz8(row, lane & 7) * 16);
    }
    const bool sa_real = wave < C::NSA;
    const uint32_t oS = (uint32_t)token_of(sa_real ? 64 * wave + lane : 0) * (uint32_t)(KB * 4);
    // this lane's weight row: A-operand row r of the wave's 32
    int wrow;
    if (GATEUP) wrow = (r < 16 ? 0 : a.N) + t.n0 + 16 * wave + (r & 15);
    else wrow = t.n0 + 32 * wave + r;
    const uint32_t oW = (uint32_t)wrow * (uint32_t)a.K + 16 * h;
    const uint8_t *gS = reinterpret_cast<const uint8_t *>(a.As);

    auto issue_a = [&](int kb) {   // A rows + row scales of step kb into its ring stage
        const int kk = kb < 0 ? 0 : (kb < KB ? kb : KB - 1);
        const bool live = kb >= 0;
        const uint32_t st = ring_lds + (uint32_t)((live ? kb % C::NST : 0) * C::STAGE);
#pragma unroll
        for (int u = 0; u < C::NA; ++u) {
            const int q = wave + kNW * u;
            dma16(a.A + (size_t)kk * 128, oA[u], (live && q < C::A_INSTR) ? st + 1024 * q : trash_lds);
        }
        dma4(gS + (size_t)kk * 4, oS, (live && sa_real) ? st + C::A_BYTES + 256 * wave : trash_lds);
    };

    v4i wb[C::NWB][4];
#pragma unroll
    for (int b = 0; b < C::NWB; ++b)
#pragma unroll
        for (int j = 0; j < 4; ++j) wb[b][j] = v4i{0, 0, 0, 0};

    v16f acc[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[s][v] = 0.f;

    __syncthreads();   // weight scale table visible; previous users of the ring done
    // prologue: the steady-state issue pattern for iterations -PRO .. -1
#pragma unroll
    for (int j = -C::PRO; j < 0; ++j) {
        const int kw = j + C::NWB - 1;
        load_w(wb[((kw % C::NWB) + C::NWB) % C::NWB], t.Bexp + (size_t)(kw < 0 ? 0 : (kw < KB ? kw : KB - 1)) * 128, oW);
        issue_a(j + C::NST - 1);
    }

    const int wblk = GATEUP ? 0 : (wave >> 2);       // down: the wave's 128-row scale block
    for (int kb0 = 0; kb0 < KB; kb0 += C::NWB) {
#pragma unroll
        for (int u = 0; u < C::NWB; ++u) {   // K/128 is a multiple of NWB: no guards
            const int kb = kb0 + u;
            {
                wait_w<C::X>(wb[u]);
                __syncthreads();                      // A(kb) of every wave landed; stage kb-1 free
                {
                    const int kw = kb + C::NWB - 1;
                    load_w(wb[(u + C::NWB - 1) % C::NWB], t.Bexp + (size_t)(kw < KB ? kw : KB - 1) * 128, oW);
                    issue_a(kb + C::NST - 1);
                }
                const uint8_t *sA = smem + (kb % C::NST) * C::STAGE;
                const float *sS = reinterpret_cast<const float *>(sA + C::A_BYTES);
                const float sb0 = t.sB[wblk * KB + kb];
                const float sb1 = GATEUP ? t.sB[KB + kb] : sb0;
                const v8i w01 = cat(wb[u][0], wb[u][1]), w23 = cat(wb[u][2], wb[u][3]);
                // One subtile at a time (the other wave of the SIMD covers the LDS
                // latency); the scheduling barrier keeps the compiler from hoisting
                // every subtile's reads to the top of the step (NS x 16 live VGPRs).
                auto read_b = [&](int s, v4i (&b)[4]) {
                    const int row = 32 * s + r;
                    const uint8_t *rp = sA + row * 128;
#pragma unroll
                    for (int j = 0; j < 4; ++j) b[j] = *reinterpret_cast<const v4i *>(rp + swz8(row, 2 * j + h) * 16);
                };
#pragma unroll
                for (int s = 0; s < NS; ++s) {
                    v4i bc[4];
                    read_b(s, bc);
                    const float sa = sS[32 * s + r];
                    v16f p = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(w01, cat(bc[0], bc[1]), v16f{}, 0, 0, 0, 0, 0, 0);
                    p = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(w23, cat(bc[2], bc[3]), p, 0, 0, 0, 0, 0, 0);
                    const float c0 = sa * sb0, c1 = sa * sb1;
#pragma unroll
                    for (int v = 0; v < 16; ++v) acc[s][v] = __builtin_fmaf(p[v], v < 8 ? c0 : c1, acc[s][v]);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        }
    }
    wait_vm<0>();      // the clamped DMAs past the last step must land before the ring is reused
    __syncthreads();

    // ------------------------------------------------------------ epilogue
    // acc[s][v]: token row 32 s + r; A-operand row 8 (v / 4) + 4 h + (v % 4).
    if (GATEUP) {
        // act feature (within the block's 128 columns) of v < 8: 16 w + 8 (v/4) + 4 h + v%4
        float *red = reinterpret_cast<float *>(smem);          // [kNW][kBM] wave amax per token
        float act[NS][8];
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            float m = 0.f;
#pragma unroll
            for (int v = 0; v < 8; ++v) {
                const float g = acc[s][v], u = acc[s][v + 8];
                act[s][v] = g * fast_sigmoid(g) * u;
                m = fmaxf(m, __builtin_fabsf(act[s][v]));
            }
            m = fmaxf(m, __shfl_xor(m, 32, WAVE));
            if (h == 0) red[wave * kBM + 32 * s + r] = m;
        }
        __syncthreads();
        float *Cs = reinterpret_cast<float *>(a.Cs);
        const int nsc = a.N / 128;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const int row = 32 * s + r;
            float amax = 0.f;
#pragma unroll
            for (int w = 0; w < kNW; ++w) amax = fmaxf(amax, red[w * kBM + row]);
            const float inv = amax == 0.f ? 0.f : __fdiv_rn(448.0f, amax);
            if (row < t.rows) {
                const size_t pos = (size_t)(t.pos0 + row);
                uint8_t *dst = a.Cq + pos * a.N + t.n0 + 16 * wave + 4 * h;
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    float x[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) x[i] = fminf(fmaxf(act[s][4 * q + i] * inv, -448.f), 448.f);
                    *reinterpret_cast<uint32_t *>(dst + 8 * q) =
                        e4m3_pack2_hw(x[0], x[1]) | (e4m3_pack2_hw(x[2], x[3]) << 16);
                }
                if (wave == 0 && h == 0) Cs[pos * nsc + t.n0 / 128] = amax == 0.f ? 1.0f : __fdiv_rn(amax, 448.0f);
            }
        }
    } else {
        // output column n0 + 32 w + 8 q + 4 h + i holds acc[s][4 q + i]
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const int row = 32 * s + r;
            if (row < t.rows) {
                uint16_t *dst = a.Cy + (size_t)(t.pos0 + row) * a.ldc + t.n0 + 32 * wave + 4 * h;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    v2i pk;
                    pk[0] = (int)((uint32_t)bf16_from_f32(acc[s][4 * q]) | ((uint32_t)bf16_from_f32(acc[s][4 * q + 1]) << 16));
                    pk[1] = (int)((uint32_t)bf16_from_f32(acc[s][4 * q + 2]) |
                                  ((uint32_t)bf16_from_f32(acc[s][4 * q + 3]) << 16));
                    *reinterpret_cast<v2i *>(dst + 8 * q) = pk;
                }
            }
        }
    }
}

template <bool GATEUP>
__global__ __launch_bounds__(kNT) void moe_gemm_wide_kernel(GemmArgs a)
{
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    TileCtx t;
    int m0;
    if (!find_tile(a, t.e, m0, t.rows)) return;
    if (t.rows > kBM) t.rows = kBM;
    const bool shared = t.e == a.E;
    t.pos0 = a.offsets[t.e] + m0;
    t.KB = a.K / 128;
    t.lane = threadIdx.x & 63;
    t.wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    t.r = t.lane & 31;
    t.h = t.lane >> 5;
    t.n0 = blockIdx.x * (GATEUP ? 128 : 256);
    t.smem = smem;
    const int Nrows = GATEUP ? 2 * a.N : a.N;
    t.Bexp = shared ? a.Bsh : a.B + (size_t)t.e * Nrows * a.K;

    // weight block scales of the slab: gate_up [gate block][KB], [up block][KB];
    // down [n0/128][KB], [n0/128 + 1][KB]
    float *sB = reinterpret_cast<float *>(smem + kRing + kTrash);
    {
        const float *Bsf = shared ? a.Bssh : reinterpret_cast<const float *>(a.Bs) + (size_t)t.e * (Nrows / 128) * t.KB;
        for (int q = threadIdx.x; q < 2 * t.KB; q += kNT) {
            const int b = q / t.KB, kb = q % t.KB;
            const int nb = GATEUP ? (b ? a.N + t.n0 : t.n0) / 128 : t.n0 / 128 + b;
            sB[q] = Bsf[(size_t)nb * t.KB + kb];
        }
    }
    t.sB = sB;

    switch ((t.rows + 31) >> 5) {
    case 1: run_tile<GATEUP, 1>(a, t); break;
    case 2: run_tile<GATEUP, 2>(a, t); break;
    case 3: run_tile<GATEUP, 3>(a, t); break;
    case 4: run_tile<GATEUP, 4>(a, t); break;
    case 5: run_tile<GATEUP, 5>(a, t); break;
    default: run_tile<GATEUP, 6>(a, t); break;
    }
}

template <bool GATEUP>
int launch_wide(const GemmArgs &a, int grid_y, hipStream_t st)
{
    if (grid_y <= 0) return XS_OK;
    const size_t smem = (size_t)kRing + kTrash + 8 * (size_t)(a.K / 128);
    if (smem > 160 * 1024) return set_error(XS_ERR_UNSUPPORTED, "K=%d needs %zu bytes of LDS", a.K, smem);
    auto fn = moe_gemm_wide_kernel<GATEUP>;
    static bool attr_set = false;
    if (!attr_set) {
        XS_HIP(hipFuncSetAttribute((const void *)fn, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
        attr_set = true;
    }
    const int grid_x = GATEUP ? a.N / 128 : a.N / 256;
    fn<<<dim3((unsigned)grid_x, (unsigned)grid_y), dim3(kNT), smem, st>>>(a);
    XS_LAUNCH_CHECK();
    return XS_OK;
}

}  // namespace

int wide_tile_rows() { return kBM; }

int launch_gemm_wide(const GemmArgs &a, bool gateup, int grid_y, hipStream_t st)
{
    if (a.bm != kBM) return set_error(XS_ERR_INVALID, "wide GEMM needs tile offsets for %d-row tiles", kBM);
    if (a.K % 1024 || (gateup ? a.N % 128 : a.N % 256))
        return set_error(XS_ERR_UNSUPPORTED, "wide GEMM shape K=%d N=%d", a.K, a.N);
    return gateup ? launch_wide<true>(a, grid_y, st) : launch_wide<false>(a, grid_y, st);
}

}  // namespace xs
