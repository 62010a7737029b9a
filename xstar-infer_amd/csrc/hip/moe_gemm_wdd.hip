// moe_gemm_wdd.hip -- grouped FP8 block-scaled expert GEMMs for decode-sized
// tiles (at most 16 token rows per expert tile) with the weights loaded
// straight into VGPRs (gfx950), when the layer holds a fragment-packed copy of
// its FP8 weights.
//
// Nearest reference code: gemm_silu_and_mul_kernel (xstar_cpp/src/ops/mlp.cu:52-200)
// and gemm_kernel (xstar_cpp/src/ops/gemm.cu:41-210).  Numerics are those of
// the 16-row tiles of moe_gemm.hip, step for step: each 128-K block is summed
// by one v_mfma_f32_16x16x128_f8f6f4 (weights operand A, tokens operand B),
// folded into f32 as fma(partial, row scale x block scale, acc) in K order;
// SwiGLU in f32; 1x128 FP8 requantisation over the block's 128 act columns.
// The two kernels give the same bits.
//
// Decode streams every selected expert's weights once, so the bound is HBM,
// and what limits a CU is the bytes it keeps in flight.  In the LDS-ring
// kernels that is the ring (about 100 KB).  Here no operand passes through
// LDS:
//   * the weights are packed in MFMA fragment order ([rows/16][K/128][2][64
//     lanes][16 B], xs_pack_weight_fp8_frag): one 16-row tile's K step is
//     2 KB, loaded by a wave as two coalesced 1 KB instructions straight into
//     the 8 registers the MFMA reads;
//   * the token fragment (16 rows x 128 K, gathered through row_token) is
//     loaded the same way, by every wave (L2-resident);
//   * a block is 8 waves over 128 output columns: gate_up, wave w owns the 16
//     gate rows n0 + 16 w and the matching 16 up rows, so SwiGLU and the
//     requantisation's 128-column amax stay inside the block; down, wave w
//     owns the 16 rows n0 + 16 w;
//   * each wave keeps PD K steps of loads in flight (4 or 8: 8 waves x PD x 4-6 KB
//     per block), and the K loop is unrolled in full (KB is a template argument),
//     so the compiler waits for exactly the step it uses: there is no loop back
//     edge to make it wait for everything;
//   * the row scales and block scales are staged in LDS once per block.
#include "moe_gemm.hpp"

namespace xs {
namespace {

constexpr int kNW = 8, kNT = 64 * kNW;       // waves per block, threads
constexpr int kBN = 16 * kNW;                // output columns per block (act columns for gate_up)
typedef const __attribute__((address_space(1))) v4i gv4i;

__device__ __forceinline__ v8i cat(v4i a, v4i b) { return v8i{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]}; }
// a wave-uniform pointer, made visibly uniform (SGPRs): the loads then take
// the scalar-base form with a 32-bit lane offset
__device__ __forceinline__ const uint8_t *uniform(const uint8_t *p)
{
    const uint64_t u = (uint64_t)(uintptr_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)u), hi = __builtin_amdgcn_readfirstlane((uint32_t)(u >> 32));
    return reinterpret_cast<const uint8_t *>((uintptr_t)(((uint64_t)hi << 32) | lo));
}

// KB K steps of 128; PD steps of loads in flight; NTW 16-row weight tiles per wave
template <bool GATEUP, int KB, int PD>
__global__ __launch_bounds__(kNT) void moe_gemm_wdd_kernel(GemmArgs a)
{
    constexpr int NTW = GATEUP ? 2 : 1;
    constexpr int SS = KB + 1;                   // row-scale stride in LDS (words): conflict-free reads
    __shared__ float sB[2 * KB];                 // block scales: gate_up [gate, up][KB]; down [KB]
    __shared__ float sS[16 * SS];                // row scales [16 rows][KB]
    __shared__ float red[kNW * 16];              // epilogue amax [wave][row]

    // tile of blockIdx.y from the tile table: {tiles, shared tiles}, then
    // {expert, first position, rows}
    const int4 *tab = reinterpret_cast<const int4 *>(a.tile_tab);
    if ((int)blockIdx.y >= tab[0].x) return;
    const int4 d = tab[1 + blockIdx.y];
    const int e = d.x, pos0 = d.y, rows = min(d.z, 16);
    if (rows <= 0) return;
    const bool shared = e == a.E;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r16 = lane & 15, g = lane >> 4;
    const int n0 = (int)blockIdx.x * kBN;
    const int Nrows = GATEUP ? 2 * a.N : a.N;
    const int K = KB * 128;

    auto token_of = [&](int r) -> int {
        const int p = pos0 + min(r, rows - 1);
        return a.row_token ? a.row_token[p] : p;
    };
    {
        const float *Bsf = shared ? a.Bssh : reinterpret_cast<const float *>(a.Bs) + (size_t)e * (Nrows / 128) * KB;
        for (int q = tid; q < (GATEUP ? 2 : 1) * KB; q += kNT) {
            const int b = q / KB, kb = q % KB;
            const int nb = (GATEUP && b ? a.N + n0 : n0) / 128;
            sB[q] = Bsf[(size_t)nb * KB + kb];
        }
        const float *As = reinterpret_cast<const float *>(a.As);
        for (int q = tid; q < 16 * KB; q += kNT) {
            const int r = q / KB, kb = q % KB;
            sS[r * SS + kb] = As[(size_t)token_of(r) * KB + kb];
        }
    }

    // The wave's weight tiles and the token rows.  Every load is a wave-uniform
    // base (SGPRs, advanced per K step) plus one 32-bit lane offset, so the
    // unrolled steps share their address registers.
    const uint8_t *Wexp = shared ? a.Bshp : a.Bp + (size_t)e * Nrows * K;
    const uint8_t *Wb[NTW];
#pragma unroll
    for (int j = 0; j < NTW; ++j) {
        const int row = (j ? a.N : 0) + n0 + 16 * wave;   // gate_up: j = 1 the up rows
        Wb[j] = Wexp + (size_t)(row / 16) * KB * 2048;
    }
    // an expert with one tile reads its weights once: stream them
    const bool stream_w = a.offsets[e + 1] - a.offsets[e] <= 16;
    const uint32_t ow = 16 * (uint32_t)lane;
    const uint32_t ox = (uint32_t)token_of(r16) * (uint32_t)K + 16 * (uint32_t)g;

    v8i wf[PD][NTW], xf[PD];
    auto load = [&](int kb, int s) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < NTW; ++j) {
            const uint8_t *b = uniform(Wb[j] + (size_t)kb * 2048);
            if (stream_w)
                wf[s][j] = cat(__builtin_nontemporal_load((gv4i *)(b + ow)),
                               __builtin_nontemporal_load((gv4i *)(b + ow + 1024)));
            else
                wf[s][j] = cat(*(gv4i *)(b + ow), *(gv4i *)(b + ow + 1024));
        }
        const uint8_t *xb = uniform(a.A + (size_t)kb * 128);
        xf[s] = cat(*(gv4i *)(xb + ox), *(gv4i *)(xb + ox + 64));
    };
#pragma unroll
    for (int s = 0; s < PD; ++s) load(s, s);
    __syncthreads();   // sB, sS visible

    v4f acc[NTW];
#pragma unroll
    for (int j = 0; j < NTW; ++j) acc[j] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
        const int s = kb % PD;
        const float sx = sS[r16 * SS + kb];
#pragma unroll
        for (int j = 0; j < NTW; ++j) {
            const v4f q = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(wf[s][j], xf[s], v4f{0.f, 0.f, 0.f, 0.f}, 0,
                                                                          0, 0, 0, 0, 0);
            const float c = sx * sB[(GATEUP && j ? KB : 0) + kb];
#pragma unroll
            for (int v = 0; v < 4; ++v) acc[j][v] = __builtin_fmaf(q[v], c, acc[j][v]);
            // fold here: left to itself the compiler sinks the whole chain to
            // the epilogue and keeps every step's products live
            asm volatile("" : "+v"(acc[j]));
        }
        if (kb + PD < KB) load(kb + PD, s);
        __builtin_amdgcn_sched_barrier(0);   // keep the steps (and their prefetch distance) in order
    }

    // ------------------------------------------------------------ epilogue
    // lane 16 g + r16: token row r16; gate_up act column (and down output
    // column) n0 + 16 wave + 4 g + v
    const int col = n0 + 16 * wave + 4 * g;
    if (GATEUP) {
        float act[4];
        float m = 0.f;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const float gt = acc[0][v], up = acc[1][v];
            act[v] = gt * fast_sigmoid(gt) * up;
            m = fmaxf(m, __builtin_fabsf(act[v]));
        }
        m = fmaxf(m, __shfl_xor(m, 16, WAVE));
        m = fmaxf(m, __shfl_xor(m, 32, WAVE));
        if (g == 0) red[wave * 16 + r16] = m;
        __syncthreads();
        float amax = 0.f;
#pragma unroll
        for (int w = 0; w < kNW; ++w) amax = fmaxf(amax, red[w * 16 + r16]);
        const float inv = amax == 0.f ? 0.f : __fdiv_rn(448.0f, amax);
        float x[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) x[v] = fminf(fmaxf(act[v] * inv, -448.f), 448.f);
        if (r16 < rows) {
            *reinterpret_cast<uint32_t *>(a.Cq + (size_t)(pos0 + r16) * a.N + col) =
                e4m3_pack2_hw(x[0], x[1]) | (e4m3_pack2_hw(x[2], x[3]) << 16);
            if (wave == 0 && g == 0)
                reinterpret_cast<float *>(a.Cs)[(size_t)(pos0 + r16) * (a.N / 128) + n0 / 128] =
                    amax == 0.f ? 1.0f : __fdiv_rn(amax, 448.0f);
        }
    } else if (r16 < rows) {
        *reinterpret_cast<v4f *>(a.Cf + (size_t)(pos0 + r16) * a.ldc + col) = acc[0];
    }
}

// Prefetch depth: 8 steps where a CU holds one block anyway (gate_up: 136
// VGPRs at 4 steps, 199-215 at 8) or the launch has fewer blocks than two per
// CU (decode down at T = 1: 224); 4 steps otherwise, so that the down GEMM's
// blocks (63-76 VGPRs) can share a CU.
template <bool GATEUP, int KB>
int launch_wdd(const GemmArgs &a, int grid_y, hipStream_t st)
{
    constexpr int PD4 = KB < 4 ? KB : 4, PD8 = KB < 8 ? KB : 8;
    const int gx = a.N / kBN;
    const bool deep = GATEUP || (int64_t)gx * grid_y < 512;
    if (deep) moe_gemm_wdd_kernel<GATEUP, KB, PD8><<<dim3((unsigned)gx, (unsigned)grid_y), dim3(kNT), 0, st>>>(a);
    else moe_gemm_wdd_kernel<GATEUP, KB, PD4><<<dim3((unsigned)gx, (unsigned)grid_y), dim3(kNT), 0, st>>>(a);
    XS_LAUNCH_CHECK();
    return XS_OK;
}

bool kb_supported(int64_t K) { return K == 512 || K == 1024 || K == 2048 || K == 4096; }

}  // namespace

bool wdd_supported(int64_t H, int64_t I) { return kb_supported(H) && kb_supported(I); }

int launch_gemm_wdd(const GemmArgs &a, bool gateup, int grid_y, hipStream_t st)
{
    if (grid_y <= 0) return XS_OK;
    if (a.bm != 16) return set_error(XS_ERR_INVALID, "weight-direct decode GEMM needs 16-row tiles");
    if (!kb_supported(a.K) || a.N % kBN || !a.tile_tab || !a.Bp || (a.e_hi > a.E && !a.Bshp) || (!gateup && !a.Cf))
        return set_error(XS_ERR_UNSUPPORTED, "weight-direct decode GEMM shape K=%d N=%d", a.K, a.N);
#define XS_WDD(KBV)                                                                            \
    case KBV:                                                                                  \
        return gateup ? launch_wdd<true, KBV>(a, grid_y, st) : launch_wdd<false, KBV>(a, grid_y, st);
    switch (a.K / 128) {
        XS_WDD(4)
        XS_WDD(8)
        XS_WDD(16)
        XS_WDD(32)
    default:
        break;
    }
#undef XS_WDD
    return set_error(XS_ERR_UNSUPPORTED, "weight-direct decode GEMM: K=%d", a.K);
}

}  // namespace xs
