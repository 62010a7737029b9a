// moe_router.hip -- router logits, top-k routing, activation and weight
// quantizers for gfx950.
//
// Router logits replace linear(x, router_w, nullptr) (xstar_cpp/src/ops/linear.cpp:9-66).
// Two variants: an exact kernel that reproduces gemm_cpu's sequential f32
// accumulation (xstar_cpp/include/ops/gemm.h:57-83) bit for bit, and a bf16
// MFMA kernel (v_mfma_f32_16x16x32_bf16, f32 accumulate).
// Routing uses the branched sigmoid of xstar_cpp/src/ops/mlp.cpp:10-21 over a
// reproducible exp, so indices and weights are bit-identical to the CPU
// restatement given the same logits.
#include "moe_internal.hpp"

namespace xs {

// Upper bound on the K slices of the split-K router GEMM.
static constexpr int kMaxSplits = 16;

// Zero the per-expert token bitmask the route kernel ORs into (folded into the
// router launch so the layer needs no separate fill).
__device__ __forceinline__ void clear_mask(uint32_t *mask, int64_t words)
{
    if (!mask) return;
    const int64_t nb = (int64_t)gridDim.x * gridDim.y * gridDim.z;
    const int64_t b = ((int64_t)blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x;
    for (int64_t i = b * blockDim.x + threadIdx.x; i < words; i += nb * blockDim.x) mask[i] = 0u;
}

// ------------------------------------------------------------ exact logits
// gemm_cpu order: each logit is one sequential f32 chain over k (a separately
// rounded product added to the running sum, no contraction), so the work is
// latency-bound chains.  A lane owns TB chains: one expert, TB tokens (one
// token for small batches, where the chains' latency is the cost; four for
// large ones, where the LDS reads shared by the four chains are).  The block
// holds 64 experts x 4 TB tokens (TB per wave).  K moves in chunks of 256: the
// chunk of the 64 router rows is converted to f32 into LDS (rows padded to
// 260 floats, so a lane's 16-byte reads of its own row hit distinct banks),
// the token rows too (read as broadcasts), and the next chunk's loads are in
// flight while the chains run over the current one.
constexpr int kXC = 256;                 // K chunk
constexpr int kXR = kXC + 4;             // padded LDS row (floats)

template <typename T>
struct ChainLoad;
template <>
struct ChainLoad<uint16_t> {
    static constexpr int N = 8;          // 16-byte loads per thread per chunk (64 bf16)
    v4i r[N];
};
template <>
struct ChainLoad<float> {
    static constexpr int N = 16;         // 64 f32
    v4i r[N];
};

template <typename T, int TB>
__global__ __launch_bounds__(256) void router_logits_exact_kernel(const T *__restrict__ x,
                                                                  const T *__restrict__ wr,
                                                                  int Tn, int E, int H,
                                                                  float *__restrict__ logits,
                                                                  uint32_t *__restrict__ mask, int64_t mask_words)
{
#pragma clang fp contract(off)
    clear_mask(mask, mask_words);
    extern __shared__ __attribute__((aligned(16))) float xsm[];
    float *Ws = xsm;                      // [64][kXR]
    float *Xs = xsm + 64 * kXR;           // [4 TB][kXC]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int e0 = blockIdx.x * 64, t0 = blockIdx.y * 4 * TB + wave * TB;
    // loader mapping: router row lr (4 threads per row, 64 consecutive k each);
    // this wave's TB token rows, 4 consecutive k per lane.  H is a multiple of
    // 128: a last chunk of 128 loads (and runs) half.
    const int lr = tid >> 2, lc = (tid & 3) * 64;
    const T *wrow = wr + (size_t)min(e0 + lr, E - 1) * H + lc;
    ChainLoad<T> ld;
    float xv[TB][4];
    auto fetch = [&](int k0) {
        const int rem = min(kXC, H - k0);
        if (lc < rem) {
#pragma unroll
            for (int i = 0; i < ChainLoad<T>::N; ++i)
                ld.r[i] = *reinterpret_cast<const v4i *>(wrow + k0 + i * (16 / sizeof(T)));
        }
        if (lane * 4 < rem) {
#pragma unroll
            for (int j = 0; j < TB; ++j) load4(x + (size_t)min(t0 + j, Tn - 1) * H + k0 + lane * 4, xv[j]);
        }
    };
    auto store = [&]() {
        float *dst = Ws + lr * kXR + lc;
        if constexpr (sizeof(T) == 2) {
#pragma unroll
            for (int i = 0; i < ChainLoad<T>::N; ++i) {
                v4f lo, hi;
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    lo[2 * j] = __uint_as_float((uint32_t)ld.r[i][j] << 16);
                    lo[2 * j + 1] = __uint_as_float((uint32_t)ld.r[i][j] & 0xFFFF0000u);
                    hi[2 * j] = __uint_as_float((uint32_t)ld.r[i][j + 2] << 16);
                    hi[2 * j + 1] = __uint_as_float((uint32_t)ld.r[i][j + 2] & 0xFFFF0000u);
                }
                *reinterpret_cast<v4f *>(dst + 8 * i) = lo;
                *reinterpret_cast<v4f *>(dst + 8 * i + 4) = hi;
            }
        } else {
#pragma unroll
            for (int i = 0; i < ChainLoad<T>::N; ++i)
                *reinterpret_cast<v4i *>(dst + 4 * i) = ld.r[i];
        }
#pragma unroll
        for (int j = 0; j < TB; ++j)
            *reinterpret_cast<v4f *>(Xs + (wave * TB + j) * kXC + lane * 4) = v4f{xv[j][0], xv[j][1], xv[j][2], xv[j][3]};
    };
    float acc[TB];
#pragma unroll
    for (int j = 0; j < TB; ++j) acc[j] = 0.0f;
    fetch(0);
    for (int k0 = 0; k0 < H; k0 += kXC) {
        __syncthreads();                  // the previous chunk's chains are done with LDS
        store();
        if (k0 + kXC < H) fetch(k0 + kXC);
        __syncthreads();
        const float *wl = Ws + lane * kXR;
        const float *xl = Xs + wave * TB * kXC;
        const int rem = min(kXC, H - k0);
#pragma unroll 4
        for (int k = 0; k < rem; k += 4) {
            const v4f w4 = *reinterpret_cast<const v4f *>(wl + k);
            v4f x4[TB];
#pragma unroll
            for (int j = 0; j < TB; ++j) x4[j] = *reinterpret_cast<const v4f *>(xl + j * kXC + k);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < TB; ++j) acc[j] = acc[j] + x4[j][i] * w4[i];   // no contraction (pragma above)
        }
    }
    const int e = e0 + lane;
#pragma unroll
    for (int j = 0; j < TB; ++j)
        if (t0 + j < Tn && e < E) logits[(size_t)(t0 + j) * E + e] = acc[j];
}

template <typename T, int TB>
static int launch_exact(const T *x, const T *wr, int64_t T_, int64_t E, int64_t H, float *logits, uint32_t *mask,
                        int64_t mask_words, hipStream_t st)
{
    const size_t smem = sizeof(float) * (64 * kXR + 4 * TB * kXC);
    static bool attr_set = false;
    if (!attr_set) {
        XS_HIP(hipFuncSetAttribute((const void *)router_logits_exact_kernel<T, TB>,
                                   hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem));
        attr_set = true;
    }
    dim3 grid((unsigned)((E + 63) / 64), (unsigned)((T_ + 4 * TB - 1) / (4 * TB))), block(256);
    router_logits_exact_kernel<T, TB><<<grid, block, smem, st>>>(x, wr, (int)T_, (int)E, (int)H, logits, mask,
                                                                 mask_words);
    XS_LAUNCH_CHECK();
    return XS_OK;
}

// FP8 1x128 of one 8-column chunk c8 of a row: the 16 lanes of an aligned
// 16-lane group hold the 16 chunks of one 128-column group.
template <typename T>
__device__ __forceinline__ void quant_chunk_fp8(const T *__restrict__ xr, int cols, int c8,
                                                uint8_t *__restrict__ qr, float *__restrict__ sr)
{
    float v[8];
    load8(xr + c8 * 8, v);
    quant8_fp8(v, qr + c8 * 8, (c8 & 15) == 0 ? sr + c8 / 16 : nullptr);
}

// ------------------------------------------------------------- MFMA logits
// Block = 2 x 2 waves; a wave owns MT x NT subtiles of 16 tokens x 16 experts
// over one K slice (blockIdx.z; several slices = split-K for few tokens, the
// partials are summed in slice order by the route kernel, so the result does
// not depend on scheduling).  Operands come straight from global memory, 16 B
// per lane per MFMA, a whole 128-wide K step in flight at once (the router
// weight is 2 MB and stays L2-resident).  MFMA 16x16x32 bf16: lane l supplies
// row (l % 16) and k-slice (l / 16) of 8 elements for both A and B, so the
// k-pairing is consistent whatever the hardware's internal k order.
template <int MT, int NT>
__global__ __launch_bounds__(256) void router_logits_mfma_kernel(const uint16_t *__restrict__ x,
                                                                 const uint16_t *__restrict__ wr,
                                                                 int Tn, int E, int H, int klen,
                                                                 float *__restrict__ part,
                                                                 uint32_t *__restrict__ mask, int64_t mask_words,
                                                                 uint8_t *__restrict__ q, float *__restrict__ qs)
{
    clear_mask(mask, mask_words);
    if (q && blockIdx.x == 0) {
        // the FP8 1x128 activation quant of this block's tokens and K slice
        // (klen % 128 == 0, so each aligned 16-lane group is one 128-column group)
        const int per_row = klen / 8, rows = 32 * MT;
        for (int c = threadIdx.x; c < rows * per_row; c += 256) {
            const int t = blockIdx.y * rows + c / per_row;
            if (t < Tn)
                quant_chunk_fp8(x + (size_t)t * H, H, blockIdx.z * per_row + c % per_row, q + (size_t)t * H,
                                qs + (size_t)t * (H / 128));
        }
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int wm = wave >> 1, wn = wave & 1;
    const int t0 = blockIdx.y * (32 * MT) + wm * 16 * MT, e0 = blockIdx.x * (32 * NT) + wn * 16 * NT;
    const int kbeg = blockIdx.z * klen;
    const v8bf *xa[MT];
    const v8bf *wb[NT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
        xa[i] = reinterpret_cast<const v8bf *>(x + (size_t)min(t0 + 16 * i + r, Tn - 1) * H + kbeg + g * 8);
#pragma unroll
    for (int j = 0; j < NT; ++j)
        wb[j] = reinterpret_cast<const v8bf *>(wr + (size_t)min(e0 + 16 * j + r, E - 1) * H + kbeg + g * 8);
    v4f acc[MT][NT] = {};
    for (int k = 0; k < klen; k += 128) {
        v8bf a[MT][4], b[NT][4];
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
            for (int u = 0; u < 4; ++u) a[i][u] = xa[i][(k + 32 * u) / 8];
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
            for (int u = 0; u < 4; ++u) b[j][u] = wb[j][(k + 32 * u) / 8];
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int i = 0; i < MT; ++i)
#pragma unroll
                for (int j = 0; j < NT; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i][u], b[j][u], acc[i][j], 0, 0, 0);
    }
    // output layout: lane holds column (l % 16), rows 4*(l/16) + v
    float *out = part + (size_t)blockIdx.z * Tn * E;
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            int e = e0 + 16 * j + r;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                int t = t0 + 16 * i + 4 * g + v;
                if (t < Tn && e < E) out[(size_t)t * E + e] = acc[i][j][v];
            }
        }
}

// ------------------------------------------------------- tiled MFMA logits
// Prefill (many tokens): 128 tokens x 128 experts per block over one K slice.
// Both operand tiles move global -> LDS by wave-wide DMA (global_load_lds,
// 8 lanes per 128-byte row, so each load instruction is fully coalesced) into a
// 3-stage ring of 64-wide K steps; 16-byte chunks are XOR-swizzled per row so
// the fragment reads are bank-conflict free.  (Loading MFMA fragments straight
// from global memory touches 16 rows per instruction, which the vector memory
// path serves ~4x slower than coalesced rows.)  4 waves as 2 x 2, each 64 x 64;
// v_mfma_f32_16x16x32_bf16 with the router weight as operand A, so a lane's 4
// results are 4 consecutive experts of one token (one 16-byte store).
namespace {
constexpr int kRtBT = 128, kRtBE = 128, kRtNST = 3;
constexpr int kRtStage = (kRtBT + kRtBE) * 128;       // bytes per K step of 64

__device__ __forceinline__ int rt_swz(int r, int c) { return c ^ ((r >> 1) & 7); }
__device__ __forceinline__ uint32_t rt_lds(const void *p)
{
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}
// Wave-wide DMA global -> LDS: lane i's 16 bytes land at lds + 16 i.  M0 carries
// the wave-uniform LDS base; it is written only here.
// Wait state inside the asm (the compiler's hazard checks do not look into an
// asm string): an LDS DMA that reads M0 needs one after the SALU write of M0.
__device__ __forceinline__ void rt_dma16(const void *g, uint32_t lds)
{
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(__builtin_amdgcn_readfirstlane(lds))
                 : "memory");
}
template <int N>
__device__ __forceinline__ void rt_wait_vm()
{
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
}  // namespace

__global__ __launch_bounds__(256) void router_logits_tile_kernel(const uint16_t *__restrict__ x,
                                                                 const uint16_t *__restrict__ wr,
                                                                 int Tn, int E, int H, int klen,
                                                                 float *__restrict__ part,
                                                                 uint32_t *__restrict__ mask, int64_t mask_words)
{
    clear_mask(mask, mask_words);
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int l16 = lane & 15, g = lane >> 4;
    const int t0 = blockIdx.y * kRtBT, e0 = blockIdx.x * kRtBE;
    const int kbeg = blockIdx.z * klen, KS = klen / 64;

    // DMA sources: instruction q = wave + 4 u covers LDS rows 8q .. 8q+7 (rows
    // 0..127 tokens, 128..255 experts), lane -> (row, swizzled 16-byte chunk).
    const uint16_t *src[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        const int p = 64 * (wave + 4 * u) + lane, row = p >> 3, c = rt_swz(row, p & 7);
        const uint16_t *base = row < kRtBT ? x + (size_t)min(t0 + row, Tn - 1) * H
                                           : wr + (size_t)min(e0 + row - kRtBT, E - 1) * H;
        src[u] = base + kbeg + c * 8;
    }
    const uint32_t ring = __builtin_amdgcn_readfirstlane(rt_lds(smem));
    auto issue = [&](int ks) {
        const int kk = ks < KS ? ks : KS - 1;      // past the end: reload the last step (never read)
        const uint32_t st = ring + (uint32_t)((ks % kRtNST) * kRtStage);
#pragma unroll
        for (int u = 0; u < 8; ++u) rt_dma16(src[u] + (size_t)kk * 64, st + (uint32_t)((wave + 4 * u) * 1024));
    };

    v4f acc[4][4] = {};        // [expert subtile j][token subtile i]
#pragma unroll
    for (int s = 0; s < kRtNST - 1; ++s) issue(s);
    for (int ks = 0; ks < KS; ++ks) {
        rt_wait_vm<(kRtNST - 2) * 8>();     // this wave's loads of step ks landed
        __syncthreads();                    // ... and every wave's; stage (ks-1) % NST is free
        issue(ks + kRtNST - 1);
        const uint8_t *st = smem + (ks % kRtNST) * kRtStage;
        // bf16 16x16x32 operands: lane 16g + r holds row r, K elements [8g, 8g+8)
        // of the 32-wide slice: 16-byte chunk 4u + g of the 128-byte row for
        // slice u of this 64-wide step.
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            v8bf xf[4], wf[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = wm * 64 + 16 * i + l16;
                xf[i] = *reinterpret_cast<const v8bf *>(st + row * 128 + rt_swz(row, 4 * u + g) * 16);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int row = kRtBT + wn * 64 + 16 * j + l16;
                wf[j] = *reinterpret_cast<const v8bf *>(st + row * 128 + rt_swz(row, 4 * u + g) * 16);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[j][i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf[j], xf[i], acc[j][i], 0, 0, 0);
        }
    }
    rt_wait_vm<0>();
    // result layout: lane 16g + r holds token r and experts 4g..4g+3 of the subtile
    float *out = part + (size_t)blockIdx.z * Tn * E;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int t = t0 + wm * 64 + 16 * i + l16;
        if (t >= Tn) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int e = e0 + wn * 64 + 16 * j + 4 * g;
            if (e + 3 < E && (E & 3) == 0) {
                *reinterpret_cast<v4f *>(out + (size_t)t * E + e) = acc[j][i];
            } else {
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    if (e + v < E) out[(size_t)t * E + e + v] = acc[j][i][v];
            }
        }
    }
}

// ----------------------------------------------------------------- routing
struct Cand {
    float key;
    float s;
    int e;
};

// a is better than b: larger key, ties to the lower expert index; e < 0 = empty.
__device__ __forceinline__ bool better(const Cand &a, const Cand &b)
{
    if (a.e < 0) return false;
    if (b.e < 0) return true;
    return a.key > b.key || (a.key == b.key && a.e < b.e);
}

__device__ __forceinline__ Cand wave_best(Cand c)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        Cand d;
        d.key = __shfl_xor(c.key, o, WAVE);
        d.s = __shfl_xor(c.s, o, WAVE);
        d.e = __shfl_xor(c.e, o, WAVE);
        if (better(d, c)) c = d;
    }
    return c;
}

// 64-bit rank of a routing candidate: larger rank = better.  The key's bits
// are mapped to an unsigned order (-0 is folded into +0 first, as the float
// comparison treats them equal); the low word is ~expert, so equal keys rank
// the lower expert index higher.
__device__ __forceinline__ uint64_t route_rank(float key, int e)
{
    const uint32_t u = __builtin_bit_cast(uint32_t, key + 0.0f);
    const uint32_t o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)o << 32) | (uint32_t)(0xffffffffu - (uint32_t)e);
}

template <int CTRL>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t v)
{
    const int lo = __builtin_amdgcn_update_dpp((int)(uint32_t)v, (int)(uint32_t)v, CTRL, 0xf, 0xf, false);
    const int hi = __builtin_amdgcn_update_dpp((int)(uint32_t)(v >> 32), (int)(uint32_t)(v >> 32), CTRL, 0xf, 0xf, false);
    return ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo;
}

// Wave-wide maximum (uniform result): DPP within each row of 16 lanes
// (quad xor 1, quad xor 2, half-row mirror, row mirror), then the four row
// results through readlane.  No LDS round trips.
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v)
{
    uint64_t o;
    o = dpp_u64<0xB1>(v);  v = o > v ? o : v;    // quad_perm [1,0,3,2]
    o = dpp_u64<0x4E>(v);  v = o > v ? o : v;    // quad_perm [2,3,0,1]
    o = dpp_u64<0x141>(v); v = o > v ? o : v;    // row_half_mirror
    o = dpp_u64<0x140>(v); v = o > v ? o : v;    // row_mirror
    uint64_t r = 0;
#pragma unroll
    for (int row = 0; row < 4; ++row) {
        const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, 16 * row);
        const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), 16 * row);
        const uint64_t x = ((uint64_t)hi << 32) | lo;
        r = x > r ? x : r;
    }
    return r;
}

// One wave per token.  Lane l holds experts l + 64*i, i < NV.
template <int NV>
__global__ __launch_bounds__(256) void route_kernel(const float *__restrict__ logits,
                                                    const float *__restrict__ bias, int Tn, int E,
                                                    int k, int n_group, int topk_group, int renorm,
                                                    float scaling, int32_t *__restrict__ idx,
                                                    float *__restrict__ wout,
                                                    uint32_t *__restrict__ mask, int mask_words,
                                                    int nsplit, float *__restrict__ logits_out)
{
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= Tn) return;
    float s[NV], key[NV];
    bool ok[NV];
    const size_t TE = (size_t)Tn * E;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        int e = lane + 64 * i;
        ok[i] = e < E;
        // split-K partials of the router GEMM, summed in slice order
        float lg = 0.0f;
        if (ok[i]) {
            float part[kMaxSplits];
#pragma unroll
            for (int sp = 0; sp < kMaxSplits; ++sp)
                if (sp < nsplit) part[sp] = logits[sp * TE + (size_t)t * E + e];
            lg = part[0];
#pragma unroll
            for (int sp = 1; sp < kMaxSplits; ++sp)
                if (sp < nsplit) lg = __fadd_rn(lg, part[sp]);
            if (logits_out) logits_out[(size_t)t * E + e] = lg;
        }
        s[i] = xs_sigmoid(lg);
        key[i] = (ok[i] && bias) ? __fadd_rn(s[i], bias[e]) : s[i];
    }
    if (n_group > 1) {
        const int gs = E / n_group;
        float my_score = -__builtin_inff();
        for (int gidx = 0; gidx < n_group; ++gidx) {
            // top-2 keys of the group: lane-local, then a wave merge of pairs
            float b1 = -__builtin_inff(), b2 = -__builtin_inff();
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                int e = lane + 64 * i;
                if (ok[i] && e / gs == gidx) {
                    if (key[i] > b1) { b2 = b1; b1 = key[i]; }
                    else if (key[i] > b2) b2 = key[i];
                }
            }
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) {
                float c1 = __shfl_xor(b1, o, WAVE), c2 = __shfl_xor(b2, o, WAVE);
                float n1 = fmaxf(b1, c1);
                float n2 = fmaxf(fminf(b1, c1), fmaxf(b2, c2));
                b1 = n1;
                b2 = n2;
            }
            if (lane == gidx) my_score = __fadd_rn(b1, b2);
        }
        // keep the topk_group best groups (ties -> lower group index)
        uint64_t keep = 0;
        for (int rnd = 0; rnd < topk_group; ++rnd) {
            Cand c;
            c.key = my_score;
            c.s = 0.0f;
            c.e = (lane < n_group && !((keep >> lane) & 1ull)) ? lane : -1;
            c = wave_best(c);
            keep |= 1ull << c.e;
        }
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            int e = lane + 64 * i;
            if (ok[i]) ok[i] = (keep >> (e / gs)) & 1ull;
        }
    }
    // top-k: k rounds of a wave arg-max over 64-bit ranks (order-preserving
    // key bits, then the complement of the expert index: ties go to the lower
    // index, as in the reference's comparison); empty candidates rank 0
    uint64_t rk[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) rk[i] = ok[i] ? route_rank(key[i], lane + 64 * i) : 0ull;
    // lane j keeps pick j; the weight denominator is summed in pick order
    int my_e = -1;
    float my_s = 0.0f, denom = 0.0f;
#pragma unroll 1
    for (int j = 0; j < k; ++j) {
        uint64_t b = rk[0];
#pragma unroll
        for (int i = 1; i < NV; ++i) b = rk[i] > b ? rk[i] : b;
        b = wave_max_u64(b);
        const int e = b ? (int)(0xffffffffu - (uint32_t)b) : -1;
        // the winner's score, from its lane
        float sv = 0.0f;
#pragma unroll
        for (int i = 0; i < NV; ++i)
            if ((e >> 6) == i) sv = s[i];
        sv = e >= 0 ? __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sv), e & 63)) : 0.0f;
        denom = __fadd_rn(denom, sv);
        if (lane == j) { my_e = e; my_s = sv; }
#pragma unroll
        for (int i = 0; i < NV; ++i)
            if (lane + 64 * i == e) rk[i] = 0ull;
    }
    if (lane < k) {
        const float wv = renorm ? __fmul_rn(__fdiv_rn(my_s, denom), scaling) : __fmul_rn(my_s, scaling);
        idx[(size_t)t * k + lane] = my_e;
        wout[(size_t)t * k + lane] = wv;
        if (mask && my_e >= 0) atomicOr(&mask[(size_t)my_e * mask_words + (t >> 5)], 1u << (t & 31));
    }
}

int launch_route(const float *logits, const float *bias, int64_t T, int64_t E, int64_t k,
                 int64_t n_group, int64_t topk_group, int renorm, float scaling, int32_t *idx,
                 float *w, uint32_t *mask, int mask_words, int nsplit, float *logits_out,
                 hipStream_t st)
{
    if (T == 0) return XS_OK;
    dim3 grid((unsigned)((T + 3) / 4)), block(256);
    int nv = (int)((E + 63) / 64);
#define XS_ROUTE(NVV)                                                                       \
    route_kernel<NVV><<<grid, block, 0, st>>>(logits, bias, (int)T, (int)E, (int)k,         \
                                              (int)n_group, (int)topk_group, renorm, scaling, \
                                              idx, w, mask, mask_words, nsplit, logits_out)
    if (nv <= 1) XS_ROUTE(1);
    else if (nv <= 2) XS_ROUTE(2);
    else if (nv <= 4) XS_ROUTE(4);
    else if (nv <= 8) XS_ROUTE(8);
    else XS_ROUTE(16);
#undef XS_ROUTE
    XS_LAUNCH_CHECK();
    return XS_OK;
}

int router_logits_splits(int64_t T, int64_t H, int exact, int dtype)
{
    if (exact || dtype == XS_F32) return 1;
    // decode: enough K slices to fill the GPU; prefill (tiled kernel, 64-wide
    // K steps): 2 slices from 2048 tokens, 4 below
    int ns = T <= 64 ? 16 : (T <= 256 ? 8 : (T < 2048 ? 4 : 2));
    while (ns > 1 && (H % (128 * ns)) != 0) ns >>= 1;
    return ns;
}

bool router_quantizes(int64_t T, int exact, int dtype)
{
    return !exact && dtype == XS_BF16 && T <= 256;   // the decode (router_logits_mfma_kernel) path
}

int launch_router_logits(const void *x, const void *wr, int dtype, int64_t T, int64_t E, int64_t H,
                         int exact, float *logits, int nsplit, hipStream_t st, uint32_t *mask_clear,
                         int64_t mask_words, uint8_t *q, float *qs)
{
    if (q && !router_quantizes(T, exact, dtype))
        return set_error(XS_ERR_INVALID, "router: the activation quant is folded into the decode path only");
    if (T == 0) return XS_OK;
    if (exact || dtype == XS_F32) {
        // one token per lane while the chains' latency is the cost (measured up to
        // 256 tokens: 4 per lane was 2.5x slower there), four for large batches
        if (dtype == XS_F32)
            return T <= 2048 ? launch_exact<float, 1>((const float *)x, (const float *)wr, T, E, H, logits, mask_clear,
                                                    mask_words, st)
                           : launch_exact<float, 4>((const float *)x, (const float *)wr, T, E, H, logits, mask_clear,
                                                    mask_words, st);
        return T <= 2048 ? launch_exact<uint16_t, 1>((const uint16_t *)x, (const uint16_t *)wr, T, E, H, logits,
                                                   mask_clear, mask_words, st)
                       : launch_exact<uint16_t, 4>((const uint16_t *)x, (const uint16_t *)wr, T, E, H, logits,
                                                   mask_clear, mask_words, st);
    } else if (T > 256) {
        // prefill: 128 tokens x 128 experts per block through an LDS ring, K split nsplit ways
        static bool attr_set = false;
        if (!attr_set) {
            XS_HIP(hipFuncSetAttribute((const void *)router_logits_tile_kernel,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, kRtNST * kRtStage));
            attr_set = true;
        }
        dim3 grid((unsigned)((E + kRtBE - 1) / kRtBE), (unsigned)((T + kRtBT - 1) / kRtBT), (unsigned)nsplit), block(256);
        router_logits_tile_kernel<<<grid, block, kRtNST * kRtStage, st>>>((const uint16_t *)x, (const uint16_t *)wr,
                                                                          (int)T, (int)E, (int)H, (int)(H / nsplit),
                                                                          logits, mask_clear, mask_words);
    } else {
        // decode: 32 tokens x 64 experts per block, K split nsplit ways
        dim3 grid((unsigned)((E + 63) / 64), (unsigned)((T + 31) / 32), (unsigned)nsplit), block(256);
        router_logits_mfma_kernel<1, 2><<<grid, block, 0, st>>>((const uint16_t *)x, (const uint16_t *)wr,
                                                                (int)T, (int)E, (int)H, (int)(H / nsplit), logits,
                                                                mask_clear, mask_words, q, qs);
    }
    XS_LAUNCH_CHECK();
    return XS_OK;
}

// ---------------------------------------------------- activation quantizers
// Each thread owns 8 consecutive columns (rows are whole multiples of 16
// threads, so the 16-lane groups stay aligned).
template <typename T>
__global__ __launch_bounds__(256) void quant_act_fp8_kernel(const T *__restrict__ x, int64_t rows,
                                                            int cols, uint8_t *__restrict__ q,
                                                            float *__restrict__ s, int32_t *zero, int zero_n)
{
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (gid < zero_n) zero[gid] = 0;
    const int per_row = cols / 8;
    const int64_t row = gid / per_row;
    if (row >= rows) return;
    quant_chunk_fp8(x + row * cols, cols, (int)(gid - row * per_row), q + row * cols, s + row * (cols / 128));
}

// MXFP8 1x32: 4 lanes per block of 32.
template <typename T>
__global__ __launch_bounds__(256) void quant_act_mxfp8_kernel(const T *__restrict__ x, int64_t rows,
                                                              int cols, uint8_t *__restrict__ q,
                                                              uint8_t *__restrict__ s)
{
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int per_row = cols / 8;
    const int64_t row = gid / per_row;
    if (row >= rows) return;
    const int c8 = (int)(gid - row * per_row);
    float v[8];
    load8(x + row * cols + c8 * 8, v);
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, __builtin_fabsf(v[i]));
    amax = fmaxf(amax, __shfl_xor(amax, 1, WAVE));
    amax = fmaxf(amax, __shfl_xor(amax, 2, WAVE));
    int se = mx_exponent(amax, 8);
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) lo |= e4m3_encode_sw(__builtin_ldexpf(v[i], -se)) << (8 * i);
#pragma unroll
    for (int i = 0; i < 4; ++i) hi |= e4m3_encode_sw(__builtin_ldexpf(v[4 + i], -se)) << (8 * i);
    *reinterpret_cast<v2i *>(q + row * cols + c8 * 8) = v2i{(int)lo, (int)hi};
    if ((c8 & 3) == 0) s[row * (cols / 32) + c8 / 4] = (uint8_t)(se + 127);
}

int launch_quant_act(const void *x, int dtype, int64_t rows, int64_t cols, uint8_t *q, void *s,
                     int mx, hipStream_t st, int32_t *zero, int zero_n)
{
    if (rows == 0) return XS_OK;
    int64_t threads = std::max(rows * (cols / 8), (int64_t)zero_n);
    dim3 grid((unsigned)((threads + 255) / 256)), block(256);
    if (mx) {
        if (dtype == XS_F32)
            quant_act_mxfp8_kernel<float><<<grid, block, 0, st>>>((const float *)x, rows, (int)cols, q, (uint8_t *)s);
        else
            quant_act_mxfp8_kernel<uint16_t><<<grid, block, 0, st>>>((const uint16_t *)x, rows, (int)cols, q, (uint8_t *)s);
    } else {
        if (dtype == XS_F32)
            quant_act_fp8_kernel<float><<<grid, block, 0, st>>>((const float *)x, rows, (int)cols, q, (float *)s, zero, zero_n);
        else
            quant_act_fp8_kernel<uint16_t><<<grid, block, 0, st>>>((const uint16_t *)x, rows, (int)cols, q, (float *)s, zero, zero_n);
    }
    XS_LAUNCH_CHECK();
    return XS_OK;
}

// ------------------------------------------------------- weight quantizers
// FP8 128x128 block: one 256-thread block per (batch, nb, kb) block.
template <typename T>
__global__ __launch_bounds__(256) void quant_weight_fp8_block_kernel(const T *__restrict__ w, int n,
                                                                     int k, uint8_t *__restrict__ q,
                                                                     float *__restrict__ s)
{
    __shared__ float red[4];
    const int KB = k / 128, NB = n / 128;
    const int64_t b = blockIdx.z;
    const int nb = blockIdx.y, kb = blockIdx.x;
    const T *wb = w + b * (int64_t)n * k;
    uint8_t *qb = q + b * (int64_t)n * k;
    // thread: row = tid / 2 (0..127), 64 columns = 8 chunks of 8
    const int r = threadIdx.x >> 1, half = threadIdx.x & 1;
    const int64_t base = (int64_t)(nb * 128 + r) * k + kb * 128 + half * 64;
    float amax = 0.0f;
    for (int c = 0; c < 64; c += 8) {
        float v[8];
        load8(wb + base + c, v);
#pragma unroll
        for (int i = 0; i < 8; ++i) amax = fmaxf(amax, __builtin_fabsf(v[i]));
    }
    amax = wave_max(amax);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float inv = amax == 0.0f ? 0.0f : __fdiv_rn(448.0f, amax);
    for (int c = 0; c < 64; c += 8) {
        float v[8];
        load8(wb + base + c, v);
        uint32_t lo = 0, hi = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) lo |= e4m3_encode_sw(__fmul_rn(v[i], inv)) << (8 * i);
#pragma unroll
        for (int i = 0; i < 4; ++i) hi |= e4m3_encode_sw(__fmul_rn(v[4 + i], inv)) << (8 * i);
        *reinterpret_cast<v2i *>(qb + base + c) = v2i{(int)lo, (int)hi};
    }
    if (threadIdx.x == 0) s[(b * NB + nb) * KB + kb] = amax == 0.0f ? 1.0f : __fdiv_rn(amax, 448.0f);
}

// MXFP4: 4 lanes per 32-element block, each lane packs 8 values into 4 bytes.
template <typename T>
__global__ __launch_bounds__(256) void quant_weight_mxfp4_kernel(const T *__restrict__ w, int64_t rows,
                                                                 int k, uint8_t *__restrict__ q,
                                                                 uint8_t *__restrict__ s)
{
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int per_row = k / 8;
    const int64_t row = gid / per_row;
    if (row >= rows) return;
    const int c8 = (int)(gid - row * per_row);
    float v[8];
    load8(w + row * k + c8 * 8, v);
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, __builtin_fabsf(v[i]));
    amax = fmaxf(amax, __shfl_xor(amax, 1, WAVE));
    amax = fmaxf(amax, __shfl_xor(amax, 2, WAVE));
    int se = mx_exponent(amax, 2);
    uint32_t packed = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) packed |= e2m1_encode_sw(__builtin_ldexpf(v[i], -se)) << (4 * i);
    *reinterpret_cast<uint32_t *>(q + row * (k / 2) + c8 * 4) = packed;
    if ((c8 & 3) == 0) s[row * (k / 32) + c8 / 4] = (uint8_t)(se + 127);
}

}  // namespace xs

using namespace xs;

extern "C" {

int xs_moe_router_logits(const void *x, const void *router_w, int dtype, int64_t T, int64_t E,
                         int64_t H, int exact, float *logits, void *stream)
{
    XS_REQUIRE(x && router_w && logits, "null pointer");
    XS_REQUIRE(dtype == XS_F32 || dtype == XS_BF16, "unsupported dtype");
    XS_REQUIRE(T >= 0 && E >= 1 && H >= 128 && H % 128 == 0, "shape mismatch: H %% 128 != 0");
    return launch_router_logits(x, router_w, dtype, T, E, H, exact, logits, 1, (hipStream_t)stream);
}

int xs_moe_route(const float *logits, const float *bias, int64_t T, int64_t E, int64_t k,
                 int64_t n_group, int64_t topk_group, int renormalize, float scaling,
                 int32_t *idx, float *w, void *stream)
{
    XS_REQUIRE(logits && idx && w, "null pointer");
    XS_REQUIRE(E >= 1 && E <= 1024, "E must be in [1, 1024]");
    XS_REQUIRE(k >= 1 && k <= 16 && k <= E, "top_k must be in [1, min(16, E)]");
    if (n_group > 1) {
        XS_REQUIRE(n_group <= 64 && E % n_group == 0 && E / n_group >= 2,
                   "n_group must divide E into groups of >= 2 (n_group <= 64)");
        XS_REQUIRE(topk_group >= 1 && topk_group <= n_group && topk_group * (E / n_group) >= k,
                   "topk_group must keep at least top_k experts");
    }
    return launch_route(logits, bias, T, E, k, n_group, topk_group, renormalize, scaling, idx, w,
                        nullptr, 0, 1, nullptr, (hipStream_t)stream);
}

int xs_quant_act_fp8(const void *x, int dtype, int64_t rows, int64_t cols, uint8_t *q, float *s,
                     void *stream)
{
    XS_REQUIRE(x && q && s, "null pointer");
    XS_REQUIRE(dtype == XS_F32 || dtype == XS_BF16, "unsupported dtype");
    XS_REQUIRE(rows >= 0 && cols > 0 && cols % 128 == 0, "cols must be a multiple of 128");
    XS_REQUIRE(((uintptr_t)x & 15) == 0 && ((uintptr_t)q & 7) == 0 && ((uintptr_t)s & 3) == 0,
               "misaligned operand: x needs 16-byte, q 8-byte, s 4-byte alignment");
    return launch_quant_act(x, dtype, rows, cols, q, s, 0, (hipStream_t)stream);
}

int xs_quant_act_mxfp8(const void *x, int dtype, int64_t rows, int64_t cols, uint8_t *q,
                       uint8_t *s, void *stream)
{
    XS_REQUIRE(x && q && s, "null pointer");
    XS_REQUIRE(dtype == XS_F32 || dtype == XS_BF16, "unsupported dtype");
    XS_REQUIRE(rows >= 0 && cols > 0 && cols % 32 == 0, "cols must be a multiple of 32");
    XS_REQUIRE(((uintptr_t)x & 15) == 0 && ((uintptr_t)q & 7) == 0,
               "misaligned operand: x needs 16-byte, q 8-byte alignment");
    return launch_quant_act(x, dtype, rows, cols, q, s, 1, (hipStream_t)stream);
}

int xs_quant_weight_fp8_block(const void *w, int dtype, int64_t batch, int64_t n, int64_t k,
                              uint8_t *q, float *s, void *stream)
{
    XS_REQUIRE(w && q && s, "null pointer");
    XS_REQUIRE(dtype == XS_F32 || dtype == XS_BF16, "unsupported dtype");
    XS_REQUIRE(batch >= 1 && n > 0 && k > 0 && n % 128 == 0 && k % 128 == 0,
               "n and k must be multiples of 128");
    XS_REQUIRE(batch <= 65535, "batch too large");
    dim3 grid((unsigned)(k / 128), (unsigned)(n / 128), (unsigned)batch), block(256);
    hipStream_t st = (hipStream_t)stream;
    if (dtype == XS_F32)
        quant_weight_fp8_block_kernel<float><<<grid, block, 0, st>>>((const float *)w, (int)n, (int)k, q, s);
    else
        quant_weight_fp8_block_kernel<uint16_t><<<grid, block, 0, st>>>((const uint16_t *)w, (int)n, (int)k, q, s);
    XS_LAUNCH_CHECK();
    return XS_OK;
}

int xs_quant_weight_mxfp4(const void *w, int dtype, int64_t batch, int64_t n, int64_t k,
                          uint8_t *q, uint8_t *s, void *stream)
{
    XS_REQUIRE(w && q && s, "null pointer");
    XS_REQUIRE(dtype == XS_F32 || dtype == XS_BF16, "unsupported dtype");
    XS_REQUIRE(batch >= 1 && n > 0 && k > 0 && k % 32 == 0, "k must be a multiple of 32");
    int64_t rows = batch * n;
    int64_t threads = rows * (k / 8);
    dim3 grid((unsigned)((threads + 255) / 256)), block(256);
    hipStream_t st = (hipStream_t)stream;
    if (dtype == XS_F32)
        quant_weight_mxfp4_kernel<float><<<grid, block, 0, st>>>((const float *)w, rows, (int)k, q, s);
    else
        quant_weight_mxfp4_kernel<uint16_t><<<grid, block, 0, st>>>((const uint16_t *)w, rows, (int)k, q, s);
    XS_LAUNCH_CHECK();
    return XS_OK;
}

}  // extern "C"
