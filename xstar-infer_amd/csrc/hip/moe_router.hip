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
// gemm_cpu order: each logit is one sequential f32 chain over k, a separately
// rounded product added to the running sum (no contraction).  The chains are
// latency-bound, so a block splits each chain's work between waves: wave 0
// runs 64 chains (one (token, expert) pair per lane), and waves 1..4 compute
// the rounded products x[t][k] * w[e][k] of the next K chunk into LDS
// (double-buffered), so the chain wave issues one LDS read per 4 adds and
// nothing else.  A product computed by a helper is the same f32 value the
// reference rounds (the helpers only multiply, the chain only adds), so the
// bits are gemm_cpu's for f32 and bf16 operands alike.
// Pairs: implicit (pair p = token p / E, expert p % E: every logit) or a list
// of (token, expert) int32 pairs with its count in device memory (the pairs
// the certified router could not settle).  Blocks loop over groups of 64
// pairs, so the grid is sized without knowing the count.
constexpr int kCK = 128;                 // K chunk per buffer
constexpr int kCR = kCK + 4;             // padded LDS row (floats): a lane's 16-byte reads of its own row hit distinct banks
constexpr int kChainThreads = 320;       // 1 chain wave + 4 product waves

template <typename T>
struct ChainUnit {
    // one unit = 8 consecutive k of one pair: x and w, 16 bytes (bf16) or 32 (f32) each
    static constexpr int V = sizeof(T) == 2 ? 1 : 2;
    v4i x[V], w[V];
};

template <typename T>
__device__ __forceinline__ void chain_unit_load(ChainUnit<T> &u, const T *xr, const T *wr)
{
#pragma unroll
    for (int i = 0; i < ChainUnit<T>::V; ++i) {
        u.x[i] = *reinterpret_cast<const v4i *>(xr + i * (16 / sizeof(T)));
        u.w[i] = *reinterpret_cast<const v4i *>(wr + i * (16 / sizeof(T)));
    }
}

template <typename T>
__device__ __forceinline__ void chain_unit_products(const ChainUnit<T> &u, float *dst)
{
#pragma clang fp contract(off)
    float xv[8], wv[8];
    if constexpr (sizeof(T) == 2) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            xv[2 * j] = __uint_as_float((uint32_t)u.x[0][j] << 16);
            xv[2 * j + 1] = __uint_as_float((uint32_t)u.x[0][j] & 0xFFFF0000u);
            wv[2 * j] = __uint_as_float((uint32_t)u.w[0][j] << 16);
            wv[2 * j + 1] = __uint_as_float((uint32_t)u.w[0][j] & 0xFFFF0000u);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                xv[4 * i + j] = __int_as_float(u.x[i][j]);
                wv[4 * i + j] = __int_as_float(u.w[i][j]);
            }
    }
    v4f lo, hi;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        lo[j] = __fmul_rn(xv[j], wv[j]);
        hi[j] = __fmul_rn(xv[4 + j], wv[4 + j]);
    }
    *reinterpret_cast<v4f *>(dst) = lo;
    *reinterpret_cast<v4f *>(dst + 4) = hi;
}

// One group of up to 64 pairs (pair_of(l) -> {token, expert}, l < cnt) by all
// kChainThreads threads of the block: wave 0's lane l runs pair l's chain and
// stores it to out[token * E + expert]; the other waves compute the products.
template <typename T, typename PairOf>
__device__ __forceinline__ void chain_group(const T *__restrict__ x, const T *__restrict__ wr, int E, int H,
                                            int cnt, PairOf pair_of, float *__restrict__ out, float *prod)
{
#pragma clang fp contract(off)
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nc = H / kCK;
    if (wave == 0) {
        float acc = 0.0f;
        for (int c = 0; c < nc; ++c) {
            __syncthreads();              // chunk c's products are in buffer c & 1
            const float *row = prod + (c & 1) * 64 * kCR + lane * kCR;
#pragma unroll
            for (int k = 0; k < kCK; k += 4) {
                const v4f pv = *reinterpret_cast<const v4f *>(row + k);
                acc = acc + pv[0];
                acc = acc + pv[1];
                acc = acc + pv[2];
                acc = acc + pv[3];
            }
        }
        __syncthreads();                  // the last chunk: the product waves' final barrier
        if (lane < cnt) {
            const v2i te = pair_of(lane);
            out[(size_t)te[0] * E + te[1]] = acc;
        }
    } else {
        // product waves: 256 threads x 4 units = 64 pairs x 16 units of 8 k per
        // chunk; 16 consecutive threads cover one pair's 128 k (256 contiguous
        // bytes of bf16)
        const int htid = tid - 64;
        const T *xr[4], *wrow[4];
        int l[4], k8[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int u = i * 256 + htid;
            l[i] = u >> 4;
            k8[i] = u & 15;
            const v2i te = pair_of(l[i] < cnt ? l[i] : 0);
            xr[i] = x + (size_t)te[0] * H + 8 * k8[i];
            wrow[i] = wr + (size_t)te[1] * H + 8 * k8[i];
        }
        ChainUnit<T> ua[4], ub[4];
        // chunk 0 into buffer 0 and chunk 1's loads in flight, then per
        // iteration c: products of chunk c + 1 (loaded one iteration ago)
        // into buffer (c + 1) & 1 and chunk c + 2's loads issued
#pragma unroll
        for (int i = 0; i < 4; ++i) chain_unit_load(ua[i], xr[i], wrow[i]);
        if (nc > 1) {
#pragma unroll
            for (int i = 0; i < 4; ++i) chain_unit_load(ub[i], xr[i] + kCK, wrow[i] + kCK);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) chain_unit_products(ua[i], prod + l[i] * kCR + 8 * k8[i]);
        for (int c = 0; c < nc; ++c) {
            __syncthreads();
            if (c + 1 < nc) {
                ChainUnit<T> *cur = (c & 1) ? ua : ub;   // chunk c + 1
                ChainUnit<T> *nxt = (c & 1) ? ub : ua;   // chunk c + 2 goes where chunk c was
                float *dst = prod + ((c + 1) & 1) * 64 * kCR;
#pragma unroll
                for (int i = 0; i < 4; ++i) chain_unit_products(cur[i], dst + l[i] * kCR + 8 * k8[i]);
                if (c + 2 < nc) {
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        chain_unit_load(nxt[i], xr[i] + (size_t)(c + 2) * kCK, wrow[i] + (size_t)(c + 2) * kCK);
                }
            }
        }
        __syncthreads();
    }
}

template <typename T>
__global__ __launch_bounds__(kChainThreads) void router_chain_kernel(const T *__restrict__ x,
                                                                     const T *__restrict__ wr, int E, int H,
                                                                     const int32_t *__restrict__ pairs,
                                                                     const int32_t *__restrict__ npairs_dev,
                                                                     int64_t npairs, float *__restrict__ out,
                                                                     uint32_t *__restrict__ mask, int64_t mask_words)
{
    clear_mask(mask, mask_words);
    extern __shared__ __attribute__((aligned(16))) float prod[];   // [2][64][kCR]
    const int64_t n = pairs ? (int64_t)*npairs_dev : npairs;
    for (int64_t base = (int64_t)blockIdx.x * 64; base < n; base += (int64_t)gridDim.x * 64) {
        const int cnt = (int)min((int64_t)64, n - base);
        chain_group(x, wr, E, H, cnt,
                    [&](int l) -> v2i {
                        const int64_t pp = base + l;
                        if (pairs) return v2i{pairs[2 * pp], pairs[2 * pp + 1]};
                        return v2i{(int)(pp / E), (int)(pp % E)};
                    },
                    out, prod);
    }
}

// Chain launch: every logit of [T, E] (pairs == NULL) or the listed pairs.
template <typename T>
static int launch_chain(const T *x, const T *wr, int64_t T_, int64_t E, int64_t H, const int32_t *pairs,
                        const int32_t *npairs_dev, int64_t max_pairs, float *out, uint32_t *mask,
                        int64_t mask_words, hipStream_t st)
{
    const size_t smem = sizeof(float) * 2 * 64 * kCR;
    static bool attr_set = false;
    if (!attr_set) {
        XS_HIP(hipFuncSetAttribute((const void *)router_chain_kernel<T>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                   (int)smem));
        attr_set = true;
    }
    const int64_t groups = (max_pairs + 63) / 64;
    // two blocks per CU fit (67.6 KB of LDS each); a list launch is sized for
    // its worst case and loops, so it stays small
    const int64_t cap = pairs ? 512 : 4096;
    dim3 grid((unsigned)std::max((int64_t)1, std::min(groups, cap))), block(kChainThreads);
    router_chain_kernel<T><<<grid, block, smem, st>>>(x, wr, (int)E, (int)H, pairs, npairs_dev,
                                                      pairs ? 0 : T_ * E, out, mask, mask_words);
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
    quant8_fp8(v, qr ? qr + c8 * 8 : nullptr, (qr && (c8 & 15) == 0) ? sr + c8 / 16 : nullptr);
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
// The certified router's error bound (CERT): besides each logit L, the kernel
// tracks R = sum over the 32-wide K blocks of |acc| after the block's MFMA, and
// A = sum |x_k| |w_k| (the same MFMA over the operands' magnitudes, exact
// bf16 values), and writes D = 98 R + 101 A per (slice, token, expert) into
// dpart.  The route kernel turns D into a bound on |L - L_ref|, L_ref the
// sequential gemm_cpu sum (see route_token).
__device__ __forceinline__ v8bf bf16_abs8(v8bf v)
{
    v4i u = __builtin_bit_cast(v4i, v);
    u &= 0x7fff7fff;
    return __builtin_bit_cast(v8bf, u);
}
__device__ __forceinline__ v4f abs4(v4f v)
{
    return v4f{__builtin_fabsf(v[0]), __builtin_fabsf(v[1]), __builtin_fabsf(v[2]), __builtin_fabsf(v[3])};
}
__device__ __forceinline__ v4f cert_d(v4f r, v4f a) { return 98.0f * r + 101.0f * a; }

// Zeroes n int32 words (the certified router's counters) from the first
// block's first threads.
__device__ __forceinline__ void clear_words(int32_t *z, int n)
{
    if (z && blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0 && (int)threadIdx.x < n) z[threadIdx.x] = 0;
}

template <int MT, int NT, bool CERT>
__global__ __launch_bounds__(256) void router_logits_mfma_kernel(const uint16_t *__restrict__ x,
                                                                 const uint16_t *__restrict__ wr,
                                                                 int Tn, int E, int H, int klen,
                                                                 float *__restrict__ part,
                                                                 uint32_t *__restrict__ mask, int64_t mask_words,
                                                                 uint8_t *__restrict__ q, float *__restrict__ qs,
                                                                 float *__restrict__ dpart, int32_t *__restrict__ zero,
                                                                 int zero_n)
{
    clear_mask(mask, mask_words);
    clear_words(zero, zero_n);
    if (q && blockIdx.x == 0) {
        // the FP8 1x128 activation quant of this block's tokens and K slice
        // (klen % 128 == 0, so each aligned 16-lane group is one 128-column group)
        const int per_row = klen / 8, rows = 32 * MT;
        for (int c = threadIdx.x; c < rows * per_row; c += 256) {
            // every lane takes part in the group's amax shuffles; rows past
            // the batch read the last row and store nothing
            const int t = blockIdx.y * rows + c / per_row;
            const bool live = t < Tn;
            const int tr = live ? t : Tn - 1;
            quant_chunk_fp8(x + (size_t)tr * H, H, blockIdx.z * per_row + c % per_row,
                            live ? q + (size_t)t * H : nullptr, live ? qs + (size_t)t * (H / 128) : nullptr);
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
    v4f aacc[MT][NT] = {}, rr[MT][NT] = {};
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
                for (int j = 0; j < NT; ++j) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i][u], b[j][u], acc[i][j], 0, 0, 0);
                    if constexpr (CERT) {
                        aacc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bf16_abs8(a[i][u]), bf16_abs8(b[j][u]),
                                                                            aacc[i][j], 0, 0, 0);
                        rr[i][j] += abs4(acc[i][j]);
                    }
                }
    }
    // output layout: lane holds column (l % 16), rows 4*(l/16) + v
    float *out = part + (size_t)blockIdx.z * Tn * E;
    float *dout = CERT ? dpart + (size_t)blockIdx.z * Tn * E : nullptr;
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            int e = e0 + 16 * j + r;
            const v4f d = cert_d(rr[i][j], aacc[i][j]);
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                int t = t0 + 16 * i + 4 * g + v;
                if (t < Tn && e < E) {
                    out[(size_t)t * E + e] = acc[i][j][v];
                    if constexpr (CERT) dout[(size_t)t * E + e] = d[v];
                }
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

template <bool CERT>
__global__ __launch_bounds__(256) void router_logits_tile_kernel(const uint16_t *__restrict__ x,
                                                                 const uint16_t *__restrict__ wr,
                                                                 int Tn, int E, int H, int klen,
                                                                 float *__restrict__ part,
                                                                 uint32_t *__restrict__ mask, int64_t mask_words,
                                                                 float *__restrict__ dpart, int32_t *__restrict__ zero,
                                                                 int zero_n)
{
    clear_mask(mask, mask_words);
    clear_words(zero, zero_n);
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
    v4f aacc[4][4] = {}, rr[4][4] = {};   // CERT: magnitude sums and |partial| sums
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
            if constexpr (CERT) {
#pragma unroll
                for (int j = 0; j < 4; ++j) wf[j] = bf16_abs8(wf[j]);
#pragma unroll
                for (int i = 0; i < 4; ++i) xf[i] = bf16_abs8(xf[i]);
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        aacc[j][i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf[j], xf[i], aacc[j][i], 0, 0, 0);
                        rr[j][i] += abs4(acc[j][i]);
                    }
            }
        }
    }
    rt_wait_vm<0>();
    // result layout: lane 16g + r holds token r and experts 4g..4g+3 of the subtile
    float *out = part + (size_t)blockIdx.z * Tn * E;
    float *dout = CERT ? dpart + (size_t)blockIdx.z * Tn * E : nullptr;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int t = t0 + wm * 64 + 16 * i + l16;
        if (t >= Tn) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int e = e0 + wn * 64 + 16 * j + 4 * g;
            const v4f d = cert_d(rr[j][i], aacc[j][i]);
            if (e + 3 < E && (E & 3) == 0) {
                *reinterpret_cast<v4f *>(out + (size_t)t * E + e) = acc[j][i];
                if constexpr (CERT) *reinterpret_cast<v4f *>(dout + (size_t)t * E + e) = d;
            } else {
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    if (e + v < E) {
                        out[(size_t)t * E + e + v] = acc[j][i][v];
                        if constexpr (CERT) dout[(size_t)t * E + e + v] = d[v];
                    }
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

// Inclusive prefix sum over the wave's lanes.
__device__ __forceinline__ int wave_prefix(int v, int lane)
{
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int u = __shfl_up(v, o, WAVE);
        if (lane >= o) v += u;
    }
    return v;
}
__device__ __forceinline__ float wave_minf(float v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fminf(v, __shfl_xor(v, o, WAVE));
    return v;
}

// The certified router's state for one forward (route_token MODE 1 and 2).
struct CertArgs {
    const float *dpart;   // [nsplit][T][E]: D = 98 R + 101 A of each logit slice (MODE 1)
    int kblocks;          // 32-wide K blocks per slice
    float *flog;          // [T][E]: the logit rows of flagged tokens (MODE 1 writes, MODE 2 reads)
    int32_t *pairs;       // [T * E][2]: (token, expert) pairs to recompute in gemm_cpu order
    int32_t *cnt;         // [0] pairs, [1] flagged tokens (zeroed by the logits launch)
    int32_t *flagged;     // [T]: tokens whose routing waits for their exact logits
    int32_t *fbase;       // [T]: first pair of flagged token j in the pair list
    int32_t *fcnt;        // [T]: its number of pairs
    float margin_scale;   // 1; larger values widen every interval (tests of the exact path)
};

// Routing of token t by one wave; lane l holds experts l + 64 i, i < NV.
//   MODE 0: route on the sum (in slice order) of the nsplit logit slices.
//   MODE 1 (certified): the slices are the bf16 MFMA router's.  With
//     u = 2^-24, the gemm_cpu sum L_ref of exact bf16 products p_k differs
//     from the exact sum by at most u sum_k |S_k| (S_k its partial sums,
//     each add rounding by at most u |S_k|).  For k in the 32-wide block
//     starting at j0, |S_k| <= |S_j0| + a_j (a_j the block's sum of |p|),
//     so sum_k |S_k| <= 32 sum_j |S_j0| + 32 A.  The MFMA's own result is
//     allowed 66 u (|acc| + a_j) per instruction: 33 additions of at most
//     one unit in the last place of a magnitude below |acc| + a_j, whatever
//     the hardware's internal order and rounding (truncation included).
//     Products that underflow are covered by the 2^-100 absolute term.
//     Slice s starts its accumulator at 0 while L_ref's partial sums carry
//     P_s (the slices before it), which adds 32 n_s |P_s| for its n_s
//     blocks; summing the slices rounds by at most u |P_s+1| per add.  Hence
//       |L - L_ref| <= delta = u (1 + 2^-4) (sum_s D_s + (32 n_s + 1) sum_s |P_s|
//                                            + |L|),
//     the factor absorbing second-order terms (errors of the tracked |acc|,
//     of A's own MFMA, f32 rounding of the bound).  The sigmoid is
//     1/4-Lipschitz and xs_sigmoid is within 2^-22 of it over all floats, and
//     the bias add rounds by at most 2^-24 (|key| + 1), so the reference's
//     key lies in [key - m, key + m] with
//       m = (delta / 4)(1 + 2^-8) + 2^-20 + 2^-22 |bias|.
//     (The two keys' sigmoid and rounding errors take at most
//     2^-21 + 2^-23 (1 + |bias|) of the fixed part, leaving 3 2^-23.  An MFMA
//     that flushed subnormal bf16 operands would lose products totalling less
//     than H M 2^-126, M the largest operand magnitude, which moves a key by a
//     quarter of that: within the leftover whenever H M <= 2^106, e.g. any
//     H <= 65536 with operands below 10^27.  So the bound does not depend on
//     how the MFMA treats subnormal operands.)
//     Let T be the top-k on these keys and U the experts whose interval
//     meets the interval of another expert where either is in T.  Every
//     expert outside T and U lies below all of T under the reference's keys
//     too, and every pair in T + U with a member outside U is ordered the
//     same by both keys, so recomputing the logits of U in gemm_cpu order and
//     routing again on the mixed keys gives the reference's top-k, order and
//     ties included.  A token with U empty is routed here; otherwise its
//     pairs (t, e in U) and the token are listed, its logit row goes to flog,
//     and routing waits for MODE 2.  Group-limited routing is certified at the
//     group step the same way (group scores bounded by the top-2 sums of the
//     interval ends); when that step is not settled, or a logit or bound is
//     not finite, every expert of the token is recomputed.
//   MODE 2: route on flog (the exact logits of U patched in).
// Returns (MODE 1) the token's listed pair range {first, count}; count 0: routed here.
template <int NV, int MODE>
__device__ __forceinline__ v2i route_token(int t, int lane, const float *__restrict__ logits,
                                            const float *__restrict__ bias, int Tn, int E, int k, int n_group,
                                            int topk_group, int renorm, float scaling, int32_t *__restrict__ idx,
                                            float *__restrict__ wout, uint32_t *__restrict__ mask, int mask_words,
                                            int nsplit, float *__restrict__ logits_out, const CertArgs &ca)
{
    float s[NV], key[NV], lgv[NV];
    float lo[NV], hi[NV];   // MODE 1: the interval of the reference's key
    bool ok[NV], valid[NV];
    bool bad = false;       // MODE 1: a non-finite logit or bound, or an unsettled group step
    const size_t TE = (size_t)Tn * E;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        int e = lane + 64 * i;
        ok[i] = valid[i] = e < E;
        float lg = 0.0f, mm = 0.0f;
        if (ok[i]) {
            if constexpr (MODE == 2) {
                lg = ca.flog[(size_t)t * E + e];
            } else {
                // split-K partials of the router GEMM, summed in slice order
                float part[kMaxSplits], dp[kMaxSplits];
#pragma unroll
                for (int sp = 0; sp < kMaxSplits; ++sp)
                    if (sp < nsplit) {
                        part[sp] = logits[sp * TE + (size_t)t * E + e];
                        if constexpr (MODE == 1) dp[sp] = ca.dpart[sp * TE + (size_t)t * E + e];
                    }
                lg = part[0];
                float dsum = 0.0f, carry = 0.0f;
                if constexpr (MODE == 1) dsum = dp[0];
#pragma unroll
                for (int sp = 1; sp < kMaxSplits; ++sp)
                    if (sp < nsplit) {
                        if constexpr (MODE == 1) {
                            carry += __builtin_fabsf(lg);
                            dsum += dp[sp];
                        }
                        lg = __fadd_rn(lg, part[sp]);
                    }
                if constexpr (MODE == 1) {
                    const float delta = 0x1.1p-24f * (dsum + 32.0f * (float)ca.kblocks * carry + carry +
                                                      __builtin_fabsf(lg)) + 0x1p-100f;
                    mm = 0.25f * delta * 1.00390625f * ca.margin_scale + 0x1p-20f +
                         (bias ? 0x1p-22f * __builtin_fabsf(bias[e]) : 0.0f);
                    if (!__builtin_isfinite(lg) || !__builtin_isfinite(mm)) bad = true;
                }
            }
        }
        lgv[i] = lg;
        s[i] = xs_sigmoid(lg);
        key[i] = (ok[i] && bias) ? __fadd_rn(s[i], bias[e]) : s[i];
        lo[i] = key[i] - mm;
        hi[i] = key[i] + mm;
    }
    if (n_group > 1) {
        const int gs = E / n_group;
        float my_score = -__builtin_inff(), my_lo = -__builtin_inff(), my_hi = -__builtin_inff();
        for (int gidx = 0; gidx < n_group; ++gidx) {
            // top-2 keys of the group (MODE 1: also of the interval ends):
            // lane-local, then a wave merge of pairs
            float b[3][2];
#pragma unroll
            for (int q = 0; q < 3; ++q) b[q][0] = b[q][1] = -__builtin_inff();
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                int e = lane + 64 * i;
                if (ok[i] && e / gs == gidx) {
#pragma unroll
                    for (int q = 0; q < (MODE == 1 ? 3 : 1); ++q) {
                        const float v = q == 0 ? key[i] : (q == 1 ? lo[i] : hi[i]);
                        if (v > b[q][0]) { b[q][1] = b[q][0]; b[q][0] = v; }
                        else if (v > b[q][1]) b[q][1] = v;
                    }
                }
            }
#pragma unroll
            for (int q = 0; q < (MODE == 1 ? 3 : 1); ++q) {
#pragma unroll
                for (int o = 32; o > 0; o >>= 1) {
                    float c1 = __shfl_xor(b[q][0], o, WAVE), c2 = __shfl_xor(b[q][1], o, WAVE);
                    float n1 = fmaxf(b[q][0], c1);
                    float n2 = fmaxf(fminf(b[q][0], c1), fmaxf(b[q][1], c2));
                    b[q][0] = n1;
                    b[q][1] = n2;
                }
            }
            if (lane == gidx) {
                my_score = __fadd_rn(b[0][0], b[0][1]);
                if constexpr (MODE == 1) {
                    // the top-2 sum is increasing in every key; its rounding is
                    // below 2^-22 (1 + |sum|)
                    const float l2 = b[1][0] + b[1][1], h2 = b[2][0] + b[2][1];
                    my_lo = l2 - 0x1p-22f * (1.0f + __builtin_fabsf(l2));
                    my_hi = h2 + 0x1p-22f * (1.0f + __builtin_fabsf(h2));
                }
            }
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
        if constexpr (MODE == 1) {
            // settled when every kept group's score is surely above every other's
            const bool kept = lane < n_group && ((keep >> lane) & 1ull);
            const float kl = wave_minf(kept ? my_lo : __builtin_inff());
            const float nh = wave_max((lane < n_group && !kept) ? my_hi : -__builtin_inff());
            if (!(kl > nh)) bad = true;
        }
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            int e = lane + 64 * i;
            if (ok[i]) ok[i] = (keep >> (e / gs)) & 1ull;
        }
    }
    if constexpr (MODE == 1) bad = __builtin_amdgcn_readfirstlane((int)__any(bad)) != 0;
    // top-k: k rounds of a wave arg-max over 64-bit ranks (order-preserving
    // key bits, then the complement of the expert index: ties go to the lower
    // index, as in the reference's comparison); empty candidates rank 0
    uint64_t rk[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) rk[i] = ok[i] ? route_rank(key[i], lane + 64 * i) : 0ull;
    // lane j keeps pick j; the weight denominator is summed in pick order
    int my_e = -1;
    float my_s = 0.0f, denom = 0.0f, my_lo = 0.0f, my_hi = 0.0f, min_lo = __builtin_inff();
#pragma unroll 1
    for (int j = 0; j < k; ++j) {
        uint64_t b = rk[0];
#pragma unroll
        for (int i = 1; i < NV; ++i) b = rk[i] > b ? rk[i] : b;
        b = wave_max_u64(b);
        const int e = b ? (int)(0xffffffffu - (uint32_t)b) : -1;
        // the winner's score (and interval), from its lane
        float sv = 0.0f, lv = 0.0f, hv = 0.0f;
#pragma unroll
        for (int i = 0; i < NV; ++i)
            if ((e >> 6) == i) {
                sv = s[i];
                lv = lo[i];
                hv = hi[i];
            }
        sv = e >= 0 ? __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sv), e & 63)) : 0.0f;
        if constexpr (MODE == 1) {
            lv = e >= 0 ? __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, lv), e & 63)) : 0.0f;
            hv = e >= 0 ? __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, hv), e & 63)) : 0.0f;
            min_lo = fminf(min_lo, lv);
        }
        denom = __fadd_rn(denom, sv);
        if (lane == j) { my_e = e; my_s = sv; my_lo = lv; my_hi = hv; }
#pragma unroll
        for (int i = 0; i < NV; ++i)
            if (lane + 64 * i == e) rk[i] = 0ull;
    }
    if constexpr (MODE == 1) {
        // U: non-picks whose interval reaches the lowest pick's, picks that
        // reach a non-pick's or another pick's
        float mx = -__builtin_inff();
#pragma unroll
        for (int i = 0; i < NV; ++i)
            if (rk[i]) mx = fmaxf(mx, hi[i]);
        const float max_hi = wave_max(mx);
        int n_amb = 0;
        uint32_t amb_bits = 0;   // bit i: expert lane + 64 i is in U (non-picks, or all when bad)
#pragma unroll
        for (int i = 0; i < NV; ++i)
            if (bad ? valid[i] : (rk[i] && hi[i] >= min_lo)) {
                amb_bits |= 1u << i;
                ++n_amb;
            }
        bool pick_amb = false;
        if (!bad) {   // wave-uniform: every lane takes part in the readlanes
            const bool mine = lane < k && my_e >= 0;
            if (mine && my_lo <= max_hi) pick_amb = true;
            for (int jj = 0; jj < k; ++jj) {
                const float l2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_lo), jj));
                const float h2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_hi), jj));
                const int e2 = __builtin_amdgcn_readlane(my_e, jj);
                if (mine && jj != lane && e2 >= 0 && my_lo <= h2 && l2 <= my_hi) pick_amb = true;
            }
        }
        n_amb += pick_amb ? 1 : 0;
        const int incl = wave_prefix(n_amb, lane);
        const int total = __builtin_amdgcn_readlane(incl, 63);
        if (total > 0) {
            int pbase = 0;
            if (lane == 0) {
                pbase = atomicAdd(&ca.cnt[0], total);
                const int slot = atomicAdd(&ca.cnt[1], 1);
                ca.flagged[slot] = t;
                ca.fbase[slot] = pbase;
                ca.fcnt[slot] = total;
            }
            pbase = __builtin_amdgcn_readlane(pbase, 0);
            int o = pbase + incl - n_amb;
#pragma unroll
            for (int i = 0; i < NV; ++i)
                if ((amb_bits >> i) & 1u) {
                    ca.pairs[2 * (size_t)o] = t;
                    ca.pairs[2 * (size_t)o + 1] = lane + 64 * i;
                    ++o;
                }
            if (pick_amb) {
                ca.pairs[2 * (size_t)o] = t;
                ca.pairs[2 * (size_t)o + 1] = my_e;
            }
#pragma unroll
            for (int i = 0; i < NV; ++i)
                if (valid[i]) ca.flog[(size_t)t * E + lane + 64 * i] = lgv[i];
            return v2i{pbase, total};   // routed by MODE 2 once the pairs are exact
        }
    }
    if (logits_out) {
#pragma unroll
        for (int i = 0; i < NV; ++i)
            if (valid[i]) logits_out[(size_t)t * E + lane + 64 * i] = lgv[i];
    }
    if (lane < k) {
        const float wv = renorm ? __fmul_rn(__fdiv_rn(my_s, denom), scaling) : __fmul_rn(my_s, scaling);
        idx[(size_t)t * k + lane] = my_e;
        wout[(size_t)t * k + lane] = wv;
        if (mask && my_e >= 0) atomicOr(&mask[(size_t)my_e * mask_words + (t >> 5)], 1u << (t & 31));
    }
    return v2i{0, 0};
}

// One wave per token (MODE 0, 1), or per listed token (MODE 2: the flagged
// tokens, a grid-stride loop over their count).
template <int NV, int MODE>
__global__ __launch_bounds__(256) void route_kernel(const float *__restrict__ logits,
                                                    const float *__restrict__ bias, int Tn, int E,
                                                    int k, int n_group, int topk_group, int renorm,
                                                    float scaling, int32_t *__restrict__ idx,
                                                    float *__restrict__ wout,
                                                    uint32_t *__restrict__ mask, int mask_words,
                                                    int nsplit, float *__restrict__ logits_out, CertArgs ca)
{
    const int lane = threadIdx.x & 63;
    const int w = blockIdx.x * 4 + (threadIdx.x >> 6);
    if constexpr (MODE == 2) {
        const int n = ca.cnt[1];
        for (int j = w; j < n; j += gridDim.x * 4)
            route_token<NV, 2>(ca.flagged[j], lane, logits, bias, Tn, E, k, n_group, topk_group, renorm, scaling,
                               idx, wout, mask, mask_words, 1, logits_out, ca);
    } else {
        if (w >= Tn) return;
        route_token<NV, MODE>(w, lane, logits, bias, Tn, E, k, n_group, topk_group, renorm, scaling, idx, wout,
                              mask, mask_words, nsplit, logits_out, ca);
    }
}

// Certified routing of decode batches in one launch: a block of
// kChainThreads threads per token.  Wave 0 routes the token (MODE 1); when
// the bound leaves experts undecided, the whole block computes their logits in
// gemm_cpu order (chain_group over the pairs wave 0 listed) into the token's
// flog row, and wave 0 routes it again (MODE 2).  Block barriers order wave
// 0's listing before the other waves read it, and the chain lanes' stores
// before wave 0's second routing reads them.  No launch is added to the
// approximate router's.
template <typename T, int NV>
__global__ __launch_bounds__(kChainThreads) void route_block_kernel(
    const T *__restrict__ x, const T *__restrict__ wr, const float *__restrict__ logits,
    const float *__restrict__ bias, int Tn, int E, int H, int k, int n_group, int topk_group, int renorm,
    float scaling, int32_t *__restrict__ idx, float *__restrict__ wout, uint32_t *__restrict__ mask, int mask_words,
    int nsplit, float *__restrict__ logits_out, CertArgs ca)
{
    extern __shared__ __attribute__((aligned(16))) float prod[];   // [2][64][kCR]; [0..1] first the pair range
    int *range = reinterpret_cast<int *>(prod);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int t = blockIdx.x;
    if (wave == 0) {
        const v2i r = route_token<NV, 1>(t, lane, logits, bias, Tn, E, k, n_group, topk_group, renorm, scaling, idx,
                                         wout, mask, mask_words, nsplit, logits_out, ca);
        if (lane == 0) {
            range[0] = r[0];
            range[1] = r[1];
        }
    }
    __syncthreads();
    const int base = range[0], np = range[1];
    if (np == 0) return;                  // routed by wave 0 (the whole block leaves together)
    __syncthreads();                      // every wave has its copy: the chain may reuse the LDS
    for (int g = 0; g < np; g += 64)
        chain_group(x, wr, E, H, min(64, np - g),
                    [&](int l) -> v2i {
                        const int pp = base + g + l;
                        return v2i{ca.pairs[2 * (size_t)pp], ca.pairs[2 * (size_t)pp + 1]};
                    },
                    ca.flog, prod);
    __syncthreads();
    if (wave == 0)
        route_token<NV, 2>(t, lane, nullptr, bias, Tn, E, k, n_group, topk_group, renorm, scaling, idx, wout, mask,
                           mask_words, 1, logits_out, ca);
}

int launch_route_block(const void *x, const void *wr, int dtype, const float *logits, const float *bias, int64_t T,
                       int64_t E, int64_t H, int64_t k, int64_t n_group, int64_t topk_group, int renorm, float scaling,
                       int32_t *idx, float *w, uint32_t *mask, int mask_words, int nsplit, float *logits_out,
                       const CertState &cert, hipStream_t st)
{
    if (T == 0) return XS_OK;
    // the certified router takes bf16 inputs only (f32 inputs use the chain router)
    if (dtype != XS_BF16) return set_error(XS_ERR_INVALID, "certified router: bf16 inputs only");
    CertArgs ca = {cert.dpart, cert.kblocks, cert.flog, cert.pairs, cert.cnt, cert.flagged, cert.fbase, cert.fcnt,
                   cert.margin_scale};
    const size_t smem = sizeof(float) * 2 * 64 * kCR;
    dim3 grid((unsigned)T), block(kChainThreads);
    const int nv = (int)((E + 63) / 64);
#define XS_ROUTE_BLOCK(NVV)                                                                                    \
    do {                                                                                                       \
        static bool attr_set = false;                                                                          \
        if (!attr_set) {                                                                                       \
            XS_HIP(hipFuncSetAttribute((const void *)route_block_kernel<uint16_t, NVV>,                         \
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem));                 \
            attr_set = true;                                                                                   \
        }                                                                                                      \
        route_block_kernel<uint16_t, NVV><<<grid, block, smem, st>>>(                                          \
            (const uint16_t *)x, (const uint16_t *)wr, logits, bias, (int)T, (int)E, (int)H, (int)k, (int)n_group, \
            (int)topk_group, renorm, scaling, idx, w, mask, mask_words, nsplit, logits_out, ca);               \
    } while (0)
    if (nv <= 1) XS_ROUTE_BLOCK(1);
    else if (nv <= 2) XS_ROUTE_BLOCK(2);
    else if (nv <= 4) XS_ROUTE_BLOCK(4);
    else if (nv <= 8) XS_ROUTE_BLOCK(8);
    else XS_ROUTE_BLOCK(16);
#undef XS_ROUTE_BLOCK
    XS_LAUNCH_CHECK();
    return XS_OK;
}

int launch_route(const float *logits, const float *bias, int64_t T, int64_t E, int64_t k,
                 int64_t n_group, int64_t topk_group, int renorm, float scaling, int32_t *idx,
                 float *w, uint32_t *mask, int mask_words, int nsplit, float *logits_out,
                 hipStream_t st, const CertState *cert, int mode)
{
    if (T == 0) return XS_OK;
    CertArgs ca = {};
    if (cert) {
        ca.dpart = cert->dpart;
        ca.kblocks = cert->kblocks;
        ca.flog = cert->flog;
        ca.pairs = cert->pairs;
        ca.cnt = cert->cnt;
        ca.flagged = cert->flagged;
        ca.fbase = cert->fbase;
        ca.fcnt = cert->fcnt;
        ca.margin_scale = cert->margin_scale;
    }
    // MODE 2 loops over the flagged tokens: a grid for a quarter of them at most
    dim3 grid((unsigned)(mode == 2 ? std::min((T + 3) / 4, (int64_t)256) : (T + 3) / 4)), block(256);
    int nv = (int)((E + 63) / 64);
#define XS_ROUTE(NVV, M)                                                                         \
    route_kernel<NVV, M><<<grid, block, 0, st>>>(logits, bias, (int)T, (int)E, (int)k,           \
                                                 (int)n_group, (int)topk_group, renorm, scaling, \
                                                 idx, w, mask, mask_words, nsplit, logits_out, ca)
#define XS_ROUTE_NV(M)                       \
    if (nv <= 1) XS_ROUTE(1, M);             \
    else if (nv <= 2) XS_ROUTE(2, M);        \
    else if (nv <= 4) XS_ROUTE(4, M);        \
    else if (nv <= 8) XS_ROUTE(8, M);        \
    else XS_ROUTE(16, M);
    if (mode == 1) {
        XS_ROUTE_NV(1)
    } else if (mode == 2) {
        XS_ROUTE_NV(2)
    } else {
        XS_ROUTE_NV(0)
    }
#undef XS_ROUTE_NV
#undef XS_ROUTE
    XS_LAUNCH_CHECK();
    return XS_OK;
}

// Router kinds by params.router_exact and the input dtype: 0 the bf16 MFMA
// router (approximate); 1 exact routing: bf16 inputs take the certified MFMA
// router (route_token MODE 1) plus the chain kernel for the pairs it lists;
// 2, and f32 inputs, the chain kernel for every logit.
int router_kind(int exact, int dtype)
{
    if (dtype == XS_F32 || exact >= 2) return XS_ROUTER_CHAIN;
    return exact == 1 ? XS_ROUTER_CERTIFIED : XS_ROUTER_MFMA;
}

int router_logits_splits(int64_t T, int64_t H, int exact, int dtype)
{
    if (router_kind(exact, dtype) == XS_ROUTER_CHAIN) return 1;
    // decode: enough K slices to fill the GPU; prefill (tiled kernel, 64-wide
    // K steps): 2 slices from 2048 tokens, 4 below
    int ns = T <= 64 ? 16 : (T <= 256 ? 8 : (T < 2048 ? 4 : 2));
    while (ns > 1 && (H % (128 * ns)) != 0) ns >>= 1;
    return ns;
}

bool router_quantizes(int64_t T, int exact, int dtype)
{
    // the decode (router_logits_mfma_kernel) path
    return router_kind(exact, dtype) != XS_ROUTER_CHAIN && T <= 256;
}

int launch_router_logits(const void *x, const void *wr, int dtype, int64_t T, int64_t E, int64_t H,
                         int exact, float *logits, int nsplit, hipStream_t st, uint32_t *mask_clear,
                         int64_t mask_words, uint8_t *q, float *qs, const CertState *cert)
{
    if (q && !router_quantizes(T, exact, dtype))
        return set_error(XS_ERR_INVALID, "router: the activation quant is folded into the decode path only");
    if (T == 0) return XS_OK;
    const int kind = router_kind(exact, dtype);
    if (kind == XS_ROUTER_CHAIN || (kind == XS_ROUTER_CERTIFIED && !cert)) {
        // every logit in gemm_cpu order (a certified router needs the routing
        // stage: without it, the logits alone are computed exactly)
        if (dtype == XS_F32)
            return launch_chain<float>((const float *)x, (const float *)wr, T, E, H, nullptr, nullptr, T * E, logits,
                                       mask_clear, mask_words, st);
        return launch_chain<uint16_t>((const uint16_t *)x, (const uint16_t *)wr, T, E, H, nullptr, nullptr, T * E,
                                      logits, mask_clear, mask_words, st);
    }
    const bool c = kind == XS_ROUTER_CERTIFIED;
    float *dpart = c ? cert->dpart : nullptr;
    int32_t *zero = c ? cert->cnt : nullptr;
    const int zero_n = c ? 2 : 0;
    if (T > 256) {
        // prefill: 128 tokens x 128 experts per block through an LDS ring, K split nsplit ways
        static bool attr_set[2] = {false, false};
        const void *fn = c ? (const void *)router_logits_tile_kernel<true> : (const void *)router_logits_tile_kernel<false>;
        if (!attr_set[c]) {
            XS_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, kRtNST * kRtStage));
            attr_set[c] = true;
        }
        dim3 grid((unsigned)((E + kRtBE - 1) / kRtBE), (unsigned)((T + kRtBT - 1) / kRtBT), (unsigned)nsplit), block(256);
        if (c)
            router_logits_tile_kernel<true><<<grid, block, kRtNST * kRtStage, st>>>(
                (const uint16_t *)x, (const uint16_t *)wr, (int)T, (int)E, (int)H, (int)(H / nsplit), logits,
                mask_clear, mask_words, dpart, zero, zero_n);
        else
            router_logits_tile_kernel<false><<<grid, block, kRtNST * kRtStage, st>>>(
                (const uint16_t *)x, (const uint16_t *)wr, (int)T, (int)E, (int)H, (int)(H / nsplit), logits,
                mask_clear, mask_words, nullptr, nullptr, 0);
    } else {
        // decode: 32 tokens x 64 experts per block, K split nsplit ways
        dim3 grid((unsigned)((E + 63) / 64), (unsigned)((T + 31) / 32), (unsigned)nsplit), block(256);
        if (c)
            router_logits_mfma_kernel<1, 2, true><<<grid, block, 0, st>>>(
                (const uint16_t *)x, (const uint16_t *)wr, (int)T, (int)E, (int)H, (int)(H / nsplit), logits,
                mask_clear, mask_words, q, qs, dpart, zero, zero_n);
        else
            router_logits_mfma_kernel<1, 2, false><<<grid, block, 0, st>>>(
                (const uint16_t *)x, (const uint16_t *)wr, (int)T, (int)E, (int)H, (int)(H / nsplit), logits,
                mask_clear, mask_words, q, qs, nullptr, nullptr, 0);
    }
    XS_LAUNCH_CHECK();
    return XS_OK;
}

int launch_router_fix(const void *x, const void *wr, int dtype, int64_t T, int64_t E, int64_t H,
                      const CertState &cert, hipStream_t st)
{
    if (T == 0) return XS_OK;
    if (dtype == XS_F32)
        return launch_chain<float>((const float *)x, (const float *)wr, T, E, H, cert.pairs, cert.cnt, T * E,
                                   cert.flog, nullptr, 0, st);
    return launch_chain<uint16_t>((const uint16_t *)x, (const uint16_t *)wr, T, E, H, cert.pairs, cert.cnt, T * E,
                                  cert.flog, nullptr, 0, st);
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
    XS_REQUIRE(T * E < ((int64_t)1 << 31), "too many logits: T x E must stay below 2^31 (split the batch)");
    XS_REQUIRE(((uintptr_t)x & 15) == 0 && ((uintptr_t)router_w & 15) == 0 && ((uintptr_t)logits & 3) == 0,
               "misaligned operand: x and router_w need 16-byte, logits 4-byte alignment");
    return launch_router_logits(x, router_w, dtype, T, E, H, exact, logits, 1, (hipStream_t)stream);
}

int xs_moe_route(const float *logits, const float *bias, int64_t T, int64_t E, int64_t k,
                 int64_t n_group, int64_t topk_group, int renormalize, float scaling,
                 int32_t *idx, float *w, void *stream)
{
    XS_REQUIRE(logits && idx && w, "null pointer");
    XS_REQUIRE(E >= 1 && E <= 1024, "E must be in [1, 1024]");
    XS_REQUIRE(T >= 0 && T * E < ((int64_t)1 << 31), "too many logits: T x E must stay below 2^31 (split the batch)");
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
