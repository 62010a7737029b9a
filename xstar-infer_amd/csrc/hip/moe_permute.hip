// moe_permute.hip -- stable counting sort of the routed slots by expert.
//
// No reference counterpart (README.md:28 plans it).  Contract: slot s = t*k + j
// goes to position offsets[e] + #{t' < t : token t' routed to e}, i.e. a stable
// sort by (expert, token).  Built from per-expert token bitmasks: the route
// kernel sets bit t of mask[e] (an OR, so the result does not depend on the
// order of the atomics), a single-block scan turns popcounts into per-word
// prefixes and expert offsets, and a scatter kernel computes each slot's
// position with one popcount.  Fully deterministic.
#include "moe_internal.hpp"

namespace xs {

int mask_words_for(int64_t T) { return (int)((T + 31) / 32); }

__global__ void fill_u32_kernel(uint32_t *p, int64_t n, uint32_t v)
{
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (; i < n; i += (int64_t)gridDim.x * blockDim.x) p[i] = v;
}

int launch_mask_clear(uint32_t *mask, int64_t words, hipStream_t st)
{
    if (words == 0) return XS_OK;
    int64_t blocks = (words + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    fill_u32_kernel<<<dim3((unsigned)blocks), dim3(256), 0, st>>>(mask, words, 0u);
    XS_LAUNCH_CHECK();
    return XS_OK;
}

// Sets bit t of mask[e] for every slot; flags (bit 0) an expert outside [0, E)
// and (bit 1) an expert named twice in one row: the second atomicOr of a bit
// finds it already set, whichever order the atomics run in.
__global__ void build_mask_kernel(const int32_t *__restrict__ idx, int64_t S, int k, int E,
                                  uint32_t *__restrict__ mask, int W, uint32_t *__restrict__ bad)
{
    int64_t s = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= S) return;
    int e = idx[s];
    if (e < 0 || e >= E) {
        atomicOr(bad, 1u);
        return;
    }
    int t = (int)(s / k);
    const uint32_t bit = 1u << (t & 31);
    if (atomicOr(&mask[(size_t)e * W + (t >> 5)], bit) & bit) atomicOr(bad, 2u);
}

// Exclusive scan of one int per thread over a 1024-thread block.
__device__ int block_exclusive_scan(int v, int *lds_waves, int *total)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int x = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        int y = __shfl_up(x, o, WAVE);
        if (lane >= o) x += y;
    }
    if (lane == 63) lds_waves[wave] = x;
    __syncthreads();
    if (threadIdx.x == 0) {
        int run = 0;
        for (int w = 0; w < (int)(blockDim.x >> 6); ++w) {
            int c = lds_waves[w];
            lds_waves[w] = run;
            run += c;
        }
        lds_waves[16] = run;
    }
    __syncthreads();
    int r = x - v + lds_waves[wave];
    *total = lds_waves[16];
    __syncthreads();
    return r;
}

// Per-expert word prefixes and token counts, one block per expert (large T).
__global__ __launch_bounds__(256) void permute_count_kernel(const uint32_t *__restrict__ mask, int W,
                                                            int32_t *__restrict__ wordprefix,
                                                            int32_t *__restrict__ counts)
{
    __shared__ int lds[17];
    const int e = blockIdx.x;
    int run = 0;
    for (int base = 0; base < W; base += 256) {
        const int w = base + (int)threadIdx.x;
        const int c = w < W ? __builtin_popcount(mask[(size_t)e * W + w]) : 0;
        int tot;
        const int ex = block_exclusive_scan(c, lds, &tot);
        if (w < W) wordprefix[(size_t)e * W + w] = run + ex;
        run += tot;
    }
    if (threadIdx.x == 0) counts[e] = run;
}

struct ScatterArgs {
    const int32_t *idx;
    const uint32_t *mask;
    const int32_t *wordprefix;   // NULL: W <= kSmallWords, prefixes counted inline
    int32_t *counts;             // computed here when wordprefix is NULL, else read
    int32_t *offsets;
    int32_t *tile_off;           // [E+2] or NULL
    int4 *tab;                   // tile table or NULL
    int bm;
    int64_t T;
    int k, E, W, shared_rows, offsets_ext;
    int32_t *perm, *inv, *row_token;
    int32_t *zero;
    int64_t zero_n;
};
constexpr int kSmallWords = 8;

// 1024 threads per block: every block scans the E counts (thread e owns expert
// e) into LDS offsets; block 0 also writes counts, offsets, tile offsets and
// the tile table; then each thread places one slot (or one shared row).
__global__ __launch_bounds__(1024) void permute_scatter_kernel(ScatterArgs a)
{
    __shared__ int lds[17];
    __shared__ int offs[1024];
    const int e = threadIdx.x;
    const bool small = a.wordprefix == nullptr;
    int cnt = 0;
    if (e < a.E) {
        if (small) {
            for (int w = 0; w < a.W; ++w) cnt += __builtin_popcount(a.mask[(size_t)e * a.W + w]);
        } else {
            cnt = a.counts[e];
        }
    }
    int total;
    const int off = block_exclusive_scan(cnt, lds, &total);
    if (e < a.E) offs[e] = off;
    if (blockIdx.x == 0) {
        if (e < a.E) {
            if (small) a.counts[e] = cnt;
            a.offsets[e] = off;
        }
        if (e == 0) {
            a.offsets[a.E] = total;
            if (a.offsets_ext) a.offsets[a.E + 1] = total + a.shared_rows;
        }
        if (a.tile_off || a.tab) {
            const int nt = e < a.E ? (cnt + a.bm - 1) / a.bm : 0;
            int tt;
            const int toff = block_exclusive_scan(nt, lds, &tt);
            const int nsh = (a.shared_rows + a.bm - 1) / a.bm;
            if (a.tile_off) {
                if (e < a.E) a.tile_off[e] = toff;
                if (e == 0) {
                    a.tile_off[a.E] = tt;
                    a.tile_off[a.E + 1] = tt + nsh;
                }
            }
            if (a.tab) {
                // entry 0: {tiles, shared tiles}; the shared segment's tiles first
                if (e == 0) a.tab[0] = int4{tt + nsh, nsh, 0, 0};
                if (e < a.E)
                    for (int t = 0; t < nt; ++t)
                        a.tab[1 + nsh + toff + t] = int4{e, off + t * a.bm, min(a.bm, cnt - t * a.bm), t | (min(nt, 0x7fff) << 16)};
                for (int t = e; t < nsh; t += blockDim.x)
                    a.tab[1 + t] = int4{a.E, total + t * a.bm, min(a.bm, a.shared_rows - t * a.bm), t | (min(nsh, 0x7fff) << 16)};
            }
        }
    }
    if (a.zero)
        for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < a.zero_n; i += (int64_t)gridDim.x * blockDim.x)
            a.zero[i] = 0;
    __syncthreads();
    const int64_t S = a.T * a.k;
    const int64_t s = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (s < S) {
        const int ex = a.idx[s];
        if (ex < 0 || ex >= a.E) return;
        const int t = (int)(s / a.k);
        const int wi = t >> 5;
        const uint32_t *m = a.mask + (size_t)ex * a.W;
        int pre = __builtin_popcount(m[wi] & ((1u << (t & 31)) - 1u));
        if (small) {
            for (int w = 0; w < wi; ++w) pre += __builtin_popcount(m[w]);
        } else {
            pre += a.wordprefix[(size_t)ex * a.W + wi];
        }
        const int pos = offs[ex] + pre;
        if (a.perm) a.perm[pos] = (int32_t)s;
        if (a.inv) a.inv[s] = pos;
        if (a.row_token) a.row_token[pos] = t;
    } else if (s < S + a.shared_rows) {
        const int t = (int)(s - S);
        if (a.row_token) a.row_token[S + t] = t;
    }
}

int launch_permute(const int32_t *idx, const uint32_t *mask, int64_t T, int64_t E, int64_t k,
                   int shared_rows, int32_t *wordprefix, const PermuteOut &o, hipStream_t st)
{
    const int W = mask_words_for(T);
    const bool small = W <= kSmallWords;
    if (!small && W > 0) {
        permute_count_kernel<<<dim3((unsigned)E), dim3(256), 0, st>>>(mask, W, wordprefix, o.counts);
        XS_LAUNCH_CHECK();
    }
    ScatterArgs a;
    a.idx = idx;
    a.mask = mask;
    a.wordprefix = small ? nullptr : wordprefix;
    a.counts = o.counts;
    a.offsets = o.offsets;
    a.tile_off = o.tile_off;
    a.tab = reinterpret_cast<int4 *>(o.tab);
    a.bm = o.tile_bm > 0 ? o.tile_bm : 1;
    a.T = T;
    a.k = (int)k;
    a.E = (int)E;
    a.W = W;
    a.shared_rows = shared_rows;
    a.offsets_ext = o.offsets_ext;
    a.perm = o.perm;
    a.inv = o.inv;
    a.row_token = o.row_token;
    a.zero = o.zero;
    a.zero_n = o.zero ? o.zero_n : 0;
    const int64_t n = T * k + shared_rows;
    const unsigned blocks = (unsigned)(n > 0 ? (n + 1023) / 1024 : 1);
    permute_scatter_kernel<<<dim3(blocks), dim3(1024), 0, st>>>(a);
    XS_LAUNCH_CHECK();
    return XS_OK;
}

size_t tile_table_bytes(int64_t rows_routed, int64_t rows_shared, int64_t E, int bm)
{
    return (size_t)16 * (size_t)(rows_routed / bm + E + rows_shared / bm + 3);
}

}  // namespace xs

using namespace xs;

static size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

extern "C" {

size_t xs_moe_permute_workspace_size(int64_t T, int64_t E)
{
    size_t W = (size_t)mask_words_for(T);
    return 2 * align256(sizeof(uint32_t) * W * (size_t)E) + 256;
}

int xs_moe_permute(const int32_t *idx, int64_t T, int64_t E, int64_t k, int32_t *counts,
                   int32_t *offsets, int32_t *perm, int32_t *inv, void *workspace,
                   size_t workspace_bytes, void *stream)
{
    XS_REQUIRE(idx && counts && offsets && perm && inv, "null pointer");
    XS_REQUIRE(E >= 1 && E <= 1024 && k >= 1 && k <= E && T >= 0, "shape mismatch");
    XS_REQUIRE(T * k < (int64_t)1 << 31, "too many slots");
    XS_REQUIRE(workspace && workspace_bytes >= xs_moe_permute_workspace_size(T, E),
               "workspace too small");
    hipStream_t st = (hipStream_t)stream;
    const int W = mask_words_for(T);
    uint32_t *mask = (uint32_t *)workspace;
    int32_t *wordprefix = (int32_t *)((char *)workspace + align256(sizeof(uint32_t) * W * (size_t)E));
    uint32_t *bad = (uint32_t *)((char *)wordprefix + align256(sizeof(uint32_t) * W * (size_t)E));
    int rc = launch_mask_clear(mask, (int64_t)W * E, st);
    if (rc) return rc;
    if (T * k > 0) {
        if ((rc = launch_mask_clear(bad, 1, st))) return rc;
        build_mask_kernel<<<dim3((unsigned)((T * k + 255) / 256)), dim3(256), 0, st>>>(
            idx, T * k, (int)k, (int)E, mask, W, bad);
        XS_LAUNCH_CHECK();
        // the caller's idx is checked before anything is placed (this entry
        // point therefore waits for its stream once)
        uint32_t flags = 0;
        XS_HIP(hipMemcpyAsync(&flags, bad, 4, hipMemcpyDeviceToHost, st));
        XS_HIP(hipStreamSynchronize(st));
        if (flags & 1u) return set_error(XS_ERR_INVALID, "idx: expert index outside [0, E)");
        if (flags & 2u) return set_error(XS_ERR_INVALID, "idx: expert named twice in one row");
    }
    PermuteOut o = {};   // caller's offsets has E+1 entries: offsets_ext = 0
    o.counts = counts;
    o.offsets = offsets;
    o.perm = perm;
    o.inv = inv;
    return launch_permute(idx, mask, T, E, k, 0, wordprefix, o, st);
}

}  // extern "C"
