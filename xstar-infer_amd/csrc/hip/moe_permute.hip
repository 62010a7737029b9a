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

__global__ void build_mask_kernel(const int32_t *__restrict__ idx, int64_t S, int k, int E,
                                  uint32_t *__restrict__ mask, int W)
{
    int64_t s = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= S) return;
    int e = idx[s];
    if (e < 0 || e >= E) return;
    int t = (int)(s / k);
    atomicOr(&mask[(size_t)e * W + (t >> 5)], 1u << (t & 31));
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

struct ScanArgs {
    const uint32_t *mask;
    int32_t *wordprefix;
    int32_t *counts;
    int32_t *offsets;
    int32_t *tile_off0, *tile_off1, *tile_off2;
    int bm0, bm1, bm2;
    int E, W, shared_rows;
    int offsets_ext;   // 1: offsets has E+2 entries (shared-segment end at [E+1])
};

// One block of 1024 threads; thread e < E owns expert e.
__global__ __launch_bounds__(1024) void permute_scan_kernel(ScanArgs a)
{
    __shared__ int lds[17];
    const int e = threadIdx.x;
    int cnt = 0;
    if (e < a.E) {
        const uint32_t *m = a.mask + (size_t)e * a.W;
        int32_t *wp = a.wordprefix + (size_t)e * a.W;
        for (int w = 0; w < a.W; ++w) {
            wp[w] = cnt;
            cnt += __builtin_popcount(m[w]);
        }
        a.counts[e] = cnt;
    }
    int total;
    int off = block_exclusive_scan(e < a.E ? cnt : 0, lds, &total);
    if (e < a.E) a.offsets[e] = off;
    if (e == 0) {
        a.offsets[a.E] = total;
        if (a.offsets_ext) a.offsets[a.E + 1] = total + a.shared_rows;
    }
    int32_t *tiles[3] = {a.tile_off0, a.tile_off1, a.tile_off2};
    int bms[3] = {a.bm0, a.bm1, a.bm2};
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        if (!tiles[i]) continue;
        int nt = e < a.E ? (cnt + bms[i] - 1) / bms[i] : 0;
        int tt;
        int toff = block_exclusive_scan(nt, lds, &tt);
        if (e < a.E) tiles[i][e] = toff;
        if (e == 0) {
            tiles[i][a.E] = tt;
            tiles[i][a.E + 1] = tt + (a.shared_rows + bms[i] - 1) / bms[i];
        }
    }
}

__global__ void permute_scatter_kernel(const int32_t *__restrict__ idx, const uint32_t *__restrict__ mask,
                                       const int32_t *__restrict__ wordprefix,
                                       const int32_t *__restrict__ offsets, int64_t T, int k, int E,
                                       int W, int shared_rows, int32_t *__restrict__ perm,
                                       int32_t *__restrict__ inv, int32_t *__restrict__ row_token)
{
    const int64_t S = T * k;
    int64_t s = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (s < S) {
        int e = idx[s];
        if (e < 0 || e >= E) return;
        int t = (int)(s / k);
        size_t wi = (size_t)e * W + (t >> 5);
        uint32_t below = mask[wi] & ((1u << (t & 31)) - 1u);
        int pos = offsets[e] + wordprefix[wi] + __builtin_popcount(below);
        if (perm) perm[pos] = (int32_t)s;
        if (inv) inv[s] = pos;
        if (row_token) row_token[pos] = t;
    } else if (s < S + shared_rows) {
        int t = (int)(s - S);
        if (row_token) row_token[S + t] = t;
    }
}

int launch_permute(const int32_t *idx, const uint32_t *mask, int64_t T, int64_t E, int64_t k,
                   int shared_rows, int32_t *wordprefix, const PermuteOut &o, hipStream_t st)
{
    const int W = mask_words_for(T);
    ScanArgs a;
    a.mask = mask;
    a.wordprefix = wordprefix;
    a.counts = o.counts;
    a.offsets = o.offsets;
    a.tile_off0 = o.n_tile_sizes > 0 ? o.tile_off[0] : nullptr;
    a.tile_off1 = o.n_tile_sizes > 1 ? o.tile_off[1] : nullptr;
    a.tile_off2 = o.n_tile_sizes > 2 ? o.tile_off[2] : nullptr;
    a.bm0 = o.tile_bm[0];
    a.bm1 = o.tile_bm[1];
    a.bm2 = o.tile_bm[2];
    a.E = (int)E;
    a.W = W;
    a.shared_rows = shared_rows;
    a.offsets_ext = o.offsets_ext;
    permute_scan_kernel<<<dim3(1), dim3(1024), 0, st>>>(a);
    XS_LAUNCH_CHECK();
    int64_t n = T * k + shared_rows;
    if (n > 0) {
        permute_scatter_kernel<<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st>>>(
            idx, mask, wordprefix, o.offsets, T, (int)k, (int)E, W, shared_rows, o.perm, o.inv,
            o.row_token);
        XS_LAUNCH_CHECK();
    }
    return XS_OK;
}

}  // namespace xs

using namespace xs;

static size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

extern "C" {

size_t xs_moe_permute_workspace_size(int64_t T, int64_t E)
{
    size_t W = (size_t)mask_words_for(T);
    return 2 * align256(sizeof(uint32_t) * W * (size_t)E);
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
    int rc = launch_mask_clear(mask, (int64_t)W * E, st);
    if (rc) return rc;
    if (T * k > 0) {
        build_mask_kernel<<<dim3((unsigned)((T * k + 255) / 256)), dim3(256), 0, st>>>(
            idx, T * k, (int)k, (int)E, mask, W);
        XS_LAUNCH_CHECK();
    }
    PermuteOut o = {};   // caller's offsets has E+1 entries: offsets_ext = 0
    o.counts = counts;
    o.offsets = offsets;
    o.perm = perm;
    o.inv = inv;
    o.row_token = nullptr;
    o.n_tile_sizes = 0;
    return launch_permute(idx, mask, T, E, k, 0, wordprefix, o, st);
}

}  // extern "C"
