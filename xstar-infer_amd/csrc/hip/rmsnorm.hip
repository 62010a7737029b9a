// rmsnorm.hip -- RMSNorm over rows of `hidden` values, optionally fused with
// the FP8 1x128 quantization of its output (the MoE layer's pre-norm: one read
// of x gives the normalized row for the router and the FP8 activations for the
// expert GEMMs).
//
// Numerics follow the reference CPU path (xstar_cpp/src/ops/rmsnorm.cpp:27-73):
// f32 sum of squares, inv = 1 / sqrt(sum / hidden + eps) with correctly rounded
// sqrt and divisions, f32 y = (x * inv) * w, bf16 y = bf16(bf16(x * inv) * w).
// Only the order of the sum differs (per lane, then a butterfly), so outputs
// may differ from the sequential CPU sum by an ulp of inv.
//
// HBM-bound: per row, 2H (bf16) read + 2H written (+ H + H/32 for the fused
// FP8 output).  One wave per row keeps the row in registers, so x is read once.
#include "moe_internal.hpp"

namespace xs {
namespace {

constexpr int kTPB = 256;
constexpr int kWavesPerBlock = kTPB / WAVE;
constexpr int kMaxChunks = 16;   // 8 columns per lane per chunk: hidden <= 64 * 8 * 16 = 8192

// __builtin_sqrtf is lowered to a correctly rounded sequence (HIP's __fsqrt_rn
// maps to the approximate native sqrt in this toolchain); the divisions are
// correctly rounded.
__device__ __forceinline__ float norm_inv(float sum, int hidden, float eps)
{
    return __fdiv_rn(1.0f, __builtin_sqrtf(__fadd_rn(__fdiv_rn(sum, (float)hidden), eps)));
}

__device__ __forceinline__ float norm_apply(float x, float inv, float w, bool bf16)
{
    if (bf16) {
        float n = f32_from_bf16(bf16_from_f32(__fmul_rn(x, inv)));
        return f32_from_bf16(bf16_from_f32(__fmul_rn(n, w)));
    }
    return __fmul_rn(__fmul_rn(x, inv), w);
}

// 8 consecutive elements in their storage format.
template <typename T> struct Raw8Of { typedef v4i type; };   // 8 bf16
template <> struct Raw8Of<float> { typedef struct { v4f a, b; } type; };
template <typename T> using Raw8 = typename Raw8Of<T>::type;

__device__ __forceinline__ Raw8<uint16_t> load_raw8(const uint16_t *p) { return *reinterpret_cast<const v4i *>(p); }
__device__ __forceinline__ Raw8<float> load_raw8(const float *p)
{
    return Raw8<float>{*reinterpret_cast<const v4f *>(p), *reinterpret_cast<const v4f *>(p + 4)};
}
__device__ __forceinline__ void unpack8(const v4i &r, float *v)
{
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[2 * i] = __uint_as_float((uint32_t)r[i] << 16);
        v[2 * i + 1] = __uint_as_float((uint32_t)r[i] & 0xFFFF0000u);
    }
}
__device__ __forceinline__ void unpack8(const Raw8<float> &r, float *v)
{
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[i] = r.a[i];
        v[4 + i] = r.b[i];
    }
}

// One wave per row.  Lane l holds the 8-column chunks c8 = l + 64 i, i < NC.
// With q: hidden % 128 == 0, so every aligned 16-lane group is one 128-column
// quantization group, wholly inside or outside the row.
template <typename T, int NC>
__global__ __launch_bounds__(kTPB) void rmsnorm_wave_kernel(const T *__restrict__ x, const T *__restrict__ w,
                                                            int64_t rows, int hidden, float eps,
                                                            T *__restrict__ y, uint8_t *__restrict__ q,
                                                            float *__restrict__ s)
{
    const int64_t row = (int64_t)blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int lane = threadIdx.x & (WAVE - 1);
    const int nc8 = hidden >> 3;
    const T *xr = x + row * hidden;
    // the row stays in registers in its own format (bf16: 4 VGPRs per chunk)
    Raw8<T> v[NC];
#pragma unroll
    for (int i = 0; i < NC; ++i)
        if (lane + WAVE * i < nc8) v[i] = load_raw8(xr + (lane + WAVE * i) * 8);
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < NC; ++i)
        if (lane + WAVE * i < nc8) {
            float f[8];
            unpack8(v[i], f);
#pragma unroll
            for (int j = 0; j < 8; ++j) sum = __fadd_rn(sum, __fmul_rn(f[j], f[j]));
        }
    // xor butterfly: every lane ends with the same bits (a + b == b + a)
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) sum = __fadd_rn(sum, __shfl_xor(sum, o, WAVE));
    const float inv = norm_inv(sum, hidden, eps);
    constexpr bool kBf16 = sizeof(T) == 2;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
        const int c8 = lane + WAVE * i;
        if (c8 < nc8) {
            float f[8], g[8], o[8];
            unpack8(v[i], f);
            load8(w + c8 * 8, g);
#pragma unroll
            for (int j = 0; j < 8; ++j) o[j] = norm_apply(f[j], inv, g[j], kBf16);
            store8(y + row * hidden + c8 * 8, o);
            if (q) quant8_fp8(o, q + row * hidden + c8 * 8, (c8 & 15) == 0 ? s + row * (hidden >> 7) + (c8 >> 4) : nullptr);
        }
    }
}

// Any hidden: one block per row, two passes over x (the second hits L2).
template <typename T>
__global__ __launch_bounds__(kTPB) void rmsnorm_block_kernel(const T *__restrict__ x, const T *__restrict__ w,
                                                             int64_t rows, int hidden, float eps,
                                                             T *__restrict__ y)
{
    __shared__ float part[kWavesPerBlock];
    const int64_t row = blockIdx.x;
    const T *xr = x + row * hidden;
    float sum = 0.0f;
    for (int j = threadIdx.x; j < hidden; j += kTPB) {
        float v = to_f32(xr[j]);
        sum = __fadd_rn(sum, __fmul_rn(v, v));
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) sum = __fadd_rn(sum, __shfl_xor(sum, o, WAVE));
    if ((threadIdx.x & (WAVE - 1)) == 0) part[threadIdx.x >> 6] = sum;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int i = 0; i < kWavesPerBlock; ++i) tot = __fadd_rn(tot, part[i]);
    const float inv = norm_inv(tot, hidden, eps);
    constexpr bool kBf16 = sizeof(T) == 2;
    for (int j = threadIdx.x; j < hidden; j += kTPB) {
        float o = norm_apply(to_f32(xr[j]), inv, to_f32(w[j]), kBf16);
        if constexpr (kBf16)
            y[row * hidden + j] = bf16_from_f32(o);
        else
            y[row * hidden + j] = o;
    }
}

template <typename T, int NC>
void launch_wave(const void *x, const void *w, int64_t rows, int hidden, float eps, void *y, uint8_t *q, float *s,
                 hipStream_t st)
{
    const unsigned blocks = (unsigned)((rows + kWavesPerBlock - 1) / kWavesPerBlock);
    rmsnorm_wave_kernel<T, NC><<<blocks, kTPB, 0, st>>>((const T *)x, (const T *)w, rows, hidden, eps, (T *)y, q, s);
}

template <typename T>
int dispatch_wave(int nc, const void *x, const void *w, int64_t rows, int hidden, float eps, void *y, uint8_t *q,
                  float *s, hipStream_t st)
{
    switch (nc) {
#define XS_NC(n) \
    case n: launch_wave<T, n>(x, w, rows, hidden, eps, y, q, s, st); break;
        XS_NC(1) XS_NC(2) XS_NC(3) XS_NC(4) XS_NC(5) XS_NC(6) XS_NC(7) XS_NC(8)
        XS_NC(9) XS_NC(10) XS_NC(11) XS_NC(12) XS_NC(13) XS_NC(14) XS_NC(15) XS_NC(16)
#undef XS_NC
        default: return set_error(XS_ERR_INVALID, "rmsnorm: internal chunk count %d", nc);
    }
    XS_LAUNCH_CHECK();
    return XS_OK;
}

}  // namespace

int launch_rmsnorm(const void *x, const void *w, int dtype, int64_t rows, int64_t hidden, float eps, void *y,
                   uint8_t *q, float *s, hipStream_t st)
{
    if (rows == 0) return XS_OK;
    const size_t es = dtype == XS_BF16 ? 2 : 4;
    const uintptr_t align = 8 * es;   // one 8-column chunk per load / store
    const int nc8 = (int)(hidden / 8);
    const int nc = (nc8 + WAVE - 1) / WAVE;
    const bool wave = hidden % 8 == 0 && nc <= kMaxChunks && ((uintptr_t)x % align) == 0 &&
                      ((uintptr_t)w % align) == 0 && ((uintptr_t)y % align) == 0;
    if (wave) {
        return dtype == XS_BF16 ? dispatch_wave<uint16_t>(nc, x, w, rows, (int)hidden, eps, y, q, s, st)
                                : dispatch_wave<float>(nc, x, w, rows, (int)hidden, eps, y, q, s, st);
    }
    if (dtype == XS_BF16)
        rmsnorm_block_kernel<uint16_t><<<(unsigned)rows, kTPB, 0, st>>>((const uint16_t *)x, (const uint16_t *)w,
                                                                        rows, (int)hidden, eps, (uint16_t *)y);
    else
        rmsnorm_block_kernel<float><<<(unsigned)rows, kTPB, 0, st>>>((const float *)x, (const float *)w, rows,
                                                                     (int)hidden, eps, (float *)y);
    XS_LAUNCH_CHECK();
    // the quantization then reads the normalized rows back (same values, same codes)
    if (q) return launch_quant_act(y, dtype, rows, hidden, q, s, 0, st);
    return XS_OK;
}

}  // namespace xs

using namespace xs;

extern "C" int xs_rmsnorm(const void *x, const void *weight, int dtype, int64_t rows, int64_t hidden, float eps,
                          void *y, uint8_t *q, float *s, void *stream)
{
    XS_REQUIRE(dtype == XS_F32 || dtype == XS_BF16, "unsupported dtype");
    XS_REQUIRE(rows >= 0 && rows < ((int64_t)1 << 31), "rows out of range");
    XS_REQUIRE(hidden >= 1 && hidden < ((int64_t)1 << 30), "shape mismatch: hidden must be >= 1");
    XS_REQUIRE((q == nullptr) == (s == nullptr), "q and s must both be set or both be null");
    XS_REQUIRE(q == nullptr || hidden % 128 == 0, "shape mismatch: FP8 output needs hidden % 128 == 0");
    XS_REQUIRE(rows * hidden < ((int64_t)1 << 40), "too many elements");
    if (rows == 0) return XS_OK;
    XS_REQUIRE(x && weight && y, "null pointer");
    XS_REQUIRE(q == nullptr || (((uintptr_t)q & 7) == 0 && ((uintptr_t)s & 3) == 0 && ((uintptr_t)y & 15) == 0),
               "misaligned operand: with the FP8 output, y needs 16-byte, q 8-byte, s 4-byte alignment");
    return launch_rmsnorm(x, weight, dtype, rows, hidden, eps, y, q, s, (hipStream_t)stream);
}
