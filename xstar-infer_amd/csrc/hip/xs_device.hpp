// xs_device.hpp -- device-side helpers shared by the gfx950 MoE kernels:
// number-format conversions, the reproducible exp/sigmoid, wave reductions,
// MFMA operand vector types and host-side error plumbing.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "xs_moe.h"

// ----------------------------------------------------------------- host side
namespace xs {

// Records `msg` as the calling thread's last error and returns `code`.
int set_error(int code, const char *fmt, ...);

}  // namespace xs

#define XS_REQUIRE(cond, ...)                                                 \
    do {                                                                      \
        if (!(cond)) return ::xs::set_error(XS_ERR_INVALID, __VA_ARGS__);     \
    } while (0)

#define XS_HIP(call)                                                          \
    do {                                                                      \
        hipError_t e_ = (call);                                               \
        if (e_ != hipSuccess)                                                 \
            return ::xs::set_error(XS_ERR_HIP, "HIP error: %s (%s) at %s:%d", \
                                   hipGetErrorString(e_), #call, __FILE__, __LINE__); \
    } while (0)

#define XS_LAUNCH_CHECK() XS_HIP(hipGetLastError())

// --------------------------------------------------------------- vector types
typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

namespace xs {

static constexpr int WAVE = 64;

// ---------------------------------------------------------------- bf16 codec
// f32 -> bf16 by adding 0x7FFF + lsb (xstar_cpp/src/bfloat16.cpp:5-25; no
// NaN/Inf special case, same as the reference).
__device__ __forceinline__ uint16_t bf16_from_f32(float f)
{
    uint32_t u = __float_as_uint(f);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
__device__ __forceinline__ float f32_from_bf16(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// ---------------------------------------------------------------- e4m3 codec
// f32 -> E4M3FN, round to nearest even, saturating to +-448 (integer
// arithmetic on the f32 bit pattern; the same steps as the CPU restatement).
__device__ __forceinline__ uint32_t e4m3_encode_sw(float f)
{
    uint32_t u = __float_as_uint(f);
    uint32_t sign = (u >> 31) << 7;
    float a = __builtin_fabsf(f);
    if (a != a) return 0x7fu;
    if (a >= 448.0f) return sign | 0x7eu;
    if (a < 0x1p-6f) return sign | (uint32_t)__builtin_rintf(a * 512.0f);
    uint32_t ua = __float_as_uint(a);
    uint32_t r = (ua + 0x7FFFFu + ((ua >> 20) & 1u)) >> 20;
    uint32_t code = r - ((127u - 7u) << 3);
    return sign | (code > 0x7eu ? 0x7eu : code);
}

// Hardware pair conversion (v_cvt_pk_fp8_f32, OCP E4M3 on gfx950, RNE).  Only
// used where |v| <= 448 * (1 + 2^-22) by construction, so no saturation is
// needed; pinned against e4m3_encode_sw by the GPU tests.
__device__ __forceinline__ uint32_t e4m3_pack2_hw(float a, float b)
{
    return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false) & 0xFFFFu;
}

// ---------------------------------------------------------------- e2m1 codec
__device__ __forceinline__ uint32_t e2m1_encode_sw(float f)
{
    uint32_t u = __float_as_uint(f);
    uint32_t sign = (u >> 31) << 3;
    float a = __builtin_fabsf(f);
    if (a != a || a >= 6.0f) return sign | 7u;
    if (a < 1.0f) return sign | (uint32_t)__builtin_rintf(a * 2.0f);
    uint32_t ua = __float_as_uint(a);
    uint32_t r = (ua + 0x1FFFFFu + ((ua >> 22) & 1u)) >> 22;
    uint32_t code = r - ((127u - 1u) << 1);
    return sign | (code > 7u ? 7u : code);
}

// floor(log2(a)) for finite a > 0 (v_frexp_exp: a = m * 2^e, m in [0.5, 1)).
__device__ __forceinline__ int ilog2f(float a) { return __builtin_amdgcn_frexp_expf(a) - 1; }

// OCP MX shared exponent for a block with max magnitude amax and element emax.
__device__ __forceinline__ int mx_exponent(float amax, int emax_elem)
{
    if (amax == 0.0f) return -127;
    int se = ilog2f(amax) - emax_elem;
    return se < -127 ? -127 : (se > 127 ? 127 : se);
}

// ------------------------------------------------------------ exp / sigmoid
// exp(x) = 2^n * p(r): Cody-Waite reduction with ln2 split into a 12-bit head
// and an f32 tail, degree-7 Taylor polynomial (coefficients 1/k!), ldexp.  Every
// step is a correctly rounded f32 operation, so the CPU restatement gets the
// same bits.
__device__ __forceinline__ float xs_expf(float x)
{
    if (x != x) return x;
    if (x > 88.75f) return __builtin_inff();
    if (x < -104.0f) return 0.0f;
    float n = __builtin_rintf(__fmul_rn(x, 0x1.715476p+0f));
    float r = __builtin_fmaf(-n, 0x1.62ep-1f, x);
    r = __builtin_fmaf(-n, 0x1.0bfbe8p-15f, r);
    float p = 0x1.a01a02p-13f;
    p = __builtin_fmaf(p, r, 0x1.6c16c2p-10f);
    p = __builtin_fmaf(p, r, 0x1.111112p-7f);
    p = __builtin_fmaf(p, r, 0x1.555556p-5f);
    p = __builtin_fmaf(p, r, 0x1.555556p-3f);
    p = __builtin_fmaf(p, r, 0x1.0p-1f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    return __builtin_ldexpf(p, (int)n);
}

// Branched, overflow-safe sigmoid of xstar_cpp/src/ops/mlp.cpp:10-21.
__device__ __forceinline__ float xs_sigmoid(float x)
{
    if (x >= 0.0f) return __fdiv_rn(1.0f, __fadd_rn(1.0f, xs_expf(-x)));
    float e = xs_expf(x);
    return __fdiv_rn(e, __fadd_rn(1.0f, e));
}

// Fast sigmoid for the SwiGLU epilogue (tolerance-checked, not bit-exact):
// the same branch structure with the hardware exp2 and reciprocal.
__device__ __forceinline__ float fast_sigmoid(float x)
{
    float e = __builtin_amdgcn_exp2f(-__builtin_fabsf(x) * 1.4426950408889634f);
    float r = __builtin_amdgcn_rcpf(1.0f + e);
    return x >= 0.0f ? r : e * r;
}

// ----------------------------------------------------------- wave reductions
__device__ __forceinline__ float wave_max(float v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, WAVE));
    return v;
}

}  // namespace xs
