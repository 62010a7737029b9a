// ref_driver.cpp -- exposes the reference's own CPU numerics through a C ABI so
// the oracle can be checked against them.  TEST INFRASTRUCTURE ONLY.
//
// Compiled together with, from /root/reference (never copied into this repo):
//   xstar_cpp/include/ops/gemm.h   gemm_cpu<T> (header template, gemm.h:57-83)
//   xstar_cpp/src/bfloat16.cpp     f32 <-> bf16 RNE (bfloat16.cpp:5-36)
//   xstar_cpp/src/ops/mlp.cpp      sigmoid / silu (mlp.cpp:10-26)
// mlp.cpp's Tensor-level mlp() is discarded by --gc-sections (nothing calls it);
// only its scalar sigmoid/silu are reachable.
#include <cstdint>
#include <cstring>
#include "ops/gemm.h"
#include "bfloat16.h"

float sigmoid(float x);   // defined in mlp.cpp:10-21
float silu(float x);      // defined in mlp.cpp:23-26

#define EXPORT extern "C" __attribute__((visibility("default")))

EXPORT void xsref_gemm_f32(const float *A, const float *B, float *C, std::int64_t m,
                           std::int64_t k, std::int64_t n, int transB)
{
    gemm_cpu<float>(A, B, C, m, k, n, transB != 0, k, transB ? k : n, n);
}

EXPORT void xsref_gemm_bf16(const std::uint16_t *A, const std::uint16_t *B, std::uint16_t *C,
                            std::int64_t m, std::int64_t k, std::int64_t n, int transB)
{
    gemm_cpu<bfloat16>(reinterpret_cast<const bfloat16 *>(A), reinterpret_cast<const bfloat16 *>(B),
                       reinterpret_cast<bfloat16 *>(C), m, k, n, transB != 0, k, transB ? k : n, n);
}

EXPORT void xsref_bf16_from_f32(const float *x, std::uint16_t *y, std::int64_t n)
{
    for (std::int64_t i = 0; i < n; ++i) y[i] = bfloat16(x[i]).bits;
}

EXPORT void xsref_sigmoid(const float *x, float *y, std::int64_t n)
{
    for (std::int64_t i = 0; i < n; ++i) y[i] = sigmoid(x[i]);
}

EXPORT void xsref_silu(const float *x, float *y, std::int64_t n)
{
    for (std::int64_t i = 0; i < n; ++i) y[i] = silu(x[i]);
}
