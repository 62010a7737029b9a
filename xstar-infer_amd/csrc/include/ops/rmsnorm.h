#pragma once
#include <tuple>

#include "tensor.h"

/**
 * RMSNorm over the last axis: y = x * inv_rms * weight, inv_rms =
 * 1 / sqrt(mean(x^2) + eps) in f32.  Same signature, checks and messages as the
 * reference op (xstar_cpp/include/ops/rmsnorm.h, xstar_cpp/src/ops/rmsnorm.cpp:6-20):
 *   x [..., hidden] Float32 | BFloat16, weight [hidden] of the same dtype.
 * Numerics of the reference CPU path (rmsnorm.cpp:27-73): bf16 rounds x * inv_rms
 * to bf16 before the weight multiply; the f32 sum of squares is taken in a
 * different order (per lane, then across lanes), so results may differ from the
 * sequential CPU sum by an ulp of inv_rms.
 * Device CUDA only: a CPU tensor throws "unsupported device" (this library has
 * no CPU compute path).  Synchronous at return.
 * Throws: "rmsnorm: x and weight must have the same dtype", "rmsnorm expects x
 * rank >= 1 and weight 1D", "shape mismatch", "device mismatch",
 * "unsupported dtype", "unsupported device".
 */
Tensor rmsnorm(const Tensor &x, const Tensor &weight, float eps);

/** rmsnorm fused with the FP8 1x128 activation quantization of its output:
 * (y, q Float8E4M3 [..., hidden], scales Float32 [..., hidden/128]).
 * hidden % 128 == 0.  q and scales equal quant_act_fp8(y). */
std::tuple<Tensor, Tensor, Tensor> rmsnorm_quant_fp8(const Tensor &x, const Tensor &weight, float eps);
