#pragma once
#include <cstdint>
#include <tuple>

#include "ops/moe_weights.h"
#include "tensor.h"

/**
 * Mixture-of-experts FFN layer (DeepSeek-V4-Flash shape: sigmoid router with
 * bias, top-k routed experts + optional shared expert, SwiGLU experts).
 * Drop-in for mlp(x, gate_up_weight, down_weight) (xstar_cpp/include/ops/mlp.h:51)
 * at the transformer_block call sites; same op idiom: validate, allocate the
 * output on x.device(), dispatch.
 *
 *   x                [..., H]            Float32 | BFloat16, device CUDA
 *   router_w         [E, H]              same dtype as x
 *   router_bias      [E] Float32 or nullptr
 *   w13              [E, 2I, H] Float8E4M3 with w13_scale [E, 2I/128, H/128] Float32
 *                    or [E, 2I, H/2] Float4E2M1x2 with w13_scale [E, 2I, H/32] Float8E8M0
 *                    rows are [gate ; up] (xstar_cpp/include/ops/mlp.h:4-14)
 *   w2               [E, H, I] Float8E4M3 with w2_scale [E, H/128, I/128] Float32
 *                    or [E, H, I/2] Float4E2M1x2 with w2_scale [E, H, I/32] Float8E8M0
 *   shared_*         one FP8 expert (2-D shapes of the above) or all nullptr
 *   top_k, n_group, topk_group, renormalize, routed_scaling: routing options
 *   residual         [..., H] dtype of x, or nullptr: added to the output (in f32,
 *                    before its one rounding)
 *   norm_weight      [H] dtype of x, or nullptr: the layer computes
 *                    moe(rmsnorm(x, norm_weight, norm_eps)) with the norm fused
 *                    into the activation quantization (ops/rmsnorm.h numerics)
 *   returns          [..., H], dtype of x, device CUDA
 *
 *   router           0 bf16 MFMA logits (approximate routing); 1 (default)
 *                    certified: top-k indices, order and counts bit-exact with
 *                    the reference's gemm_cpu logits; 2 every logit in
 *                    gemm_cpu order (xs_moe.h, XS_ROUTER_*)
 *
 * Numerics: routing bit-exact with the CPU restatement (router 1 or 2);
 * expert GEMMs in FP8 (or MXFP4 x MXFP8) with f32 accumulation; SwiGLU in f32
 * (branched sigmoid, xstar_cpp/src/ops/mlp.cpp:10-26); combine in f32 with one
 * cast to the output dtype.
 *
 * Throws std::runtime_error: "rank mismatch", "dtype mismatch", "shape mismatch",
 * "device mismatch", "unsupported dtype", "unsupported device" (the reference's
 * messages, xstar_cpp/src/ops/mlp.cpp:49-58), "HIP error: ..." from the library.
 * Synchronous at return, like the reference's launchers.
 */
Tensor moe(const Tensor &x, const Tensor &router_w, const Tensor *router_bias,
           const Tensor &w13, const Tensor &w13_scale, const Tensor &w2, const Tensor &w2_scale,
           const Tensor *shared_w13, const Tensor *shared_w13_scale,
           const Tensor *shared_w2, const Tensor *shared_w2_scale,
           std::int64_t top_k, std::int64_t n_group = 1, std::int64_t topk_group = 1,
           bool renormalize = true, float routed_scaling = 1.0f, int router = 1,
           const Tensor *norm_weight = nullptr, float norm_eps = 1e-6f, const Tensor *residual = nullptr);

/**
 * The FFN half of a MoE transformer block in one call: h + moe(rmsnorm(h, ln2_w, eps)),
 * the line `add(attention_x, mlp(rmsnorm(attention_x, ln2_w, eps), gate_up_w, down_w))`
 * of xstar_cpp/src/ops/transformer_block.cpp:75,353 with the MoE in place of mlp().
 * The norm is fused into the activation quantization and the residual into the
 * combine (added in f32 before the output's one rounding).  `w` comes from
 * load_moe_layer (ops/moe_weights.h); after pack_moe_layer_frag(w) its packed
 * FP8 weights go to the GEMMs that load weights straight into registers (same
 * bits).  Same checks and messages as moe().
 */
Tensor moe_block_ffn(const Tensor &h, const Tensor &ln2_w, float eps, const MoeLayerWeights &w, std::int64_t top_k,
                     std::int64_t n_group = 1, std::int64_t topk_group = 1, bool renormalize = true,
                     float routed_scaling = 1.0f, int router = 1);

/** Router logits x . router_w^T in f32 ([T, E]); exact: bit-identical to
 * gemm_cpu's sequential accumulation (xstar_cpp/include/ops/gemm.h:57-83). */
Tensor moe_router_logits(const Tensor &x, const Tensor &router_w, bool exact);

/** Top-k routing on f32 logits [T, E] -> (idx [T, k] Int32, weights [T, k] Float32). */
std::tuple<Tensor, Tensor> moe_route(const Tensor &logits, const Tensor *bias, std::int64_t top_k,
                                     std::int64_t n_group, std::int64_t topk_group,
                                     bool renormalize, float routed_scaling);

/** Stable sort of slots by expert: idx [T, k] Int32 ->
 * (counts [E], offsets [E+1], perm [T*k], inv [T*k]), all Int32. */
std::tuple<Tensor, Tensor, Tensor, Tensor> moe_permute(const Tensor &idx, std::int64_t num_experts);

/** Activation quantizers: x [rows, cols] -> (q Float8E4M3, scales Float32 [rows, cols/128])
 * or MXFP8 (q Float8E4M3, scales Float8E8M0 [rows, cols/32]). */
std::tuple<Tensor, Tensor> quant_act_fp8(const Tensor &x);
std::tuple<Tensor, Tensor> quant_act_mxfp8(const Tensor &x);

/** Weight quantizers: w [..., n, k] -> FP8 128x128 (q, Float32 scales) or MXFP4. */
std::tuple<Tensor, Tensor> quant_weight_fp8_block(const Tensor &w);
std::tuple<Tensor, Tensor> quant_weight_mxfp4(const Tensor &w);

/** C = x . dequant(B)^T for bf16 x [M, K] and FP8 B [N, K] with 128x128 scales;
 * bf16 [M, N]. */
Tensor gemm_fp8_blockscale(const Tensor &x, const Tensor &b, const Tensor &b_scale);
