#pragma once
#include <cstdint>
#include <optional>
#include <string>
#include <vector>

#include "tensor.h"

/**
 * One MoE layer's weights in the layout moe() takes, assembled from
 * safetensors checkpoints (DeepSeek-V3-style names under `prefix`, e.g.
 * "model.layers.3.mlp"):
 *   {prefix}.gate.weight                          router [E, H], F32 or BF16
 *   {prefix}.gate.e_score_correction_bias         [E] (optional; stored as F32)
 *   {prefix}.experts.{e}.{gate,up,down}_proj.weight
 *   {prefix}.experts.{e}.{gate,up,down}_proj.weight_scale_inv   (FP8 checkpoints)
 *   {prefix}.shared_experts.{gate,up,down}_proj.weight[_scale_inv]   (optional)
 * FP8 checkpoints (F8_E4M3 weights with F32 128x128 dequant scales) are copied
 * as they are; gate and up are stacked per expert into w13 = [gate ; up]
 * (the reference's fused gate_up, xstar_cpp/src/qwen2_model.cpp:187-206).
 * Dense checkpoints (BF16 / F32 expert weights, no scales) are quantized on the
 * GPU to FP8 with 128x128 block scales while loading (xs_quant_weight_fp8_block).
 * The reference reads F32 / BF16 only (xstar_cpp/src/weight_io.cpp:122-127).
 */
struct MoeLayerWeights
{
    std::int64_t E = 0, H = 0, I = 0;
    // always set by load_moe_layer
    std::optional<Tensor> router_w;            // [E, H], dtype as stored
    std::optional<Tensor> w13, w13_scale;      // [E, 2I, H] Float8E4M3, [E, 2I/128, H/128] Float32
    std::optional<Tensor> w2, w2_scale;        // [E, H, I] Float8E4M3, [E, H/128, I/128] Float32
    // set when present in the checkpoint
    std::optional<Tensor> router_bias;         // [E] Float32
    std::optional<Tensor> shared_w13, shared_w13_scale, shared_w2, shared_w2_scale;  // 2-D, same formats
    // set by pack_moe_layer_frag: the weights again, in MFMA fragment order
    // (MXFP4 layers: also their scales; the shared expert is FP8)
    std::optional<Tensor> w13_frag, w2_frag, shared_w13_frag, shared_w2_frag, w13_scale_frag, w2_scale_frag;
};

/**
 * Loads the layer under `prefix` from one or more safetensors files (a sharded
 * checkpoint: each name must appear in exactly one file) onto `device`.
 * Device::CPU keeps FP8 checkpoints on the host (dense ones need the GPU).
 * Throws std::runtime_error: "missing weight key: <name>", "shape mismatch: <name>",
 * "dtype mismatch: <name>", "duplicate weight key: <name>", "unsupported device",
 * and the parser's messages.
 */
MoeLayerWeights load_moe_layer(const std::vector<std::string> &paths, const std::string &prefix, Device device);

/**
 * Adds fragment-packed copies of the layer's expert weights (CUDA only;
 * xs_pack_weight_fp8_frag, and for MXFP4 routed experts
 * xs_pack_weight_mxfp4_frag with their scales), which moe_block_ffn then hands
 * to the GEMMs that load weights straight into registers.  The results are the
 * same bits.  packed_only = false keeps the row-major weights too (twice the
 * device memory); true drops them (w13, w2 and the shared expert's become
 * empty), and every GEMM of the layer is then a weight-direct one.  No
 * reference counterpart.  Throws "unsupported device" (host weights) and
 * "unsupported dtype".
 */
void pack_moe_layer_frag(MoeLayerWeights &w, bool packed_only = false);
