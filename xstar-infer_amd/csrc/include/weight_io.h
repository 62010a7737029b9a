#pragma once
#include <cstddef>
#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

#include "mmap_file.h"
#include "tensor.h"

/**
 * One tensor of a safetensors header (the reference's TensorMeta,
 * xstar_cpp/include/weight_io.h:13-18): offset from the FILE START (8-byte
 * length prefix and header included), shape, dtype.
 */
struct TensorMeta
{
    std::size_t offset;
    std::vector<std::int64_t> shape;
    DType dtype;
};

/**
 * Host view (non-owning, Device::CPU) of `shape` x `dtype` at `offset` in the
 * mapping (xstar_cpp/include/weight_io.h:23).  Throws "offset not aligned to
 * dtype size" and "weight view exceeds mmap region".
 */
Tensor make_weight_view(MMapFile &mf, std::size_t offset, std::vector<std::int64_t> shape, DType dtype);

/**
 * Parses the safetensors header of `mf` (xstar_cpp/include/weight_io.h:25-56):
 * [u64 LE header length][JSON object name -> {dtype, shape, data_offsets}][data].
 * "__metadata__" is skipped.  Accepted dtypes: F32, BF16 (the reference's),
 * and F8_E4M3, F8_E8M0, U8, I32 for quantized checkpoints (FP8 weights with
 * their f32 weight_scale_inv, packed FP4 bytes with e8m0 scales).
 * Throws std::runtime_error with the reference's messages: "file smaller than 8
 * bytes", "header_len exceeds remaining file bytes (truncated header)",
 * "dtype not supported ...", "header inconsistent: ...", JSON syntax errors.
 */
std::unordered_map<std::string, TensorMeta> parse_safetensors_header(const MMapFile &mf);
