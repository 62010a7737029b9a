#pragma once
#include <cstddef>
#include <stdexcept>

/**
 * Element types of a Tensor.  Float32 / BFloat16 keep the reference's names and
 * order (xstar_cpp/include/dtype.h:8-12) and their numeric values match
 * xs_dtype in include/xs_moe.h.  The quantized types follow torch's storage
 * convention: Float4E2M1x2 is one byte holding two E2M1 values (element 2i in
 * the low nibble), so a packed [n, k] matrix is a [n, k/2] tensor and
 * nbytes == numel * dtype_size for every dtype.
 */
enum class DType
{
    Float32 = 0,      // 4 bytes
    BFloat16 = 1,     // 2 bytes
    Float8E4M3 = 2,   // 1 byte, OCP E4M3FN
    Float4E2M1x2 = 3, // 1 byte = 2 x OCP E2M1
    Float8E8M0 = 4,   // 1 byte, OCP E8M0 scale
    Int32 = 5,        // 4 bytes
    UInt8 = 6,        // 1 byte (raw workspace)
};

inline std::size_t dtype_size(DType d)
{
    switch (d)
    {
    case DType::Float32:
    case DType::Int32:
        return 4;
    case DType::BFloat16:
        return 2;
    case DType::Float8E4M3:
    case DType::Float4E2M1x2:
    case DType::Float8E8M0:
    case DType::UInt8:
        return 1;
    }
    throw std::runtime_error("unknown DType");
}
