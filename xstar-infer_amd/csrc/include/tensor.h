#pragma once
#include <cstddef>
#include <cstdint>
#include <vector>

#include "dtype.h"
#include "device.h"

/**
 * Contiguous row-major buffer of one dtype on one device, owned or borrowed.
 * Same contract as the reference's Tensor (xstar_cpp/include/tensor.h:16-75):
 *   - Tensor(shape, dtype, device) OWNS: 64-byte aligned host memory, or device
 *     memory from xs_malloc (256-byte aligned), freed on destruction;
 *   - Tensor(ptr, shape, dtype, device) BORROWS external memory (not freed);
 *   - move-only (copy would double free).
 */
class Tensor
{
public:
    Tensor(std::vector<std::int64_t> shape, DType dtype, Device device = Device::CPU);
    Tensor(const void *ptr, std::vector<std::int64_t> shape, DType dtype, Device device);
    ~Tensor();

    Tensor(const Tensor &) = delete;
    Tensor &operator=(const Tensor &) = delete;
    Tensor(Tensor &&other) noexcept;
    Tensor &operator=(Tensor &&other) noexcept;

    const std::vector<std::int64_t> &shape() const { return shape_; }
    const std::vector<std::int64_t> &strides() const { return strides_; }
    DType dtype() const { return dtype_; }
    Device device() const { return device_; }
    std::int64_t numel() const;
    std::size_t nbytes() const;
    void *data() { return data_; }
    const void *data() const { return data_; }

private:
    void *data_ = nullptr;
    std::vector<std::int64_t> shape_;
    std::vector<std::int64_t> strides_;
    DType dtype_ = DType::Float32;
    Device device_ = Device::CPU;
    bool owns_data_ = false;

    void release();
};

/** H2D copy into a new owned device Tensor; throws unless t is on the CPU
 * (reference: xstar_cpp/include/tensor.h:77-93). */
Tensor to_cuda(const Tensor &t);
/** D2H copy into a new owned host Tensor; throws unless t is on the device. */
Tensor to_cpu(const Tensor &t);
/** Free device memory in bytes (reference: cuda_free_bytes). */
std::size_t cuda_free_bytes();

/** Throws std::runtime_error("HIP error: <message>") for a non-zero xs_status,
 * the CHECK_CUDA convention of xstar_cpp/include/cuda/cuda_check.h:23-31. */
void xs_check(int rc);
