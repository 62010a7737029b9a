// tensor.cpp -- owned/borrowed contiguous buffers (reference contract:
// xstar_cpp/src/tensor.cpp:10-194), device memory through the C ABI.
#include "tensor.h"

#include <cstdlib>
#include <cstring>
#include <new>
#include <stdexcept>
#include <string>

#include "xs_moe.h"

void xs_check(int rc)
{
    if (rc != 0) throw std::runtime_error(std::string("HIP error: ") + xs_last_error());
}

static std::vector<std::int64_t> row_major(const std::vector<std::int64_t> &shape)
{
    std::vector<std::int64_t> s(shape.size());
    std::int64_t st = 1;
    for (std::size_t i = shape.size(); i-- > 0;) {
        s[i] = st;
        st *= shape[i];
    }
    return s;
}

Tensor::Tensor(std::vector<std::int64_t> shape, DType dtype, Device device)
    : shape_(std::move(shape)), dtype_(dtype), device_(device), owns_data_(true)
{
    for (auto d : shape_)
        if (d < 0) throw std::runtime_error("shape mismatch");
    strides_ = row_major(shape_);
    std::size_t nb = nbytes();
    if (device == Device::CPU) {
        std::size_t a = (nb + 63) & ~std::size_t(63);
        data_ = std::aligned_alloc(64, a ? a : 64);
        if (!data_) throw std::bad_alloc();
    } else if (device == Device::CUDA) {
        xs_check(xs_malloc(&data_, nb));
    } else {
        throw std::runtime_error("unsupported device");
    }
}

Tensor::Tensor(const void *ptr, std::vector<std::int64_t> shape, DType dtype, Device device)
    : data_(const_cast<void *>(ptr)), shape_(std::move(shape)), dtype_(dtype), device_(device),
      owns_data_(false)
{
    strides_ = row_major(shape_);
}

Tensor::~Tensor() { release(); }

Tensor::Tensor(Tensor &&o) noexcept
    : data_(o.data_), shape_(std::move(o.shape_)), strides_(std::move(o.strides_)), dtype_(o.dtype_),
      device_(o.device_), owns_data_(o.owns_data_)
{
    o.data_ = nullptr;
    o.owns_data_ = false;
}

Tensor &Tensor::operator=(Tensor &&o) noexcept
{
    if (this != &o) {
        release();
        data_ = o.data_;
        shape_ = std::move(o.shape_);
        strides_ = std::move(o.strides_);
        dtype_ = o.dtype_;
        device_ = o.device_;
        owns_data_ = o.owns_data_;
        o.data_ = nullptr;
        o.owns_data_ = false;
    }
    return *this;
}

std::int64_t Tensor::numel() const
{
    std::int64_t n = 1;
    for (auto d : shape_) n *= d;
    return n;
}

std::size_t Tensor::nbytes() const { return static_cast<std::size_t>(numel()) * dtype_size(dtype_); }

void Tensor::release()
{
    if (data_ && owns_data_) {
        if (device_ == Device::CPU) std::free(data_);
        else xs_free(data_);
    }
    data_ = nullptr;
}

Tensor to_cuda(const Tensor &t)
{
    if (t.device() != Device::CPU) throw std::runtime_error("to_cuda: tensor is not on the CPU");
    Tensor r(t.shape(), t.dtype(), Device::CUDA);
    xs_check(xs_memcpy_h2d(r.data(), t.data(), t.nbytes()));
    return r;
}

Tensor to_cpu(const Tensor &t)
{
    if (t.device() != Device::CUDA) throw std::runtime_error("to_cpu: tensor is not on the device");
    Tensor r(t.shape(), t.dtype(), Device::CPU);
    xs_check(xs_memcpy_d2h(r.data(), t.data(), t.nbytes()));
    return r;
}

std::size_t cuda_free_bytes()
{
    std::size_t f = 0;
    xs_check(xs_free_bytes(&f));
    return f;
}
