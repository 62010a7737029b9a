// rmsnorm.cpp -- Tensor-level RMSNorm ops over the C ABI (xs_rmsnorm), with the
// validation order and messages of xstar_cpp/src/ops/rmsnorm.cpp:6-20.
#include "ops/rmsnorm.h"

#include <stdexcept>

#include "xs_moe.h"

namespace {

void check_args(const Tensor &x, const Tensor &weight, bool quant)
{
    if (x.dtype() != weight.dtype())
        throw std::runtime_error("rmsnorm: x and weight must have the same dtype");
    if (x.shape().size() < 1 || weight.shape().size() != 1)
        throw std::runtime_error("rmsnorm expects x rank >= 1 and weight 1D");
    if (x.shape().back() != weight.shape()[0]) throw std::runtime_error("shape mismatch");
    if (quant && x.shape().back() % 128 != 0) throw std::runtime_error("shape mismatch");
    if (x.device() != weight.device()) throw std::runtime_error("device mismatch");
    if (x.dtype() != DType::Float32 && x.dtype() != DType::BFloat16) throw std::runtime_error("unsupported dtype");
    if (x.device() != Device::CUDA) throw std::runtime_error("unsupported device");
}

std::int64_t rows_of(const Tensor &x)
{
    const std::int64_t h = x.shape().back();
    return h ? x.numel() / h : 0;
}

}  // namespace

Tensor rmsnorm(const Tensor &x, const Tensor &weight, float eps)
{
    check_args(x, weight, false);
    Tensor y(x.shape(), x.dtype(), x.device());
    xs_check(xs_rmsnorm(x.data(), weight.data(), static_cast<int>(x.dtype()), rows_of(x), x.shape().back(), eps,
                        y.data(), nullptr, nullptr, nullptr));
    xs_check(xs_stream_synchronize(nullptr));
    return y;
}

std::tuple<Tensor, Tensor, Tensor> rmsnorm_quant_fp8(const Tensor &x, const Tensor &weight, float eps)
{
    check_args(x, weight, true);
    const std::int64_t h = x.shape().back();
    Tensor y(x.shape(), x.dtype(), x.device());
    Tensor q(x.shape(), DType::Float8E4M3, x.device());
    std::vector<std::int64_t> ss(x.shape());
    ss.back() = h / 128;
    Tensor s(ss, DType::Float32, x.device());
    xs_check(xs_rmsnorm(x.data(), weight.data(), static_cast<int>(x.dtype()), rows_of(x), h, eps, y.data(),
                        static_cast<std::uint8_t *>(q.data()), static_cast<float *>(s.data()), nullptr));
    xs_check(xs_stream_synchronize(nullptr));
    return {std::move(y), std::move(q), std::move(s)};
}
