// python_bindings.cpp -- the xstar_cpp module: Tensor, raw-byte bridges and
// the MoE ops, following the reference's binding contract
// (bindings/python_bindings.cpp:389-550: enums, Tensor class, from_numpy_raw /
// to_numpy_raw, to_cuda / to_cpu, optional tensors as py::object None ->
// nullptr as in linear_py at :148-162).
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <cstring>
#include <stdexcept>
#include <vector>

#include "ops/moe.h"
#include "ops/moe_weights.h"
#include "ops/rmsnorm.h"
#include "weight_io.h"
#include "tensor.h"

namespace py = pybind11;

// Copy raw bytes from `array`, interpreted as `dtype`; the numpy dtype only
// has to match the element size (bf16 travels as uint16, quantized types as
// uint8).  Reference semantics: bindings/python_bindings.cpp:80-104.
Tensor from_numpy_raw(py::array array, std::vector<std::int64_t> shape, DType dtype)
{
    if (static_cast<std::size_t>(array.itemsize()) != dtype_size(dtype))
        throw std::runtime_error("itemsize mismatch: array itemsize != dtype size");
    std::int64_t numel = 1;
    for (auto s : shape) numel *= s;
    if (array.size() != numel) throw std::runtime_error("byte count mismatch");
    if (!(array.flags() & py::array::c_style)) throw std::runtime_error("array must be C-contiguous");
    Tensor t(shape, dtype, Device::CPU);
    std::memcpy(t.data(), array.data(), t.nbytes());
    return t;
}

// Raw bytes of a host Tensor as a flat uint8 array (inverse of from_numpy_raw).
py::array to_numpy_raw(const Tensor &t)
{
    if (t.device() != Device::CPU) throw std::runtime_error("unsupported device");
    py::array_t<std::uint8_t> a(static_cast<py::ssize_t>(t.nbytes()));
    std::memcpy(a.mutable_data(), t.data(), t.nbytes());
    return a;
}

static const Tensor *opt(py::object o) { return o.is_none() ? nullptr : &o.cast<Tensor &>(); }

Tensor moe_py(Tensor &x, Tensor &router_w, py::object router_bias, Tensor &w13, Tensor &w13_scale,
              Tensor &w2, Tensor &w2_scale, py::object shared_w13, py::object shared_w13_scale,
              py::object shared_w2, py::object shared_w2_scale, std::int64_t top_k, std::int64_t n_group,
              std::int64_t topk_group, bool renormalize, float routed_scaling, int router,
              py::object norm_weight, float norm_eps, py::object residual)
{
    return moe(x, router_w, opt(router_bias), w13, w13_scale, w2, w2_scale, opt(shared_w13),
               opt(shared_w13_scale), opt(shared_w2), opt(shared_w2_scale), top_k, n_group, topk_group,
               renormalize, routed_scaling, router, opt(norm_weight), norm_eps, opt(residual));
}

py::tuple rmsnorm_quant_fp8_py(Tensor &x, Tensor &weight, float eps)
{
    auto r = rmsnorm_quant_fp8(x, weight, eps);
    return py::make_tuple(std::move(std::get<0>(r)), std::move(std::get<1>(r)), std::move(std::get<2>(r)));
}

py::tuple moe_route_py(Tensor &logits, py::object bias, std::int64_t top_k, std::int64_t n_group,
                       std::int64_t topk_group, bool renormalize, float routed_scaling)
{
    auto r = moe_route(logits, opt(bias), top_k, n_group, topk_group, renormalize, routed_scaling);
    return py::make_tuple(std::move(std::get<0>(r)), std::move(std::get<1>(r)));
}

py::tuple moe_permute_py(Tensor &idx, std::int64_t E)
{
    auto r = moe_permute(idx, E);
    return py::make_tuple(std::move(std::get<0>(r)), std::move(std::get<1>(r)), std::move(std::get<2>(r)),
                          std::move(std::get<3>(r)));
}

template <std::tuple<Tensor, Tensor> (*F)(const Tensor &)>
py::tuple pair_py(Tensor &t)
{
    auto r = F(t);
    return py::make_tuple(std::move(std::get<0>(r)), std::move(std::get<1>(r)));
}

// An optional tensor member as a Python attribute: the Tensor (kept alive by
// its owner) or None.
template <std::optional<Tensor> MoeLayerWeights::*F>
py::object opt_member(py::object self)
{
    auto &w = self.cast<MoeLayerWeights &>();
    if (!(w.*F)) return py::none();
    return py::cast(&*(w.*F), py::return_value_policy::reference_internal, self);
}

PYBIND11_MODULE(xstar_cpp, m)
{
    m.doc() = "Xstar MoE operator on MI355X (gfx950): Tensor runtime + MoE ops";

    py::enum_<DType>(m, "DType")
        .value("Float32", DType::Float32)
        .value("BFloat16", DType::BFloat16)
        .value("Float8E4M3", DType::Float8E4M3)
        .value("Float4E2M1x2", DType::Float4E2M1x2)
        .value("Float8E8M0", DType::Float8E8M0)
        .value("Int32", DType::Int32)
        .value("UInt8", DType::UInt8)
        .export_values();
    py::enum_<Device>(m, "Device").value("CPU", Device::CPU).value("CUDA", Device::CUDA).export_values();

    py::class_<Tensor>(m, "Tensor")
        .def(py::init<std::vector<std::int64_t>, DType, Device>(), py::arg("shape"), py::arg("dtype"),
             py::arg("device") = Device::CPU)
        .def("numel", &Tensor::numel)
        .def("nbytes", &Tensor::nbytes)
        .def("shape", &Tensor::shape)
        .def("dtype", &Tensor::dtype)
        .def("device", &Tensor::device);

    m.def("from_numpy_raw", &from_numpy_raw, py::arg("array"), py::arg("shape"), py::arg("dtype"));
    m.def("to_numpy_raw", &to_numpy_raw, py::arg("tensor"));
    m.def("to_cuda", &to_cuda, py::arg("t"));
    m.def("to_cpu", &to_cpu, py::arg("t"));
    m.def("cuda_free_bytes", &cuda_free_bytes);

    m.def("moe", &moe_py, py::arg("x"), py::arg("router_w"), py::arg("router_bias"), py::arg("w13"),
          py::arg("w13_scale"), py::arg("w2"), py::arg("w2_scale"), py::arg("shared_w13") = py::none(),
          py::arg("shared_w13_scale") = py::none(), py::arg("shared_w2") = py::none(),
          py::arg("shared_w2_scale") = py::none(), py::arg("top_k") = 6, py::arg("n_group") = 1,
          py::arg("topk_group") = 1, py::arg("renormalize") = true, py::arg("routed_scaling") = 1.0f,
          py::arg("router") = 1, py::arg("norm_weight") = py::none(), py::arg("norm_eps") = 1e-6f,
          py::arg("residual") = py::none());
    m.def("moe_block_ffn", &moe_block_ffn, py::arg("h"), py::arg("ln2_w"), py::arg("eps"), py::arg("w"),
          py::arg("top_k") = 6, py::arg("n_group") = 1, py::arg("topk_group") = 1, py::arg("renormalize") = true,
          py::arg("routed_scaling") = 1.0f, py::arg("router") = 1);
    m.def("rmsnorm", &rmsnorm, py::arg("x"), py::arg("weight"), py::arg("eps"));
    m.def("rmsnorm_quant_fp8", &rmsnorm_quant_fp8_py, py::arg("x"), py::arg("weight"), py::arg("eps"));
    // safetensors reading (the reference's names and signatures, bindings/python_bindings.cpp:412-424,519-522)
    py::class_<MMapFile>(m, "MMapFile")
        .def(py::init<const std::string &>(), py::arg("path"))
        .def("addr", [](const MMapFile &f) { return reinterpret_cast<std::uintptr_t>(f.addr()); })
        .def("size", &MMapFile::size);
    py::class_<TensorMeta>(m, "TensorMeta")
        .def_readonly("offset", &TensorMeta::offset)
        .def_readonly("shape", &TensorMeta::shape)
        .def_readonly("dtype", &TensorMeta::dtype);
    m.def("make_weight_view", &make_weight_view, py::arg("mf"), py::arg("offset"), py::arg("shape"), py::arg("dtype"),
          py::keep_alive<0, 1>());
    m.def("parse_safetensors_header", &parse_safetensors_header, py::arg("mf"));
    py::class_<MoeLayerWeights>(m, "MoeLayerWeights")
        .def_readonly("E", &MoeLayerWeights::E)
        .def_readonly("H", &MoeLayerWeights::H)
        .def_readonly("I", &MoeLayerWeights::I)
        .def_property_readonly("router_w", &opt_member<&MoeLayerWeights::router_w>)
        .def_property_readonly("router_bias", &opt_member<&MoeLayerWeights::router_bias>)
        .def_property_readonly("w13", &opt_member<&MoeLayerWeights::w13>)
        .def_property_readonly("w13_scale", &opt_member<&MoeLayerWeights::w13_scale>)
        .def_property_readonly("w2", &opt_member<&MoeLayerWeights::w2>)
        .def_property_readonly("w2_scale", &opt_member<&MoeLayerWeights::w2_scale>)
        .def_property_readonly("shared_w13", &opt_member<&MoeLayerWeights::shared_w13>)
        .def_property_readonly("shared_w13_scale", &opt_member<&MoeLayerWeights::shared_w13_scale>)
        .def_property_readonly("shared_w2", &opt_member<&MoeLayerWeights::shared_w2>)
        .def_property_readonly("shared_w2_scale", &opt_member<&MoeLayerWeights::shared_w2_scale>)
        .def_property_readonly("w13_frag", &opt_member<&MoeLayerWeights::w13_frag>)
        .def_property_readonly("w2_frag", &opt_member<&MoeLayerWeights::w2_frag>)
        .def_property_readonly("shared_w13_frag", &opt_member<&MoeLayerWeights::shared_w13_frag>)
        .def_property_readonly("shared_w2_frag", &opt_member<&MoeLayerWeights::shared_w2_frag>)
        .def_property_readonly("w13_scale_frag", &opt_member<&MoeLayerWeights::w13_scale_frag>)
        .def_property_readonly("w2_scale_frag", &opt_member<&MoeLayerWeights::w2_scale_frag>);
    m.def("pack_moe_layer_frag", &pack_moe_layer_frag, py::arg("w"), py::arg("packed_only") = false);
    m.def("load_moe_layer", &load_moe_layer, py::arg("paths"), py::arg("prefix"), py::arg("device") = Device::CUDA);

    m.def("moe_router_logits", &moe_router_logits, py::arg("x"), py::arg("router_w"), py::arg("exact") = false);
    m.def("moe_route", &moe_route_py, py::arg("logits"), py::arg("bias"), py::arg("top_k"),
          py::arg("n_group") = 1, py::arg("topk_group") = 1, py::arg("renormalize") = true,
          py::arg("routed_scaling") = 1.0f);
    m.def("moe_permute", &moe_permute_py, py::arg("idx"), py::arg("num_experts"));
    m.def("quant_act_fp8", &pair_py<quant_act_fp8>, py::arg("x"));
    m.def("quant_act_mxfp8", &pair_py<quant_act_mxfp8>, py::arg("x"));
    m.def("quant_weight_fp8_block", &pair_py<quant_weight_fp8_block>, py::arg("w"));
    m.def("quant_weight_mxfp4", &pair_py<quant_weight_mxfp4>, py::arg("w"));
    m.def("gemm_fp8_blockscale", &gemm_fp8_blockscale, py::arg("x"), py::arg("b"), py::arg("b_scale"));
}
