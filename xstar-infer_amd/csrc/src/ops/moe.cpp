// moe.cpp -- Tensor-level MoE ops: validate, allocate outputs on x.device(),
// call the C ABI, synchronise (the op idiom of xstar_cpp/src/ops/mlp.cpp:47-86).
#include "ops/moe.h"

#include <stdexcept>

#include "xs_moe.h"

namespace {

int code(DType d) { return static_cast<int>(d); }

void require_cuda(const Tensor &t)
{
    if (t.device() != Device::CUDA) throw std::runtime_error("unsupported device");
}

void same_device(const Tensor &a, const Tensor &b)
{
    if (a.device() != b.device()) throw std::runtime_error("device mismatch");
}

bool is_act(DType d) { return d == DType::Float32 || d == DType::BFloat16; }

std::int64_t rows_of(const Tensor &x) { return x.numel() / x.shape().back(); }

void sync() { xs_check(xs_stream_synchronize(nullptr)); }

}  // namespace

namespace {
// fragment-packed copies of the FP8 weights (pack_moe_layer_frag), or none
struct Frag {
    const Tensor *w13 = nullptr, *w2 = nullptr, *shared_w13 = nullptr, *shared_w2 = nullptr;
    const Tensor *w13_scale = nullptr, *w2_scale = nullptr;   // MXFP4 layers
    bool only = false;   // packed copies alone: the weight arguments are the packed tensors
};
}  // namespace

static Tensor moe_core(const Tensor &x, const Tensor &router_w, const Tensor *router_bias,
                       const Tensor &w13, const Tensor &w13_scale, const Tensor &w2, const Tensor &w2_scale,
                       const Tensor *shared_w13, const Tensor *shared_w13_scale,
                       const Tensor *shared_w2, const Tensor *shared_w2_scale,
                       std::int64_t top_k, std::int64_t n_group, std::int64_t topk_group,
                       bool renormalize, float routed_scaling, int router,
                       const Tensor *norm_weight, float norm_eps, const Tensor *residual, const Frag &frag)
{
    // ---- dtype ----
    if (!is_act(x.dtype())) throw std::runtime_error("unsupported dtype");
    if (router_w.dtype() != x.dtype()) throw std::runtime_error("dtype mismatch");
    if (router_bias && router_bias->dtype() != DType::Float32) throw std::runtime_error("dtype mismatch");
    if (norm_weight && norm_weight->dtype() != x.dtype()) throw std::runtime_error("dtype mismatch");
    if (residual && residual->dtype() != x.dtype()) throw std::runtime_error("dtype mismatch");
    const bool fp4 = w13.dtype() == DType::Float4E2M1x2;
    const DType wq = fp4 ? DType::Float4E2M1x2 : DType::Float8E4M3;
    const DType ws = fp4 ? DType::Float8E8M0 : DType::Float32;
    if (w13.dtype() != DType::Float8E4M3 && !fp4) throw std::runtime_error("unsupported dtype");
    if (w2.dtype() != wq || w13_scale.dtype() != ws || w2_scale.dtype() != ws)
        throw std::runtime_error("dtype mismatch");
    const int n_shared = (shared_w13 != nullptr) + (shared_w13_scale != nullptr) +
                         (shared_w2 != nullptr) + (shared_w2_scale != nullptr);
    if (n_shared != 0 && n_shared != 4) throw std::runtime_error("shape mismatch");
    const bool has_shared = n_shared == 4;
    if (has_shared && (shared_w13->dtype() != DType::Float8E4M3 || shared_w2->dtype() != DType::Float8E4M3 ||
                       shared_w13_scale->dtype() != DType::Float32 || shared_w2_scale->dtype() != DType::Float32))
        throw std::runtime_error("dtype mismatch");
    // ---- rank ----
    if (x.shape().size() < 1 || router_w.shape().size() != 2 || w13.shape().size() != 3 ||
        w2.shape().size() != 3 || w13_scale.shape().size() != 3 || w2_scale.shape().size() != 3 ||
        (router_bias && router_bias->shape().size() != 1) || (norm_weight && norm_weight->shape().size() != 1))
        throw std::runtime_error("rank mismatch");
    if (has_shared && (shared_w13->shape().size() != 2 || shared_w2->shape().size() != 2 ||
                       shared_w13_scale->shape().size() != 2 || shared_w2_scale->shape().size() != 2))
        throw std::runtime_error("rank mismatch");
    // ---- shape ----
    const std::int64_t H = x.shape().back();
    const std::int64_t E = router_w.shape()[0];
    const std::int64_t I = fp4 ? w2.shape()[2] * 2 : w2.shape()[2];
    const std::int64_t hk = fp4 ? H / 2 : H;
    auto eq = [](const std::vector<std::int64_t> &s, std::initializer_list<std::int64_t> v) {
        return s == std::vector<std::int64_t>(v);
    };
    bool ok = router_w.shape()[1] == H && eq(w13.shape(), {E, 2 * I, hk}) && eq(w2.shape(), {E, H, fp4 ? I / 2 : I}) &&
              (!router_bias || router_bias->shape()[0] == E) && (!norm_weight || norm_weight->shape()[0] == H) &&
              (!residual || residual->shape() == x.shape()) &&
              H % 256 == 0 && I % 128 == 0;
    if (ok) {
        if (fp4) ok = eq(w13_scale.shape(), {E, 2 * I, H / 32}) && eq(w2_scale.shape(), {E, H, I / 32});
        else ok = eq(w13_scale.shape(), {E, 2 * I / 128, H / 128}) && eq(w2_scale.shape(), {E, H / 128, I / 128});
    }
    if (ok && has_shared)
        ok = eq(shared_w13->shape(), {2 * I, H}) && eq(shared_w2->shape(), {H, I}) &&
             eq(shared_w13_scale->shape(), {2 * I / 128, H / 128}) && eq(shared_w2_scale->shape(), {H / 128, I / 128});
    if (!ok || top_k < 1 || top_k > E) throw std::runtime_error("shape mismatch");
    // ---- device ----
    for (const Tensor *t : {&router_w, &w13, &w13_scale, &w2, &w2_scale}) same_device(x, *t);
    if (router_bias) same_device(x, *router_bias);
    if (norm_weight) same_device(x, *norm_weight);
    if (residual) same_device(x, *residual);
    if (has_shared)
        for (const Tensor *t : {shared_w13, shared_w13_scale, shared_w2, shared_w2_scale}) same_device(x, *t);
    require_cuda(x);

    Tensor out(x.shape(), x.dtype(), x.device());
    xs_moe_params p{};
    p.T = rows_of(x);
    p.H = H;
    p.I = I;
    p.E = E;
    p.top_k = top_k;
    p.n_group = n_group;
    p.topk_group = topk_group;
    p.renormalize = renormalize ? 1 : 0;
    p.routed_scaling = routed_scaling;
    p.x_dtype = code(x.dtype());
    p.routed_format = fp4 ? XS_FP4_E2M1X2 : XS_FP8_E4M3;
    p.has_shared = has_shared ? 1 : 0;
    if (router < XS_ROUTER_MFMA || router > XS_ROUTER_CHAIN) throw std::runtime_error("unsupported router");
    p.router_exact = router;
    p.has_norm = norm_weight ? 1 : 0;
    p.norm_eps = norm_eps;
    std::size_t wsb = xs_moe_workspace_size(&p);
    if (wsb == 0) throw std::runtime_error("shape mismatch");
    Tensor wsp({static_cast<std::int64_t>(wsb)}, DType::UInt8, Device::CUDA);
    xs_moe_tensors t{};
    t.x = x.data();
    t.router_w = router_w.data();
    t.router_bias = router_bias ? static_cast<const float *>(router_bias->data()) : nullptr;
    t.w13 = w13.data();
    t.w13_scale = w13_scale.data();
    t.w2 = w2.data();
    t.w2_scale = w2_scale.data();
    if (has_shared) {
        t.shared_w13 = shared_w13->data();
        t.shared_w13_scale = static_cast<const float *>(shared_w13_scale->data());
        t.shared_w2 = shared_w2->data();
        t.shared_w2_scale = static_cast<const float *>(shared_w2_scale->data());
    }
    if (frag.w13 && frag.w2 && (!fp4 || (frag.w13_scale && frag.w2_scale))) {
        for (const Tensor *f : {frag.w13, frag.w2, frag.shared_w13, frag.shared_w2, frag.w13_scale, frag.w2_scale})
            if (f) same_device(x, *f);
        if (frag.w13->nbytes() != w13.nbytes() || frag.w2->nbytes() != w2.nbytes() ||
            (fp4 && (frag.w13_scale->nbytes() != w13_scale.nbytes() || frag.w2_scale->nbytes() != w2_scale.nbytes())) ||
            (frag.shared_w13 && has_shared && frag.shared_w13->nbytes() != shared_w13->nbytes()) ||
            (frag.shared_w2 && has_shared && frag.shared_w2->nbytes() != shared_w2->nbytes()))
            throw std::runtime_error("shape mismatch");
        t.w13_frag = frag.w13->data();
        t.w2_frag = frag.w2->data();
        if (fp4) {
            t.w13_scale_frag = frag.w13_scale->data();
            t.w2_scale_frag = frag.w2_scale->data();
        }
        if (has_shared && frag.shared_w13 && frag.shared_w2) {
            t.shared_w13_frag = frag.shared_w13->data();
            t.shared_w2_frag = frag.shared_w2->data();
        }
        if (frag.only) {   // no row-major copies: every GEMM reads the packed ones
            t.w13 = nullptr;
            t.w2 = nullptr;
            t.shared_w13 = nullptr;
            t.shared_w2 = nullptr;
        }
    }
    t.out = out.data();
    t.norm_weight = norm_weight ? norm_weight->data() : nullptr;
    t.residual = residual ? residual->data() : nullptr;
    xs_check(xs_moe_forward(&p, &t, wsp.data(), wsb, nullptr));
    sync();
    return out;
}

Tensor moe(const Tensor &x, const Tensor &router_w, const Tensor *router_bias,
           const Tensor &w13, const Tensor &w13_scale, const Tensor &w2, const Tensor &w2_scale,
           const Tensor *shared_w13, const Tensor *shared_w13_scale,
           const Tensor *shared_w2, const Tensor *shared_w2_scale,
           std::int64_t top_k, std::int64_t n_group, std::int64_t topk_group,
           bool renormalize, float routed_scaling, int router,
           const Tensor *norm_weight, float norm_eps, const Tensor *residual)
{
    return moe_core(x, router_w, router_bias, w13, w13_scale, w2, w2_scale, shared_w13, shared_w13_scale, shared_w2,
                    shared_w2_scale, top_k, n_group, topk_group, renormalize, routed_scaling, router, norm_weight,
                    norm_eps, residual, Frag{});
}

Tensor moe_block_ffn(const Tensor &h, const Tensor &ln2_w, float eps, const MoeLayerWeights &w, std::int64_t top_k,
                     std::int64_t n_group, std::int64_t topk_group, bool renormalize, float routed_scaling,
                     int router)
{
    // packed-only layers (pack_moe_layer_frag(w, true)) carry their shapes and
    // dtypes in the packed tensors
    const bool only = !w.w13 && !w.w2 && w.w13_frag && w.w2_frag;
    if (!w.router_w || !w.w13_scale || !w.w2_scale || (!only && (!w.w13 || !w.w2)))
        throw std::runtime_error("shape mismatch");
    auto p = [](const std::optional<Tensor> &t) { return t ? &*t : nullptr; };
    Frag f{p(w.w13_frag), p(w.w2_frag), p(w.shared_w13_frag), p(w.shared_w2_frag), p(w.w13_scale_frag),
           p(w.w2_scale_frag)};
    f.only = only;
    const Tensor &w13 = only ? *w.w13_frag : *w.w13, &w2 = only ? *w.w2_frag : *w.w2;
    const Tensor *sw13 = only ? p(w.shared_w13_frag) : p(w.shared_w13), *sw2 = only ? p(w.shared_w2_frag) : p(w.shared_w2);
    return moe_core(h, *w.router_w, p(w.router_bias), w13, *w.w13_scale, w2, *w.w2_scale, sw13, p(w.shared_w13_scale),
                    sw2, p(w.shared_w2_scale), top_k, n_group, topk_group, renormalize, routed_scaling, router,
                    &ln2_w, eps, &h, f);
}

Tensor moe_router_logits(const Tensor &x, const Tensor &router_w, bool exact)
{
    if (!is_act(x.dtype())) throw std::runtime_error("unsupported dtype");
    if (x.dtype() != router_w.dtype()) throw std::runtime_error("dtype mismatch");
    if (x.shape().size() < 1 || router_w.shape().size() != 2) throw std::runtime_error("rank mismatch");
    const std::int64_t H = x.shape().back(), E = router_w.shape()[0];
    if (router_w.shape()[1] != H || H % 128 != 0) throw std::runtime_error("shape mismatch");
    same_device(x, router_w);
    require_cuda(x);
    std::vector<std::int64_t> os(x.shape());
    os.back() = E;
    Tensor out(os, DType::Float32, Device::CUDA);
    xs_check(xs_moe_router_logits(x.data(), router_w.data(), code(x.dtype()), rows_of(x), E, H, exact ? 1 : 0,
                                  static_cast<float *>(out.data()), nullptr));
    sync();
    return out;
}

std::tuple<Tensor, Tensor> moe_route(const Tensor &logits, const Tensor *bias, std::int64_t top_k,
                                     std::int64_t n_group, std::int64_t topk_group, bool renormalize,
                                     float routed_scaling)
{
    if (logits.dtype() != DType::Float32 || (bias && bias->dtype() != DType::Float32))
        throw std::runtime_error("dtype mismatch");
    if (logits.shape().size() != 2 || (bias && bias->shape().size() != 1)) throw std::runtime_error("rank mismatch");
    const std::int64_t T = logits.shape()[0], E = logits.shape()[1];
    if ((bias && bias->shape()[0] != E) || top_k < 1 || top_k > E) throw std::runtime_error("shape mismatch");
    if (bias) same_device(logits, *bias);
    require_cuda(logits);
    Tensor idx({T, top_k}, DType::Int32, Device::CUDA);
    Tensor w({T, top_k}, DType::Float32, Device::CUDA);
    xs_check(xs_moe_route(static_cast<const float *>(logits.data()),
                          bias ? static_cast<const float *>(bias->data()) : nullptr, T, E, top_k, n_group,
                          topk_group, renormalize ? 1 : 0, routed_scaling, static_cast<int32_t *>(idx.data()),
                          static_cast<float *>(w.data()), nullptr));
    sync();
    return {std::move(idx), std::move(w)};
}

std::tuple<Tensor, Tensor, Tensor, Tensor> moe_permute(const Tensor &idx, std::int64_t E)
{
    if (idx.dtype() != DType::Int32) throw std::runtime_error("dtype mismatch");
    if (idx.shape().size() != 2) throw std::runtime_error("rank mismatch");
    require_cuda(idx);
    const std::int64_t T = idx.shape()[0], k = idx.shape()[1];
    Tensor counts({E}, DType::Int32, Device::CUDA), offsets({E + 1}, DType::Int32, Device::CUDA);
    Tensor perm({T * k}, DType::Int32, Device::CUDA), inv({T * k}, DType::Int32, Device::CUDA);
    std::size_t wsb = xs_moe_permute_workspace_size(T, E);
    Tensor ws({static_cast<std::int64_t>(wsb)}, DType::UInt8, Device::CUDA);
    xs_check(xs_moe_permute(static_cast<const int32_t *>(idx.data()), T, E, k, static_cast<int32_t *>(counts.data()),
                            static_cast<int32_t *>(offsets.data()), static_cast<int32_t *>(perm.data()),
                            static_cast<int32_t *>(inv.data()), ws.data(), wsb, nullptr));
    sync();
    return {std::move(counts), std::move(offsets), std::move(perm), std::move(inv)};
}

static std::tuple<Tensor, Tensor> quant_act(const Tensor &x, bool mx)
{
    if (!is_act(x.dtype())) throw std::runtime_error("unsupported dtype");
    if (x.shape().size() != 2) throw std::runtime_error("rank mismatch");
    const std::int64_t R = x.shape()[0], Cc = x.shape()[1];
    if (Cc % (mx ? 32 : 128) != 0) throw std::runtime_error("shape mismatch");
    require_cuda(x);
    Tensor q({R, Cc}, DType::Float8E4M3, Device::CUDA);
    if (mx) {
        Tensor s({R, Cc / 32}, DType::Float8E8M0, Device::CUDA);
        xs_check(xs_quant_act_mxfp8(x.data(), code(x.dtype()), R, Cc, static_cast<uint8_t *>(q.data()),
                                    static_cast<uint8_t *>(s.data()), nullptr));
        sync();
        return {std::move(q), std::move(s)};
    }
    Tensor s({R, Cc / 128}, DType::Float32, Device::CUDA);
    xs_check(xs_quant_act_fp8(x.data(), code(x.dtype()), R, Cc, static_cast<uint8_t *>(q.data()),
                              static_cast<float *>(s.data()), nullptr));
    sync();
    return {std::move(q), std::move(s)};
}

std::tuple<Tensor, Tensor> quant_act_fp8(const Tensor &x) { return quant_act(x, false); }
std::tuple<Tensor, Tensor> quant_act_mxfp8(const Tensor &x) { return quant_act(x, true); }

static std::tuple<Tensor, Tensor> quant_weight(const Tensor &w, bool fp4)
{
    if (!is_act(w.dtype())) throw std::runtime_error("unsupported dtype");
    if (w.shape().size() < 2) throw std::runtime_error("rank mismatch");
    const std::int64_t n = w.shape()[w.shape().size() - 2], k = w.shape().back();
    const std::int64_t b = w.numel() / (n * k);
    if (fp4 ? (k % 32 != 0) : (n % 128 != 0 || k % 128 != 0)) throw std::runtime_error("shape mismatch");
    require_cuda(w);
    std::vector<std::int64_t> qs(w.shape()), ss(w.shape());
    if (fp4) {
        qs.back() = k / 2;
        ss.back() = k / 32;
        Tensor q(qs, DType::Float4E2M1x2, Device::CUDA), s(ss, DType::Float8E8M0, Device::CUDA);
        xs_check(xs_quant_weight_mxfp4(w.data(), code(w.dtype()), b, n, k, static_cast<uint8_t *>(q.data()),
                                       static_cast<uint8_t *>(s.data()), nullptr));
        sync();
        return {std::move(q), std::move(s)};
    }
    ss[ss.size() - 2] = n / 128;
    ss.back() = k / 128;
    Tensor q(qs, DType::Float8E4M3, Device::CUDA), s(ss, DType::Float32, Device::CUDA);
    xs_check(xs_quant_weight_fp8_block(w.data(), code(w.dtype()), b, n, k, static_cast<uint8_t *>(q.data()),
                                       static_cast<float *>(s.data()), nullptr));
    sync();
    return {std::move(q), std::move(s)};
}

std::tuple<Tensor, Tensor> quant_weight_fp8_block(const Tensor &w) { return quant_weight(w, false); }
std::tuple<Tensor, Tensor> quant_weight_mxfp4(const Tensor &w) { return quant_weight(w, true); }

Tensor gemm_fp8_blockscale(const Tensor &x, const Tensor &b, const Tensor &b_scale)
{
    if (x.dtype() != DType::BFloat16) throw std::runtime_error("unsupported dtype");
    if (b.dtype() != DType::Float8E4M3 || b_scale.dtype() != DType::Float32) throw std::runtime_error("dtype mismatch");
    if (x.shape().size() != 2 || b.shape().size() != 2 || b_scale.shape().size() != 2)
        throw std::runtime_error("rank mismatch");
    const std::int64_t M = x.shape()[0], K = x.shape()[1], N = b.shape()[0];
    if (b.shape()[1] != K || K % 128 || N % 128 || b_scale.shape()[0] != N / 128 || b_scale.shape()[1] != K / 128)
        throw std::runtime_error("shape mismatch");
    same_device(x, b);
    same_device(x, b_scale);
    require_cuda(x);
    Tensor out({M, N}, DType::BFloat16, Device::CUDA);
    std::size_t wsb = xs_gemm_fp8_blockscale_workspace_size(M, K);
    Tensor ws({static_cast<std::int64_t>(wsb)}, DType::UInt8, Device::CUDA);
    xs_check(xs_gemm_fp8_blockscale(x.data(), static_cast<const uint8_t *>(b.data()),
                                    static_cast<const float *>(b_scale.data()), M, N, K, out.data(), ws.data(),
                                    wsb, nullptr));
    sync();
    return out;
}
