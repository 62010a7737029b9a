// moe_weights.cpp -- assembles one MoE layer's weights from safetensors files
// into the layout the MoE op takes (stacked experts, w13 = [gate ; up]).
#include "ops/moe_weights.h"

#include <cstring>
#include <memory>
#include <stdexcept>
#include <unordered_map>
#include <utility>

#include "weight_io.h"
#include "xs_moe.h"

namespace {

struct Entry
{
    MMapFile *file;
    TensorMeta meta;
};

class Checkpoint
{
public:
    explicit Checkpoint(const std::vector<std::string> &paths)
    {
        if (paths.empty()) throw std::runtime_error("no checkpoint files given");
        for (const auto &p : paths) {
            files_.push_back(std::make_unique<MMapFile>(p));
            for (auto &kv : parse_safetensors_header(*files_.back())) {
                if (!index_.emplace(kv.first, Entry{files_.back().get(), std::move(kv.second)}).second)
                    throw std::runtime_error("duplicate weight key: " + kv.first);
            }
        }
    }
    bool has(const std::string &k) const { return index_.count(k) != 0; }
    const Entry &get(const std::string &k) const
    {
        auto it = index_.find(k);
        if (it == index_.end()) throw std::runtime_error("missing weight key: " + k);
        return it->second;
    }
    // Host view of `k`, checked against `shape` and one of `dtypes`.
    Tensor view(const std::string &k, const std::vector<std::int64_t> &shape, std::initializer_list<DType> dtypes) const
    {
        const Entry &e = get(k);
        if (e.meta.shape != shape) throw std::runtime_error("shape mismatch: " + k);
        bool ok = false;
        for (DType d : dtypes) ok = ok || e.meta.dtype == d;
        if (!ok) throw std::runtime_error("dtype mismatch: " + k);
        return make_weight_view(*e.file, e.meta.offset, e.meta.shape, e.meta.dtype);
    }

private:
    std::vector<std::unique_ptr<MMapFile>> files_;
    std::unordered_map<std::string, Entry> index_;
};

// Copies host bytes into `dst` at byte offset `off` (host or device tensor).
void put(Tensor &dst, std::size_t off, const Tensor &src)
{
    if (off + src.nbytes() > dst.nbytes()) throw std::runtime_error("internal: copy out of range");
    char *d = static_cast<char *>(dst.data()) + off;
    if (dst.device() == Device::CUDA)
        xs_check(xs_memcpy_h2d(d, src.data(), src.nbytes()));
    else
        std::memcpy(d, src.data(), src.nbytes());
}

bool is_dense(DType d) { return d == DType::Float32 || d == DType::BFloat16; }

// One expert (or the shared expert): gate/up/down under `base`, written into
// slice `e` of the destination tensors (slice 0 of 2-D tensors for shared).
// `stage` is a device buffer of 2I*H dense elements for dense checkpoints.
void load_expert(const Checkpoint &ck, const std::string &base, std::int64_t e, std::int64_t H, std::int64_t I,
                 Tensor &w13, Tensor &s13, Tensor &w2, Tensor &s2, std::optional<Tensor> &stage)
{
    const std::string g = base + ".gate_proj.weight", u = base + ".up_proj.weight", d = base + ".down_proj.weight";
    const DType wd = ck.get(g).meta.dtype;
    const std::size_t q13 = static_cast<std::size_t>(2 * I * H), q2 = static_cast<std::size_t>(H * I);
    const std::size_t n13 = static_cast<std::size_t>(2 * I / 128 * (H / 128)), n2 = static_cast<std::size_t>(H / 128 * (I / 128));
    if (wd == DType::Float8E4M3) {
        Tensor gv = ck.view(g, {I, H}, {DType::Float8E4M3});
        Tensor uv = ck.view(u, {I, H}, {DType::Float8E4M3});
        Tensor dv = ck.view(d, {H, I}, {DType::Float8E4M3});
        Tensor gs = ck.view(g + "_scale_inv", {I / 128, H / 128}, {DType::Float32});
        Tensor us = ck.view(u + "_scale_inv", {I / 128, H / 128}, {DType::Float32});
        Tensor ds = ck.view(d + "_scale_inv", {H / 128, I / 128}, {DType::Float32});
        put(w13, e * q13, gv);
        put(w13, e * q13 + gv.nbytes(), uv);
        put(s13, e * n13 * 4, gs);
        put(s13, e * n13 * 4 + gs.nbytes(), us);
        put(w2, e * q2, dv);
        put(s2, e * n2 * 4, ds);
        return;
    }
    if (!is_dense(wd)) throw std::runtime_error("dtype mismatch: " + g);
    if (w13.device() != Device::CUDA) throw std::runtime_error("unsupported device");
    // dense: stage [gate ; up] on the device, quantize into slice e
    Tensor gv = ck.view(g, {I, H}, {wd});
    Tensor uv = ck.view(u, {I, H}, {wd});
    Tensor dv = ck.view(d, {H, I}, {wd});
    const std::size_t es = dtype_size(wd);
    if (!stage || stage->nbytes() < q13 * es)
        stage.emplace(std::vector<std::int64_t>{static_cast<std::int64_t>(q13 * es)}, DType::UInt8, Device::CUDA);
    put(*stage, 0, gv);
    put(*stage, gv.nbytes(), uv);
    const int dt = static_cast<int>(wd);
    xs_check(xs_quant_weight_fp8_block(stage->data(), dt, 1, 2 * I, H, static_cast<std::uint8_t *>(w13.data()) + e * q13,
                                       static_cast<float *>(s13.data()) + e * n13, nullptr));
    xs_check(xs_stream_synchronize(nullptr));   // the stage is reused by the next copy
    put(*stage, 0, dv);
    xs_check(xs_quant_weight_fp8_block(stage->data(), dt, 1, H, I, static_cast<std::uint8_t *>(w2.data()) + e * q2,
                                       static_cast<float *>(s2.data()) + e * n2, nullptr));
    xs_check(xs_stream_synchronize(nullptr));
}

}  // namespace

MoeLayerWeights load_moe_layer(const std::vector<std::string> &paths, const std::string &prefix, Device device)
{
    if (device != Device::CUDA && device != Device::CPU) throw std::runtime_error("unsupported device");
    const Checkpoint ck(paths);
    MoeLayerWeights L;

    // router
    const std::string rk = prefix + ".gate.weight";
    const Entry &re = ck.get(rk);
    if (re.meta.shape.size() != 2) throw std::runtime_error("shape mismatch: " + rk);
    if (!is_dense(re.meta.dtype)) throw std::runtime_error("dtype mismatch: " + rk);
    const std::int64_t E = re.meta.shape[0], H = re.meta.shape[1];
    {
        Tensor v = ck.view(rk, {E, H}, {re.meta.dtype});
        L.router_w.emplace(std::vector<std::int64_t>{E, H}, re.meta.dtype, device);
        put(*L.router_w, 0, v);
    }
    const std::string bk = prefix + ".gate.e_score_correction_bias";
    if (ck.has(bk)) {
        Tensor v = ck.view(bk, {E}, {DType::Float32, DType::BFloat16});
        Tensor f(std::vector<std::int64_t>{E}, DType::Float32, Device::CPU);
        float *fp = static_cast<float *>(f.data());
        if (v.dtype() == DType::Float32) {
            std::memcpy(fp, v.data(), v.nbytes());
        } else {   // bf16 -> f32 is exact (zero-extend the mantissa)
            const std::uint16_t *b = static_cast<const std::uint16_t *>(v.data());
            for (std::int64_t i = 0; i < E; ++i) {
                const std::uint32_t u = static_cast<std::uint32_t>(b[i]) << 16;
                std::memcpy(fp + i, &u, 4);
            }
        }
        L.router_bias.emplace(std::vector<std::int64_t>{E}, DType::Float32, device);
        put(*L.router_bias, 0, f);
    }

    // routed experts: 0 .. E-1 must all be present
    const std::string e0 = prefix + ".experts.0.gate_proj.weight";
    const Entry &ge = ck.get(e0);
    if (ge.meta.shape.size() != 2 || ge.meta.shape[1] != H) throw std::runtime_error("shape mismatch: " + e0);
    const std::int64_t I = ge.meta.shape[0];
    if (H % 128 != 0 || I % 128 != 0) throw std::runtime_error("shape mismatch: " + e0 + " (H and I must be multiples of 128)");
    if (ck.has(prefix + ".experts." + std::to_string(E) + ".gate_proj.weight"))
        throw std::runtime_error("shape mismatch: more experts than router rows under " + prefix);
    L.E = E;
    L.H = H;
    L.I = I;
    L.w13.emplace(std::vector<std::int64_t>{E, 2 * I, H}, DType::Float8E4M3, device);
    L.w13_scale.emplace(std::vector<std::int64_t>{E, 2 * I / 128, H / 128}, DType::Float32, device);
    L.w2.emplace(std::vector<std::int64_t>{E, H, I}, DType::Float8E4M3, device);
    L.w2_scale.emplace(std::vector<std::int64_t>{E, H / 128, I / 128}, DType::Float32, device);
    std::optional<Tensor> stage;
    for (std::int64_t e = 0; e < E; ++e)
        load_expert(ck, prefix + ".experts." + std::to_string(e), e, H, I, *L.w13, *L.w13_scale, *L.w2, *L.w2_scale,
                    stage);

    // shared expert (optional)
    const std::string sb = prefix + ".shared_experts";
    if (ck.has(sb + ".gate_proj.weight")) {
        const Entry &se = ck.get(sb + ".gate_proj.weight");
        if (se.meta.shape != std::vector<std::int64_t>{I, H})
            throw std::runtime_error("shape mismatch: " + sb + ".gate_proj.weight (the shared expert must have the routed I)");
        L.shared_w13.emplace(std::vector<std::int64_t>{2 * I, H}, DType::Float8E4M3, device);
        L.shared_w13_scale.emplace(std::vector<std::int64_t>{2 * I / 128, H / 128}, DType::Float32, device);
        L.shared_w2.emplace(std::vector<std::int64_t>{H, I}, DType::Float8E4M3, device);
        L.shared_w2_scale.emplace(std::vector<std::int64_t>{H / 128, I / 128}, DType::Float32, device);
        load_expert(ck, sb, 0, H, I, *L.shared_w13, *L.shared_w13_scale, *L.shared_w2, *L.shared_w2_scale, stage);
    }
    return L;
}

void pack_moe_layer_frag(MoeLayerWeights &w, bool packed_only)
{
    if (!w.w13 || !w.w2) throw std::runtime_error("shape mismatch");
    if (w.w13->device() != Device::CUDA) throw std::runtime_error("unsupported device");
    const bool fp4 = w.w13->dtype() == DType::Float4E2M1x2;
    if ((!fp4 && w.w13->dtype() != DType::Float8E4M3) || w.w2->dtype() != w.w13->dtype() || !w.w13_scale ||
        !w.w2_scale)
        throw std::runtime_error("unsupported dtype");
    auto pack = [](const Tensor &t, std::int64_t batch, std::int64_t n, std::int64_t k) {
        Tensor out(t.shape(), t.dtype(), Device::CUDA);
        xs_check(xs_pack_weight_fp8_frag(static_cast<const std::uint8_t *>(t.data()), batch, n, k,
                                         static_cast<std::uint8_t *>(out.data()), nullptr));
        return out;
    };
    auto pack4 = [](const Tensor &t, const Tensor &s, std::int64_t batch, std::int64_t n, std::int64_t k) {
        std::pair<Tensor, Tensor> o{Tensor(t.shape(), t.dtype(), Device::CUDA), Tensor(s.shape(), s.dtype(), Device::CUDA)};
        xs_check(xs_pack_weight_mxfp4_frag(static_cast<const std::uint8_t *>(t.data()),
                                           static_cast<const std::uint8_t *>(s.data()), batch, n, k,
                                           static_cast<std::uint8_t *>(o.first.data()),
                                           static_cast<std::uint8_t *>(o.second.data()), nullptr));
        return o;
    };
    const std::int64_t E = w.E, H = w.H, I = w.I;
    if (fp4) {
        auto a = pack4(*w.w13, *w.w13_scale, E, 2 * I, H);
        auto b = pack4(*w.w2, *w.w2_scale, E, H, I);
        w.w13_frag = std::move(a.first);
        w.w13_scale_frag = std::move(a.second);
        w.w2_frag = std::move(b.first);
        w.w2_scale_frag = std::move(b.second);
    } else {
        w.w13_frag = pack(*w.w13, E, 2 * I, H);
        w.w2_frag = pack(*w.w2, E, H, I);
    }
    if (w.shared_w13 && w.shared_w2) {
        w.shared_w13_frag = pack(*w.shared_w13, 1, 2 * I, H);
        w.shared_w2_frag = pack(*w.shared_w2, 1, H, I);
    }
    xs_check(xs_stream_synchronize(nullptr));
    if (packed_only) {
        w.w13.reset();
        w.w2.reset();
        w.shared_w13.reset();
        w.shared_w2.reset();
    }
}
