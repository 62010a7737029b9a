// Host emulation of the C++ Tensor ops (csrc/src: tensor.cpp, ops/moe.cpp,
// ops/rmsnorm.cpp, ops/moe_weights.cpp, weight_io.cpp) over the emulated
// library: the ops call the library's C ABI exactly as on the card, and every
// kernel runs from its source on the CPU (gen_fwd.py, hip_emu.hpp).
//   moe()            against xs_moe_forward on the same buffers (same bits),
//                    and against the oracle's layer (routing exact, 2e-2);
//                    FP8 with the shared expert, f32 input, MXFP4 experts,
//                    the pre-norm with a residual
//   moe_block_ffn()  on weights from load_moe_layer (a two-file FP8
//                    checkpoint written here) against moe() with the norm
//                    and residual (same bits); the loaded tensors against what
//                    was written; a dense BF16 checkpoint quantized while
//                    loading against the oracle's block quantization
//   rmsnorm(), moe_router_logits(exact), moe_route(), moe_permute() against
//                    the C ABI / oracle
// usage: cpp_emu <tmp dir>   prints "<check> mismatches N" and "errors N".
#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <map>
#include <random>
#include <string>
#include <vector>

#include "ops/moe.h"
#include "ops/moe_weights.h"
#include "ops/rmsnorm.h"
#include "tensor.h"
#include "xs_moe.h"
#include "moe_oracle.h"

#include "hip_emu.hpp"

static std::mt19937 rng(7);
static std::normal_distribution<float> nd(0.f, 1.f);
static long g_bad = 0;

static void report(const char *what, long n)
{
    printf("%s mismatches %ld\n", what, n);
}
template <typename T>
static long diff(const T *a, const T *b, size_t n)
{
    long d = 0;
    for (size_t i = 0; i < n; ++i) d += memcmp(&a[i], &b[i], sizeof(T)) != 0;
    return d;
}
static std::vector<uint16_t> bf16v(size_t n, float sd)
{
    std::vector<uint16_t> v(n);
    for (auto &e : v) e = xo_bf16_from_f32(sd * nd(rng));
    return v;
}
// a device Tensor holding a copy of host data
template <typename T>
static Tensor dev(const std::vector<T> &h, std::vector<int64_t> shape, DType dt)
{
    Tensor c(h.data(), shape, dt, Device::CPU);
    return to_cuda(c);
}
template <typename T>
static std::vector<T> host(const Tensor &t)
{
    Tensor c = to_cpu(t);
    std::vector<T> v(c.nbytes() / sizeof(T));
    memcpy(v.data(), c.data(), c.nbytes());
    return v;
}

struct Layer {
    int64_t E, H, I;
    bool fp4;
    std::vector<uint16_t> router_w;
    std::vector<float> bias;
    std::vector<uint8_t> w13, w2, sw13, sw2;   // codes
    std::vector<uint8_t> s13b, s2b;            // scales as bytes (f32 or e8m0)
    std::vector<float> ss13, ss2;              // shared FP8 block scales
};
static Layer make_layer(int64_t E, int64_t H, int64_t I, bool fp4)
{
    Layer L{E, H, I, fp4, bf16v(E * H, 0.02f), {}, {}, {}, {}, {}, {}, {}, {}, {}};
    for (int e = 0; e < E; ++e) L.bias.push_back(0.1f * nd(rng));
    std::vector<float> a(2 * I * H), b(H * I);
    for (int64_t e = 0; e < E; ++e) {
        for (auto &v : a) v = 0.02f * nd(rng);
        for (auto &v : b) v = 0.02f * nd(rng);
        if (fp4) {
            std::vector<uint8_t> q1(I * H), s1(2 * I * H / 32), q2(H * I / 2), s2(H * I / 32);
            xo_quant_weight_mxfp4(a.data(), 2 * I, H, q1.data(), s1.data());
            xo_quant_weight_mxfp4(b.data(), H, I, q2.data(), s2.data());
            L.w13.insert(L.w13.end(), q1.begin(), q1.end());
            L.s13b.insert(L.s13b.end(), s1.begin(), s1.end());
            L.w2.insert(L.w2.end(), q2.begin(), q2.end());
            L.s2b.insert(L.s2b.end(), s2.begin(), s2.end());
        } else {
            std::vector<uint8_t> q1(2 * I * H), q2(H * I);
            std::vector<float> s1(2 * I / 128 * H / 128), s2(H / 128 * I / 128);
            xo_quant_weight_fp8_block(a.data(), 2 * I, H, q1.data(), s1.data());
            xo_quant_weight_fp8_block(b.data(), H, I, q2.data(), s2.data());
            L.w13.insert(L.w13.end(), q1.begin(), q1.end());
            L.w2.insert(L.w2.end(), q2.begin(), q2.end());
            const uint8_t *p1 = (const uint8_t *)s1.data(), *p2 = (const uint8_t *)s2.data();
            L.s13b.insert(L.s13b.end(), p1, p1 + 4 * s1.size());
            L.s2b.insert(L.s2b.end(), p2, p2 + 4 * s2.size());
        }
    }
    for (auto &v : a) v = 0.02f * nd(rng);
    for (auto &v : b) v = 0.02f * nd(rng);
    L.sw13.resize(2 * I * H);
    L.sw2.resize(H * I);
    L.ss13.resize(2 * I / 128 * H / 128);
    L.ss2.resize(H / 128 * I / 128);
    xo_quant_weight_fp8_block(a.data(), 2 * I, H, L.sw13.data(), L.ss13.data());
    xo_quant_weight_fp8_block(b.data(), H, I, L.sw2.data(), L.ss2.data());
    return L;
}

// moe() against xs_moe_forward on the same device buffers, and the oracle
static void check_moe(const char *name, int64_t T, const Layer &L, int64_t k, bool xf32, bool norm, bool resid)
{
    const int64_t E = L.E, H = L.H, I = L.I;
    const DType xd = xf32 ? DType::Float32 : DType::BFloat16;
    std::vector<uint16_t> xb = bf16v(T * H, 1.0f);
    std::vector<float> xf(T * H), wf(E * H);
    for (size_t i = 0; i < xf.size(); ++i) xf[i] = xo_f32_from_bf16(xb[i]);
    for (size_t i = 0; i < wf.size(); ++i) wf[i] = xo_f32_from_bf16(L.router_w[i]);
    Tensor x = xf32 ? dev(xf, {T, H}, xd) : dev(xb, {T, H}, xd);
    Tensor rw = xf32 ? dev(wf, {E, H}, xd) : dev(L.router_w, {E, H}, xd);
    Tensor bias = dev(L.bias, {E}, DType::Float32);
    const DType wd = L.fp4 ? DType::Float4E2M1x2 : DType::Float8E4M3, sd = L.fp4 ? DType::Float8E8M0 : DType::Float32;
    Tensor w13 = dev(L.w13, L.fp4 ? std::vector<int64_t>{E, 2 * I, H / 2} : std::vector<int64_t>{E, 2 * I, H}, wd);
    Tensor w2 = dev(L.w2, L.fp4 ? std::vector<int64_t>{E, H, I / 2} : std::vector<int64_t>{E, H, I}, wd);
    Tensor s13 = L.fp4 ? dev(L.s13b, {E, 2 * I, H / 32}, sd) : dev(L.s13b, {E, 2 * I / 128, H / 128}, sd);
    Tensor s2 = L.fp4 ? dev(L.s2b, {E, H, I / 32}, sd) : dev(L.s2b, {E, H / 128, I / 128}, sd);
    Tensor sw13 = dev(L.sw13, {2 * I, H}, DType::Float8E4M3), sw2 = dev(L.sw2, {H, I}, DType::Float8E4M3);
    Tensor ss13 = dev(L.ss13, {2 * I / 128, H / 128}, DType::Float32), ss2 = dev(L.ss2, {H / 128, I / 128}, DType::Float32);
    std::vector<float> nwf(H);
    for (auto &v : nwf) v = 1.f + 0.1f * nd(rng);
    std::vector<uint16_t> nwb(H);
    for (int64_t i = 0; i < H; ++i) nwb[i] = xo_bf16_from_f32(nwf[i]);
    Tensor nw = xf32 ? dev(nwf, {H}, xd) : dev(nwb, {H}, xd);
    std::vector<uint16_t> rb = bf16v(T * H, 1.0f);
    std::vector<float> rf(T * H);
    for (size_t i = 0; i < rf.size(); ++i) rf[i] = xo_f32_from_bf16(rb[i]);
    Tensor res = xf32 ? dev(rf, {T, H}, xd) : dev(rb, {T, H}, xd);

    Tensor out = moe(x, rw, &bias, w13, s13, w2, s2, &sw13, &ss13, &sw2, &ss2, k, 1, 1, true, 1.0f, 1,
                     norm ? &nw : nullptr, 1e-6f, resid ? &res : nullptr);
    // the C ABI on the same buffers
    xs_moe_params p = {};
    p.T = T; p.H = H; p.I = I; p.E = E; p.top_k = k; p.n_group = 1; p.topk_group = 1; p.renormalize = 1;
    p.routed_scaling = 1.0f; p.x_dtype = xf32 ? XS_F32 : XS_BF16; p.routed_format = L.fp4 ? XS_FP4_E2M1X2 : XS_FP8_E4M3;
    p.has_shared = 1; p.router_exact = XS_ROUTER_CERTIFIED; p.has_norm = norm; p.norm_eps = 1e-6f;
    Tensor out2({T, H}, xd, Device::CUDA);
    float *lg = (float *)emu_alloc(4 * T * E, "logits");
    xs_moe_tensors t = {};
    t.x = x.data(); t.router_w = rw.data(); t.router_bias = (const float *)bias.data();
    t.w13 = (const uint8_t *)w13.data(); t.w13_scale = s13.data(); t.w2 = (const uint8_t *)w2.data(); t.w2_scale = s2.data();
    t.shared_w13 = (const uint8_t *)sw13.data(); t.shared_w13_scale = (const float *)ss13.data();
    t.shared_w2 = (const uint8_t *)sw2.data(); t.shared_w2_scale = (const float *)ss2.data();
    t.norm_weight = norm ? nw.data() : nullptr; t.residual = resid ? res.data() : nullptr;
    t.out = out2.data(); t.logits = lg;
    const size_t wsb = xs_moe_workspace_size(&p);
    void *ws = emu_alloc(wsb, "ws");
    long bad = xs_moe_forward(&p, &t, ws, wsb, nullptr) != 0;
    const size_t el = xf32 ? 4 : 2;
    std::vector<uint8_t> o1 = host<uint8_t>(out), o2 = host<uint8_t>(out2);
    bad += diff(o1.data(), o2.data(), o1.size());
    // the oracle on the row the router read (the op's own norm when present)
    std::vector<uint8_t> xin(T * H * el);
    if (norm) {
        Tensor xn = rmsnorm(x, nw, 1e-6f);
        std::vector<uint8_t> h = host<uint8_t>(xn);
        memcpy(xin.data(), h.data(), xin.size());
    } else {
        memcpy(xin.data(), xf32 ? (const void *)xf.data() : (const void *)xb.data(), xin.size());
    }
    xo_moe_cfg cfg = {T, H, I, E, k, 1, 1, 1, 1.0f, xf32 ? 0 : 1, L.fp4 ? 1 : 0, 1, 1};
    const void *rwin = xf32 ? (const void *)wf.data() : (const void *)L.router_w.data();
    xo_moe_inputs in = {xin.data(), rwin, L.bias.data(), lg, L.w13.data(), L.s13b.data(), L.w2.data(), L.s2b.data(),
                        L.sw13.data(), L.ss13.data(), L.sw2.data(), L.ss2.data()};
    std::vector<int32_t> ridx(T * k), rcn(E), rof(E + 1), rpm(T * k), riv(T * k);
    std::vector<float> rw_(T * k), rout(T * H);
    std::vector<uint8_t> rob(T * H * el);
    xo_moe_outputs o = {nullptr, ridx.data(), rw_.data(), rcn.data(), rof.data(), rpm.data(), riv.data(), rout.data(),
                        rob.data()};
    xo_moe_forward(&cfg, &in, &o);
    // routing from x: the reference's gemm_cpu logits
    std::vector<float> xl(T * E);
    xo_router_logits(xin.data(), rwin, xf32 ? 0 : 1, T, E, H, xl.data());
    std::vector<int32_t> xidx(T * k);
    std::vector<float> xw(T * k);
    xo_route(xl.data(), L.bias.data(), T, E, k, 1, 1, 1, 1.0f, xidx.data(), xw.data());
    bad += diff(ridx.data(), xidx.data(), ridx.size());   // the forward routed like the reference
    double amax = 0, dmax = 0;
    for (int64_t i = 0; i < T * H; ++i) {
        double r = rout[i];
        if (resid) r += rf[i];
        const double g = xf32 ? ((const float *)o1.data())[i] : xo_f32_from_bf16(((const uint16_t *)o1.data())[i]);
        amax = std::max(amax, std::fabs(r));
        dmax = std::max(dmax, std::fabs(g - r));
    }
    bad += !(dmax <= 2e-2 * amax);
    std::string n = std::string("moe ") + name;
    report(n.c_str(), bad);
    g_bad += bad;
}

// ---------------------------------------------------------------- safetensors
struct StEntry { std::string dtype; std::vector<int64_t> shape; std::vector<uint8_t> data; };
static void write_safetensors(const std::string &path, const std::map<std::string, StEntry> &ts)
{
    std::string hdr = "{";
    size_t off = 0;
    for (auto &[k, e] : ts) {
        if (hdr.size() > 1) hdr += ",";
        hdr += "\"" + k + "\":{\"dtype\":\"" + e.dtype + "\",\"shape\":[";
        for (size_t i = 0; i < e.shape.size(); ++i) hdr += (i ? "," : "") + std::to_string(e.shape[i]);
        hdr += "],\"data_offsets\":[" + std::to_string(off) + "," + std::to_string(off + e.data.size()) + "]}";
        off += e.data.size();
    }
    hdr += "}";
    while (hdr.size() % 8) hdr += " ";
    std::ofstream f(path, std::ios::binary);
    const uint64_t n = hdr.size();
    f.write((const char *)&n, 8);
    f.write(hdr.data(), hdr.size());
    for (auto &[k, e] : ts) f.write((const char *)e.data.data(), e.data.size());
}
template <typename T>
static StEntry ste(const std::string &dt, std::vector<int64_t> shape, const T *p, size_t n)
{
    StEntry e{dt, shape, std::vector<uint8_t>(n * sizeof(T))};
    memcpy(e.data.data(), p, e.data.size());
    return e;
}

static void check_checkpoints(const std::string &dir)
{
    const int64_t E = 8, H = 512, I = 256, T = 24, k = 2;
    Layer L = make_layer(E, H, I, false);
    // two files: router, bias and experts 0..3 in one, the rest and the shared expert in the other
    std::map<std::string, StEntry> a, b;
    a["m.gate.weight"] = ste("BF16", {E, H}, L.router_w.data(), L.router_w.size());
    a["m.gate.e_score_correction_bias"] = ste("F32", {E}, L.bias.data(), L.bias.size());
    const int64_t n13 = 2 * I * H, n2 = H * I, s13 = 2 * I / 128 * H / 128, s2 = H / 128 * I / 128;
    for (int64_t e = 0; e < E; ++e) {
        auto &f = e < 4 ? a : b;
        const std::string base = "m.experts." + std::to_string(e);
        const uint8_t *w = L.w13.data() + e * n13;
        const float *sc = (const float *)L.s13b.data() + e * s13;
        f[base + ".gate_proj.weight"] = ste("F8_E4M3", {I, H}, w, I * H);
        f[base + ".up_proj.weight"] = ste("F8_E4M3", {I, H}, w + I * H, I * H);
        f[base + ".gate_proj.weight_scale_inv"] = ste("F32", {I / 128, H / 128}, sc, s13 / 2);
        f[base + ".up_proj.weight_scale_inv"] = ste("F32", {I / 128, H / 128}, sc + s13 / 2, s13 / 2);
        f[base + ".down_proj.weight"] = ste("F8_E4M3", {H, I}, L.w2.data() + e * n2, n2);
        f[base + ".down_proj.weight_scale_inv"] = ste("F32", {H / 128, I / 128}, (const float *)L.s2b.data() + e * s2, s2);
    }
    b["m.shared_experts.gate_proj.weight"] = ste("F8_E4M3", {I, H}, L.sw13.data(), I * H);
    b["m.shared_experts.up_proj.weight"] = ste("F8_E4M3", {I, H}, L.sw13.data() + I * H, I * H);
    b["m.shared_experts.gate_proj.weight_scale_inv"] = ste("F32", {I / 128, H / 128}, L.ss13.data(), s13 / 2);
    b["m.shared_experts.up_proj.weight_scale_inv"] = ste("F32", {I / 128, H / 128}, L.ss13.data() + s13 / 2, s13 / 2);
    b["m.shared_experts.down_proj.weight"] = ste("F8_E4M3", {H, I}, L.sw2.data(), n2);
    b["m.shared_experts.down_proj.weight_scale_inv"] = ste("F32", {H / 128, I / 128}, L.ss2.data(), s2);
    const std::string pa = dir + "/a.safetensors", pb = dir + "/b.safetensors";
    write_safetensors(pa, a);
    write_safetensors(pb, b);
    MoeLayerWeights W = load_moe_layer({pa, pb}, "m", Device::CUDA);
    long bad = !(W.E == E && W.H == H && W.I == I && W.router_bias && W.shared_w13);
    if (!bad) {
        bad += diff(host<uint8_t>(*W.w13).data(), L.w13.data(), L.w13.size());
        bad += diff(host<uint8_t>(*W.w13_scale).data(), L.s13b.data(), L.s13b.size());
        bad += diff(host<uint8_t>(*W.w2).data(), L.w2.data(), L.w2.size());
        bad += diff(host<uint8_t>(*W.w2_scale).data(), L.s2b.data(), L.s2b.size());
        bad += diff(host<uint8_t>(*W.shared_w13).data(), L.sw13.data(), L.sw13.size());
        bad += diff(host<uint16_t>(*W.router_w).data(), L.router_w.data(), L.router_w.size());
        bad += diff(host<float>(*W.router_bias).data(), L.bias.data(), L.bias.size());
    }
    report("load fp8 checkpoint", bad);
    g_bad += bad;
    // the block's FFN half from the loaded weights against moe() with the norm and residual
    std::vector<uint16_t> hb = bf16v(T * H, 1.0f), lnb(H);
    for (auto &v : lnb) v = xo_bf16_from_f32(1.f + 0.1f * nd(rng));
    Tensor h = dev(hb, {T, H}, DType::BFloat16), ln = dev(lnb, {H}, DType::BFloat16);
    bad = 0;
    try {
        Tensor f1 = moe_block_ffn(h, ln, 1e-6f, W, k);
        Tensor f2 = moe(h, *W.router_w, &*W.router_bias, *W.w13, *W.w13_scale, *W.w2, *W.w2_scale, &*W.shared_w13,
                        &*W.shared_w13_scale, &*W.shared_w2, &*W.shared_w2_scale, k, 1, 1, true, 1.0f, 1, &ln, 1e-6f, &h);
        std::vector<uint16_t> a1 = host<uint16_t>(f1), a2 = host<uint16_t>(f2);
        bad += diff(a1.data(), a2.data(), a1.size());
    } catch (const std::exception &e) {
        printf("moe_block_ffn threw: %s\n", e.what());
        bad += 1;
    }
    report("moe_block_ffn", bad);
    g_bad += bad;

    // a dense BF16 checkpoint, quantized while loading (an all-zero block included)
    std::map<std::string, StEntry> d;
    std::vector<uint16_t> rw = bf16v(E * H, 0.02f);
    d["m.gate.weight"] = ste("BF16", {E, H}, rw.data(), rw.size());
    std::vector<std::vector<uint16_t>> gate(E), up(E), down(E);
    for (int64_t e = 0; e < E; ++e) {
        gate[e] = bf16v(I * H, 0.02f);
        up[e] = bf16v(I * H, 0.02f);
        down[e] = bf16v(H * I, 0.02f);
        if (e == 1)
            for (int r = 0; r < 128; ++r) memset(&up[e][(size_t)r * H], 0, 2 * 128);
        const std::string base = "m.experts." + std::to_string(e);
        d[base + ".gate_proj.weight"] = ste("BF16", {I, H}, gate[e].data(), gate[e].size());
        d[base + ".up_proj.weight"] = ste("BF16", {I, H}, up[e].data(), up[e].size());
        d[base + ".down_proj.weight"] = ste("BF16", {H, I}, down[e].data(), down[e].size());
    }
    const std::string pd = dir + "/d.safetensors";
    write_safetensors(pd, d);
    MoeLayerWeights D = load_moe_layer({pd}, "m", Device::CUDA);
    bad = 0;
    std::vector<uint8_t> q13 = host<uint8_t>(*D.w13), q2 = host<uint8_t>(*D.w2);
    std::vector<float> sc13 = host<float>(*D.w13_scale), sc2 = host<float>(*D.w2_scale);
    for (int64_t e = 0; e < E; ++e) {
        std::vector<float> w13f(2 * I * H), w2f(H * I);
        for (int64_t i = 0; i < I * H; ++i) {
            w13f[i] = xo_f32_from_bf16(gate[e][i]);
            w13f[I * H + i] = xo_f32_from_bf16(up[e][i]);
            w2f[i] = xo_f32_from_bf16(down[e][i]);
        }
        std::vector<uint8_t> rq13(2 * I * H), rq2(H * I);
        std::vector<float> rs13(s13), rs2(s2);
        xo_quant_weight_fp8_block(w13f.data(), 2 * I, H, rq13.data(), rs13.data());
        xo_quant_weight_fp8_block(w2f.data(), H, I, rq2.data(), rs2.data());
        bad += diff(q13.data() + e * n13, rq13.data(), n13) + diff(sc13.data() + e * s13, rs13.data(), s13);
        bad += diff(q2.data() + e * n2, rq2.data(), n2) + diff(sc2.data() + e * s2, rs2.data(), s2);
    }
    report("load dense checkpoint", bad);
    g_bad += bad;
}

// rmsnorm(), moe_router_logits(exact), moe_route(), moe_permute()
static void check_stage_ops()
{
    const int64_t T = 33, H = 512, E = 72, k = 6;
    std::vector<uint16_t> xb = bf16v(T * H, 1.5f), wb(H), rwb = bf16v(E * H, 0.02f);
    for (auto &v : wb) v = xo_bf16_from_f32(1.f + 0.1f * nd(rng));
    Tensor x = dev(xb, {T, H}, DType::BFloat16), w = dev(wb, {H}, DType::BFloat16);
    Tensor y = rmsnorm(x, w, 1e-5f);
    uint16_t *y2 = (uint16_t *)emu_alloc(2 * T * H, "y2");
    long bad = xs_rmsnorm(x.data(), w.data(), XS_BF16, T, H, 1e-5f, y2, nullptr, nullptr, nullptr) != 0;
    std::vector<uint16_t> yh = host<uint16_t>(y);
    bad += diff(yh.data(), y2, yh.size());
    report("rmsnorm op", bad);
    g_bad += bad;
    Tensor rw = dev(rwb, {E, H}, DType::BFloat16);
    Tensor lg = moe_router_logits(x, rw, true);
    std::vector<float> l = host<float>(lg), rl(T * E);
    xo_router_logits(xb.data(), rwb.data(), 1, T, E, H, rl.data());
    bad = diff(l.data(), rl.data(), rl.size());
    report("router logits op", bad);
    g_bad += bad;
    std::vector<float> bias(E);
    for (auto &v : bias) v = 0.1f * nd(rng);
    Tensor bt = dev(bias, {E}, DType::Float32);
    auto [idx, wt] = moe_route(lg, &bt, k, 8, 3, false, 2.5f);
    std::vector<int32_t> ri(T * k);
    std::vector<float> rwt(T * k);
    xo_route(rl.data(), bias.data(), T, E, k, 8, 3, 0, 2.5f, ri.data(), rwt.data());
    std::vector<int32_t> ih = host<int32_t>(idx);
    std::vector<float> wh = host<float>(wt);
    bad = diff(ih.data(), ri.data(), ri.size()) + diff(wh.data(), rwt.data(), rwt.size());
    report("route op", bad);
    g_bad += bad;
    auto [cnt, off, perm, inv] = moe_permute(idx, E);
    std::vector<int32_t> rc(E), ro(E + 1), rp(T * k), rv(T * k);
    xo_permute(ri.data(), T, E, k, rc.data(), ro.data(), rp.data(), rv.data());
    bad = diff(host<int32_t>(cnt).data(), rc.data(), E) + diff(host<int32_t>(off).data(), ro.data(), E + 1) +
          diff(host<int32_t>(perm).data(), rp.data(), T * k) + diff(host<int32_t>(inv).data(), rv.data(), T * k);
    report("permute op", bad);
    g_bad += bad;
}

int main(int argc, char **argv)
{
    const std::string dir = argc > 1 ? argv[1] : "/tmp";
    g_math = true;
    try {
        Layer L8 = make_layer(16, 512, 256, false);
        check_moe("fp8", 40, L8, 4, false, false, false);
        check_moe("fp8 f32 input", 24, L8, 4, true, false, false);
        check_moe("fp8 norm residual", 40, L8, 4, false, true, true);
        Layer L4 = make_layer(16, 512, 512, true);
        check_moe("mxfp4", 48, L4, 6, false, false, false);
        check_checkpoints(dir);
        check_stage_ops();
    } catch (const std::exception &e) {
        printf("threw: %s\n", e.what());
        g_bad += 1000;
    }
    printf("total mismatches %ld\nerrors %ld\n", g_bad, (long)g_errors);
    return 0;
}
