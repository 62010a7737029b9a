// Host stand-in of the HIP runtime and of the gfx950 builtins the library's
// sources use, for the whole-forward emulation (fwd_main.cpp): the product's
// own C ABI entry points, dispatch and launchers run on the CPU, and every
// kernel launch runs the kernel's source through emu.hpp (one fiber per
// lane).  Launches are synchronous; streams and events are no-ops.
#pragma once
#include "router_emu.hpp"
#include <cstdarg>
#include <type_traits>

#define __align__(n) __attribute__((aligned(n)))
// atomics of any 4- or 8-byte type (the kernels also store and load floats)
#undef __hip_atomic_load
#undef __hip_atomic_store
#undef __hip_atomic_fetch_add
template <typename T>
inline T emu_atomic_load(const T *p, int o) { T v; __atomic_load(p, &v, o); return v; }
template <typename T, typename V>
inline void emu_atomic_store(T *p, V v, int o) { T t = (T)v; __atomic_store(p, &t, o); }
#define __hip_atomic_load(p, o, s) emu_atomic_load((p), (o))
#define __hip_atomic_store(p, v, o, s) emu_atomic_store((p), (v), (o))
#define __hip_atomic_fetch_add(p, v, o, s) __atomic_fetch_add((p), (v), (o))
#define __restrict__ __restrict
#define HIP_SYMBOL(x) (&(x))

typedef void *hipStream_t;
typedef void *hipEvent_t;
typedef int hipError_t;
typedef int hipDeviceAttribute_t;
typedef int hipFuncAttribute;
typedef int hipMemcpyKind;
enum { hipSuccess = 0 };
enum { hipFuncAttributeMaxDynamicSharedMemorySize = 1 };
enum { hipDeviceAttributeMultiprocessorCount = 1 };
enum { hipMemcpyHostToDevice = 1, hipMemcpyDeviceToHost = 2, hipMemcpyDeviceToDevice = 3 };

struct dim3 {
    unsigned x, y, z;
    dim3(unsigned a = 1, unsigned b = 1, unsigned c = 1) : x(a), y(b), z(c) {}
};

inline int emu_cus() { const char *v = getenv("EMU_CUS"); return v ? atoi(v) : 16; }
inline hipError_t hipGetLastError() { return hipSuccess; }
inline const char *hipGetErrorString(hipError_t) { return "emulated"; }
inline hipError_t hipFuncSetAttribute(const void *, int, int) { return hipSuccess; }
inline hipError_t hipGetDevice(int *d) { *d = 0; return hipSuccess; }
inline hipError_t hipGetDeviceCount(int *n) { *n = 1; return hipSuccess; }
inline hipError_t hipDeviceGetAttribute(int *v, int, int) { *v = emu_cus(); return hipSuccess; }
inline hipError_t hipMalloc(void **p, size_t n) { *p = emu_alloc(n, "hipMalloc"); return hipSuccess; }
inline hipError_t hipFree(void *) { return hipSuccess; }
inline hipError_t hipMemcpy(void *d, const void *s, size_t n, int) { memcpy(d, s, n); return hipSuccess; }
inline hipError_t hipMemcpyAsync(void *d, const void *s, size_t n, int, hipStream_t) { memcpy(d, s, n); return hipSuccess; }
inline hipError_t hipMemGetInfo(size_t *f, size_t *t) { *f = *t = (size_t)1 << 34; return hipSuccess; }
inline hipError_t hipStreamSynchronize(hipStream_t) { return hipSuccess; }
inline hipError_t hipEventCreate(hipEvent_t *e) { *e = nullptr; return hipSuccess; }
inline hipError_t hipEventRecord(hipEvent_t, hipStream_t) { return hipSuccess; }
inline hipError_t hipEventSynchronize(hipEvent_t) { return hipSuccess; }
inline hipError_t hipEventElapsedTime(float *ms, hipEvent_t, hipEvent_t) { *ms = 0; return hipSuccess; }
template <typename T>
inline hipError_t hipMemcpyFromSymbol(void *d, const T *sym, size_t n) { memcpy(d, sym, n); return hipSuccess; }
// a __device__ array's address: its host copy, registered as a device buffer
template <typename T>
inline hipError_t hipGetSymbolAddress(void **p, T *sym)
{
    *p = (void *)sym;
    for (auto &r : g_regions)
        if (r.p == (const uint8_t *)sym) return hipSuccess;
    g_regions.push_back({(const uint8_t *)sym, sizeof(T), "device symbol"});
    return hipSuccess;
}

// builtins of xs_device.hpp and the kernels
inline uint32_t emu_cvt_pk_fp8(float a, float b, int old, bool hi)
{
    const uint32_t v = e4m3_enc(a) | (e4m3_enc(b) << 8);
    return hi ? (((uint32_t)old & 0xFFFFu) | (v << 16)) : (((uint32_t)old & 0xFFFF0000u) | v);
}
#define __builtin_amdgcn_cvt_pk_fp8_f32(a, b, o, h) emu_cvt_pk_fp8((a), (b), (o), (h))
inline int emu_frexp_exp(float a) { int e = 0; std::frexp(a, &e); return e; }
#define __builtin_amdgcn_frexp_expf(a) emu_frexp_exp(a)
#define __builtin_amdgcn_rcpf(a) (1.0f / (a))
#define __builtin_amdgcn_exp2f(a) exp2f(a)
inline uint64_t wall_clock64() { return 0; }
inline unsigned atomicAdd(unsigned *p, unsigned v) { return __atomic_fetch_add(p, v, __ATOMIC_RELAXED); }
inline int atomicMax(int *p, int v)
{
    int o = __atomic_load_n(p, __ATOMIC_RELAXED);
    while (o < v && !__atomic_compare_exchange_n(p, &o, v, false, __ATOMIC_RELAXED, __ATOMIC_RELAXED)) {}
    return o;
}
inline uint32_t __shfl_xor(uint32_t v, int m, int w) { return (uint32_t)__shfl_xor((int)v, m, w); }
inline int __shfl(int v, int src, int) { return (int)(uint32_t)emu_xchg((uint32_t)v, src); }
inline float __shfl(float v, int src, int)
{
    uint32_t u;
    memcpy(&u, &v, 4);
    u = (uint32_t)emu_xchg(u, src);
    float r;
    memcpy(&r, &u, 4);
    return r;
}
inline uint64_t __ballot(int pred)
{
    const int w = wave_id(), l = lane_id();
    tb->xch[w][l] = pred != 0;
    emu_xpost(w, l, 7);
    tb->wbar[w]->arrive_and_wait();
    emu_xcheck(w, l);
    uint64_t r = 0;
    for (int i = 0; i < 64; ++i) r |= (uint64_t)(tb->xch[w][i] & 1) << i;
    tb->wbar[w]->arrive_and_wait();
    return r;
}
template <typename A, typename B, typename = std::enable_if_t<!std::is_same_v<A, B>>>
inline auto min(A a, B b) { using C = std::common_type_t<A, B>; return (C)a < (C)b ? (C)a : (C)b; }
template <typename A, typename B, typename = std::enable_if_t<!std::is_same_v<A, B>>>
inline auto max(A a, B b) { using C = std::common_type_t<A, B>; return (C)a > (C)b ? (C)a : (C)b; }

// EMU_KERNEL_LOG=<file>: every launched kernel's name is appended to the file
// (coverage of the emulated suites)
inline void emu_note_kernel(const char *name)
{
    static std::mutex m;
    if (const char *f = getenv("EMU_KERNEL_LOG")) {
        std::lock_guard<std::mutex> l(m);
        if (FILE *fp = fopen(f, "a")) { fprintf(fp, "%s\n", name); fclose(fp); }
    }
}
#define EMU_NOTE_KERNEL()                                                                              \
    do {                                                                                               \
        if (threadIdx.x == 0 && blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0 && getenv("EMU_KERNEL_LOG")) \
            emu_note_kernel(__PRETTY_FUNCTION__);                                                      \
    } while (0)
// a kernel launch: every block's lanes as fibers (emu_run_grid), synchronous;
// static __shared__ arrays follow the dynamic LDS
template <typename F>
inline void emu_kl(F fn, dim3 g, dim3 b, size_t smem = 0, hipStream_t = nullptr)
{
    const unsigned nt = b.x * b.y * b.z;
    if (nt % 64 || nt > 1024) { fprintf(stderr, "[emu] block of %u threads\n", nt); g_errors++; return; }
    const size_t dyn = (smem + 15) / 16 * 16;
    emu_run_grid(fn, {g.x, g.y, g.z}, nt, dyn + 65536, dyn);
}

// compiler-visible register loads of the weight-direct kernels: read now (the
// compiler waits for them before any use), counted in the lane's vmcnt queue
// as the hardware counts them
inline v4i wd_gload(const uint8_t *p)
{
    if (!emu_check_global(p, 16)) EMU_ERR("register load %p outside every buffer", (const void *)p);
    v4i v;
    memcpy(&v, p, 16);
    push(Op{2, nullptr, 0, 0, nullptr, nullptr});
    return v;
}
inline uint8_t wd_gload1(const uint8_t *p)
{
    if (!emu_check_global(p, 1)) EMU_ERR("scale load %p outside every buffer", (const void *)p);
    push(Op{2, nullptr, 0, 0, nullptr, nullptr});
    return *p;
}
inline v4i wd_gload_now(const uint8_t *p)
{
    if (!emu_check_global(p, 16)) EMU_ERR("register load %p outside every buffer", (const void *)p);
    v4i v;
    memcpy(&v, p, 16);
    return v;
}
