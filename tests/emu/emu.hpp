// CPU emulation shim for the DMA-ring GEMM kernels: one cooperative fiber per
// GPU lane (a block's lanes share one host thread and switch only at block
// barriers and wave exchanges; blocks run on a pool of host threads), wave
// exchanges for readfirstlane / shuffles / MFMA, DMA ops queued per lane and
// landed at s_waitcnt (LATE mode) or at issue (EARLY mode), bounds-checked
// against registered buffers and the LDS size.
#pragma once
#include <atomic>
#include <barrier>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <functional>
#include <mutex>
#include <string>
#include <thread>
#include <type_traits>
#include <vector>
#include <algorithm>
#include <sys/mman.h>
#include <unistd.h>
#include <ucontext.h>

#define __global__
#define __device__
#define __host__
#define __forceinline__ inline
#define __launch_bounds__(x)
#define __HIP_MEMORY_SCOPE_AGENT 0
#define __hip_atomic_fetch_add(p, v, o, s) __atomic_fetch_add(p, v, o)
#define __HIP_MEMORY_SCOPE_SYSTEM 0
#define __hip_atomic_load(p, o, s) __atomic_load_n(p, o)
#define __hip_atomic_store(p, v, o, s) __atomic_store_n(p, v, o)
inline float __uint_as_float(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
inline int atomicAdd(int *p, int v) { return __atomic_fetch_add(p, v, __ATOMIC_RELAXED); }
inline uint32_t __float_as_uint(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));
static constexpr int WAVE = 64;
struct alignas(16) int4 { int x, y, z, w; };
using std::min;
using std::max;
#define static_assert(...)

struct EmuDim { unsigned x = 0, y = 0, z = 0; };
inline thread_local EmuDim threadIdx, blockIdx;
inline EmuDim gridDim, blockDim;

// ------------------------------------------------------------ global buffers
struct Region { const uint8_t *p; size_t n; std::string name; };
inline std::vector<Region> g_regions;
inline std::atomic<long> g_errors{0};
inline std::mutex g_print;
#define EMU_ERR(...) do { std::lock_guard<std::mutex> _l(g_print); if (g_errors++ < 40) { fprintf(stderr, "[emu] b%u t%u: ", blockIdx.x, threadIdx.x); fprintf(stderr, __VA_ARGS__); fputc('\n', stderr); } } while (0)

// buffer that ends at a PROT_NONE page: plain out-of-bounds accesses fault
inline void *emu_alloc(size_t n, const char *name)
{
    const size_t pg = 4096, body = (n + pg - 1) / pg * pg;
    uint8_t *base = (uint8_t *)mmap(nullptr, body + pg, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS, -1, 0);
    mprotect(base + body, pg, PROT_NONE);
    uint8_t *p = base + body - n;
    g_regions.push_back({p, n, name});
    return p;
}
inline const char *emu_check_global(const void *src, size_t n)
{
    const uint8_t *s = (const uint8_t *)src;
    for (auto &r : g_regions)
        if (s >= r.p && s + n <= r.p + r.n) return r.name.c_str();
    return nullptr;
}

// ------------------------------------------------------------ block context
enum { MODE_LATE = 0, MODE_EARLY = 1 };
inline int g_mode = MODE_LATE;

struct Op { int kind; const uint8_t *src; uint32_t dst; int n; int32_t *atom; int32_t *result; };

// A barrier among the fibers of one block (the interface of std::barrier):
// a fiber that arrives before the others yields until the phase completes.
inline void emu_progress();
inline void emu_yield();
struct EmuBarrier {
    ptrdiff_t expected, arrived = 0, drops = 0;
    uint64_t phase = 0;
    explicit EmuBarrier(ptrdiff_t n) : expected(n) {}
    void complete() { arrived = 0; expected -= drops; drops = 0; ++phase; }
    void arrive_and_wait()
    {
        const uint64_t ph = phase;
        emu_progress();
        if (++arrived == expected) { complete(); return; }
        while (phase == ph) emu_yield();
    }
    void arrive_and_drop()
    {
        emu_progress();
        ++drops;
        if (++arrived == expected) complete();
    }
};
struct Blk {
    uint8_t *smem; size_t smem_size;
    EmuBarrier *bar;
    EmuBarrier *wbar[16];
    uint64_t xch[16][64];
    uint8_t wx[16][64][64];
    uint64_t xseq[16][64];   // per lane: how many wave exchanges it has entered
    bool gone[16][64];       // lane has returned from the kernel
};
inline thread_local Blk *tb;
inline thread_local std::deque<Op> tq;
inline thread_local int32_t t_claims[64];
inline thread_local int t_nclaim;
inline thread_local uint64_t t_xseq = 0;
// Wave exchanges (shuffles, readfirstlane, MFMA operand exchange) need every
// live lane of the wave: on the card they are wave-wide, here each is a
// barrier of the wave's lane threads.  A lane that skips one (divergent
// control flow around a shuffle) would pair later exchanges wrongly, so each
// lane counts the exchanges it enters and the first live lane checks that
// all live lanes are at the same one, of the same kind (1 readfirstlane,
// 2 shuffle, 3 MFMA, 4 first-lane read, 5 readlane / DPP / int shuffle, 6 any,
// 7 ballot).
inline void emu_xpost(int w, int l, int kind) { tb->xseq[w][l] = (++t_xseq << 8) | (uint64_t)kind; }
inline void emu_xcheck(int w, int l);

inline uint8_t *emu_smem() { return tb->smem; }
// static __shared__ arrays: carved from the block's LDS in declaration order
// (every lane declares them in the same order, so all get the same offsets)
inline thread_local size_t t_shoff = 0;
template <typename T>
inline T *emu_shared(size_t n)
{
    t_shoff = (t_shoff + 15) / 16 * 16;
    T *p = reinterpret_cast<T *>(tb->smem + t_shoff);
    t_shoff += n * sizeof(T);
    if (t_shoff > tb->smem_size) EMU_ERR("static LDS arrays need %zu bytes, the launch gave %zu", t_shoff, tb->smem_size);
    return p;
}
inline uint32_t lds_addr(const void *p) { return (uint32_t)((const uint8_t *)p - tb->smem); }

inline void __syncthreads() { tb->bar->arrive_and_wait(); }
inline void emu_xcheck(int w, int l)
{
    for (int i = 0; i < 64; ++i) {
        if (tb->gone[w][i]) continue;
        if (i != l) return;   // only the first live lane checks
        break;
    }
    for (int i = 0; i < 64; ++i)
        if (!tb->gone[w][i] && tb->xseq[w][i] != tb->xseq[w][l])
            EMU_ERR("wave %d: lane %d is at exchange %llu (kind %d), lane %d at %llu (kind %d): a wave exchange under divergent control flow",
                    w, i, (unsigned long long)(tb->xseq[w][i] >> 8), (int)(tb->xseq[w][i] & 255), l,
                    (unsigned long long)(tb->xseq[w][l] >> 8), (int)(tb->xseq[w][l] & 255));
}
inline int wave_id() { return threadIdx.x / 64; }
inline int lane_id() { return threadIdx.x % 64; }

// wave-wide: every lane posts v, returns lane 0's; flags non-uniform values
inline uint64_t wave_first(uint64_t v, const char *what)
{
    const int w = wave_id(), l = lane_id();
    tb->xch[w][l] = v;
    emu_xpost(w, l, 1);
    tb->wbar[w]->arrive_and_wait();
    emu_xcheck(w, l);
    const uint64_t r = tb->xch[w][0];
    if (r != v) EMU_ERR("non-uniform %s: lane %d has %llx, lane 0 %llx", what, l, (unsigned long long)v, (unsigned long long)r);
    tb->wbar[w]->arrive_and_wait();
    return r;
}
template <typename T>
inline T emu_rfl(T v)
{
    uint64_t u = 0;
    memcpy(&u, &v, sizeof(T));
    u = wave_first(u, "readfirstlane");
    T r;
    memcpy(&r, &u, sizeof(T));
    return r;
}
#define __builtin_amdgcn_readfirstlane(x) emu_rfl(x)
#define __builtin_amdgcn_sched_barrier(x) ((void)0)
#define __builtin_amdgcn_sched_group_barrier(a, b, c) ((void)0)

inline float __shfl_xor(float v, int m, int)
{
    const int w = wave_id(), l = lane_id();
    uint32_t u;
    memcpy(&u, &v, 4);
    tb->xch[w][l] = u;
    emu_xpost(w, l, 2);
    tb->wbar[w]->arrive_and_wait();
    emu_xcheck(w, l);
    uint32_t o = (uint32_t)tb->xch[w][l ^ m];
    tb->wbar[w]->arrive_and_wait();
    float r;
    memcpy(&r, &o, 4);
    return r;
}

// ------------------------------------------------------------ DMA
inline void land(const Op &o)
{
    if (o.kind == 1) {   // atomic: result delivered
        if (o.result) *o.result = *o.result;   // value fixed at issue
        return;
    }
    if (o.src) memcpy(tb->smem + o.dst, o.src, o.n);
}
inline void push(Op o)
{
    if (g_mode == MODE_EARLY) { land(o); return; }
    if (o.kind == 0) memset(tb->smem + o.dst, 0xA5, o.n);   // poison until landed
    tq.push_back(o);
}
inline void emu_wait(int n)
{
    while ((int)tq.size() > n) { land(tq.front()); tq.pop_front(); }
}
template <int N>
inline void wait_vm() { emu_wait(N); }

inline void dma_lane(const uint8_t *src, uint32_t lds_base, int bytes, const char *what)
{
    const uint32_t dst = lds_base + (uint32_t)(bytes * lane_id());
    if (!emu_check_global(src, bytes)) EMU_ERR("%s: global source %p (+%d) outside every buffer", what, (const void *)src, bytes);
    if ((size_t)dst + bytes > tb->smem_size) {
        EMU_ERR("%s: LDS destination %u..%u past the %zu-byte allocation", what, dst, dst + bytes, tb->smem_size);
        return;
    }
    bool ok = emu_check_global(src, bytes) != nullptr;
    push(Op{0, ok ? src : nullptr, dst, bytes, nullptr, nullptr});
}
// Hazard model (g_hazard bits; off by default): 1 = an LDS DMA reads M0
// before the s_mov_b32 m0 ahead of it has taken effect, so it lands at the
// previous DMA's LDS destination; 2 = a VMEM instruction reads its scalar base
// before the v_readfirstlane that wrote it has, so it uses the wave's
// previous base.  Each DMA is hit with probability g_hazard_p, the same
// choice for every lane of the wave (hash of block, wave, DMA ordinal).
inline int g_hazard = 0;
inline double g_hazard_p = 0.0;
inline unsigned g_hazard_seed = 1;
inline thread_local uint32_t t_m0 = 0;
inline thread_local const uint8_t *t_sbase = nullptr;
inline thread_local uint64_t t_ndma = 0;
inline std::atomic<long> g_hazard_hits{0};
inline bool hazard_hit(int salt)
{
    uint64_t z = ((uint64_t)blockIdx.x << 40) ^ ((uint64_t)blockIdx.y << 28) ^ ((uint64_t)wave_id() << 20) ^
                 (t_ndma * 4 + salt) ^ ((uint64_t)g_hazard_seed << 52);
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    z ^= z >> 31;
    return (double)(z >> 11) * (1.0 / 9007199254740992.0) < g_hazard_p;
}
inline uint32_t hazard_m0(uint32_t lds)
{
    uint32_t used = lds;
    if ((g_hazard & 1) && t_ndma > 0 && hazard_hit(1)) {
        used = t_m0;
        if (lane_id() == 0) {
            ++g_hazard_hits;
            if (getenv("EMU_HAZARD_LOG")) { std::lock_guard<std::mutex> _l(g_print); fprintf(stderr, "[hit] b%u w%d dma#%llu: meant LDS %u, landed at %u\n", blockIdx.x, wave_id(), (unsigned long long)t_ndma, lds, used); }
        }
    }
    t_m0 = lds;
    return used;
}
inline const uint8_t *hazard_sbase(const uint8_t *sbase)
{
    const uint8_t *used = sbase;
    if ((g_hazard & 2) && t_sbase && hazard_hit(2)) {
        used = t_sbase;
        if (lane_id() == 0) ++g_hazard_hits;
    }
    t_sbase = sbase;
    return used;
}
inline void dma16(const uint8_t *sbase, uint32_t voff, uint32_t lds)
{
    sbase = (const uint8_t *)wave_first((uint64_t)(uintptr_t)sbase, "dma16 sbase");
    lds = (uint32_t)wave_first(lds, "dma16 lds");
    sbase = hazard_sbase(sbase);
    lds = hazard_m0(lds);
    ++t_ndma;
    dma_lane(sbase + voff, lds, 16, "dma16");
}
inline void dma16_nt(const uint8_t *sbase, uint32_t voff, uint32_t lds) { dma16(sbase, voff, lds); }
inline void dma4(const uint8_t *sbase, uint32_t voff, uint32_t lds)
{
    sbase = (const uint8_t *)wave_first((uint64_t)(uintptr_t)sbase, "dma4 sbase");
    lds = (uint32_t)wave_first(lds, "dma4 lds");
    sbase = hazard_sbase(sbase);
    lds = hazard_m0(lds);
    ++t_ndma;
    dma_lane(sbase + voff, lds, 4, "dma4");
}
inline void dma4s(const void *g, uint32_t lds)
{
    lds = (uint32_t)wave_first(lds, "dma4s lds");
    lds = hazard_m0(lds);
    ++t_ndma;
    dma_lane((const uint8_t *)g, lds, 4, "dma4s");
}
// returning atomic issued by one lane: the value is fixed now, readable after its wait
inline uint32_t emu_atomic_issue(int32_t *p, uint32_t v)
{
    if (!emu_check_global(p, 4)) EMU_ERR("atomic outside every buffer");
    const int32_t old = __atomic_fetch_add(p, (int32_t)v, __ATOMIC_RELAXED);
    t_claims[t_nclaim & 63] = old;
    Op o{1, nullptr, 0, 0, p, &t_claims[t_nclaim & 63]};
    ++t_nclaim;
    if (g_mode == MODE_LATE) tq.push_back(o);
    return (uint32_t)old;
}
inline void emu_check_claim_retired()
{
    for (auto &o : tq)
        if (o.kind == 1) EMU_ERR("claim read while its atomic is still outstanding");
}

// ------------------------------------------------------------ math stand-ins
inline float __fdiv_rn(float a, float b) { return a / b; }
inline float fast_sigmoid(float x) { return 1.f / (1.f + std::exp(-x)); }
inline uint16_t bf16_from_f32(float f)
{
    uint32_t u;
    memcpy(&u, &f, 4);
    return (uint16_t)((u + 0x7fff + ((u >> 16) & 1)) >> 16);
}
inline uint32_t e4m3_enc(float f)
{
    // round-to-nearest e4m3fn, saturating (values pre-clamped to +-448)
    uint32_t s = std::signbit(f) ? 0x80 : 0;
    float a = std::fabs(f);
    if (!(a > 0)) return s;
    int e;
    float m = std::frexp(a, &e);   // a = m 2^e, m in [0.5, 1)
    int E = e - 1 + 7;
    if (E <= 0) {   // subnormal: step 2^-9
        int q = (int)std::nearbyint(a * 512.f);
        return s | (uint32_t)q;
    }
    int q = (int)std::nearbyint((m * 2 - 1) * 8);
    if (q == 8) { q = 0; ++E; }
    if (E > 15 || (E == 15 && q > 6)) { E = 15; q = 6; }
    return s | (uint32_t)(E << 3) | (uint32_t)q;
}
inline uint32_t e4m3_pack2_hw(float a, float b) { return e4m3_enc(a) | (e4m3_enc(b) << 8); }
inline float e4m3_dec(uint8_t b)
{
    const int s = b >> 7, E = (b >> 3) & 15, m = b & 7;
    float v = E ? std::ldexp(1.f + m / 8.f, E - 7) : std::ldexp(m / 8.f, -6);
    if (E == 15 && m == 7) v = NAN;
    return s ? -v : v;
}

inline float e2m1_dec(int nib)
{
    static const float mag[8] = {0.f, 0.5f, 1.f, 1.5f, 2.f, 3.f, 4.f, 6.f};
    return (nib & 8) ? -mag[nib & 7] : mag[nib & 7];
}
inline int emu_ilog2(float a)
{
    int e;
    std::frexp(a, &e);
    return e - 1;
}
inline int mx_exponent(float amax, int emax_elem)
{
    if (amax == 0.0f) return -127;
    int se = emu_ilog2(amax) - emax_elem;
    return se < -127 ? -127 : (se > 127 ? 127 : se);
}

// v_mfma_scale_f32_16x16x128_f8f6f4.  An FP8 e4m3 operand: lane 16g + r
// supplies row r, K bytes [16g, 16g+16) and [64+16g, 64+16g+16).  An FP4 e2m1
// operand (cbsz / blgp 4): lane 16g + r supplies row r, K = [32g, 32g+32) in
// its first 16 bytes (element 2i in the low nibble).  The e8m0 scale of (row
// r, 32-block b) comes from lane 16b + r's scale operand (byte opsel); scale
// 0 with every opsel 0 and all-zero scale registers is the unscaled form used
// for FP8 x FP8 (the kernels pass zeros).  Lane 16g + r receives C[4g + v][r],
// C[m][n] = sum_k A[m][k] B[n][k].
inline bool g_math = false;
inline v4f emu_mfma(v8i a, v8i b, v4f c, int cbsz, int blgp, int opa, int sa, int opb, int sb)
{
    if (!g_math) return c;
    const int w = wave_id(), l = lane_id();
    memcpy(tb->wx[w][l], &a, 32);
    memcpy(tb->wx[w][l] + 32, &b, 32);
    tb->xch[w][l] = ((uint64_t)(uint8_t)(sa >> (8 * opa)) << 8) | (uint8_t)(sb >> (8 * opb));
    emu_xpost(w, l, 3);
    tb->wbar[w]->arrive_and_wait();
    emu_xcheck(w, l);
    const int r = l & 15, g = l >> 4;
    v4f out = c;
    // element decodes and scales from tables; each lane decodes its own A
    // rows and B row once.  The products keep the order ((a * sa) * b) * sb.
    static const std::vector<float> e4m3 = [] { std::vector<float> t(256); for (int i = 0; i < 256; ++i) t[i] = e4m3_dec((uint8_t)i); return t; }();
    static const std::vector<float> pow2 = [] { std::vector<float> t(256); for (int i = 0; i < 256; ++i) t[i] = std::ldexp(1.f, i - 127); return t; }();
    auto elem = [&](int lane_row, int k, int off, bool fp4) -> float {   // element k of row lane_row
        if (fp4) {
            const uint8_t by = tb->wx[w][16 * (k / 32) + lane_row][off + (k % 32) / 2];
            return e2m1_dec((k & 1) ? by >> 4 : by & 15);
        }
        const int chunk = k / 16, gg = chunk & 3, hi = chunk >> 2;
        return e4m3[tb->wx[w][16 * gg + lane_row][off + 16 * hi + (k & 15)]];
    };
    const bool scaled = cbsz == 4 || blgp == 4;
    auto scl = [&](int lane_row, int blk, bool isa) -> float {
        if (!scaled) return 1.f;
        const uint64_t x = tb->xch[w][16 * blk + lane_row];
        return pow2[isa ? (x >> 8) & 0xff : x & 0xff];
    };
    float bv[128], bscl[4];
    for (int k = 0; k < 128; ++k) bv[k] = elem(r, k, 32, blgp == 4);
    for (int q = 0; q < 4; ++q) bscl[q] = scl(r, q, false);
    for (int v = 0; v < 4; ++v) {
        float ascl[4], av[128];
        for (int q = 0; q < 4; ++q) ascl[q] = scl(4 * g + v, q, true);
        for (int k = 0; k < 128; ++k) av[k] = elem(4 * g + v, k, 0, cbsz == 4) * ascl[k / 32];
        float s = 0;
        for (int k = 0; k < 128; ++k) s += av[k] * bv[k] * bscl[k / 32];
        out[v] += s;
    }
    tb->wbar[w]->arrive_and_wait();
    return out;
}
#define __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4 emu_mfma

// ------------------------------------------------------------ launch
// Lanes run as fibers: a host thread takes one block at a time and resumes
// its lanes in turn; a lane runs until it waits at a barrier (block barrier or
// wave exchange) or returns.  The per-lane state above (thread_local, shared
// by the fibers of one host thread) is saved and restored around each resume.
// The card runs a block's waves in no fixed order either, and no kernel here
// spins on a flag written by another lane of its block, so cooperative
// scheduling changes no result; blocks never wait for one another.
struct EmuLane {
    ucontext_t ctx;
    bool done = false;
    EmuDim tid, bid;
    Blk *b = nullptr;
    std::deque<Op> q;
    int32_t claims[64];
    int nclaim = 0;
    uint64_t xseq = 0, ndma = 0;
    size_t shoff = 0;
    uint32_t m0 = 0;
    const uint8_t *sbase = nullptr;
};
struct EmuSched {
    ucontext_t main;
    std::vector<EmuLane> lanes;
    std::vector<uint8_t *> stacks;
    size_t cur = 0;
    long idle = 0;               // resumes since the last barrier arrival or lane exit
    const std::function<void()> *body = nullptr;
};
inline thread_local EmuSched *t_sched = nullptr;
static constexpr size_t kEmuStack = 1u << 20;
inline void emu_progress() { if (t_sched) t_sched->idle = 0; }
inline void emu_yield()
{
    EmuSched *s = t_sched;
    swapcontext(&s->lanes[s->cur].ctx, &s->main);
}
inline void emu_lane_load(EmuLane &c)
{
    threadIdx = c.tid; blockIdx = c.bid; tb = c.b;
    std::swap(tq, c.q);
    memcpy(t_claims, c.claims, sizeof c.claims);
    t_nclaim = c.nclaim; t_xseq = c.xseq; t_ndma = c.ndma; t_shoff = c.shoff; t_m0 = c.m0; t_sbase = c.sbase;
}
inline void emu_lane_save(EmuLane &c)
{
    std::swap(tq, c.q);
    memcpy(c.claims, t_claims, sizeof c.claims);
    c.nclaim = t_nclaim; c.xseq = t_xseq; c.ndma = t_ndma; c.shoff = t_shoff; c.m0 = t_m0; c.sbase = t_sbase;
}
inline void emu_lane_entry()
{
    EmuSched *s = t_sched;
    (*s->body)();
    const unsigned t = threadIdx.x;
    if (!tq.empty()) EMU_ERR("lane exits with %zu DMA ops outstanding", tq.size());
    emu_wait(0);
    tb->gone[t / 64][t % 64] = true;
    tb->wbar[t / 64]->arrive_and_drop();
    tb->bar->arrive_and_drop();
    s->lanes[s->cur].done = true;   // returning resumes the scheduler (uc_link)
}
// Runs every block of the grid: lanes as fibers of one host thread per block,
// blocks spread over a pool of host threads.  smem: the block's LDS bytes;
// shoff: where static __shared__ arrays start within it.
inline void emu_run_grid(std::function<void()> fn, EmuDim g, unsigned nt, size_t smem, size_t shoff)
{
    gridDim = g;
    blockDim = {nt, 1, 1};
    std::vector<EmuDim> blocks;
    for (unsigned z = 0; z < g.z; ++z)
        for (unsigned y = 0; y < g.y; ++y)
            for (unsigned x = 0; x < g.x; ++x) blocks.push_back({x, y, z});
    std::atomic<size_t> next{0};
    auto worker = [&] {
        EmuSched S;
        S.body = &fn;
        S.lanes.resize(nt);
        for (unsigned t = 0; t < nt; ++t) {
            uint8_t *st = (uint8_t *)mmap(nullptr, kEmuStack, PROT_READ | PROT_WRITE,
                                          MAP_PRIVATE | MAP_ANONYMOUS | MAP_NORESERVE, -1, 0);
            mprotect(st, 4096, PROT_NONE);   // guard page below the stack
            S.stacks.push_back(st);
        }
        t_sched = &S;
        for (size_t bi; (bi = next.fetch_add(1)) < blocks.size();) {
            Blk *B = new Blk();
            B->smem_size = smem;
            B->smem = (uint8_t *)aligned_alloc(256, (smem + 255) / 256 * 256 + 256);
            memset(B->smem, 0x5A, smem);
            B->bar = new EmuBarrier(nt);
            for (unsigned w = 0; w < nt / 64; ++w) B->wbar[w] = new EmuBarrier(64);
            for (unsigned t = 0; t < nt; ++t) {
                EmuLane &c = S.lanes[t];
                c.done = false;
                c.tid = {t, 0, 0};
                c.bid = blocks[bi];
                c.b = B;
                c.q.clear();
                c.nclaim = 0; c.xseq = 0; c.ndma = 0; c.shoff = shoff; c.m0 = 0; c.sbase = nullptr;
                getcontext(&c.ctx);
                c.ctx.uc_stack.ss_sp = S.stacks[t];
                c.ctx.uc_stack.ss_size = kEmuStack;
                c.ctx.uc_link = &S.main;
                makecontext(&c.ctx, emu_lane_entry, 0);
            }
            S.idle = 0;
            for (size_t live = nt; live > 0;) {
                live = 0;
                for (unsigned t = 0; t < nt; ++t) {
                    EmuLane &c = S.lanes[t];
                    if (c.done) continue;
                    S.cur = t;
                    emu_lane_load(c);
                    swapcontext(&S.main, &c.ctx);
                    emu_lane_save(c);
                    if (!c.done) ++live;
                    else S.idle = 0;
                    if (++S.idle > 4l * nt + 8) {
                        threadIdx = c.tid; blockIdx = c.bid;
                        EMU_ERR("every live lane waits at a barrier the others never reach (divergent barrier)");
                        fflush(stderr);
                        abort();
                    }
                }
            }
            free(B->smem);
            delete B->bar;
            for (unsigned w = 0; w < nt / 64; ++w) delete B->wbar[w];
            delete B;
        }
        t_sched = nullptr;
        for (auto *st : S.stacks) munmap(st, kEmuStack);
    };
    const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
    const size_t nw = std::min<size_t>({blocks.size(), (size_t)std::min(hw, 8u), 8});
    std::vector<std::thread> th;
    for (size_t i = 1; i < nw; ++i) th.emplace_back(worker);
    worker();
    for (auto &t : th) t.join();
}
template <typename F>
inline void emu_launch(F fn, unsigned gx, unsigned gy, unsigned nt, size_t smem, unsigned /*conc*/)
{
    emu_run_grid(fn, {gx, gy, 1}, nt, smem, 0);
}
inline uint32_t emu_first_lane(uint32_t v)
{
    const int w = wave_id(), l = lane_id();
    tb->xch[w][l] = v;
    emu_xpost(w, l, 4);
    tb->wbar[w]->arrive_and_wait();
    emu_xcheck(w, l);
    const uint32_t r = (uint32_t)tb->xch[w][0];
    tb->wbar[w]->arrive_and_wait();
    return r;
}
