// Self-test of the emulator's lane scheduling (emu.hpp): a kernel with block
// barriers and wave shuffles must give its known result with no error; a
// shuffle that only some lanes of a wave reach must be reported; lanes that
// wait at barriers the others never reach must be reported (and the run
// stopped) instead of hanging.
//   selftest_main ok | div_shuffle | deadlock
#include "emu.hpp"

static float *g_out;

static void sum_kernel(int diverge)
{
    float *part = emu_shared<float>(16);
    const int t = threadIdx.x, w = t / 64, l = t % 64;
    float v = (float)(t + 1);
    if (diverge == 2 && t == 0) __syncthreads();   // the other lanes go to the shuffle below
    if (diverge == 1) {        // one exchange each, of different kinds
        if (l < 32) v += __shfl_xor(v, 1, 64);
        else v += 0.0f * (float)__builtin_amdgcn_readfirstlane(t);
    }
    for (int m = 1; m < 64; m <<= 1) v += __shfl_xor(v, m, 64);
    if (l == 0) part[w] = v;
    __syncthreads();
    if (t == 0) {
        float s = 0;
        for (unsigned i = 0; i < blockDim.x / 64; ++i) s += part[i];
        g_out[blockIdx.x] = s;
    }
    __syncthreads();
}

int main(int argc, char **argv)
{
    const std::string mode = argc > 1 ? argv[1] : "ok";
    const int diverge = mode == "div_shuffle" ? 1 : mode == "deadlock" ? 2 : 0;
    const unsigned nb = 5, nt = diverge == 2 ? 64 : 256;
    g_out = (float *)emu_alloc(sizeof(float) * nb, "out");
    emu_launch([&] { sum_kernel(diverge); }, nb, 1, nt, 64, 1);
    int bad = 0;
    for (unsigned b = 0; b < nb; ++b) bad += g_out[b] != (float)(nt * (nt + 1) / 2);
    printf("result mismatches %d\nerrors %ld\n", bad, g_errors.load());
    return 0;
}
