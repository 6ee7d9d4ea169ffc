// ff_issue_probe.hip -- what bounds the int8 conv kernels on gfx950: the
// i8 MFMA rate with random and with constant operands, the same MFMAs fed from
// LDS, and how MFMA work and requantization-style VALU work share a SIMD when
// they come from the same wave or from different waves.
//
//   fastface_amd/bin/ff_issue_probe [steps]
//
// Prints one JSON line per measurement: kernel time (HIP events, mean of 5
// launches after one warm-up) and the int8 rate against MI355X's 5.0 POP/s
// dense spec.  Every launch fills all 256 CUs; nothing is read from or
// written to memory in the timed loops except the result guard at the end.
// Run it under rocprofv3 --pmc GRBM_GUI_ACTIVE SQ_VALU_MFMA_BUSY_CYCLES to
// see the clock each case runs at.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

namespace {

#define PROBE_CHECK(x)                                                                  \
    do {                                                                                \
        hipError_t e_ = (x);                                                            \
        if (e_ != hipSuccess) {                                                         \
            fprintf(stderr, "ff_issue_probe: %s: %s\n", #x, hipGetErrorString(e_));     \
            exit(1);                                                                    \
        }                                                                               \
    } while (0)

__device__ __forceinline__ unsigned mix(unsigned h) {
    h ^= h >> 13;
    h *= 0x5bd1e995u;
    h ^= h >> 15;
    return h;
}

// Operand words: uniformly random bytes, or a constant pattern (low toggle rate).
__device__ __forceinline__ int operand(unsigned seed, bool random) {
    return random ? (int)mix(mix(seed) + 0x9e3779b9u) : (int)0x01010101;
}

constexpr int LDS_BYTES = 64 * 1024;

// MODE 0: MFMAs on register operands; 1: operands read from LDS (2x2 wave
// tile: 4 b128 reads per 4 MFMAs per K half, conflict-free 80-byte pitch);
// 2: MFMAs plus, in the same wave, VALU elements of the conv epilogue's
// arithmetic (10 operations each); 3: the VALU elements alone; 4: waves 0-3
// of each workgroup run mode 0's MFMAs, waves 4-7 mode 3's VALU work (each
// SIMD holds MFMA waves and VALU waves); 5: mode 1's LDS-fed MFMAs with VEL
// epilogue elements interleaved in the same wave (an epilogue spread over
// the next tile's main loop).
// VEL: VALU elements per step (16 MFMAs per step in modes 0-2).
template <int MODE, int VEL>
__global__ __launch_bounds__(512) void probe_kernel(int steps, int random, int* guard) {
    __shared__ __align__(1024) int8_t smem[LDS_BYTES];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool do_mfma = MODE <= 2 || MODE == 5 || (MODE == 4 && (wave & 4) == 0);
    const bool do_valu = MODE == 2 || MODE == 3 || MODE == 5 || (MODE == 4 && (wave & 4) != 0);
    if (MODE == 1 || MODE == 5) {
        for (int i = tid; i < LDS_BYTES / 16; i += 512) {
            v4i v;
            for (int q = 0; q < 4; q++) v[q] = operand(i * 4 + q, random != 0);
            reinterpret_cast<v4i*>(smem)[i] = v;
        }
        __syncthreads();
    }
    v16i acc[2][2];
    for (int i = 0; i < 2; i++)
        for (int j = 0; j < 2; j++)
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0;
    v4i ra[2], rb[2];
    for (int i = 0; i < 2; i++)
        for (int q = 0; q < 4; q++) {
            ra[i][q] = operand(lane * 977 + i * 131 + q * 7 + wave * 65537 + blockIdx.x * 3, random != 0);
            rb[i][q] = operand(lane * 613 + i * 71 + q * 11 + wave * 4099 + blockIdx.x * 5 + 1, random != 0);
        }
    // (A operands in the first 32 KB, B in the second; every read stays below 64 KB)
    const int base = (lane & 31) * 80 + (lane >> 5) * 16 + (wave & 3) * 2560;
    float f[16];
    for (int r = 0; r < 16; r++) f[r] = (float)(int)(mix(tid * 16 + r) & 0xffff);
    const float ws = 0.0037f + lane * 1e-6f, bias = 0.5f, slope = 0.25f, inv = 0.031f;
    int q = 0;
    for (int s = 0; s < steps; s++) {
        if (do_mfma) {
#pragma unroll
            for (int ks = 0; ks < 4; ks++) {
                v4i af[2], bf[2];
                if (MODE == 1 || MODE == 5) {
                    const int off = ((s * 4 + ks) & 7) * 1024;
#pragma unroll
                    for (int i = 0; i < 2; i++) af[i] = *reinterpret_cast<const v4i*>(smem + base + off + i * 8192 + (ks & 1) * 32);
#pragma unroll
                    for (int j = 0; j < 2; j++) bf[j] = *reinterpret_cast<const v4i*>(smem + base + off + 32768 + j * 8192 + (ks & 1) * 32);
                } else {
                    af[0] = ra[0]; af[1] = ra[1]; bf[0] = rb[0]; bf[1] = rb[1];
                }
#pragma unroll
                for (int i = 0; i < 2; i++)
#pragma unroll
                    for (int j = 0; j < 2; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
            }
        }
        if (do_valu) {
#pragma unroll
            for (int r = 0; r < VEL; r++) {
                float x = f[r & 15];
                x = x * ws;
                x = x + bias;
                x = __builtin_fmaxf(x, x * slope);
                x = x * inv;
                x = x + __builtin_copysignf(0.5f, x);
                const int v = (int)__builtin_amdgcn_fmed3f(x, -128.0f, 127.0f);
                q ^= v;
                f[r & 15] = (float)(v + s);
            }
        }
        if (MODE == 2 || MODE == 5) {
            // one MFMA, then its share of the VALU work, in the wave's order
#pragma unroll
            for (int i = 0; i < 16; i++) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, VEL * 10 / 16, 0);
            }
        }
    }
    int sum = q;
    for (int i = 0; i < 2; i++)
        for (int j = 0; j < 2; j++)
            for (int r = 0; r < 16; r++) sum += acc[i][j][r];
    if (sum == 0x7a5a5a5a) guard[tid] = sum;
}

template <int MODE, int VEL>
void run(const char* name, int grid, int steps, int random, int* guard) {
    hipEvent_t e0, e1;
    PROBE_CHECK(hipEventCreate(&e0));
    PROBE_CHECK(hipEventCreate(&e1));
    hipLaunchKernelGGL((probe_kernel<MODE, VEL>), dim3(grid), dim3(512), 0, 0, steps, random, guard);
    PROBE_CHECK(hipGetLastError());
    PROBE_CHECK(hipDeviceSynchronize());
    PROBE_CHECK(hipEventRecord(e0, 0));
    for (int i = 0; i < 5; i++) hipLaunchKernelGGL((probe_kernel<MODE, VEL>), dim3(grid), dim3(512), 0, 0, steps, random, guard);
    PROBE_CHECK(hipEventRecord(e1, 0));
    PROBE_CHECK(hipEventSynchronize(e1));
    float ms = 0;
    PROBE_CHECK(hipEventElapsedTime(&ms, e0, e1));
    ms /= 5;
    // 8 waves per workgroup; mode 4: half of them run each kind of work
    const double mw = MODE <= 2 || MODE == 5 ? 8 : (MODE == 4 ? 4 : 0);
    const double vw = MODE == 2 || MODE == 3 || MODE == 5 ? 8 : (MODE == 4 ? 4 : 0);
    const double mfma = (double)grid * mw * steps * 16;
    const double tops = mfma * 32 * 32 * 32 * 2 / (ms * 1e-3) / 1e12;
    const double valu = (double)grid * vw * steps * VEL * 10;
    printf("{\"case\": \"%s\", \"workgroups\": %d, \"waves_per_simd\": %d, \"random_operands\": %s, \"ms\": %.4f, "
           "\"int8_tops\": %.1f, \"frac_of_5pops\": %.3f, \"valu_ops_per_mfma\": %.1f}\n",
           name, grid, grid / 128, random ? "true" : "false", ms, tops, tops / 5000.0,
           mfma > 0 ? valu / mfma : 0.0);
    fflush(stdout);
    PROBE_CHECK(hipEventDestroy(e0));
    PROBE_CHECK(hipEventDestroy(e1));
}

}  // namespace

int main(int argc, char** argv) {
    const int steps = argc > 1 ? atoi(argv[1]) : 1000;
    if (steps <= 0 || steps > 100000) {
        fprintf(stderr, "ff_issue_probe: steps must be 1..100000\n");
        return 2;
    }
    int* guard = nullptr;
    PROBE_CHECK(hipMalloc(&guard, 512 * sizeof(int)));
    // 512 workgroups of 8 waves (64 KB of LDS each): two per CU, 4 waves per
    // SIMD; 256 workgroups: one per CU, 2 waves per SIMD
    run<0, 0>("mfma_registers", 512, steps, 0, guard);
    run<0, 0>("mfma_registers", 512, steps, 1, guard);
    run<1, 0>("mfma_from_lds", 512, steps, 1, guard);
    run<0, 0>("mfma_registers", 256, steps, 1, guard);
    run<3, 32>("valu_only", 256, steps, 1, guard);
    run<2, 32>("mfma_and_valu_same_wave", 256, steps, 1, guard);
    run<3, 32>("valu_only", 512, steps, 1, guard);
    run<2, 32>("mfma_and_valu_same_wave", 512, steps, 1, guard);
    run<4, 32>("mfma_waves_beside_valu_waves", 512, steps, 1, guard);
    // the conv's ratio (~2.5 VALU per MFMA): 4 epilogue elements per 16 MFMAs
    run<1, 0>("mfma_from_lds", 256, steps, 1, guard);
    run<5, 4>("mfma_from_lds_and_epilogue_same_wave", 256, steps, 1, guard);
    run<3, 4>("valu_only", 256, steps, 1, guard);
    run<5, 4>("mfma_from_lds_and_epilogue_same_wave", 512, steps, 1, guard);
    run<3, 4>("valu_only", 512, steps, 1, guard);
    PROBE_CHECK(hipFree(guard));
    return 0;
}
