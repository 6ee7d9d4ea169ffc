// ff_phase_probe.hip -- where the time of a 3x3 conv launch goes, per
// workgroup: the library's own kernel templates and launchers, compiled here
// with FF_PHASE_STAMPS so that wave 0 of every workgroup records the real-time
// counter at the kernel's entry, its main loop's first barrier (the first
// patch and weights have landed), the end of the main loop, the start of the
// epilogue (after the K-group reduction of the small-grid kernel) and its end.
//
//   fastface_amd/bin/ff_phase_probe
//
// Cases: the 256 -> 256 3x3 layer at 14x14 (the network's dominant shape)
//   - at N = 8 and N = 64 through the small-grid kernel
//     the library runs there (conv3_patch_kg_kernel, FF_PMID),
//   - at N = 1024 through the large-batch patch kernel (conv3_patch_kernel,
//     two workgroups per CU: their phases overlap in time).
// Synthetic random int8 activations and weights, the PReLU epilogue in the
// in-range form the network runs.  Per case one JSON line: the mean launch
// time of 20 back-to-back launches (HIP events), the span from the first
// workgroup's entry to the last one's end, the median and maximum over
// workgroups of each phase, the last workgroup's start and the times by which
// 50 / 90 / 98 / 100 % of the workgroups had ended, all of the last of those
// launches.
#define FF_PHASE_STAMPS 4096
#include "ff_conv_table.h"

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <vector>

namespace {

#define PROBE_CHECK(x)                                                                  \
    do {                                                                                \
        hipError_t e_ = (x);                                                            \
        if (e_ != hipSuccess) {                                                         \
            fprintf(stderr, "ff_phase_probe: %s: %s\n", #x, hipGetErrorString(e_));     \
            exit(1);                                                                    \
        }                                                                               \
    } while (0)

constexpr int CIN = 256, COUT = 256, HW = 14;

double median(std::vector<double> v) {
    std::sort(v.begin(), v.end());
    return v[v.size() / 2];
}

void run_case(const char* kernel, ffconv::launch_fn fn, int batch, int bm, int bn) {
    const int M = batch * HW * HW;
    const int tiles_n = COUT / bn;
    const int grid = (M + bm - 1) / bm * tiles_n;
    if (grid > FF_PHASE_STAMPS) {
        fprintf(stderr, "ff_phase_probe: grid %d exceeds the stamp buffer\n", grid);
        exit(1);
    }
    std::mt19937 rng(1);
    std::vector<int8_t> hin((size_t)M * CIN), hw((size_t)9 * CIN * COUT);
    for (auto& v : hin) v = (int8_t)((int)(rng() % 255) - 127);
    for (auto& v : hw) v = (int8_t)((int)(rng() % 255) - 127);
    std::vector<float> hp((size_t)FFK_NPARAM * COUT, 0.0f);
    for (int c = 0; c < COUT; c++) {
        hp[FFK_P_WS * COUT + c] = 1e-4f;
        hp[FFK_P_BIAS * COUT + c] = 0.1f;
        hp[FFK_P_SLOPE * COUT + c] = 0.25f;
        hp[FFK_P_INV * COUT + c] = 1.0f / 40.0f;
    }
    int8_t *din = nullptr, *dw = nullptr, *dout = nullptr;
    float* dp = nullptr;
    PROBE_CHECK(hipMalloc(&din, hin.size()));
    PROBE_CHECK(hipMalloc(&dw, hw.size()));
    PROBE_CHECK(hipMalloc(&dp, hp.size() * sizeof(float)));
    PROBE_CHECK(hipMalloc(&dout, (size_t)M * COUT));
    PROBE_CHECK(hipMemcpy(din, hin.data(), hin.size(), hipMemcpyHostToDevice));
    PROBE_CHECK(hipMemcpy(dw, hw.data(), hw.size(), hipMemcpyHostToDevice));
    PROBE_CHECK(hipMemcpy(dp, hp.data(), hp.size() * sizeof(float), hipMemcpyHostToDevice));
    ConvArgs a = {};
    a.in = din;
    a.w = dw;
    a.params = dp;
    a.out = dout;
    a.M = M;
    a.in_scale = 1.0f;
    a.tiles_n = tiles_n;
    a.flags = FFK_EPI_PRELU | FFK_EPI_PRELU_LE1 | FFK_EPI_BIAS | FFK_EPI_IN_RANGE;

    hipEvent_t e0, e1;
    PROBE_CHECK(hipEventCreate(&e0));
    PROBE_CHECK(hipEventCreate(&e1));
    for (int i = 0; i < 5; i++) fn(a, grid, 0);
    PROBE_CHECK(hipGetLastError());
    PROBE_CHECK(hipDeviceSynchronize());
    PROBE_CHECK(hipEventRecord(e0, 0));
    for (int i = 0; i < 20; i++) fn(a, grid, 0);
    PROBE_CHECK(hipEventRecord(e1, 0));
    PROBE_CHECK(hipEventSynchronize(e1));
    float ms = 0;
    PROBE_CHECK(hipEventElapsedTime(&ms, e0, e1));

    std::vector<unsigned long long> t((size_t)grid * 5);
    PROBE_CHECK(hipMemcpyFromSymbol(t.data(), HIP_SYMBOL(ff_phase_stamps), t.size() * sizeof(unsigned long long)));
    int khz = 0;
    PROBE_CHECK(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, 0));
    const double us_per_tick = 1e3 / khz;
    std::vector<double> ph[5];
    unsigned long long first = ~0ull, last = 0;
    for (int b = 0; b < grid; b++) {
        const unsigned long long* r = &t[(size_t)b * 5];
        first = std::min(first, r[0]);
        last = std::max(last, r[4]);
        for (int i = 0; i < 4; i++) ph[i].push_back((double)(r[i + 1] - r[i]) * us_per_tick);
        ph[4].push_back((double)(r[4] - r[0]) * us_per_tick);
    }
    // when the workgroups start and end, from the first entry: the last start, and the time
    // by which 50 / 90 / 98 % of them had ended and the last one did
    std::vector<double> st, en;
    for (int b = 0; b < grid; b++) {
        st.push_back((double)(t[(size_t)b * 5] - first) * us_per_tick);
        en.push_back((double)(t[(size_t)b * 5 + 4] - first) * us_per_tick);
    }
    std::sort(en.begin(), en.end());
    auto pct = [&](double q) { return en[std::min(grid - 1, (int)(q * grid))]; };
    const char* name[5] = {"prologue", "main_loop", "reduction", "epilogue", "workgroup"};
    printf("{\"kernel\": \"%s\", \"batch\": %d, \"grid\": %d, \"launch_us\": %.2f, \"span_us\": %.2f",
           kernel, batch, grid, ms * 1e3 / 20, (double)(last - first) * us_per_tick);
    for (int i = 0; i < 5; i++)
        printf(", \"%s_us\": [%.2f, %.2f]", name[i], median(ph[i]), *std::max_element(ph[i].begin(), ph[i].end()));
    printf(", \"last_start_us\": %.2f, \"ended_50_90_98_100_us\": [%.2f, %.2f, %.2f, %.2f]", *std::max_element(st.begin(), st.end()),
           pct(0.5), pct(0.9), pct(0.98), en.back());
    printf("}\n");
    fflush(stdout);
    PROBE_CHECK(hipEventDestroy(e0));
    PROBE_CHECK(hipEventDestroy(e1));
    PROBE_CHECK(hipFree(din));
    PROBE_CHECK(hipFree(dw));
    PROBE_CHECK(hipFree(dp));
    PROBE_CHECK(hipFree(dout));
}

}  // namespace

int main() {
    // ([median, max] over workgroups; the patch kernel has no reduction phase)
    run_case("conv3_patch_kg_kernel", FF_PMID(CIN, COUT, HW), 8, 128, 128);
    run_case("conv3_patch_kg_kernel", FF_PMID(CIN, COUT, HW), 64, 128, 128);
    run_case("conv3_patch_kernel", &ffconv::launch_patch<CIN, COUT, HW, FF_TPATCH>, 1024, 256, 128);
    return 0;
}
