// ff_internal.h -- shared between the HIP translation units (not exported).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../../include/fastface_kernels.h"

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

void ffk_set_error(const char* fmt, const char* a, const char* b);
int ffk_hip_fail(hipError_t e, const char* what);

// Launch-time check: a kernel launch error (bad configuration) is reported
// right away instead of surfacing at the next synchronization.
static inline int ffk_check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? FFK_OK : ffk_hip_fail(e, what);
}

// Packed weight layout shared by every int8 MFMA kernel: the reduction index
// k = (kh*KW + kw)*Cin + ci is cut into steps of 64; step s of output channel
// n lives at  w[(s*Cout + n)*64 .. +64).  One K step of a whole output-channel
// tile is therefore one contiguous block of BN*64 bytes.
static constexpr int FF_KSTEP = 64;

// A conv workspace starts with the split-K arrival counters, which every
// split launch leaves at zero for the next one.
static constexpr size_t FF_WS_COUNTER_AREA = 2048;

// Integer Winograd F(2,3) path of the 64-channel 3x3 stride-1 layers
// (ff_winograd.hip), taken by ffk_conv for FFK_ALGO_WINOGRAD.
int ffk_winograd_eligible(const ffk_conv_desc* d);
int ffk_winograd_conv(const ffk_conv_desc* d, hipStream_t s);
