// ff_runtime.hip -- device memory, streams, events and graph capture behind
// the plain-C ABI of fastface_kernels.h.  Every HIP error is turned into a
// negative return code plus a per-thread message (no exceptions cross the
// ABI, matching the reference C API's NULL / non-zero convention,
// libfastface.c:235-237,313).
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <string.h>

#include "ff_internal.h"

static thread_local char g_err[512];

void ffk_set_error(const char* fmt, const char* a, const char* b) {
    snprintf(g_err, sizeof g_err, fmt, a ? a : "", b ? b : "");
}

int ffk_hip_fail(hipError_t e, const char* what) {
    ffk_set_error("%s: %s", what, hipGetErrorString(e));
    return FFK_ERR_HIP;
}

// n bytes from a 16-byte aligned d: 16-byte vector stores, then the tail
__global__ void zero_kernel(int8_t* d, size_t n) {
    const size_t n16 = n / 16;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride)
        reinterpret_cast<v4i*>(d)[i] = v4i{0, 0, 0, 0};
    if (blockIdx.x == 0 && threadIdx.x < n - n16 * 16) d[n16 * 16 + threadIdx.x] = 0;
}

extern "C" {

const char* ffk_last_error(void) { return g_err; }

int ffk_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

void* ffk_malloc(size_t bytes) {
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, bytes ? bytes : 1);
    if (e != hipSuccess) { ffk_hip_fail(e, "hipMalloc"); return nullptr; }
    return p;
}

int ffk_free(void* p) {
    if (!p) return FFK_OK;
    hipError_t e = hipFree(p);
    return e == hipSuccess ? FFK_OK : ffk_hip_fail(e, "hipFree");
}

void* ffk_host_alloc(size_t bytes) {
    void* p = nullptr;
    hipError_t e = hipHostMalloc(&p, bytes ? bytes : 1, hipHostMallocDefault);
    if (e != hipSuccess) { ffk_hip_fail(e, "hipHostMalloc"); return nullptr; }
    return p;
}

int ffk_host_free(void* p) {
    if (!p) return FFK_OK;
    hipError_t e = hipHostFree(p);
    return e == hipSuccess ? FFK_OK : ffk_hip_fail(e, "hipHostFree");
}

static int copy(void* dst, const void* src, size_t n, hipMemcpyKind k, void* s, const char* w) {
    if (n == 0) return FFK_OK;
    if (!dst || !src) { ffk_set_error("%s: null pointer", w, nullptr); return FFK_ERR_ARG; }
    hipError_t e = hipMemcpyAsync(dst, src, n, k, (hipStream_t)s);
    return e == hipSuccess ? FFK_OK : ffk_hip_fail(e, w);
}

int ffk_memcpy_h2d(void* d, const void* h, size_t n, void* s) {
    return copy(d, h, n, hipMemcpyHostToDevice, s, "memcpy h2d");
}
int ffk_memcpy_d2h(void* h, const void* d, size_t n, void* s) {
    return copy(h, d, n, hipMemcpyDeviceToHost, s, "memcpy d2h");
}
int ffk_memcpy_d2d(void* d, const void* s2, size_t n, void* s) {
    return copy(d, s2, n, hipMemcpyDeviceToDevice, s, "memcpy d2d");
}

int ffk_zero(void* d, size_t n, void* s) {
    if (n == 0) return FFK_OK;
    if (!d || ((uintptr_t)d & 15)) {
        ffk_set_error("zero: null or unaligned pointer%s%s", nullptr, nullptr);
        return FFK_ERR_ARG;
    }
    const size_t n16 = n / 16;
    const int grid = (int)(n16 / 256 + 1 < 4096 ? n16 / 256 + 1 : 4096);
    hipLaunchKernelGGL(zero_kernel, dim3(grid), dim3(256), 0, (hipStream_t)s, (int8_t*)d, n);
    return ffk_check_launch("zero launch");
}

int ffk_stream_create(void** s) {
    hipStream_t st;
    // default priority only: a non-blocking stream at normal priority
    hipError_t e = hipStreamCreateWithFlags(&st, hipStreamNonBlocking);
    if (e != hipSuccess) return ffk_hip_fail(e, "hipStreamCreate");
    *s = st;
    return FFK_OK;
}

int ffk_stream_destroy(void* s) {
    if (!s) return FFK_OK;
    hipError_t e = hipStreamDestroy((hipStream_t)s);
    return e == hipSuccess ? FFK_OK : ffk_hip_fail(e, "hipStreamDestroy");
}

int ffk_stream_sync(void* s) {
    hipError_t e = s ? hipStreamSynchronize((hipStream_t)s) : hipDeviceSynchronize();
    return e == hipSuccess ? FFK_OK : ffk_hip_fail(e, "synchronize");
}

int ffk_event_create(void** ev) {
    hipEvent_t e0;
    hipError_t e = hipEventCreate(&e0);
    if (e != hipSuccess) return ffk_hip_fail(e, "hipEventCreate");
    *ev = e0;
    return FFK_OK;
}

int ffk_event_destroy(void* ev) {
    if (!ev) return FFK_OK;
    hipError_t e = hipEventDestroy((hipEvent_t)ev);
    return e == hipSuccess ? FFK_OK : ffk_hip_fail(e, "hipEventDestroy");
}

int ffk_event_record(void* ev, void* s) {
    hipError_t e = hipEventRecord((hipEvent_t)ev, (hipStream_t)s);
    return e == hipSuccess ? FFK_OK : ffk_hip_fail(e, "hipEventRecord");
}

int ffk_event_sync(void* ev) {
    hipError_t e = hipEventSynchronize((hipEvent_t)ev);
    return e == hipSuccess ? FFK_OK : ffk_hip_fail(e, "hipEventSynchronize");
}

int ffk_stream_wait_event(void* s, void* ev) {
    hipError_t e = hipStreamWaitEvent((hipStream_t)s, (hipEvent_t)ev, 0);
    return e == hipSuccess ? FFK_OK : ffk_hip_fail(e, "hipStreamWaitEvent");
}

int ffk_event_elapsed_ms(void* a, void* b, float* ms) {
    hipError_t e = hipEventSynchronize((hipEvent_t)b);
    if (e != hipSuccess) return ffk_hip_fail(e, "hipEventSynchronize");
    e = hipEventElapsedTime(ms, (hipEvent_t)a, (hipEvent_t)b);
    return e == hipSuccess ? FFK_OK : ffk_hip_fail(e, "hipEventElapsedTime");
}

int ffk_graph_begin(void* s) {
    hipError_t e = hipStreamBeginCapture((hipStream_t)s, hipStreamCaptureModeThreadLocal);
    return e == hipSuccess ? FFK_OK : ffk_hip_fail(e, "hipStreamBeginCapture");
}

int ffk_graph_end(void* s, void** exec) {
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture((hipStream_t)s, &g);
    if (e != hipSuccess) return ffk_hip_fail(e, "hipStreamEndCapture");
    hipGraphExec_t ge = nullptr;
    e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return ffk_hip_fail(e, "hipGraphInstantiate");
    *exec = ge;
    return FFK_OK;
}

int ffk_graph_launch(void* exec, void* s) {
    hipError_t e = hipGraphLaunch((hipGraphExec_t)exec, (hipStream_t)s);
    return e == hipSuccess ? FFK_OK : ffk_hip_fail(e, "hipGraphLaunch");
}

int ffk_graph_destroy(void* exec) {
    if (!exec) return FFK_OK;
    hipError_t e = hipGraphExecDestroy((hipGraphExec_t)exec);
    return e == hipSuccess ? FFK_OK : ffk_hip_fail(e, "hipGraphExecDestroy");
}

}  // extern "C"
