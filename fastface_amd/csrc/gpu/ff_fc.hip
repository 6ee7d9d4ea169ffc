// ff_fc.hip -- FC head 25088 -> 512 (the reference's XOR-0x80 +
// fastface_gemm_i8_matvec_vnni, libfastface.c:441-455,
// kernels/gemm_int8_matvec.c:33-81) and the MFMA layout self check.
//
// Small batches: HBM-bound matvec.  Each output row's 25088 weight bytes are
// streamed once, split over FC_KSPLIT waves (contiguous ranges of K steps,
// 16 B per lane per load, v_dot4 signed int8 products into exact int32), so
// that the whole 12.8 MB weight matrix is in flight at once; the batch's
// activation rows come from L2.  Cross-lane and then cross-wave (LDS) sums
// give the exact dot product per face.  Larger batches use the MFMA conv
// kernel as a 1x1 GEMM (ff_conv.hip).
#include <cstring>
#include "ff_internal.h"
#include "ff_numerics.h"

int ffk_fc_gemm_launch(const ffk_fc_desc* d, hipStream_t s);
size_t ffk_fc_split_ws_bytes(int batch);

namespace {

constexpr int FC_MAXB = 16;   // matvec path handles up to this many faces

__device__ __forceinline__ int dot16(v4i a, v4i w, int acc) {
    acc = __builtin_amdgcn_sdot4(a.x, w.x, acc, false);
    acc = __builtin_amdgcn_sdot4(a.y, w.y, acc, false);
    acc = __builtin_amdgcn_sdot4(a.z, w.z, acc, false);
    acc = __builtin_amdgcn_sdot4(a.w, w.w, acc, false);
    return acc;
}

// Packed weights: [K/64][N][64] (the conv packing with Cin = K).  A
// workgroup takes FC_ROWS consecutive rows (they share 128-byte weight
// lines) with FC_KSPLIT waves each; wave (r, q) covers K steps
// [q*per, (q+1)*per) of row n, lane l reading piece (l & 3) of step
// q*per + it*16 + l/4.  Integer sums are exact in any order, so the split
// changes no bit of the result.
constexpr int FC_ROWS = 2;
constexpr int FC_KSPLIT = 8;
constexpr int FC_NT = FC_ROWS * FC_KSPLIT * 64;

__global__ __launch_bounds__(FC_NT) void fc_matvec_kernel(const int8_t* __restrict__ a,
                                                          const int8_t* __restrict__ w,
                                                          const float* __restrict__ ws,
                                                          const float* __restrict__ bias,
                                                          float a_scale, float* out,
                                                          const ffk_io* io, int io_face, int B, int N,
                                                          int K) {
    __shared__ int part[FC_ROWS][FC_KSPLIT][FC_MAXB];
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int r = wave / FC_KSPLIT;
    const int q = wave - r * FC_KSPLIT;
    const int n = blockIdx.x * FC_ROWS + r;
    const int ksteps = K / FF_KSTEP;
    const int per = (ksteps + FC_KSPLIT - 1) / FC_KSPLIT;
    const int s1 = min(ksteps, (q + 1) * per);
    int acc[FC_MAXB];
#pragma unroll
    for (int b = 0; b < FC_MAXB; b++) acc[b] = 0;
    if (n < N) {
#pragma unroll 4
        for (int s = q * per + (lane >> 2); s < s1; s += 16) {
            const int kofs = s * FF_KSTEP + (lane & 3) * 16;
            const v4i wv = *reinterpret_cast<const v4i*>(w + ((size_t)s * N + n) * FF_KSTEP + (lane & 3) * 16);
#pragma unroll
            for (int b = 0; b < FC_MAXB; b++) {
                if (b < B) {
                    const v4i av = *reinterpret_cast<const v4i*>(a + (size_t)b * K + kofs);
                    acc[b] = dot16(av, wv, acc[b]);
                }
            }
        }
    }
#pragma unroll
    for (int b = 0; b < FC_MAXB; b++) {
        if (b < B) {
            int v = acc[b];
#pragma unroll
            for (int sh = 32; sh >= 1; sh >>= 1) v += __shfl_xor(v, sh, 64);
            if (lane == 0) part[r][q][b] = v;
        }
    }
    __syncthreads();
    if (q == 0 && n < N && lane < B) {      // lane b: face b of row n
        int v = 0;
#pragma unroll
        for (int k = 0; k < FC_KSPLIT; k++) v += part[r][k][lane];
        float* o = out ? out : io->out + (size_t)io_face * N;
        o[(size_t)lane * N + n] = ff::fc_out(v, a_scale, ws[n], bias[n]);
    }
}

// 32x32x32 i8 MFMA with A[i][k] = (i*7 + k*3) % 17 - 8, B[k][j] = (k*5 + j) % 13 - 6.
__global__ void mfma_probe_kernel(int* out) {
    const int lane = threadIdx.x;
    uint32_t aw[4] = {0, 0, 0, 0}, bw[4] = {0, 0, 0, 0};
    for (int e = 0; e < 16; e++) {
        const int k = (lane >> 5) * 16 + e;
        const int i = lane & 31;
        const int av = (i * 7 + k * 3) % 17 - 8;
        const int bv = (k * 5 + i) % 13 - 6;   // column j = lane & 31
        aw[e >> 2] |= ((uint32_t)av & 0xffu) << ((e & 3) * 8);
        bw[e >> 2] |= ((uint32_t)bv & 0xffu) << ((e & 3) * 8);
    }
    const v4i A = {(int)aw[0], (int)aw[1], (int)aw[2], (int)aw[3]};
    const v4i Bv = {(int)bw[0], (int)bw[1], (int)bw[2], (int)bw[3]};
    v16i c;
    for (int r = 0; r < 16; r++) c[r] = 0;
    c = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, Bv, c, 0, 0, 0);
    for (int r = 0; r < 16; r++) {
        const int row = (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
        const int col = lane & 31;
        out[row * 32 + col] = c[r];
    }
}

}  // namespace

extern "C" {

size_t ffk_fc_packed_bytes(int n, int k) { return (size_t)n * (size_t)k; }

int ffk_pack_fc_weights(const int8_t* w, int n, int k, int8_t* packed) {
    if (!w || !packed || n <= 0 || k <= 0 || (k % FF_KSTEP) != 0) {
        ffk_set_error("pack_fc_weights: bad arguments (k must be a multiple of 64)%s%s", nullptr, nullptr);
        return FFK_ERR_ARG;
    }
    for (int r = 0; r < n; r++) ffk_pack_fc_row(w + (size_t)r * k, n, k, r, packed);
    return FFK_OK;
}

int ffk_pack_fc_row(const int8_t* row, int n, int k, int r, int8_t* packed) {
    if (!row || !packed || n <= 0 || k <= 0 || (k % FF_KSTEP) != 0 || r < 0 || r >= n) {
        ffk_set_error("pack_fc_row: bad arguments (k must be a multiple of 64)%s%s", nullptr, nullptr);
        return FFK_ERR_ARG;
    }
    for (int s = 0; s < k / FF_KSTEP; s++)
        memcpy(packed + ((size_t)s * n + r) * FF_KSTEP, row + (size_t)s * FF_KSTEP, FF_KSTEP);
    return FFK_OK;
}

size_t ffk_fc_workspace_bytes(const ffk_fc_desc* d) {
    if (!d || d->batch <= 0 || d->n != 512 || d->k != 25088) return 0;
    const int path = d->path ? d->path : (d->batch <= FC_MAXB ? 1 : 2);
    return path == 2 ? ffk_fc_split_ws_bytes(d->batch) : 0;
}

int ffk_fc(const ffk_fc_desc* d, void* stream) {
    if (!d || d->batch < 0 || !d->a || !d->w || !d->ws || !d->bias || (!d->out && !d->io) ||
        d->n <= 0 || d->k <= 0 || (d->k % FF_KSTEP) != 0) {
        ffk_set_error("fc: bad descriptor%s%s", nullptr, nullptr);
        return FFK_ERR_ARG;
    }
    if (d->batch == 0) return FFK_OK;
    hipStream_t s = (hipStream_t)stream;
    int path = d->path;
    // the MFMA GEMM is compiled for the IResNet head (25088 -> 512); any
    // other shape takes the matvec in chunks of FC_MAXB faces at every batch
    const bool gemm_shape = d->n == 512 && d->k == 25088;
    if (path == 0) path = (d->batch <= FC_MAXB || !gemm_shape) ? 1 : 2;
    if (path == 2) return ffk_fc_gemm_launch(d, s);
    for (int b0 = 0; b0 < d->batch; b0 += FC_MAXB) {
        const int nb = d->batch - b0 < FC_MAXB ? d->batch - b0 : FC_MAXB;
        float* out = d->out ? d->out + (size_t)b0 * d->n : nullptr;
        hipLaunchKernelGGL(fc_matvec_kernel, dim3((d->n + FC_ROWS - 1) / FC_ROWS), dim3(FC_NT), 0, s,
                           d->a + (size_t)b0 * d->k, d->w, d->ws, d->bias, d->a_scale, out, d->io, b0,
                           nb, d->n, d->k);
        int rc = ffk_check_launch("fc matvec launch");
        if (rc) return rc;
    }
    return FFK_OK;
}

int ffk_selftest_mfma(void) {
    int* d = (int*)ffk_malloc(32 * 32 * sizeof(int));
    if (!d) return FFK_ERR_NOMEM;
    hipLaunchKernelGGL(mfma_probe_kernel, dim3(1), dim3(64), 0, 0, d);
    int rc = ffk_check_launch("mfma probe launch");
    int h[32 * 32];
    if (!rc) {
        hipError_t e = hipMemcpy(h, d, sizeof h, hipMemcpyDeviceToHost);
        if (e != hipSuccess) rc = ffk_hip_fail(e, "mfma probe copy");
    }
    ffk_free(d);
    if (rc) return rc;
    for (int i = 0; i < 32; i++)
        for (int j = 0; j < 32; j++) {
            int ref = 0;
            for (int k = 0; k < 32; k++) ref += ((i * 7 + k * 3) % 17 - 8) * ((k * 5 + j) % 13 - 6);
            if (h[i * 32 + j] != ref) {
                ffk_set_error("mfma layout mismatch%s%s", nullptr, nullptr);
                return FFK_ERR_UNSUPPORTED;
            }
        }
    return FFK_OK;
}

}  // extern "C"
