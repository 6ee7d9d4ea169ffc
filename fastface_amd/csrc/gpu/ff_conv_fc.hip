// ff_conv_fc.hip -- the FC head 25088 -> 512 as an MFMA GEMM (batches over
// 16 faces): conv_i8_kernel run as a 1x1 "conv" over a 1x1 image with
// Cin = K, optionally with split-K through the conv workspace.
#include "ff_conv_table.h"


// FC head through the same kernel (a 1x1 "conv" over a 1x1 image with
// Cin = K): M = batch faces, N = 512, K = 25088.
int ffk_fc_gemm_launch(const ffk_fc_desc* d, hipStream_t s) {
    if (d->n != 512 || d->k != 25088) {
        ffk_set_error("fc gemm: unsupported shape (n must be 512, k 25088)%s%s", nullptr, nullptr);
        return FFK_ERR_UNSUPPORTED;
    }
    ConvArgs a = {};
    a.in = d->a;
    a.w = d->w;
    a.fc_ws = d->ws;
    a.fc_bias = d->bias;
    a.io = d->io;
    a.out_f32 = d->out;
    a.M = d->batch;
    a.flags = 0;
    a.in_scale = d->a_scale;
    a.tiles_n = 512 / 128;
    const int tiles = ((d->batch + 127) / 128) * a.tiles_n;
    const size_t need = ffk_fc_split_ws_bytes(d->batch);
    if (need && d->workspace && d->workspace_bytes >= need) {
        // split-K: FC_SPLIT workgroups per 128x128 output tile (the last to
        // arrive sums the int32 partial tiles and writes the fp32 outputs)
        a.counters = (unsigned*)d->workspace;
        a.ws = (int32_t*)((int8_t*)d->workspace + FF_SPLIT_COUNTER_BYTES);
        hipLaunchKernelGGL((conv_i8_kernel<25088, 512, 1, 1, 1, 1, 128, 128, 64, FF_PF, 2, 2, 2, FC_SPLIT>),
                           dim3(tiles * FC_SPLIT), dim3(256), 0, s, a);
        return ffk_check_launch("fc gemm launch");
    }
    hipLaunchKernelGGL((conv_i8_kernel<25088, 512, 1, 1, 1, 1, 128, 128, 128, FF_PF128, 2, 2, 2, 1>),
                       dim3(tiles), dim3(256), 0, s, a);
    return ffk_check_launch("fc gemm launch");
}

// FC GEMM split-K: K = 25088 is 392 stages of 64 bytes; 8 ranges of 49, one
// per XCD (conv_i8_kernel).  A batch whose tiles fit the counter area and
// leave the GPU under-filled with one workgroup per tile (fewer than two per
// CU) splits.
size_t ffk_fc_split_ws_bytes(int batch) {
    const long long tiles = ((long long)(batch + 127) / 128) * (512 / 128);
    if (batch <= 0 || tiles > FF_SPLIT_MAX_WG || tiles >= 512) return 0;
    return FF_SPLIT_COUNTER_BYTES + (size_t)tiles * FC_SPLIT * 128 * 128 * sizeof(int32_t);
}

