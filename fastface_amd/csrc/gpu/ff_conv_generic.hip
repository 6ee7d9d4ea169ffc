// ff_conv_generic.hip -- any conv geometry the tuned kernel table does not
// hold (the reference's im2col + GEMM path takes every shape:
// kernels/conv2d_nhwc.c:150-220): an implicit GEMM with the geometry in
// registers instead of template parameters.
//
// 64- or 128-wide output tiles, four waves of 32x32x32 i8 MFMAs.  Channel
// counts that are multiples of 16 load the A operand (16-byte channel runs
// of the NHWC input) and the B operand (packed weights) straight into a
// double-buffered LDS ring (conv_generic_dma_kernel); other channel counts
// stage it through registers, in 8-byte runs or byte by byte (any channel
// count; the 3-channel input layer quantizes fp32 faces or maps uint8 pixels
// on the fly).  The epilogue is the general form of the tuned kernels' per
// element (in-scale, ws, bias, residual, PReLU, round half away with the x86
// out-of-range case), then X, its even pixels only or BN(X) through the
// channel's table.  No LDS reuse of the input patch: each tap's run is read
// from L2 / HBM for every output pixel.
#include "ff_conv_table.h"
#include "ff_numerics.h"

#include <algorithm>

namespace {

struct GenGeom {
    int cin, cout, kh, kw, stride, pad, hin, win, hout, wout;
    int ktot;       // kh * kw * cin
    int kpad;       // ktot rounded up to whole 64-byte weight steps
    unsigned in_bytes;   // the launch's int8 input tensor (below 2 GiB)
};

// A thread's position k in the reduction order (kh*KW + kw)*Cin + ci: tap
// row th, tap column tw, channel ci, and off = (th*Win + tw)*Cin + ci, the
// input element's offset from the output pixel's tap (0, 0) element.
struct KCursor {
    int k, ci, th, tw, off;
};

__device__ __forceinline__ KCursor kcursor_at(const GenGeom& g, int k) {
    KCursor c;
    const int tap = k / g.cin;
    c.k = k;
    c.ci = k - tap * g.cin;
    c.th = tap / g.kw;
    c.tw = tap - c.th * g.kw;
    c.off = (c.th * g.win + c.tw) * g.cin + c.ci;
    return c;
}

// Moves the cursor n elements on without a division: each channel wrap is
// the next tap (the next pixel of the row: off runs on), each tap-column
// wrap the next tap row (off skips Win - KW pixels).
__device__ __forceinline__ void kcursor_step(KCursor& c, const GenGeom& g, int n) {
    c.k += n;
    c.ci += n;
    c.off += n;
    while (c.ci >= g.cin) {
        c.ci -= g.cin;
        if (++c.tw == g.kw) {
            c.tw = 0;
            c.th++;
            c.off += (g.win - g.kw) * g.cin;
        }
    }
}

// The 16 A-operand bytes from cursor c on of the output pixel whose tap (0, 0)
// is input pixel (ih0, iw0) at element offset base (channel counts that are
// multiples of 16 take conv_generic_dma_kernel instead).
// RUN 8: two taps' 8-byte runs (Cin % 8 == 0) through the int8 input's
// buffer resource r_in, where padding, rows past the batch and k past K take
// the out-of-range offset and read zeros.  RUN 0: byte by byte (any Cin, and
// the 3-channel input layer, which quantizes fp32 faces or maps uint8
// pixels), zeros there by branch.
template <int RUN>
__device__ __forceinline__ v4i gather_a(const ConvArgs& a, const GenGeom& g, __amdgpu_buffer_rsrc_t r_in,
                                        const void* x, bool mrow, long long base, int ih0, int iw0, KCursor c) {
    static_assert(RUN == 8 || RUN == 0, "16-byte runs: conv_generic_dma_kernel");
    if constexpr (RUN == 8) {
        v4i v;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            if (h) kcursor_step(c, g, 8);
            const int ih = ih0 + c.th, iw = iw0 + c.tw;
            const bool in = mrow && c.k < g.ktot && ih >= 0 && ih < g.hin && iw >= 0 && iw < g.win;
            const unsigned off = in ? (unsigned)(base + c.off) : FF_OOB;
            const auto u = __builtin_amdgcn_raw_buffer_load_b64(r_in, off, 0, 0);
            v[2 * h] = (int)u[0];
            v[2 * h + 1] = (int)u[1];
        }
        return v;
    } else {
        v4i v = {0, 0, 0, 0};
        if (!mrow) return v;
        const bool stem = g.cin == 3;
        const bool rgb8 = stem && (a.flags & FFK_IN_RGB8);
        // (global-space pointers: the input may come through the I/O
        // descriptor, whose pointer the compiler cannot place)
        typedef const __attribute__((address_space(1))) int8_t* gi8;
        typedef const __attribute__((address_space(1))) uint8_t* gu8;
        typedef const __attribute__((address_space(1))) float* gf32;
        for (int e = 0; e < 16; e++) {
            if (e) kcursor_step(c, g, 1);
            int q = 0;
            if (c.k < g.ktot) {
                const int ih = ih0 + c.th, iw = iw0 + c.tw;
                if (ih >= 0 && ih < g.hin && iw >= 0 && iw < g.win) {
                    const long long off = base + c.off;
                    if (!stem) q = ((gi8)x)[off];
                    else if (rgb8) q = a.in_lut[c.ci * 256 + ((gu8)x)[off]];
                    else q = ff::quant_input(((gf32)x)[off], a.in_inv[c.ci]);
                }
            }
            v[e >> 2] |= (int)((uint32_t)(uint8_t)q << (8 * (e & 3)));
        }
        return v;
    }
}

// The general epilogue per element (the tuned kernels' general form: in-scale,
// ws, bias, residual, PReLU, round half away with the x86 out-of-range
// case), then X, its even pixels only or BN(X) through the channel's table,
// stored straight from registers: lane owns column wc + 32j + lane%32 and 16
// rows of each of the wave's MI x NJ blocks at tile (m0, n0).
template <int MI, int NJ>
__device__ __forceinline__ void gen_epilogue(const v16i (&acc)[MI][NJ], const ConvArgs& a, const GenGeom& g,
                                             long long m0, int n0, int wr, int wc) {
    const int lane = threadIdx.x & 63;
    const int hw = g.hout * g.wout;
    const int C = g.cout;
    const float* P = a.params;
    const bool raw = a.out_i32 != nullptr;
    const bool x_even = (a.flags & FFK_OUT_X_EVEN) != 0;
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int n = n0 + wc + j * 32 + (lane & 31);
        if (n >= C) continue;
        float ws = 0.0f, bias = 0.0f, inv = 0.0f, slope = 0.0f, adds = 0.0f;
        if (!raw) {
            ws = P[FFK_P_WS * C + n];
            bias = P[FFK_P_BIAS * C + n];
            inv = P[FFK_P_INV * C + n];
            slope = P[FFK_P_SLOPE * C + n];
            adds = P[FFK_P_ADDSCALE * C + n];
        }
#pragma unroll
        for (int i = 0; i < MI; i++)
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const long long mm = m0 + wr + i * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
                if (mm >= a.M) continue;
                const size_t o = (size_t)mm * C + n;
                if (raw) {
                    a.out_i32[o] = acc[i][j][e];
                    continue;
                }
                float f = (float)acc[i][j][e];
                if (a.flags & FFK_EPI_INSCALE) f = f * a.in_scale;
                f = f * ws;
                f = f + bias;
                if (a.flags & FFK_EPI_ADD) f = ff::add_residual(f, (int32_t)a.add_src[o], adds);
                if (a.flags & FFK_EPI_PRELU) f = ff::prelu(f, slope);
                const int q = ff::requant_haz(f * inv);
                if (a.out) {
                    if (!x_even) {
                        a.out[o] = (int8_t)q;
                    } else {
                        const int bb = (int)(mm / hw);
                        const int rem = (int)(mm - (long long)bb * hw);
                        const int oh = rem / g.wout, ow = rem - oh * g.wout;
                        if (!((oh | ow) & 1))
                            a.out[(((size_t)bb * (g.hout / 2) + (oh >> 1)) * (g.wout / 2) + (ow >> 1)) * C + n] = (int8_t)q;
                    }
                }
                if (a.flags & FFK_EPI_BN) a.out_bn[o] = a.bn_lut[n * 256 + q + 128];
            }
    }
}

// Channel counts that are not multiples of 16: BM x BN output tiles (64 or
// 128 each) of four waves in a 2 x 2 grid, each
// wave MI x NJ 32x32 blocks; per 64-byte K step every thread stages 16 bytes
// of BM/64 A rows (output pixels) and of BN/64 B rows (output channels) in
// LDS, then each wave runs 2 * MI * NJ 32x32x32 MFMAs; the next step's loads
// are in flight meanwhile.  A 128-wide tile halves the gathers of the other
// operand per MAC: every staged A row serves BN output channels, every B row
// BM output pixels.
template <int RUN, int BM, int BN>
__global__ __launch_bounds__(256) void conv_generic_kernel(ConvArgs a, GenGeom g) {
    constexpr int AR = BM / 64, BR = BN / 64;          // operand rows each thread stages
    constexpr int MI = BM / 64, NJ = BN / 64;          // 32x32 blocks per wave (2 x 2 waves)
    // one 64-byte K step per barrier pair (two or four steps' pieces staged
    // at once, their loads in flight together, measured 7-48 % slower:
    // fewer waves per SIMD, the gathers' VALU work back to back)
    constexpr int PITCH = 80;                          // LDS row pitch of the staged operands
    __shared__ __align__(16) int8_t As[BM * PITCH];
    __shared__ __align__(16) int8_t Bs[BN * PITCH];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int tiles_n = (g.cout + BN - 1) / BN;
    // Workgroups go round-robin over the 8 XCDs: give each XCD a contiguous
    // run of tiles (N fastest), so the tiles that gather the same pixels
    // share one L2.
    const unsigned nb = gridDim.x, bid = blockIdx.x;
    const unsigned t = (nb & 7) == 0 ? (bid & 7) * (nb >> 3) + (bid >> 3) : bid;
    const long long m0 = (long long)(t / tiles_n) * BM;
    const int n0 = (int)(t % tiles_n) * BN;
    const int hw = g.hout * g.wout;
    const void* x = g.cin != 3 ? (const void*)a.in : a.in_f32 ? (const void*)a.in_f32 : (const void*)a.io->in;

    const int r = tid >> 2, kq = (tid & 3) * 16;
    bool mrow[AR];
    int ih0[AR], iw0[AR];
    long long base[AR];          // element offset of the row's tap (0, 0) input pixel
#pragma unroll
    for (int i = 0; i < AR; i++) {
        const long long m = m0 + r + 64 * i;
        mrow[i] = m < a.M;
        ih0[i] = 0; iw0[i] = 0; base[i] = 0;
        if (mrow[i]) {
            const int b = (int)(m / hw);
            const int rem = (int)(m - (long long)b * hw);
            const int oh = rem / g.wout;
            ih0[i] = oh * g.stride - g.pad;
            iw0[i] = (rem - oh * g.wout) * g.stride - g.pad;
            base[i] = (((long long)b * g.hin + ih0[i]) * g.win + iw0[i]) * g.cin;
        }
    }
    KCursor cur = kcursor_at(g, kq);
    const __amdgpu_buffer_rsrc_t r_in = ff_rsrc(a.in, RUN ? g.in_bytes : 0u);
    const int wr = (wave >> 1) * (BM / 2), wc = (wave & 1) * (BN / 2);
    auto load_b = [&](int k0, int i) {
        const int ncol = n0 + r + 64 * i;
        v4i v = {0, 0, 0, 0};
        if (ncol < g.cout) v = *reinterpret_cast<const v4i*>(a.w + ((size_t)(k0 >> 6) * g.cout + ncol) * 64 + kq);
        return v;
    };

    v16i acc[MI][NJ];
#pragma unroll
    for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[i][j][e] = 0;
    v4i ra[AR], rb[BR];
#pragma unroll
    for (int i = 0; i < AR; i++) ra[i] = gather_a<RUN>(a, g, r_in, x, mrow[i], base[i], ih0[i], iw0[i], cur);
#pragma unroll
    for (int i = 0; i < BR; i++) rb[i] = load_b(0, i);
    for (int k0 = 0; k0 < g.kpad; k0 += 64) {
        __syncthreads();                                  // the previous step's fragments are read
#pragma unroll
        for (int i = 0; i < AR; i++) *reinterpret_cast<v4i*>(As + (r + 64 * i) * PITCH + kq) = ra[i];
#pragma unroll
        for (int i = 0; i < BR; i++) *reinterpret_cast<v4i*>(Bs + (r + 64 * i) * PITCH + kq) = rb[i];
        __syncthreads();
        if (k0 + 64 < g.kpad) {
            kcursor_step(cur, g, 64);
#pragma unroll
            for (int i = 0; i < AR; i++) ra[i] = gather_a<RUN>(a, g, r_in, x, mrow[i], base[i], ih0[i], iw0[i], cur);
#pragma unroll
            for (int i = 0; i < BR; i++) rb[i] = load_b(k0 + 64, i);
        }
#pragma unroll
        for (int h = 0; h < 2; h++) {
            v4i A[MI], B[NJ];
#pragma unroll
            for (int i = 0; i < MI; i++)
                A[i] = *reinterpret_cast<const v4i*>(As + (wr + i * 32 + (lane & 31)) * PITCH + h * 32 + (lane >> 5) * 16);
#pragma unroll
            for (int j = 0; j < NJ; j++)
                B[j] = *reinterpret_cast<const v4i*>(Bs + (wc + j * 32 + (lane & 31)) * PITCH + h * 32 + (lane >> 5) * 16);
#pragma unroll
            for (int i = 0; i < MI; i++)
#pragma unroll
                for (int j = 0; j < NJ; j++) acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[i], B[j], acc[i][j], 0, 0, 0);
        }
    }

    gen_epilogue<MI, NJ>(acc, a, g, m0, n0, wr, wc);
}

// Cin % 16 == 0 (16-byte channel runs): the same tiles with the operands
// loaded straight into a GEN_NST-deep LDS ring (direct-to-LDS buffer loads:
// no register staging, the loads of GEN_NST - 1 steps in flight; two stages,
// 16-32 KB, leave room for four or five workgroups per CU, which measured
// 15-25 % faster than three or four stages with fewer workgroups).  A stage is
// BM + BN 64-byte rows in 256-byte lines of four rows, the 16-byte slot of
// (row r, piece p) ((r%4)*4 + p) XOR (r/4 % 4), as in conv_dma_kernel: the
// 16 rows a ds_read_b128 lane group reads land in 16 distinct slots.  A lane
// fetches the same piece p of its rows at every step (the swizzle picks
// which), so one K cursor per thread serves all its A rows; padding, rows
// past the batch, k past K and channels past Cout read zeros through the
// out-of-range offset.
constexpr int GEN_NST = 2;

template <int BM, int BN>
__global__ __launch_bounds__(256, 2) void conv_generic_dma_kernel(ConvArgs a, GenGeom g) {
    constexpr int MI = BM / 64, NJ = BN / 64;          // 32x32 blocks per wave (2 x 2 waves)
    constexpr int A_BYTES = BM * 64, B_BYTES = BN * 64, STAGE = A_BYTES + B_BYTES;
    constexpr int A_LD = A_BYTES / (256 * 16), B_LD = B_BYTES / (256 * 16);
    constexpr int LPS = A_LD + B_LD;                   // loads per thread and stage
    static_assert((GEN_NST - 2) * LPS < 64, "vmcnt range");
    __shared__ __align__(1024) int8_t smem[GEN_NST * STAGE];
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int tiles_n = (g.cout + BN - 1) / BN;
    const unsigned nb = gridDim.x, bid = blockIdx.x;
    const unsigned t = (nb & 7) == 0 ? (bid & 7) * (nb >> 3) + (bid >> 3) : bid;
    const long long m0 = (long long)(t / tiles_n) * BM;
    const int n0 = (int)(t % tiles_n) * BN;
    const int hw = g.hout * g.wout;
    const int nsteps = g.kpad / 64;
    const __amdgpu_buffer_rsrc_t r_in = ff_rsrc(a.in, g.in_bytes);
    const __amdgpu_buffer_rsrc_t r_w = ff_rsrc(a.w, (unsigned)(nsteps * g.cout * 64));

    // this thread's pieces: wave load j of wave w fills lines (4j + w)*4 ..
    // +3 of a stage's A (B) rows; lane L takes line +L/16, slot L%16, which
    // holds piece p = slot%4 XOR ... of row 4*line + slot/4
    const int sl = (lane & 15) ^ ((lane >> 4) & 3);
    const int p = sl & 3;
    int a_base[A_LD], a_ih0[A_LD], a_iw0[A_LD];
#pragma unroll
    for (int j = 0; j < A_LD; j++) {
        const int r = ((j * 4 + wave) * 4 + (lane >> 4)) * 4 + (sl >> 2);
        const long long m = m0 + r;
        a_base[j] = 0; a_iw0[j] = 0;
        a_ih0[j] = -(1 << 28);                         // a row past the batch fails every bounds check
        if (m < a.M) {
            const int b = (int)(m / hw);
            const int rem = (int)(m - (long long)b * hw);
            const int oh = rem / g.wout;
            a_ih0[j] = oh * g.stride - g.pad;
            a_iw0[j] = (rem - oh * g.wout) * g.stride - g.pad;
            a_base[j] = ((b * g.hin + a_ih0[j]) * g.win + a_iw0[j]) * g.cin;
        }
    }
    unsigned b_off[B_LD];
#pragma unroll
    for (int j = 0; j < B_LD; j++) {
        const int n = n0 + ((j * 4 + wave) * 4 + (lane >> 4)) * 4 + (sl >> 2);
        b_off[j] = n < g.cout ? (unsigned)(n * 64 + p * 16) : FF_OOB;
    }
    KCursor cur = kcursor_at(g, p * 16);
    auto issue = [&](int st, int buf) {
        int8_t* sb = smem + buf * STAGE;
        const bool kin = cur.k < g.ktot;
#pragma unroll
        for (int j = 0; j < A_LD; j++) {
            const int ih = a_ih0[j] + cur.th, iw = a_iw0[j] + cur.tw;
            const bool v = kin && ih >= 0 && ih < g.hin && iw >= 0 && iw < g.win;
            bdma16(r_in, v ? (unsigned)(a_base[j] + cur.off) : FF_OOB, 0u, sb + (j * 4 + wave) * 1024);
        }
        const unsigned wst = (unsigned)(st * g.cout * 64);
#pragma unroll
        for (int j = 0; j < B_LD; j++)
            bdma16(r_w, b_off[j] == FF_OOB ? FF_OOB : b_off[j] + wst, 0u, sb + A_BYTES + (j * 4 + wave) * 1024);
        kcursor_step(cur, g, 64);
    };

    const int wm = wave >> 1, wn = wave & 1;
    const int a_rd = dma_slot(wm * MI * 32 + (lane & 31), lane >> 5);
    const int b_rd = A_BYTES + dma_slot(wn * NJ * 32 + (lane & 31), lane >> 5);
    v16i acc[MI][NJ];
#pragma unroll
    for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[i][j][e] = 0;
#pragma unroll
    for (int u = 0; u < GEN_NST - 1; u++)
        if (u < nsteps) issue(u, u);
    int rbuf = 0;                                      // ring slot of step s
    for (int st = 0; st < nsteps; st++) {
        if (st + GEN_NST - 2 < nsteps) dma_wait_barrier<(GEN_NST - 2) * LPS>();
        else dma_wait_barrier<0>();
        if (st + GEN_NST - 1 < nsteps) issue(st + GEN_NST - 1, rbuf == 0 ? GEN_NST - 1 : rbuf - 1);
        const int8_t* sb = smem + rbuf * STAGE;
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
            v4i af[MI], bf[NJ];
#pragma unroll
            for (int i = 0; i < MI; i++) af[i] = *reinterpret_cast<const v4i*>(sb + ((a_rd + i * 2048) ^ (ks * 32)));
#pragma unroll
            for (int j = 0; j < NJ; j++) bf[j] = *reinterpret_cast<const v4i*>(sb + ((b_rd + j * 2048) ^ (ks * 32)));
#pragma unroll
            for (int i = 0; i < MI; i++)
#pragma unroll
                for (int j = 0; j < NJ; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        rbuf = rbuf == GEN_NST - 1 ? 0 : rbuf + 1;
    }
    gen_epilogue<MI, NJ>(acc, a, g, m0, n0, wm * (BM / 2), wn * (BN / 2));
}

// Tile shape of a launch: 128-wide in N above 64 output channels, 128-high
// in M where that still gives the 256 CUs a workgroup each, except for the
// 3-channel input layer, whose byte gather runs faster on 64-row tiles.
struct GenTile { int bm, bn; };

GenTile gen_tile(long long M, int cin, int cout) {
    GenTile t;
    t.bn = cout > 64 ? 128 : 64;
    const long long tiles_n = (cout + t.bn - 1) / t.bn;
    t.bm = cin != 3 && ((M + 127) / 128) * tiles_n >= 256 ? 128 : 64;
    return t;
}

template <int RUN>
void launch_run(GenTile t, dim3 gd, hipStream_t s, const ConvArgs& a, const GenGeom& g) {
    const dim3 bd(256);
    if constexpr (RUN == 16) {
        if (t.bm == 128 && t.bn == 128) hipLaunchKernelGGL((conv_generic_dma_kernel<128, 128>), gd, bd, 0, s, a, g);
        else if (t.bm == 128) hipLaunchKernelGGL((conv_generic_dma_kernel<128, 64>), gd, bd, 0, s, a, g);
        else if (t.bn == 128) hipLaunchKernelGGL((conv_generic_dma_kernel<64, 128>), gd, bd, 0, s, a, g);
        else hipLaunchKernelGGL((conv_generic_dma_kernel<64, 64>), gd, bd, 0, s, a, g);
    } else {
        if (t.bm == 128 && t.bn == 128) hipLaunchKernelGGL((conv_generic_kernel<RUN, 128, 128>), gd, bd, 0, s, a, g);
        else if (t.bm == 128) hipLaunchKernelGGL((conv_generic_kernel<RUN, 128, 64>), gd, bd, 0, s, a, g);
        else if (t.bn == 128) hipLaunchKernelGGL((conv_generic_kernel<RUN, 64, 128>), gd, bd, 0, s, a, g);
        else hipLaunchKernelGGL((conv_generic_kernel<RUN, 64, 64>), gd, bd, 0, s, a, g);
    }
}

}  // namespace

// Workgroups of the generic kernel for M output pixels (one per tile).
long long ff_conv_generic_grid(long long M, int cin, int cout) {
    const GenTile t = gen_tile(M, cin, cout);
    return ((M + t.bm - 1) / t.bm) * ((cout + t.bn - 1) / t.bn);
}

int ff_conv_generic_launch(const ConvArgs& a, const ffk_conv_desc* d, hipStream_t s) {
    GenGeom g;
    g.cin = d->cin; g.cout = d->cout; g.kh = d->kh; g.kw = d->kw; g.stride = d->stride; g.pad = d->pad;
    g.hin = d->hin; g.win = d->win;
    g.hout = (d->hin + 2 * d->pad - d->kh) / d->stride + 1;
    g.wout = (d->win + 2 * d->pad - d->kw) / d->stride + 1;
    g.ktot = d->kh * d->kw * d->cin;
    g.kpad = (g.ktot + FF_KSTEP - 1) / FF_KSTEP * FF_KSTEP;
    // channel runs are read as 8- / 16-byte vectors: they need the run's
    // alignment in memory (a tensor base that is not 16-byte aligned takes
    // the byte gather)
    const int run = (d->cin == 3 || d->cin % 8 || ((uintptr_t)d->in & 15)) ? 0 : d->cin % 16 ? 8 : 16;
    // The channel-run gathers address the int8 input with 32-bit offsets: a
    // batch whose input or output tensor reaches 2 GiB runs as several
    // launches over consecutive image ranges (images are independent).  The
    // byte gather uses 64-bit addresses and takes the batch in one launch.
    const long long px_out = (long long)g.hout * g.wout;
    const long long in_img = (long long)d->hin * d->win * d->cin;
    const long long img = std::max<long long>(in_img, px_out * d->cout);
    const int slice = run == 0 ? d->batch : (int)std::min<long long>(d->batch, 0x7fffffffLL / img);
    if (slice < 1) {
        ffk_set_error("conv: one image's tensors reach 2 GiB%s%s", nullptr, nullptr);
        return FFK_ERR_ARG;
    }
    const bool x_even = (d->flags & FFK_OUT_X_EVEN) != 0;
    for (int b0 = 0; b0 < d->batch; b0 += slice) {
        const int nb = std::min(slice, d->batch - b0);
        ConvArgs as = a;
        as.M = (int)((long long)nb * px_out);
        const size_t o = (size_t)b0 * px_out * d->cout;
        if (run) as.in = a.in + (size_t)b0 * in_img;
        if (a.add_src) as.add_src = a.add_src + o;
        if (a.out) as.out = a.out + (x_even ? o / 4 : o);     // even/even pixels: a quarter
        if (a.out_bn) as.out_bn = a.out_bn + o;
        if (a.out_i32) as.out_i32 = a.out_i32 + o;
        g.in_bytes = run ? (unsigned)(nb * in_img) : 0u;
        const long long grid = ff_conv_generic_grid(as.M, d->cin, d->cout);
        if (grid > 0x7fffffffLL) {
            ffk_set_error("conv: batch too large for the generic kernel%s%s", nullptr, nullptr);
            return FFK_ERR_ARG;
        }
        const GenTile t = gen_tile(as.M, d->cin, d->cout);
        const dim3 gd((unsigned)grid);
        if (run == 0) launch_run<0>(t, gd, s, as, g);
        else if (run == 8) launch_run<8>(t, gd, s, as, g);
        else launch_run<16>(t, gd, s, as, g);
        const int rc = ffk_check_launch("generic conv launch");
        if (rc != FFK_OK) return rc;
    }
    return FFK_OK;
}
