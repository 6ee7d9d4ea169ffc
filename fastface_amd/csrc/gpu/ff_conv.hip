// ff_conv.hip -- host side of the int8 convolution: layer lookup over the
// kernel tables, launch choice (tiles, split-K), packing, tables, and the
// ffk_conv entry points.  The kernels (ff_conv_kernels.h):
// NHWC int8 convolution as implicit GEMM on gfx950 i8 MFMA
// (v_mfma_i32_32x32x32_i8, int32 accumulation) with the requantization
// epilogue fused into the store stage.
//
// GEMM view of one layer: M = batch*Hout*Wout output pixels, N = Cout,
// K = KH*KW*Cin in (kh, kw, ci) order.  The reference computes exactly these
// integers with im2col + a u8 x s8 VNNI GEMM and a -128*colsum correction
// (kernels/conv2d_nhwc.c:29-220, kernels/gemm_int8_v2.c:42-110); signed i8
// MFMA needs no correction, and integer sums do not depend on their order,
// so the accumulators are bit-identical.
//
// Two kernels share the epilogue: conv_dma_kernel (large grids: operands go
// straight from global into a swizzled LDS ring with global_load_lds_dwordx4)
// and conv_i8_kernel (small grids and split-K: register-staged operands).
//
// conv_i8_kernel K loop: workgroup = 4 wave64s computing a BM x BN tile (each
// wave MI x NJ MFMA 32x32 tiles).  Per K stage of KB = 64 or 128 bytes each thread fetches
// 16-byte pieces of the implicit im2col rows (one input pixel's channel run;
// padding taps read a zero page, so there are no branches) and of the packed
// weights.  PF stages of loads are in flight in registers; each stage goes
// through a double-buffered LDS tile whose KB+16-byte row pitch makes the
// ds_read_b128 MFMA operand reads conflict-free.  Small batches of the layers
// with long K chains split the stages of a tile over several workgroups
// (split-K, int32 partial tiles in a caller workspace).
//
// Epilogue straight from the accumulator registers: in the 32x32 MFMA result
// every lane owns one output channel (column) and 16 pixels (rows), so each
// lane needs the per-channel parameters of only NJ = 2 channels.  The int8
// results go through a small per-wave LDS byte tile only to leave as
// coalesced 16-byte stores.  The BN second output is a per-channel 256-entry
// table lookup (BN is a fixed function of the int8 value; the table is built
// bit-exactly on the host, ffk_make_bn_lut).
#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "ff_conv_table.h"

namespace {

const ConvEntry* find_conv(int cin, int cout, int kh, int kw, int stride, int pad, int hin, int win) {
    if (kh != kw || pad != kh / 2) return nullptr;
    typedef const ConvEntry* (*table_fn)(int*);
    static const table_fn tables[] = {ff_conv_table_stem, ff_conv_table_c64, ff_conv_table_c128,
                                      ff_conv_table_c256, ff_conv_table_c512};
    for (table_fn t : tables) {
        int n = 0;
        const ConvEntry* es = t(&n);
        for (int k = 0; k < n; k++) {
            const ConvEntry& e = es[k];
            if (e.cin == cin && e.cout == cout && e.ks == kh && e.stride == stride && e.hin == hin &&
                e.win == win)
                return &e;
        }
    }
    return nullptr;
}

// Launch choice for one layer at M output pixels.
struct ConvLaunch {
    launch_fn fn;
    const char* kind;
    int bn;             // workgroup tile width (tiles_n = cout / bn)
    int grid;
    int split;
    size_t counter_bytes, ws_bytes;   // split > 1: workspace layout
};

// ws_avail: workspace bytes the caller provides (a split > 1 variant that
// needs more falls back to the whole-K tiling).  shared (FFK_SHARED_GPU):
// a twin launch runs at the same time, so the large tiles are kept when the
// two grids together reach FF_MID_MAX_WG.
ConvLaunch choose_launch(const ConvEntry* e, long long M, size_t ws_avail, bool shared = false) {
    long long big = ((M + e->bm - 1) / e->bm) * (e->cout / e->bn);
    ConvLaunch l = {e->fn, e->kind, e->bn, (int)big, 1, 0, 0};
    if (e->mid && big * (shared ? 2 : 1) < FF_MID_MAX_WG) {
        const int mbm = e->mid_bm ? e->mid_bm : 128, mbn = e->mid_bn ? e->mid_bn : 128;
        big = ((M + mbm - 1) / mbm) * (e->cout / mbn);
        l = {e->mid, e->mid_kind ? e->mid_kind : "staged128", mbn, (int)big, 1, 0, 0};
    }
    if (!e->small || big >= FF_SPLIT_MIN_WG) return l;
    // the small-tile kernels: e->split K ranges, 3 where e->split is larger,
    // then whole K; the first whose grid fits its limit and beats `big`
    const long long tiles = ((M + FF_SM_BM - 1) / FF_SM_BM) * (e->cout / FF_SM_BN);
    const int cand[3] = {e->split, e->split > 3 ? 3 : 1, 1};
    for (int c = 0; c < 3; c++) {
        const int sp = cand[c];
        if (c > 0 && sp == cand[c - 1]) continue;
        const long long wgs = tiles * sp;
        const long long lim = sp > 1 ? FF_SPLIT_MAX_WG : shared ? FF_TILE64_MAX_WG_SHARED : FF_TILE64_MAX_WG;
        if (wgs > lim || wgs <= big) continue;
        size_t cnt = 0, need = 0;
        if (sp > 1) {
            // the counter area has the same size at every batch (tiles <=
            // wgs), so launches of different sizes never see each other's
            // partial tiles in their counters
            cnt = FF_SPLIT_COUNTER_BYTES;
            need = cnt + (size_t)wgs * FF_SM_BM * FF_SM_BN * sizeof(int32_t);
            if (need > ws_avail) continue;
        }
        l.fn = e->small;
        l.kind = sp > 1 ? "splitk" : "tile64";
        l.bn = FF_SM_BN;
        l.grid = (int)wgs;
        l.split = sp;
        l.counter_bytes = cnt;
        l.ws_bytes = need;
        return l;
    }
    return l;
}

long long conv_pixels(const ffk_conv_desc* d) {
    const int hout = (d->hin + 2 * d->pad - d->kh) / d->stride + 1;
    const int wout = (d->win + 2 * d->pad - d->kw) / d->stride + 1;
    return (long long)d->batch * hout * wout;
}

// A geometry the generic kernel runs: positive sizes, a stride, no negative
// padding, at least one output pixel, and sizes whose products stay in range.
bool generic_geometry(int cin, int cout, int kh, int kw, int stride, int pad, int hin, int win) {
    if (cin <= 0 || cout <= 0 || kh <= 0 || kw <= 0 || stride <= 0 || pad < 0 || hin <= 0 || win <= 0)
        return false;
    if (cin > 65535 || cout > 65535 || kh > 255 || kw > 255 || pad > 255 || hin > 65535 || win > 65535)
        return false;
    return hin + 2 * pad >= kh && win + 2 * pad >= kw;
}

// kernel arguments of a descriptor (M, tiles_n and the split-K workspace are
// set per launch)
ConvArgs conv_args(const ffk_conv_desc* d) {
    ConvArgs a = {};
    if (d->cin == 3) a.in_f32 = (const float*)d->in;
    else a.in = (const int8_t*)d->in;
    a.in_inv = d->in_inv;
    a.in_lut = d->in_lut;
    a.io = d->io;
    a.w = d->w;
    a.params = d->params;
    a.add_src = d->add_src;
    a.bn_lut = d->bn_lut;
    a.out = d->out;
    a.out_bn = d->out_bn;
    a.out_i32 = d->out_i32;
    a.flags = d->flags & (FFK_EPI_PRELU | FFK_EPI_ADD | FFK_EPI_BN | FFK_EPI_BIAS | FFK_EPI_INSCALE |
                          FFK_EPI_PRELU_LE1 | FFK_OUT_X_EVEN | FFK_EPI_IN_RANGE | FFK_EPI_FMA_TAIL |
                          FFK_IN_RGB8);
    a.in_scale = d->in_scale;
    return a;
}

}  // namespace

extern "C" {

int ffk_conv_supported(int cin, int cout, int kh, int kw, int stride, int pad, int hin, int win) {
    return find_conv(cin, cout, kh, kw, stride, pad, hin, win) != nullptr;
}

int ffk_conv_runnable(int cin, int cout, int kh, int kw, int stride, int pad, int hin, int win) {
    return find_conv(cin, cout, kh, kw, stride, pad, hin, win) != nullptr ||
           generic_geometry(cin, cout, kh, kw, stride, pad, hin, win);
}

int ffk_prelu_le1_ok(const float* params, int cout, int ktotal, int with_add) {
    if (!params || cout <= 0 || ktotal <= 0) return 0;
    const double acc_max = (double)ktotal * 128.0 * 128.0;
    for (int c = 0; c < cout; c++) {
        const double s = params[FFK_P_SLOPE * cout + c];
        const double ws = params[FFK_P_WS * cout + c];
        const double bias = params[FFK_P_BIAS * cout + c];
        const double adds = with_add ? params[FFK_P_ADDSCALE * cout + c] : 0.0;
        if (!(s <= 1.0) || !std::isfinite(ws) || !std::isfinite(bias) || !std::isfinite(adds)) return 0;
        // each fp32 rounding is within a factor 1 + 2^-23 of its exact value
        const double bound = (acc_max * std::fabs(ws) + std::fabs(bias) + 128.0 * std::fabs(adds)) * 1.0001;
        if (!(bound < 3.0e38)) return 0;
    }
    return 1;
}

int ffk_requant_in_range(const float* params, int cout, int ktotal, int flags) {
    if (!params || cout <= 0 || ktotal <= 0 || (flags & FFK_EPI_INSCALE)) return 0;
    const double acc_max = (double)ktotal * 128.0 * 128.0;
    // each fp32 rounding is within a factor 1 + 2^-24 of its exact value;
    // five of them (conversion, ws, bias, residual, PReLU) before the inv one
    const double widen = 1.000001;
    for (int c = 0; c < cout; c++) {
        const double ws = params[FFK_P_WS * cout + c];
        const double bias = params[FFK_P_BIAS * cout + c];
        const double inv = params[FFK_P_INV * cout + c];
        const double adds = (flags & FFK_EPI_ADD) ? params[FFK_P_ADDSCALE * cout + c] : 0.0;
        const double slope = (flags & FFK_EPI_PRELU) ? params[FFK_P_SLOPE * cout + c] : 0.0;
        if (!std::isfinite(ws) || !std::isfinite(bias) || !std::isfinite(inv) || !std::isfinite(adds) ||
            !std::isfinite(slope))
            return 0;
        const double f = (acc_max * std::fabs(ws) + std::fabs(bias) + 128.0 * std::fabs(adds)) * widen;
        const double t = f * std::max(1.0, std::fabs(slope)) * std::fabs(inv) * widen;
        if (!(t < 2147483520.0)) return 0;              // 2^31 - 128
    }
    return 1;
}

// FFK_EPI_FMA_TAIL.  The pre-requant value f(acc) of one channel as the
// kernels and the reference compute it on the in-range forms without a
// residual: (float)acc (round to nearest even above 2^24), * ws, + bias,
// then PReLU.  With slope >= 0 it is non-decreasing in acc where ws > 0,
// non-increasing where ws < 0 and constant where ws == 0.
static float fma_tail_value(long long acc, float ws, float bias, float slope, bool prelu) {
    volatile float f = (float)acc;
    volatile float g = f * ws;
    volatile float h = g + bias;
    float v = h;
    if (prelu && v < 0.0f) {
        volatile float n = v * slope;
        v = n;
    }
    return v;
}

// 1 if f(acc) == target for some acc in [-amax, amax]: binary search for the
// smallest acc with f(s*acc) >= target, s the sign that makes f(s*acc)
// non-decreasing (the range is symmetric)
static int fma_tail_reached(float target, long long amax, float ws, float bias, float slope, bool prelu) {
    const long long s = ws < 0.0f ? -1 : 1;
    long long lo = -amax, hi = amax;
    if (fma_tail_value(s * hi, ws, bias, slope, prelu) < target) return 0;
    while (lo < hi) {
        const long long mid = lo + (hi - lo) / 2;
        if (fma_tail_value(s * mid, ws, bias, slope, prelu) >= target) hi = mid;
        else lo = mid + 1;
    }
    return fma_tail_value(s * lo, ws, bias, slope, prelu) == target;
}

int ffk_requant_fma_ok(const float* params, int cout, int ktotal, int flags) {
    if ((flags & (FFK_EPI_ADD | FFK_EPI_INSCALE)) || !ffk_requant_in_range(params, cout, ktotal, flags)) return 0;
    const bool prelu = (flags & FFK_EPI_PRELU) != 0;
    const long long amax = (long long)ktotal * 128 * 128;
    // p = f*inv exact, h = copysign(0.5, p).  The reference truncates
    // RN(RN(p) + h), the fma form RN(p + h).  At a level n >= 1 the two
    // differ only where RN(p) lands on the other side of c_n = n - 1/2 -
    // u_n/2 than p does (u_n: the float spacing just below n; r >= n exactly
    // when the addend before the final rounding reaches n - u_n/2, the final
    // tie going to n).  For n >= 2, c_n is an odd multiple of u_n/2, not a
    // float: RN(p) and p are on the same side unless p == c_n, and then RN
    // rounds the tie to n - 1/2 (an even multiple of u_n) and both forms
    // reach n.  For n = 1 (u_1 = 2^-24), c_1 = 1/2 - 2^-25 is a float of the
    // binade below: p strictly between c_1 - 2^-26 and c_1 rounds up to c_1,
    // where the reference reaches 1 and the fma form stays at 0.  Symmetric
    // for p < 0.  That window is the only place where they differ.
    const double c1 = 0.5 - std::ldexp(1.0, -25), w0 = c1 - std::ldexp(1.0, -26);
    for (int c = 0; c < cout; c++) {
        const float ws = params[FFK_P_WS * cout + c];
        const float bias = params[FFK_P_BIAS * cout + c];
        const float inv = params[FFK_P_INV * cout + c];
        const float slope = prelu ? params[FFK_P_SLOPE * cout + c] : 0.0f;
        if (!(inv > 0.0f) || (prelu && !(slope >= 0.0f))) return 0;
        const double di = inv;
        auto reached = [&](float f) {
            return fma_tail_reached(f, amax, ws, bias, slope, prelu) || fma_tail_reached(-f, amax, ws, bias, slope, prelu);
        };
        // floats f > 0 with f*inv strictly inside (c1 - 2^-26, c1) (the
        // product of two floats is exact in double): start a few floats
        // below the window's start and walk up past its end
        float f = (float)(w0 / di);
        if (!std::isfinite(f)) continue;
        f = std::nextafter(std::nextafter(f, 0.0f), 0.0f);
        int k = 0;
        for (; k < 16 && (double)f * di < c1; k++, f = std::nextafter(f, INFINITY))
            if ((double)f * di > w0 && reached(f)) return 0;
        if (k == 16) return 0;                       // (never: the window is narrower than a float step)
    }
    return 1;
}

size_t ffk_conv_packed_bytes(int cin, int cout, int kh, int kw) {
    const size_t ktot = (size_t)kh * kw * cin;
    const size_t steps = (ktot + FF_KSTEP - 1) / FF_KSTEP;
    return steps * (size_t)cout * FF_KSTEP;
}

int ffk_pack_conv_weights(const int8_t* w, int cout, int cin, int kh, int kw, int8_t* packed) {
    if (!w || !packed || cout <= 0 || cin <= 0 || kh <= 0 || kw <= 0) {
        ffk_set_error("pack_conv_weights: bad arguments%s%s", nullptr, nullptr);
        return FFK_ERR_ARG;
    }
    // Per output channel: its OIHW weights (cin x taps, read in order)
    // transposed into reduction order k = tap*cin + ci, zero-padded to whole
    // K steps, then each 64-byte K step copied to its place in the packed
    // [step][cout][64] layout.
    const int taps = kh * kw;
    const int ktot = taps * cin;
    const int steps = (ktot + FF_KSTEP - 1) / FF_KSTEP;
    std::vector<int8_t> row((size_t)steps * FF_KSTEP, 0);
    for (int n = 0; n < cout; n++) {
        const int8_t* src = w + (size_t)n * ktot;
        for (int ci = 0; ci < cin; ci++)
            for (int t = 0; t < taps; t++) row[(size_t)t * cin + ci] = src[(size_t)ci * taps + t];
        for (int s = 0; s < steps; s++)
            memcpy(packed + ((size_t)s * cout + n) * FF_KSTEP, row.data() + (size_t)s * FF_KSTEP, FF_KSTEP);
    }
    return FFK_OK;
}

int ffk_conv(const ffk_conv_desc* d, void* stream) {
    if (!d || d->batch < 0) {
        ffk_set_error("conv: bad descriptor%s%s", nullptr, nullptr);
        return FFK_ERR_ARG;
    }
    const ConvEntry* e = find_conv(d->cin, d->cout, d->kh, d->kw, d->stride, d->pad, d->hin, d->win);
    if (!e && !generic_geometry(d->cin, d->cout, d->kh, d->kw, d->stride, d->pad, d->hin, d->win)) {
        ffk_set_error("conv: invalid layer geometry%s%s", nullptr, nullptr);
        return FFK_ERR_ARG;
    }
    const long long M = conv_pixels(d);
    if (M > 0x7fffffffLL) {
        ffk_set_error("conv: batch too large%s%s", nullptr, nullptr);
        return FFK_ERR_ARG;
    }
    const bool stem = d->cin == 3;
    const bool raw = d->out_i32 != nullptr;
    const bool rgb8 = stem && (d->flags & FFK_IN_RGB8);
    if (stem && (d->flags & FFK_EPI_ADD)) {
        ffk_set_error("conv: the 3-channel input layer takes no residual input%s%s", nullptr, nullptr);
        return FFK_ERR_UNSUPPORTED;
    }
    if ((d->flags & FFK_IN_RGB8) && !stem) {
        ffk_set_error("conv: FFK_IN_RGB8 applies to the 3-channel input layer only%s%s", nullptr, nullptr);
        return FFK_ERR_ARG;
    }
    bool bad = !d->w || (!raw && !d->params) || (stem && !rgb8 && !d->in_inv) || (rgb8 && !d->in_lut) ||
               (stem && !d->in && !d->io) ||
               (!stem && !d->in);
    if (!raw) {
        if ((d->flags & FFK_EPI_ADD) && !d->add_src) bad = true;
        if ((d->flags & FFK_EPI_BN) && (!d->out_bn || !d->bn_lut)) bad = true;
        if (!(d->flags & FFK_EPI_BN) && !d->out) bad = true;
    }
    if (bad) {
        ffk_set_error("conv: missing pointer for the requested flags%s%s", nullptr, nullptr);
        return FFK_ERR_ARG;
    }
    const bool x_even = (d->flags & FFK_OUT_X_EVEN) != 0;
    if (x_even) {
        const int hout = (d->hin + 2 * d->pad - d->kh) / d->stride + 1;
        const int wout = (d->win + 2 * d->pad - d->kw) / d->stride + 1;
        if (raw || !d->out || (hout & 1) || (wout & 1)) {
            ffk_set_error("conv: FFK_OUT_X_EVEN needs an int8 output X of even height and width%s%s",
                          nullptr, nullptr);
            return FFK_ERR_ARG;
        }
    }
    if (M == 0) return FFK_OK;
    if (d->flags & FFK_ALGO_WINOGRAD) return ffk_winograd_conv(d, (hipStream_t)stream);
    const ConvArgs a = conv_args(d);
    if (!e) {                              // no tuned kernel: the generic one
        ConvArgs as = a;
        as.M = (int)M;
        return ff_conv_generic_launch(as, d, (hipStream_t)stream);
    }
    // The direct-to-LDS kernels address the int8 input and the residual
    // tensor with 32-bit offsets: a batch whose input or output tensor
    // reaches 2 GiB runs as several launches over consecutive image ranges
    // (images are independent).
    const long long px_out = M / d->batch;
    const long long in_img = (long long)d->hin * d->win * d->cin;
    const long long img = std::max<long long>(in_img, px_out * d->cout);
    const int slice = stem ? d->batch : (int)std::min<long long>(d->batch, 0x7fffffffLL / img);
    for (int b0 = 0; b0 < d->batch; b0 += slice) {
        const int nb = std::min(slice, d->batch - b0);
        const long long ms = (long long)nb * px_out;
        ConvArgs as = a;
        if (!stem) as.in = a.in + (size_t)b0 * in_img;
        const size_t o = (size_t)b0 * px_out * d->cout;
        if (a.add_src) as.add_src = a.add_src + o;
        if (a.out) as.out = a.out + (x_even ? o / 4 : o);     // even/even pixels: a quarter
        if (a.out_bn) as.out_bn = a.out_bn + o;
        if (a.out_i32) as.out_i32 = a.out_i32 + o;
        as.M = (int)ms;
        const ConvLaunch l = choose_launch(e, ms, d->workspace ? d->workspace_bytes : 0,
                                           (d->flags & FFK_SHARED_GPU) != 0);
        if (l.split > 1) {
            as.counters = (unsigned*)d->workspace;
            as.ws = (int32_t*)((int8_t*)d->workspace + l.counter_bytes);
        }
        as.tiles_n = d->cout / l.bn;
        l.fn(as, l.grid, l.split, (hipStream_t)stream);
        const int rc = ffk_check_launch("conv launch");
        if (rc != FFK_OK) return rc;
    }
    return FFK_OK;
}

int ffk_conv_s2_shortcut(const ffk_conv_desc* c, const ffk_conv_desc* s, void* stream) {
    if (!c || !s || c->batch < 0) {
        ffk_set_error("conv_s2_shortcut: bad descriptors%s%s", nullptr, nullptr);
        return FFK_ERR_ARG;
    }
    // the pair the fused kernel computes; anything else is left to ffk_conv
    const int no_c = FFK_EPI_PRELU | FFK_EPI_ADD | FFK_EPI_BN | FFK_EPI_INSCALE | FFK_ALGO_WINOGRAD | FFK_IN_RGB8 |
                     FFK_OUT_X_EVEN;
    const int no_s = FFK_EPI_PRELU | FFK_EPI_INSCALE | FFK_ALGO_WINOGRAD | FFK_IN_RGB8;
    if (c->kh != 3 || c->kw != 3 || c->stride != 2 || c->pad != 1 || c->hin != c->win || (c->hin & 1) ||
        (c->flags & no_c) || c->out_i32 || !c->in || !c->out || !c->w || !c->params)
        return 0;
    const int ho = c->hin / 2;
    if (s->batch != c->batch || s->kh != 1 || s->kw != 1 || s->stride != 1 || s->pad != 0 || s->hin != ho ||
        s->win != ho || s->cout != c->cout || !(s->flags & FFK_EPI_ADD) || (s->flags & no_s) || s->out_i32 ||
        s->add_src != c->out || !s->in || !s->w || !s->params)
        return 0;
    if ((s->flags & FFK_EPI_BN) ? (!s->out_bn || !s->bn_lut) : !s->out) return 0;
    if ((s->flags & FFK_OUT_X_EVEN) && ((ho & 1) || !s->out)) return 0;
    const ConvEntry* e = find_conv(c->cin, c->cout, 3, 3, 2, 1, c->hin, c->win);
    if (!e || !e->pair || e->pair_cx != s->cin) return 0;
    const long long M = conv_pixels(c);
    if (M == 0) return 1;
    // one launch over the whole batch: every tensor below 2 GiB
    const long long lim = 0x7fffffffLL;
    if ((long long)c->batch * c->hin * c->win * c->cin > lim || M * c->cout > lim || M * s->cin > lim) return 0;
    const ConvLaunch l = choose_launch(e, M, c->workspace ? c->workspace_bytes : 0,
                                       (c->flags & FFK_SHARED_GPU) != 0);
    if (l.fn != e->fn) return 0;
    ConvArgs a = conv_args(c), b = conv_args(s);
    a.M = b.M = (int)M;
    a.tiles_n = b.tiles_n = c->cout / l.bn;
    e->pair(a, b, l.grid, (hipStream_t)stream);
    const int rc = ffk_check_launch("conv pair launch");
    return rc != FFK_OK ? rc : 1;
}

// ---------------------------------------------------------------------------
// No-allocation variant of ffk_conv: the split-K workspace is a file-scope
// device array (each GPU holds its own copy, at its own address, for the life
// of the process) instead of caller memory.  Its size covers the largest
// split grid (FF_SPLIT_MAX_WG workgroups of 64x64 int32 partial tiles) behind
// the counter area.  In host code `scratch` names a host-side stand-in, not
// device memory: its device address comes from hipGetSymbolAddress, once per
// device, and only that address is passed on.
// ---------------------------------------------------------------------------
static_assert(FFK_NOALLOC_SCRATCH_BYTES == FF_WS_COUNTER_AREA + (size_t)FF_SPLIT_MAX_WG * FF_SM_BM * FF_SM_BN * 4,
              "the header's limit is the split-K workspace bound");
static __device__ __align__(256) int8_t scratch[FFK_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int FF_MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_addr[FF_MAX_DEVICES];

// Device address of the current device's `scratch`.  First use on a device:
// look it up and clear the counter area with a fill kernel on `stream` (the
// array is zero when the code object loads; the clear does not rely on it).
int scratch_for_current_device(hipStream_t stream, void** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return ffk_hip_fail(e, "hipGetDevice");
    if (dev < 0 || dev >= FF_MAX_DEVICES) {
        ffk_set_error("conv_noalloc: device index out of range%s%s", nullptr, nullptr);
        return FFK_ERR_UNSUPPORTED;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_addr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) return ffk_hip_fail(e, "hipGetSymbolAddress(scratch)");
        const int rc = ffk_zero(p, FF_WS_COUNTER_AREA, stream);
        if (rc != FFK_OK) return rc;
        g_scratch_addr[dev] = p;
    }
    *out = g_scratch_addr[dev];
    return FFK_OK;
}
}  // namespace

int ffk_conv_noalloc(const ffk_conv_desc* d, void* stream) {
    if (!d) {
        ffk_set_error("conv_noalloc: bad descriptor%s%s", nullptr, nullptr);
        return FFK_ERR_ARG;
    }
    ffk_conv_desc dd = *d;
    dd.workspace = nullptr;
    dd.workspace_bytes = 0;
    const size_t need = ffk_conv_workspace_bytes(&dd);
    if (need > FFK_NOALLOC_SCRATCH_BYTES) {
        ffk_set_error("conv_noalloc: this layer needs a %s-byte workspace, above the %s-byte device scratch "
                      "(use ffk_conv with a workspace)",
                      std::to_string(need).c_str(), std::to_string(FFK_NOALLOC_SCRATCH_BYTES).c_str());
        return FFK_ERR_ARG;
    }
    void* p = nullptr;
    const int rc = scratch_for_current_device((hipStream_t)stream, &p);
    if (rc != FFK_OK) return rc;
    dd.workspace = p;
    dd.workspace_bytes = FFK_NOALLOC_SCRATCH_BYTES;
    return ffk_conv(&dd, stream);
}

size_t ffk_conv_workspace_bytes(const ffk_conv_desc* d) {
    if (!d || d->batch <= 0) return 0;
    const ConvEntry* e = find_conv(d->cin, d->cout, d->kh, d->kw, d->stride, d->pad, d->hin, d->win);
    if (!e) return 0;
    if (d->flags & FFK_ALGO_WINOGRAD) return 0;       // (its transformed input stays on chip)
    const long long M = conv_pixels(d);
    if (M > 0x7fffffffLL) return 0;
    return choose_launch(e, M, (size_t)-1, (d->flags & FFK_SHARED_GPU) != 0).ws_bytes;
}

int ffk_conv_grid(const ffk_conv_desc* d) {
    if (!d || d->batch <= 0 || (d->flags & FFK_ALGO_WINOGRAD)) return -1;
    const ConvEntry* e = find_conv(d->cin, d->cout, d->kh, d->kw, d->stride, d->pad, d->hin, d->win);
    if (!e) {
        if (!generic_geometry(d->cin, d->cout, d->kh, d->kw, d->stride, d->pad, d->hin, d->win)) return -1;
        const long long g = ff_conv_generic_grid(conv_pixels(d), d->cin, d->cout);
        return g > 0x7fffffffLL ? -1 : (int)g;
    }
    if (e->cin == 3) return -1;                      // (the stem sizes its persistent grid itself)
    const long long M = conv_pixels(d);
    if (M > 0x7fffffffLL) return -1;
    return choose_launch(e, M, d->workspace ? d->workspace_bytes : 0, (d->flags & FFK_SHARED_GPU) != 0).grid;
}

const char* ffk_conv_variant(const ffk_conv_desc* d) {
    if (!d || d->batch <= 0) return nullptr;
    const ConvEntry* e = find_conv(d->cin, d->cout, d->kh, d->kw, d->stride, d->pad, d->hin, d->win);
    if (d->flags & FFK_ALGO_WINOGRAD) return ffk_winograd_eligible(d) ? "winograd" : nullptr;
    if (!e) return generic_geometry(d->cin, d->cout, d->kh, d->kw, d->stride, d->pad, d->hin, d->win)
                       ? "generic" : nullptr;
    const long long M = conv_pixels(d);
    if (M > 0x7fffffffLL) return nullptr;
    return choose_launch(e, M, d->workspace ? d->workspace_bytes : 0, (d->flags & FFK_SHARED_GPU) != 0).kind;
}

// BN second output as a table: lut[c][q + 128] = BN-requant of the int8
// value q for channel c, computed with the reference's fp32 sequence
// (bn_prelu_requant_int8 with bn != NULL, int8_epilogue.c:273-303):
//   f = fma(RN(q * s_in), bn_s, bn_o); round half away of RN(f * inv);
//   x86 cvttps2dq semantics; clamp to int8.  (The same table as a
// stand-alone BN's, ff_eltwise.hip.)
int ffk_make_bn_lut(const float* s_in, const float* bn_s, const float* bn_o, const float* bn_inv,
                    int cout, int8_t* lut) {
    if (!s_in || !bn_s || !bn_o || !bn_inv || !lut || cout <= 0) {
        ffk_set_error("make_bn_lut: bad arguments%s%s", nullptr, nullptr);
        return FFK_ERR_ARG;
    }
    return ffk_make_map_lut(s_in, bn_s, bn_o, nullptr, bn_inv, cout, lut);
}

int ffk_make_rgb8_lut(const float* in_inv, int8_t* lut) {
    if (!in_inv || !lut) {
        ffk_set_error("make_rgb8_lut: bad arguments%s%s", nullptr, nullptr);
        return FFK_ERR_ARG;
    }
    for (int c = 0; c < 3; c++)
        for (int x = 0; x < 256; x++) {
            volatile float v = (float)x - 127.5f;      // exact
            v = v / 127.5f;                            // one correctly rounded division
            volatile float t = v * in_inv[c];
            long q = lrintf(t);                        // the reference's glibc call
            int32_t qi = (int32_t)q;
            qi = qi < -128 ? -128 : (qi > 127 ? 127 : qi);
            lut[c * 256 + x] = (int8_t)qi;
        }
    return FFK_OK;
}

}  // extern "C"
