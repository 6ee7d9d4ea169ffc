"""Device-buffer helpers over the library's own C ABI (fastface_kernels.h).
torch is not used: it ships its own HIP runtime, and one process must not
load two."""
import ctypes as C

import numpy as np

import fastface_amd as fa


class Dev:
    """A device allocation; from numpy (upload) or empty."""

    def __init__(self, lib, nbytes=None, host=None):
        self.lib = lib
        if host is not None:
            host = np.ascontiguousarray(host)
            nbytes = host.nbytes
        self.nbytes = int(nbytes)
        self.ptr = lib.ffk_malloc(max(self.nbytes, 1))
        if not self.ptr:
            raise MemoryError(fa.last_error())
        if host is not None and self.nbytes:
            check(lib, lib.ffk_memcpy_h2d(self.ptr, host.ctypes.data, self.nbytes, None))
            check(lib, lib.ffk_stream_sync(None))

    def get(self, dtype, shape):
        out = np.empty(shape, dtype)
        assert out.nbytes <= self.nbytes
        check(self.lib, self.lib.ffk_memcpy_d2h(out.ctypes.data, self.ptr, out.nbytes, None))
        check(self.lib, self.lib.ffk_stream_sync(None))
        return out

    def free(self):
        if self.ptr:
            self.lib.ffk_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def check(lib, rc):
    if rc != 0:
        raise RuntimeError("ffk call failed (%d): %s" % (rc, fa.last_error()))


def pack_conv(lib, w_oihw):
    w = np.ascontiguousarray(w_oihw, np.int8)
    cout, cin, kh, kw = w.shape
    n = lib.ffk_conv_packed_bytes(cin, cout, kh, kw)
    out = np.empty(n, np.int8)
    check(lib, lib.ffk_pack_conv_weights(w.ctypes.data, cout, cin, kh, kw, out.ctypes.data))
    return out


def make_bn_lut(lib, params):
    """[cout][256] BN table from the FFK_P_BN_* rows of a parameter block."""
    P = np.ascontiguousarray(params, np.float32)
    cout = P.shape[1]
    lut = np.empty((cout, 256), np.int8)
    rows = [np.ascontiguousarray(P[i]) for i in (fa.FFK_P_BN_SIN, fa.FFK_P_BN_S, fa.FFK_P_BN_O,
                                                   fa.FFK_P_BN_INV)]
    check(lib, lib.ffk_make_bn_lut(rows[0].ctypes.data, rows[1].ctypes.data, rows[2].ctypes.data,
                                   rows[3].ctypes.data, cout, lut.ctypes.data))
    return lut


def params_block(cout, **rows):
    """[FFK_NPARAM][cout] fp32 block; rows by name (ws, bias, slope, adds, inv,
    bn_sin, bn_s, bn_o, bn_inv)."""
    names = ["ws", "bias", "slope", "adds", "inv", "bn_sin", "bn_s", "bn_o", "bn_inv"]
    P = np.zeros((fa.FFK_NPARAM, cout), np.float32)
    for k, v in rows.items():
        P[names.index(k)] = v
    return P


def conv_workspace(lib, d):
    """Zero-filled split-K workspace of the size ffk_conv asks for (or None)."""
    n = lib.ffk_conv_workspace_bytes(C.byref(d))
    if n == 0:
        return None
    ws = Dev(lib, nbytes=n)
    check(lib, lib.ffk_zero(ws.ptr, n, None))
    return ws


SPLIT_COUNTERS = 320      # uint32 arrival counters at the start of the workspace


def split_counters_zero(lib, ws):
    """The whole counter area is zero again after a launch."""
    return not ws.get(np.uint32, (SPLIT_COUNTERS,)).any()


def pack_winograd(lib, w_oihw):
    cout, cin = w_oihw.shape[:2]
    packed = np.empty(lib.ffk_winograd_packed_bytes(cin, cout), np.int8)
    check(lib, lib.ffk_pack_winograd_weights(np.ascontiguousarray(w_oihw, np.int8).ctypes.data,
                                             cout, cin, packed.ctypes.data))
    return packed


def run_conv(lib, x, w_oihw, stride, pad, params=None, flags=0, add=None, raw=False,
             want_x=True, want_bn=False, in_inv=None, in_scale=1.0, split=True, in_lut=None,
             winograd=False, workspace=None, x_even=False):
    """One ffk_conv call; returns int32 acc (raw) or (X, BN(X)) int8 arrays.
    split: give the call the split-K workspace it asks for (small batches take
    the split path); False: no workspace (whole-K tiling).
    x_even: FFK_OUT_X_EVEN -- X comes back as [B, Ho/2, Wo/2, Cout] (its
    even-row, even-column pixels), from a buffer of exactly that size."""
    B, H, W, cin = x.shape
    cout, _, kh, kw = w_oihw.shape
    ho = (H + 2 * pad - kh) // stride + 1
    wo = (W + 2 * pad - kw) // stride + 1
    keep = []
    d = fa.ffk_conv_desc()
    d.batch, d.cin, d.cout, d.kh, d.kw = B, cin, cout, kh, kw
    d.stride, d.pad, d.hin, d.win = stride, pad, H, W
    dx = Dev(lib, host=x); keep.append(dx)
    d.in_ = dx.ptr
    dw = Dev(lib, host=pack_winograd(lib, w_oihw) if winograd else pack_conv(lib, w_oihw))
    keep.append(dw)
    if winograd:
        flags |= fa.FFK_ALGO_WINOGRAD
    d.w = dw.ptr
    if in_inv is not None:
        di = Dev(lib, host=np.asarray(list(in_inv) + [0.0], np.float32)); keep.append(di)
        d.in_inv = di.ptr
    if in_lut is not None:
        dl = Dev(lib, host=np.ascontiguousarray(in_lut, np.int8)); keep.append(dl)
        d.in_lut = dl.ptr
    if params is not None:
        dp = Dev(lib, host=params); keep.append(dp)
        d.params = dp.ptr
        if flags & fa.FFK_EPI_BN:
            lut = make_bn_lut(lib, params)
            dl = Dev(lib, host=lut); keep.append(dl)
            d.bn_lut = dl.ptr
    if add is not None:
        da = Dev(lib, host=add); keep.append(da)
        d.add_src = da.ptr
    n_out = B * ho * wo * cout
    res = {}
    if raw:
        do = Dev(lib, nbytes=n_out * 4); keep.append(do)
        d.out_i32 = do.ptr
    else:
        if want_x:
            dox = Dev(lib, nbytes=n_out // 4 if x_even else n_out); keep.append(dox)
            d.out = dox.ptr
        if want_bn:
            dob = Dev(lib, nbytes=n_out); keep.append(dob)
            d.out_bn = dob.ptr
    if x_even:
        flags |= fa.FFK_OUT_X_EVEN
    d.flags = flags
    d.in_scale = in_scale
    ws = workspace if workspace is not None else (conv_workspace(lib, d) if split else None)
    if ws is not None:
        keep.append(ws)
        d.workspace, d.workspace_bytes = ws.ptr, ws.nbytes
    if winograd:
        assert lib.ffk_conv_variant(C.byref(d)) == b"winograd"
    check(lib, lib.ffk_conv(C.byref(d), None))
    check(lib, lib.ffk_stream_sync(None))
    if ws is not None:
        assert split_counters_zero(lib, ws)
    if raw:
        return do.get(np.int32, (B, ho, wo, cout))
    xshape = (B, ho // 2, wo // 2, cout) if x_even else (B, ho, wo, cout)
    x_out = dox.get(np.int8, xshape) if want_x else None
    bn_out = dob.get(np.int8, (B, ho, wo, cout)) if want_bn else None
    return x_out, bn_out


def run_fc(lib, a, W_nk, ws, bias, a_scale=1.0, path=0, split=False):
    a = np.ascontiguousarray(a, np.int8)
    B, K = a.shape
    N = W_nk.shape[0]
    packed = np.empty(lib.ffk_fc_packed_bytes(N, K), np.int8)
    check(lib, lib.ffk_pack_fc_weights(np.ascontiguousarray(W_nk, np.int8).ctypes.data, N, K,
                                       packed.ctypes.data))
    da, dw = Dev(lib, host=a), Dev(lib, host=packed)
    dws, db = Dev(lib, host=np.asarray(ws, np.float32)), Dev(lib, host=np.asarray(bias, np.float32))
    do = Dev(lib, nbytes=B * N * 4)
    d = fa.ffk_fc_desc()
    d.batch, d.n, d.k = B, N, K
    d.a, d.w, d.ws, d.bias, d.out = da.ptr, dw.ptr, dws.ptr, db.ptr, do.ptr
    d.a_scale = a_scale
    d.path = path
    wsp = None
    if split:
        n = lib.ffk_fc_workspace_bytes(C.byref(d))
        assert n > 0
        wsp = Dev(lib, nbytes=n)
        check(lib, lib.ffk_zero(wsp.ptr, n, None))
        d.workspace, d.workspace_bytes = wsp.ptr, n
    check(lib, lib.ffk_fc(C.byref(d), None))
    check(lib, lib.ffk_stream_sync(None))
    if wsp is not None:
        assert split_counters_zero(lib, wsp)
    return do.get(np.float32, (B, N))
