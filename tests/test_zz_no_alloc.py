"""ffk_conv_noalloc: the split-K workspace from the library's own device
array instead of caller memory, no allocation in the call.  Checked through
the C ABI against ffk_conv with a caller workspace, bit for bit, on two calls
in a row per layer, the second with a smaller batch (the array keeps the
first call's partial tiles; the counters must be back at zero)."""
import ctypes as C

import numpy as np
import pytest

import fastface_amd as fa
from gpu_util import Dev, check, pack_conv, params_block, make_bn_lut, conv_workspace

pytestmark = pytest.mark.gpu

# (cin, cout, k, stride, H, batches): small-batch geometries that take the
# split-K kernels (3, 6 or 9 K ranges)
LAYERS = [(256, 256, 3, 1, 14, (2, 1)), (512, 512, 3, 1, 7, (2, 1)),
          (128, 128, 3, 2, 56, (1, 1)), (256, 256, 3, 2, 28, (1, 1)), (64, 64, 3, 1, 56, (2, 1))]


def _desc(lib, keep, x, w, params, flags, add, cout, k, stride):
    B, H, W, cin = x.shape
    pad = k // 2
    ho = (H + 2 * pad - k) // stride + 1
    d = fa.ffk_conv_desc()
    d.batch, d.cin, d.cout, d.kh, d.kw = B, cin, cout, k, k
    d.stride, d.pad, d.hin, d.win = stride, pad, H, W
    for name, arr in (("in_", x), ("w", pack_conv(lib, w)), ("params", params)):
        dv = Dev(lib, host=arr)
        keep.append(dv)
        setattr(d, name, dv.ptr)
    lut = Dev(lib, host=make_bn_lut(lib, params))
    keep.append(lut)
    d.bn_lut = lut.ptr
    if add is not None:
        da = Dev(lib, host=add)
        keep.append(da)
        d.add_src = da.ptr
    n = B * ho * ho * cout
    do, db = Dev(lib, nbytes=n), Dev(lib, nbytes=n)
    keep += [do, db]
    d.out, d.out_bn = do.ptr, db.ptr
    d.flags = flags
    return d, do, db, (B, ho, ho, cout)


@pytest.mark.parametrize("cin,cout,k,stride,H,batches", LAYERS)
def test_conv_noalloc_equals_conv_with_workspace(gpu_lib, cin, cout, k, stride, H, batches):
    lib = gpu_lib
    r = np.random.default_rng(700 + cin + H)
    flags = fa.FFK_EPI_BIAS | fa.FFK_EPI_PRELU | fa.FFK_EPI_ADD | fa.FFK_EPI_BN
    P = params_block(cout, ws=r.uniform(1e-3, 1e-2, cout), bias=r.normal(0, 0.1, cout),
                     slope=0.25, adds=0.02, inv=1 / 40.0, bn_sin=0.02, bn_s=1.0, bn_o=0.01,
                     bn_inv=50.0)
    for call, B in enumerate(batches):
        x = r.integers(-128, 128, size=(B, H, H, cin), dtype=np.int8)
        w = r.integers(-128, 128, size=(cout, cin, k, k), dtype=np.int8)
        ho = (H + 2 * (k // 2) - k) // stride + 1
        add = r.integers(-128, 128, size=(B, ho, ho, cout), dtype=np.int8)
        print("noalloc layer %d->%d k%d s%d @%d batch %d call %d" % (cin, cout, k, stride, H, B, call),
              flush=True)
        keep = []
        d1, o1, b1, shp = _desc(lib, keep, x, w, P, flags, add, cout, k, stride)
        ws = conv_workspace(lib, d1)
        if ws is not None:
            keep.append(ws)
            d1.workspace, d1.workspace_bytes = ws.ptr, ws.nbytes
        kind = lib.ffk_conv_variant(C.byref(d1))
        check(lib, lib.ffk_conv(C.byref(d1), None))
        d2, o2, b2, _ = _desc(lib, keep, x, w, P, flags, add, cout, k, stride)
        # the no-alloc call ignores the descriptor's workspace fields
        d2.workspace, d2.workspace_bytes = None, 0
        check(lib, lib.ffk_conv_noalloc(C.byref(d2), None))
        check(lib, lib.ffk_stream_sync(None))
        assert np.array_equal(o1.get(np.int8, shp), o2.get(np.int8, shp))
        assert np.array_equal(b1.get(np.int8, shp), b2.get(np.int8, shp))
        if (cin, H) != (64, 56):
            assert kind == b"splitk"


def test_conv_noalloc_winograd_and_generic(gpu_lib):
    """Layers that need no workspace at all (the Winograd path, whose
    transformed input stays on chip, and a geometry on the generic kernel)
    run through the no-allocation entry point too, equal to ffk_conv, on two
    calls in a row, the second with a smaller batch."""
    lib = gpu_lib
    r = np.random.default_rng(760)
    P = params_block(64, ws=r.uniform(1e-3, 1e-2, 64), bias=r.normal(0, 0.1, 64), slope=0.25, adds=0.02,
                     inv=1 / 40.0, bn_sin=0.02, bn_s=1.0, bn_o=0.01, bn_inv=50.0)
    flags = fa.FFK_EPI_BIAS | fa.FFK_EPI_PRELU | fa.FFK_EPI_BN
    for case, (cin, H, extra) in enumerate([(64, 56, fa.FFK_ALGO_WINOGRAD), (96, 20, 0)]):
        for call, B in enumerate((3, 1)):
            x = r.integers(-128, 128, size=(B, H, H, cin), dtype=np.int8)
            w = r.integers(-128, 128, size=(64, cin, 3, 3), dtype=np.int8)
            print("noalloc case %d batch %d call %d" % (case, B, call), flush=True)
            keep = []
            d1, o1, b1, shp = _desc(lib, keep, x, w, P, flags, None, 64, 3, 1)
            d2, o2, b2, _ = _desc(lib, keep, x, w, P, flags, None, 64, 3, 1)
            if extra:
                wp = Dev(lib, host=_wino_pack(lib, w))
                keep.append(wp)
                d1.w = d2.w = wp.ptr
                d1.flags = d2.flags = flags | extra
            assert lib.ffk_conv_workspace_bytes(C.byref(d1)) == 0
            kind = lib.ffk_conv_variant(C.byref(d1))
            assert kind == (b"winograd" if extra else b"generic")
            check(lib, lib.ffk_conv(C.byref(d1), None))
            check(lib, lib.ffk_conv_noalloc(C.byref(d2), None))
            check(lib, lib.ffk_stream_sync(None))
            assert np.array_equal(o1.get(np.int8, shp), o2.get(np.int8, shp))
            assert np.array_equal(b1.get(np.int8, shp), b2.get(np.int8, shp))


def _wino_pack(lib, w):
    cout, cin = w.shape[:2]
    packed = np.empty(lib.ffk_winograd_packed_bytes(cin, cout), np.int8)
    check(lib, lib.ffk_pack_winograd_weights(np.ascontiguousarray(w).ctypes.data, cout, cin, packed.ctypes.data))
    return packed
