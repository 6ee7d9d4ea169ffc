"""Per-kernel parity on the GPU, through the C ABI, against the pinned oracle.

Bar: bit-exact int32 accumulators and bit-exact int8 / fp32 outputs.
"""
import ctypes as C

import numpy as np
import pytest

import fastface_amd as fa
from conftest import rng
import gpu_util
from gpu_util import params_block, run_conv, run_fc

pytestmark = pytest.mark.gpu
F32 = np.float32

# every conv geometry of IResNet-50 at 112x112 (Cin, Cout, k, stride, Hin)
SHAPES = [
    (64, 64, 3, 1, 112), (64, 64, 3, 2, 112), (64, 64, 1, 2, 112), (64, 64, 3, 1, 56),
    (64, 128, 3, 1, 56), (128, 128, 3, 2, 56), (64, 128, 1, 2, 56), (128, 128, 3, 1, 28),
    (128, 256, 3, 1, 28), (256, 256, 3, 2, 28), (128, 256, 1, 2, 28), (256, 256, 3, 1, 14),
    (256, 512, 3, 1, 14), (512, 512, 3, 2, 14), (256, 512, 1, 2, 14), (512, 512, 3, 1, 7),
]


def _batch_for(H):
    return 1 if H >= 112 else (3 if H >= 28 else 5)    # odd batches: ragged last tile


def test_mfma_lane_layout(gpu_lib):
    assert gpu_lib.ffk_selftest_mfma() == 0, fa.last_error()


# geometries with a split-K small-batch variant (one face takes it)
SPLIT_SHAPES = [(128, 128, 3, 2, 56), (128, 128, 3, 1, 28), (128, 256, 3, 1, 28),
                (256, 256, 3, 2, 28), (256, 256, 3, 1, 14), (256, 512, 3, 1, 14),
                (512, 512, 3, 2, 14), (512, 512, 3, 1, 7)]


def _assert_split_taken(lib, cin, cout, k, s, H, B):
    import ctypes as C
    d = fa.ffk_conv_desc()
    d.batch, d.cin, d.cout, d.kh, d.kw = B, cin, cout, k, k
    d.stride, d.pad, d.hin, d.win = s, k // 2, H, H
    assert lib.ffk_conv_workspace_bytes(C.byref(d)) > 0


@pytest.mark.parametrize("split", [True, False], ids=["splitk", "wholek"])
@pytest.mark.parametrize("cin,cout,k,s,H", SHAPES)
def test_conv_int32_accumulators(gpu_lib, oracle, cin, cout, k, s, H, split):
    if split and (cin, cout, k, s, H) not in SPLIT_SHAPES:
        pytest.skip("no split-K variant for this geometry")
    r = rng(100 + cin + cout + k * 7 + s * 3 + H)
    B = 1 if split else _batch_for(H)
    if split:
        _assert_split_taken(gpu_lib, cin, cout, k, s, H, B)
    x = r.integers(-128, 128, size=(B, H, H, cin), dtype=np.int8)
    w = r.integers(-128, 128, size=(cout, cin, k, k), dtype=np.int8)
    x[0, 0, :, :] = -128                      # extreme products
    w[0] = -128
    got = run_conv(gpu_lib, x, w, s, k // 2, raw=True, split=split)
    assert np.array_equal(got, oracle.conv_i32(x, w, s, k // 2))


@pytest.mark.parametrize("B", [2, 23])
def test_stem_int32_with_fused_input_quant(gpu_lib, oracle, B):
    """The input layer quantizes the fp32 faces on load (glibc lrintf
    semantics: +-inf, NaN, |v| >= 2^31, .5 ties) and accumulates int32
    exactly.  At 23 faces each workgroup walks several tiles, so most tiles
    fetch only their two new input rows into the ring of patch rows."""
    r = rng(7 + B)
    x = r.uniform(-1, 1, size=(B, 112, 112, 3)).astype(F32)
    x[0, 0, :4, 0] = [0.5 / 127, -2.5 / 127, 1e10, -1e10]
    x[0, 1, :3, 1] = [np.inf, -np.inf, np.nan]
    x[1, 5, 5, :] = [3e9, -3e9, 2.5 / 127]
    x[B - 1, 57, 100, :] = [np.nan, 1e10, -0.0]
    x[B - 1, 111, 111, :] = [np.inf, 3e9, -1e10]
    x[B // 2, 64, :3, 2] = [1.5 / 127, -1.5 / 127, 0.49999997 / 127]
    inv = np.array([127.0, 127.00001, 126.5], F32)
    w = r.integers(-128, 128, size=(64, 3, 3, 3), dtype=np.int8)
    got = run_conv(gpu_lib, x, w, 1, 1, raw=True, in_inv=inv)
    q = oracle.quant_input(x, inv)
    assert np.array_equal(got, oracle.conv_i32(q, w, 1, 1))


# (cin, cout, k, s, H, batch, kind, grid): the small-tile kernels of small
# batches -- the 3-way K split of layers whose own split (6, 9) gives too
# large a grid, and the whole-K 64x64 tiles of layers without a split or
# where no split grid fits
SMALL_TILE_CASES = [
    (256, 256, 3, 2, 28, 5, "splitk", 16 * 4 * 3), (512, 512, 3, 2, 14, 8, "splitk", 7 * 8 * 3),
    (512, 512, 3, 1, 7, 8, "splitk", 7 * 8 * 3), (128, 128, 3, 1, 28, 8, "tile64", 98 * 2),
    (256, 512, 3, 1, 14, 8, "tile64", 25 * 8), (64, 64, 3, 1, 56, 8, "tile64", 392),
    (64, 64, 3, 2, 112, 1, "tile64", 49), (128, 256, 1, 1, 14, 1, "tile64", 4 * 4),
    (64, 128, 3, 1, 56, 1, "tile64", 49 * 2),
]


@pytest.mark.parametrize("cin,cout,k,s,H,B,kind,grid", SMALL_TILE_CASES)
def test_small_tile_variants(gpu_lib, oracle, cin, cout, k, s, H, B, kind, grid):
    """The small-tile kernels on the batches that take them: int32
    accumulators and the PReLU + BN epilogue exact against the oracle."""
    import ctypes as C
    d = fa.ffk_conv_desc()
    d.batch, d.cin, d.cout, d.kh, d.kw, d.stride, d.pad, d.hin, d.win = B, cin, cout, k, k, s, k // 2, H, H
    n = gpu_lib.ffk_conv_workspace_bytes(C.byref(d))
    d.workspace, d.workspace_bytes = (4096, n) if n else (None, 0)
    assert gpu_lib.ffk_conv_variant(C.byref(d)).decode() == kind
    assert gpu_lib.ffk_conv_grid(C.byref(d)) == grid
    r = rng(1800 + cin + cout + H + B)
    x = r.integers(-128, 128, size=(B, H, H, cin), dtype=np.int8)
    w = r.integers(-128, 128, size=(cout, cin, k, k), dtype=np.int8)
    acc = oracle.conv_i32(x, w, s, k // 2)
    assert np.array_equal(run_conv(gpu_lib, x, w, s, k // 2, raw=True), acc)
    ws, bias, inv = _unsaturated_params(r, cout, k * k * cin)
    slope = r.uniform(0, 0.3, cout).astype(F32)
    bsin = r.uniform(1e-3, 5e-2, cout).astype(F32)
    bns = r.uniform(0.5, 1.5, cout).astype(F32)
    bno = r.normal(0, 0.05, cout).astype(F32)
    binv = (1.0 / r.uniform(0.01, 0.1, cout)).astype(F32)
    P = params_block(cout, ws=ws, bias=bias, inv=inv, slope=slope, bn_sin=bsin, bn_s=bns, bn_o=bno, bn_inv=binv)
    flags = fa.FFK_EPI_BIAS | fa.FFK_EPI_PRELU | fa.FFK_EPI_BN
    got_x, got_bn = run_conv(gpu_lib, x, w, s, k // 2, params=P, flags=flags, want_bn=True)
    exp_x = oracle.fused_epilogue(acc, ws=ws, bias=bias, prelu=slope, inv_pc=inv)
    assert 0.05 < np.mean(np.abs(exp_x) < 127)
    assert np.array_equal(got_x, exp_x)
    exp_bn = oracle.bn_prelu_requant(exp_x, in_scale_pc=bsin, bn_scale=bns, bn_offset=bno, inv_pc=binv)
    assert np.array_equal(got_bn, exp_bn)


def test_split_partials_back_to_back(gpu_lib, oracle):
    """Split-K launches queued back to back on one stream with no host
    synchronization between them, alternating two layers that share one
    workspace: each launch's partial tiles overwrite the previous launch's at
    the same addresses, and each last-arriving workgroup must sum the current
    launch's partials (written by workgroups on any XCD), never a previous
    launch's.  Every output is exact."""
    import ctypes as C
    from gpu_util import Dev, check, pack_conv, split_counters_zero
    lib = gpu_lib
    r = rng(77)
    layers = [(256, 256, 1, 14), (512, 512, 1, 7)]
    descs, ws_need = [], 0
    for cin, cout, s, H in layers:
        w = r.integers(-128, 128, size=(cout, cin, 3, 3), dtype=np.int8)
        d = fa.ffk_conv_desc()
        d.batch, d.cin, d.cout, d.kh, d.kw, d.stride, d.pad, d.hin, d.win = 1, cin, cout, 3, 3, s, 1, H, H
        ws_need = max(ws_need, lib.ffk_conv_workspace_bytes(C.byref(d)))
        descs.append((d, w, Dev(lib, host=pack_conv(lib, w))))
    assert ws_need > 0
    ws = Dev(lib, nbytes=ws_need)
    check(lib, lib.ffk_zero(ws.ptr, ws_need, None))
    runs = []
    for k in range(24):
        d, w, dw = descs[k % 2]
        H, cin, cout = d.hin, d.cin, d.cout
        x = r.integers(-128, 128, size=(1, H, H, cin), dtype=np.int8)
        dx, do = Dev(lib, host=x), Dev(lib, nbytes=H * H * cout * 4)
        d.w, d.in_, d.out_i32, d.workspace, d.workspace_bytes = dw.ptr, dx.ptr, do.ptr, ws.ptr, ws_need
        assert lib.ffk_conv_variant(C.byref(d)) == b"splitk"
        check(lib, lib.ffk_conv(C.byref(d), None))
        runs.append((x, w, dx, do, H, cout))
    check(lib, lib.ffk_stream_sync(None))
    assert split_counters_zero(lib, ws)
    for k, (x, w, _dx, do, H, cout) in enumerate(runs):
        assert np.array_equal(do.get(np.int32, (1, H, H, cout)), oracle.conv_i32(x, w, 1, 1)), k


@pytest.mark.parametrize("cin,cout,s,H,batches", [(512, 512, 1, 7, (2, 1, 2)),
                                                   (512, 512, 2, 14, (1, 2))])
def test_split_workspace_reused_across_calls(gpu_lib, oracle, cin, cout, s, H, batches):
    """Split-K launches of different batch sizes in a row on one workspace
    (sized for the largest): the arrival counters are back at zero after each,
    and every result is exact."""
    import ctypes as C
    from gpu_util import Dev, check, pack_conv, split_counters_zero
    lib = gpu_lib
    r = rng(41 + cin)
    w = r.integers(-128, 128, size=(cout, cin, 3, 3), dtype=np.int8)
    dw = Dev(lib, host=pack_conv(lib, w))
    d = fa.ffk_conv_desc()
    d.cin, d.cout, d.kh, d.kw, d.stride, d.pad, d.hin, d.win = cin, cout, 3, 3, s, 1, H, H
    Ho = (H - 1) // s + 1
    n = 0
    for B in batches:
        d.batch = B
        need = lib.ffk_conv_workspace_bytes(C.byref(d))
        assert need > 0
        n = max(n, need)
    ws = Dev(lib, nbytes=n)
    check(lib, lib.ffk_zero(ws.ptr, n, None))
    d.w, d.workspace, d.workspace_bytes = dw.ptr, ws.ptr, n
    for B in batches:
        x = r.integers(-128, 128, size=(B, H, H, cin), dtype=np.int8)
        dx, do = Dev(lib, host=x), Dev(lib, nbytes=B * Ho * Ho * cout * 4)
        d.batch, d.in_, d.out_i32 = B, dx.ptr, do.ptr
        check(lib, lib.ffk_conv(C.byref(d), None))
        check(lib, lib.ffk_stream_sync(None))
        assert split_counters_zero(lib, ws)
        assert np.array_equal(do.get(np.int32, (B, Ho, Ho, cout)), oracle.conv_i32(x, w, s, 1)), B


def _special_params(r, C):
    ws = r.uniform(1e-3, 1e-2, C).astype(F32)
    bias = r.normal(0, 0.1, C).astype(F32)
    inv = (1.0 / r.uniform(0.5, 5.0, C)).astype(F32)
    ws[0], bias[0], inv[0] = 0.5, 0.0, 1.0 / 64        # exact .5 ties after scaling
    ws[1], inv[1] = 1e-3, 3.0e38                        # overflow -> -128
    ws[2] = np.float32(1.4e-44)                         # denormal
    inv[2] = 1e30
    ws[3] = np.nan
    ws[4], bias[4] = -1e-3, -0.0
    inv[5] = 1e9
    return ws, bias, inv


EPI_MODES = ["none", "prelu", "add", "add_bn", "prelu_bn", "bn_only", "prelu_le1", "prelu_bn_le1"]
EPI_SHAPES = [(64, 64, 3, 1, 56), (64, 64, 1, 2, 112), (128, 256, 1, 2, 28),
              (256, 256, 3, 1, 14), (512, 512, 3, 1, 7)]


def _variant(lib, cin, cout, k, s, H, B):
    import ctypes as C
    d = fa.ffk_conv_desc()
    d.batch, d.cin, d.cout, d.kh, d.kw = B, cin, cout, k, k
    d.stride, d.pad, d.hin, d.win = s, k // 2, H, H
    v = lib.ffk_conv_variant(C.byref(d))
    return v.decode() if v else None


BIG_GRID_VARIANTS = ("direct", "patch", "phase")


def _direct_batch(lib, cin, cout, k, s, H):
    """Smallest odd batch of the list at which the layer runs its large-grid
    kernel (direct-to-LDS tiles, or the 3x3 patch kernel) with a ragged last
    tile."""
    for B in (1, 3, 5, 45, 91, 171, 341, 401, 701):
        if _variant(lib, cin, cout, k, s, H, B) in BIG_GRID_VARIANTS:
            return B
    raise AssertionError("no batch takes the large-grid kernel")


def test_patch_kernel_takes_the_3x3_stride1_layers(gpu_lib):
    for cin, cout, k, s, H in SHAPES:
        if k == 3 and s == 1 and H in (7, 14, 28) or (cin, cout, k, s, H) in ((64, 64, 3, 1, 56), (64, 64, 3, 1, 112),
                                                                         (64, 128, 3, 1, 56)):
            assert _variant(gpu_lib, cin, cout, k, s, H, 1024) == "patch", (cin, cout, H)


@pytest.mark.parametrize("cin,cout,k,s,H", SHAPES)
def test_conv_direct_tiles_large_batch(gpu_lib, oracle, cin, cout, k, s, H):
    """The large-grid kernels (direct-to-LDS tiles; the 3x3 stride-1 patch
    kernel) on sampled images of a batch big enough to take them: first,
    middle and last image (ragged last tile)."""
    r = rng(200 + cin + cout + k * 7 + s * 3 + H)
    B = _direct_batch(gpu_lib, cin, cout, k, s, H)
    x = r.integers(-128, 128, size=(B, H, H, cin), dtype=np.int8)
    w = r.integers(-128, 128, size=(cout, cin, k, k), dtype=np.int8)
    x[B - 1, -1, :, :] = -128
    w[-1] = -128
    got = run_conv(gpu_lib, x, w, s, k // 2, raw=True, split=False)
    idx = [0, B // 2, B - 1]
    assert np.array_equal(got[idx], oracle.conv_i32(x[idx], w, s, k // 2))


@pytest.mark.parametrize("split", [True, False, "direct"], ids=["splitk", "wholek", "direct"])
@pytest.mark.parametrize("mode", EPI_MODES)
@pytest.mark.parametrize("cin,cout,k,s,H", EPI_SHAPES)
def test_conv_fused_epilogue(gpu_lib, oracle, mode, cin, cout, k, s, H, split):
    if split is True and (cin, cout, k, s, H) not in SPLIT_SHAPES:
        pytest.skip("no split-K variant for this geometry")
    r = rng(300 + cin + cout + H + EPI_MODES.index(mode))
    if split == "direct":
        B = _direct_batch(gpu_lib, cin, cout, k, s, H)
        idx = [0, B // 2, B - 1]
        split = False
    else:
        B = 1 if split else 2
        idx = list(range(B))
    if split:
        _assert_split_taken(gpu_lib, cin, cout, k, s, H, B)
    x = r.integers(-128, 128, size=(B, H, H, cin), dtype=np.int8)
    w = r.integers(-128, 128, size=(cout, cin, k, k), dtype=np.int8)
    Ho = (H + 2 * (k // 2) - k) // s + 1
    ws, bias, inv = _special_params(r, cout)
    rows = dict(ws=ws, bias=bias, inv=inv)
    flags = fa.FFK_EPI_BIAS
    ekw = dict(ws=ws, bias=bias, inv_pc=inv)
    add = None
    if "prelu" in mode:
        slope = r.uniform(0, 0.3, cout).astype(F32)
        if mode.endswith("le1"):
            # PReLU taken as max(f, f*slope): slopes up to exactly 1, zero and
            # negative slopes, a NaN pre-activation (ws[3]) and denormals
            slope[7:12] = [1.0, 0.0, -0.0, -0.5, np.float32(1e-45)]
            flags |= fa.FFK_EPI_PRELU_LE1
        rows["slope"] = slope; ekw["prelu"] = slope; flags |= fa.FFK_EPI_PRELU
    if "add" in mode:
        add = r.integers(-128, 128, size=(B, Ho, Ho, cout), dtype=np.int8)
        adds = r.uniform(1e-3, 5e-2, cout).astype(F32)
        rows["adds"] = adds; ekw.update(add_src=add, add_scale_pc=adds); flags |= fa.FFK_EPI_ADD
    want_bn = "bn" in mode
    if want_bn:
        bsin = r.uniform(1e-3, 5e-2, cout).astype(F32)
        bsin[6] = np.float32(3e-45)
        bns = r.uniform(0.5, 1.5, cout).astype(F32)
        bno = r.normal(0, 0.05, cout).astype(F32)
        binv = (1.0 / r.uniform(0.01, 0.1, cout)).astype(F32)
        rows.update(bn_sin=bsin, bn_s=bns, bn_o=bno, bn_inv=binv)
        flags |= fa.FFK_EPI_BN
    acc = oracle.conv_i32(x[idx], w, s, k // 2)
    if add is not None:
        ekw["add_src"] = add[idx]
    exp_x = oracle.fused_epilogue(acc, **ekw)
    got_x, got_bn = run_conv(gpu_lib, x, w, s, k // 2, params=params_block(cout, **rows),
                             flags=flags, add=add, want_x=(mode != "bn_only"), want_bn=want_bn,
                             split=split)
    if mode != "bn_only":
        assert np.array_equal(got_x[idx], exp_x)
    if want_bn:
        exp_bn = oracle.bn_prelu_requant(exp_x, in_scale_pc=bsin, bn_scale=bns, bn_offset=bno,
                                         inv_pc=binv)
        assert np.array_equal(got_bn[idx], exp_bn)


def test_inscale_path(gpu_lib, oracle):
    """FFW2/FFW3 models dequantize with a runtime input scale first."""
    r = rng(9)
    x = r.integers(-128, 128, size=(3, 14, 14, 256), dtype=np.int8)
    w = r.integers(-128, 128, size=(256, 256, 3, 3), dtype=np.int8)
    ws = r.uniform(1e-3, 1e-2, 256).astype(F32)
    bias = r.normal(0, 0.1, 256).astype(F32)
    inv = (1.0 / r.uniform(0.5, 5, 256)).astype(F32)
    acc = oracle.conv_i32(x, w, 1, 1)
    exp = oracle.fused_epilogue(acc, ws=ws, bias=bias, in_scale=0.0173, inv_pc=inv)
    got, _ = run_conv(gpu_lib, x, w, 1, 1, params=params_block(256, ws=ws, bias=bias, inv=inv),
                      flags=fa.FFK_EPI_BIAS | fa.FFK_EPI_INSCALE, in_scale=0.0173)
    assert np.array_equal(got, exp)


def test_config2_microbench_layer(gpu_lib, oracle):
    """N=64, 14x14, 256->256 3x3 s1 p1; act/weights int8
    U[-127,127]; ws U[1e-3,1e-2]; bias N(0,0.1); PReLU 0.25; seed 1.  The
    output scale (unspecified) is the per-channel absmax/127 of the fp32
    pre-requant tensor."""
    r = rng(1)
    x = r.integers(-127, 128, size=(64, 14, 14, 256), dtype=np.int8)
    w = r.integers(-127, 128, size=(256, 256, 3, 3), dtype=np.int8)
    ws = r.uniform(1e-3, 1e-2, 256).astype(F32)
    bias = r.normal(0, 0.1, 256).astype(F32)
    slope = np.full(256, 0.25, F32)
    acc = oracle.conv_i32(x, w, 1, 1)
    assert np.array_equal(run_conv(gpu_lib, x, w, 1, 1, raw=True), acc)
    f = acc.astype(F32) * ws + bias
    f = np.where(f < 0, f * slope, f)
    s_out = (np.abs(f).reshape(-1, 256).max(axis=0) / 127).astype(F32)
    inv = (F32(1.0) / (s_out + F32(1e-9))).astype(F32)
    exp = oracle.fused_epilogue(acc, ws=ws, bias=bias, prelu=slope, inv_pc=inv)
    got, _ = run_conv(gpu_lib, x, w, 1, 1,
                      params=params_block(256, ws=ws, bias=bias, slope=slope, inv=inv),
                      flags=fa.FFK_EPI_BIAS | fa.FFK_EPI_PRELU)
    assert np.array_equal(got, exp)
    assert np.abs(exp.astype(np.int32)).max() == 127       # the scale reaches full range


@pytest.mark.parametrize("B,path,split", [(1, 0, False), (3, 1, False), (16, 0, False), (17, 0, False),
                                          (40, 2, False), (5, 2, False), (130, 0, False),
                                          (17, 0, True), (130, 0, True), (1024, 0, True)])
def test_fc_head(gpu_lib, oracle, B, path, split):
    """FC head in every path: matvec (b <= 16), one MFMA GEMM workgroup per
    128x128 output tile, and split-K (several workgroups share a tile's K
    reduction through the workspace)."""
    r = rng(500 + B + path)
    K, N = 25088, 512
    a = r.integers(-128, 128, size=(B, K), dtype=np.int8)
    W = r.integers(-127, 128, size=(N, K), dtype=np.int8)
    ws = r.uniform(1e-7, 1e-5, N).astype(F32)
    bias = r.normal(0, 0.05, N).astype(F32)
    got = run_fc(gpu_lib, a, W, ws, bias, path=path, split=split)
    for b in (range(B) if B <= 130 else [0, 1, 127, 128, 500, B - 1]):
        assert np.array_equal(got[b], oracle.fc(a[b], W, ws, bias)), "face %d" % b


@pytest.mark.parametrize("B,via_io", [(40, False), (40, True), (3, True)])
def test_fc_other_head_shapes(gpu_lib, oracle, B, via_io):
    """A head other than 25088 -> 512 (here K = 4096) takes the matvec at
    every batch, 16 faces per launch, writing to `out` or, as a captured
    chain does, through the I/O descriptor (each launch at its first face's
    rows); the GEMM path refuses the shape."""
    lib = gpu_lib
    r = rng(570 + B)
    K, N = 4096, 512
    a = r.integers(-128, 128, size=(B, K), dtype=np.int8)
    W = r.integers(-127, 128, size=(N, K), dtype=np.int8)
    ws = r.uniform(1e-7, 1e-5, N).astype(F32)
    bias = r.normal(0, 0.05, N).astype(F32)
    exp = np.stack([oracle.fc(a[b], W, ws, bias) for b in range(B)])
    if not via_io:
        assert np.array_equal(run_fc(lib, a, W, ws, bias), exp)
        with pytest.raises(RuntimeError):
            run_fc(lib, a, W, ws, bias, path=2)
        return
    packed = np.empty(lib.ffk_fc_packed_bytes(N, K), np.int8)
    gpu_util.check(lib, lib.ffk_pack_fc_weights(W.ctypes.data, N, K, packed.ctypes.data))
    da, dw = gpu_util.Dev(lib, host=a), gpu_util.Dev(lib, host=packed)
    dws, db = gpu_util.Dev(lib, host=ws), gpu_util.Dev(lib, host=bias)
    do = gpu_util.Dev(lib, nbytes=B * N * 4)
    dio = gpu_util.Dev(lib, host=np.array([0, do.ptr], np.uint64))
    d = fa.ffk_fc_desc()
    d.batch, d.n, d.k = B, N, K
    d.a, d.w, d.ws, d.bias, d.out, d.io = da.ptr, dw.ptr, dws.ptr, db.ptr, None, dio.ptr
    d.a_scale = 1.0
    gpu_util.check(lib, lib.ffk_fc(C.byref(d), None))
    gpu_util.check(lib, lib.ffk_stream_sync(None))
    assert np.array_equal(do.get(np.float32, (B, N)), exp)


@pytest.mark.parametrize("B", [1, 2, 16])
def test_fc_matvec_extreme_values(gpu_lib, oracle, B):
    """Matvec path (each row's K range split over several waves, partial sums
    added through LDS) at the largest dot products int8 allows: every product
    +-128*127, |dot| = 25088*128*127 ~ 4.08e8, plus rows of mixed sign."""
    r = rng(560 + B)
    K, N = 25088, 512
    a = np.full((B, K), -128, np.int8)
    if B > 1:
        a[1] = r.integers(-128, 128, size=K, dtype=np.int8)
    W = np.where(np.arange(N)[:, None] % 2 == 0, 127, -127).astype(np.int8) * np.ones((1, K), np.int8)
    W[5] = r.integers(-127, 128, size=K, dtype=np.int8)
    ws = r.uniform(1e-9, 1e-8, N).astype(F32)
    bias = r.normal(0, 0.05, N).astype(F32)
    got = run_fc(gpu_lib, a, W, ws, bias, path=1)
    for b in range(B):
        assert np.array_equal(got[b], oracle.fc(a[b], W, ws, bias)), "face %d" % b


# ---- integer Winograd F(2,3) path of the 64-channel 3x3 stride-1 layers ----

@pytest.mark.parametrize("H,B", [(56, 3), (112, 1)])
def test_winograd_int32_accumulators(gpu_lib, oracle, H, B):
    """The Winograd path's int32 accumulators equal the direct conv (brute
    force) and, times 4, the restated kernels/winograd_int8_ref.c output --
    the reference's own exactness statement (F(2,3) with G' = 2G is 4x the
    direct conv).  Extreme operands make the limb products reach their
    bounds (|v| = 510, |u| = 1152)."""
    r = rng(700 + H)
    x = r.integers(-128, 128, size=(B, H, H, 64), dtype=np.int8)
    w = r.integers(-128, 128, size=(64, 64, 3, 3), dtype=np.int8)
    x[0, 0:4, :, :] = -128
    x[0, 4:8, ::2, :] = 127                 # alternating rows: |v| = 510
    x[-1, -3:, :, :] = 127
    w[0] = -128
    w[1] = 127
    w[2, :, 0, :] = -128; w[2, :, 1, :] = 127; w[2, :, 2, :] = -128   # |u| = 1152
    got = run_conv(gpu_lib, x, w, 1, 1, raw=True, winograd=True)
    assert np.array_equal(got, oracle.conv_i32(x, w, 1, 1))
    u = oracle.winograd_weights(w)
    assert np.abs(u.astype(np.int32)).max() == 1152
    assert np.array_equal(4 * got.astype(np.int64), oracle.conv_winograd(x, u).astype(np.int64))


@pytest.mark.parametrize("mode", ["none", "prelu", "prelu_le1", "add_bn", "prelu_bn", "bn_only"])
@pytest.mark.parametrize("H,B", [(56, 2), (112, 1)])
def test_winograd_fused_epilogue(gpu_lib, oracle, mode, H, B):
    """The Winograd path's requant epilogue: bit-exact with the oracle in
    every mode, with the special parameters (ties, overflow, NaN and denormal
    scales, -0) of the direct kernels' test."""
    r = rng(750 + H + len(mode))
    x = r.integers(-128, 128, size=(B, H, H, 64), dtype=np.int8)
    w = r.integers(-128, 128, size=(64, 64, 3, 3), dtype=np.int8)
    ws, bias, inv = _special_params(r, 64)
    rows = dict(ws=ws, bias=bias, inv=inv)
    flags = fa.FFK_EPI_BIAS
    ekw = dict(ws=ws, bias=bias, inv_pc=inv)
    add = None
    if "prelu" in mode:
        slope = r.uniform(0, 0.3, 64).astype(F32)
        if mode.endswith("le1"):
            slope[7:12] = [1.0, 0.0, -0.0, -0.5, np.float32(1e-45)]
            flags |= fa.FFK_EPI_PRELU_LE1
        rows["slope"] = slope; ekw["prelu"] = slope; flags |= fa.FFK_EPI_PRELU
    if "add" in mode:
        add = r.integers(-128, 128, size=(B, H, H, 64), dtype=np.int8)
        adds = r.uniform(1e-3, 5e-2, 64).astype(F32)
        rows["adds"] = adds; ekw.update(add_src=add, add_scale_pc=adds); flags |= fa.FFK_EPI_ADD
    want_bn = "bn" in mode
    if want_bn:
        bsin = r.uniform(1e-3, 5e-2, 64).astype(F32)
        bns = r.uniform(0.5, 1.5, 64).astype(F32)
        bno = r.normal(0, 0.05, 64).astype(F32)
        binv = (1.0 / r.uniform(0.01, 0.1, 64)).astype(F32)
        rows.update(bn_sin=bsin, bn_s=bns, bn_o=bno, bn_inv=binv)
        flags |= fa.FFK_EPI_BN
    exp_x = oracle.fused_epilogue(oracle.conv_i32(x, w, 1, 1), **ekw)
    got_x, got_bn = run_conv(gpu_lib, x, w, 1, 1, params=params_block(64, **rows), flags=flags,
                             add=add, want_x=(mode != "bn_only"), want_bn=want_bn, winograd=True)
    if mode != "bn_only":
        assert np.array_equal(got_x, exp_x)
    if want_bn:
        exp_bn = oracle.bn_prelu_requant(exp_x, in_scale_pc=bsin, bn_scale=bns, bn_offset=bno,
                                         inv_pc=binv)
        assert np.array_equal(got_bn, exp_bn)


def test_winograd_large_batch(gpu_lib, oracle):
    """A 112x112 batch of 400 images in one launch (1.25 M 2x2 blocks; the
    transformed input stays on chip, so no workspace at any batch): sampled
    images exact, the last one with a ragged last tile."""
    import ctypes as C
    d = fa.ffk_conv_desc()
    d.batch, d.cin, d.cout, d.kh, d.kw, d.stride, d.pad, d.hin, d.win = 400, 64, 64, 3, 3, 1, 1, 112, 112
    d.flags = fa.FFK_ALGO_WINOGRAD
    assert gpu_lib.ffk_conv_workspace_bytes(C.byref(d)) == 0
    r = rng(790)
    B = 401
    x = r.integers(-128, 128, size=(B, 112, 112, 64), dtype=np.int8)
    w = r.integers(-128, 128, size=(64, 64, 3, 3), dtype=np.int8)
    got = run_conv(gpu_lib, x, w, 1, 1, raw=True, winograd=True)
    idx = [0, 333, 334, B - 1]
    assert np.array_equal(got[idx], oracle.conv_i32(x[idx], w, 1, 1))


def test_winograd_and_splitk_share_a_workspace(gpu_lib, oracle):
    """One workspace serves a whole launch chain: a Winograd layer given the
    chain's workspace leaves it alone, so a b=1 split-K layer after it still
    sums exactly and leaves its counters at 0."""
    import ctypes as C
    from gpu_util import Dev, check
    r = rng(795)
    d = fa.ffk_conv_desc()
    d.batch, d.cin, d.cout, d.kh, d.kw, d.stride, d.pad, d.hin, d.win = 1, 64, 64, 3, 3, 1, 1, 112, 112
    d.flags = fa.FFK_ALGO_WINOGRAD
    n = gpu_lib.ffk_conv_workspace_bytes(C.byref(d))
    d.cin, d.cout, d.hin, d.win, d.flags = 512, 512, 7, 7, 0
    n = max(n, gpu_lib.ffk_conv_workspace_bytes(C.byref(d)))
    ws = Dev(gpu_lib, nbytes=n)
    check(gpu_lib, gpu_lib.ffk_zero(ws.ptr, n, None))
    x1 = r.integers(-128, 128, size=(1, 112, 112, 64), dtype=np.int8)
    w1 = r.integers(-128, 128, size=(64, 64, 3, 3), dtype=np.int8)
    x2 = r.integers(-128, 128, size=(1, 7, 7, 512), dtype=np.int8)
    w2 = r.integers(-128, 128, size=(512, 512, 3, 3), dtype=np.int8)
    for _ in range(2):
        got1 = run_conv(gpu_lib, x1, w1, 1, 1, raw=True, winograd=True, workspace=ws)
        got2 = run_conv(gpu_lib, x2, w2, 1, 1, raw=True, workspace=ws)
        assert np.array_equal(got1, oracle.conv_i32(x1, w1, 1, 1))
        assert np.array_equal(got2, oracle.conv_i32(x2, w2, 1, 1))


# ---- X stored at its even pixels only (FFK_OUT_X_EVEN), and the 1x1 stride-1
# shortcuts that read it in place of the 1x1 stride-2 ones over the whole X ----
SHORTCUT_S1 = [(64, 64, 56), (64, 128, 28), (128, 256, 14), (256, 512, 7)]

# (cin, cout, k, s, H, batch, kernel variant): the stage outputs on their
# large-batch kernels, the split-K and 128x128 variants of small batches, a
# direct-to-LDS layer
X_EVEN_CASES = [
    (64, 64, 3, 1, 56, "big", "patch"), (128, 128, 3, 1, 28, "big", "patch"),
    (256, 256, 3, 1, 14, "big", "patch"), (256, 256, 3, 1, 14, 1, "splitk"),
    (256, 256, 3, 1, 14, 53, "patch_kg"), (256, 256, 3, 1, 14, 9, "tile64"), (64, 64, 3, 2, 112, "big", "phase"),
    (64, 128, 3, 1, 56, 7, "patch_kg"), (64, 128, 3, 1, 56, 2, "tile64"),
]


def _unsaturated_params(r, cout, ktot):
    """ws, bias, inv putting most outputs well inside int8 for uniform int8
    operands (accumulator spread ~ sqrt(K) * 74^2)."""
    ws = r.uniform(1e-3, 1e-2, cout).astype(F32)
    bias = r.normal(0, 0.1, cout).astype(F32)
    inv = (40.0 / (ws * np.sqrt(ktot) * 5460.0)).astype(F32)
    return ws, bias, inv


@pytest.mark.parametrize("mode", ["add_bn", "prelu"])
@pytest.mark.parametrize("cin,cout,k,s,H,B,variant", X_EVEN_CASES)
def test_x_even_output(gpu_lib, oracle, cin, cout, k, s, H, B, variant, mode):
    """FFK_OUT_X_EVEN: X comes out at its even-row, even-column pixels only,
    as a compact tensor, bit-exact with the oracle's X there; BN(X) stays whole."""
    r = rng(900 + cin + cout + H + (B if isinstance(B, int) else 0) + len(mode))
    if B == "big":
        B = _direct_batch(gpu_lib, cin, cout, k, s, H)
        idx = sorted({0, B // 2, B - 1})
    else:
        idx = list(range(B)) if B <= 16 else sorted({0, B // 2, B - 1})
    assert _variant_ws(gpu_lib, cin, cout, k, s, H, B) == variant
    x = r.integers(-128, 128, size=(B, H, H, cin), dtype=np.int8)
    w = r.integers(-128, 128, size=(cout, cin, k, k), dtype=np.int8)
    Ho = (H + 2 * (k // 2) - k) // s + 1
    ws, bias, inv = _unsaturated_params(r, cout, k * k * cin)
    rows = dict(ws=ws, bias=bias, inv=inv)
    ekw = dict(ws=ws, bias=bias, inv_pc=inv)
    flags = fa.FFK_EPI_BIAS
    add = None
    bn = mode == "add_bn"
    if bn:
        add = r.integers(-128, 128, size=(B, Ho, Ho, cout), dtype=np.int8)
        adds = r.uniform(1e-3, 5e-2, cout).astype(F32)
        bsin = r.uniform(1e-3, 5e-2, cout).astype(F32)
        bns = r.uniform(0.5, 1.5, cout).astype(F32)
        bno = r.normal(0, 0.05, cout).astype(F32)
        binv = (1.0 / r.uniform(0.01, 0.1, cout)).astype(F32)
        rows.update(adds=adds, bn_sin=bsin, bn_s=bns, bn_o=bno, bn_inv=binv)
        ekw.update(add_src=add[idx], add_scale_pc=adds)
        flags |= fa.FFK_EPI_ADD | fa.FFK_EPI_BN
    else:
        slope = r.uniform(0, 0.3, cout).astype(F32)
        rows["slope"] = slope
        ekw["prelu"] = slope
        flags |= fa.FFK_EPI_PRELU
    got_x, got_bn = run_conv(gpu_lib, x, w, s, k // 2, params=params_block(cout, **rows), flags=flags,
                             add=add, want_bn=bn, x_even=True)
    exp_x = oracle.fused_epilogue(oracle.conv_i32(x[idx], w, s, k // 2), **ekw)
    assert 0.05 < np.mean(np.abs(exp_x) < 127)          # not a saturated test
    assert got_x.shape == (B, Ho // 2, Ho // 2, cout)
    assert np.array_equal(got_x[idx], exp_x[:, ::2, ::2])
    if bn:
        exp_bn = oracle.bn_prelu_requant(exp_x, in_scale_pc=bsin, bn_scale=bns, bn_offset=bno, inv_pc=binv)
        assert np.array_equal(got_bn[idx], exp_bn)


def _variant_ws(lib, cin, cout, k, s, H, B):
    """Kernel variant of a layer at batch B when given the workspace it asks for."""
    import ctypes as C
    d = fa.ffk_conv_desc()
    d.batch, d.cin, d.cout, d.kh, d.kw = B, cin, cout, k, k
    d.stride, d.pad, d.hin, d.win = s, k // 2, H, H
    n = lib.ffk_conv_workspace_bytes(C.byref(d))
    d.workspace, d.workspace_bytes = (4096, n) if n else (None, 0)
    v = lib.ffk_conv_variant(C.byref(d))
    return v.decode() if v else None


@pytest.mark.parametrize("in_range", [False, True], ids=["checked", "in_range"])
@pytest.mark.parametrize("rgb8", [False, True], ids=["fp32", "rgb8"])
def test_x_even_stem(gpu_lib, oracle, rgb8, in_range):
    """The input layer with its production epilogue (PReLU + BN second output)
    and X at its even pixels, with and without FFK_EPI_IN_RANGE."""
    r = rng(951 + rgb8)
    B = 3
    w = r.integers(-128, 128, size=(64, 3, 3, 3), dtype=np.int8)
    inv = np.array([127.0, 126.9, 127.3], np.float32)
    imgs = r.integers(0, 256, size=(B, 112, 112, 3), dtype=np.uint8)
    faces = (imgs.astype(np.float32) - 127.5) / 127.5
    ws, bias, winv = _unsaturated_params(r, 64, 27)
    slope = r.uniform(0, 0.3, 64).astype(F32)
    bsin = r.uniform(1e-3, 5e-2, 64).astype(F32)
    bns = r.uniform(0.5, 1.5, 64).astype(F32)
    bno = r.normal(0, 0.05, 64).astype(F32)
    binv = (1.0 / r.uniform(0.01, 0.1, 64)).astype(F32)
    P = params_block(64, ws=ws, bias=bias, inv=winv, slope=slope, bn_sin=bsin, bn_s=bns, bn_o=bno,
                     bn_inv=binv)
    flags = fa.FFK_EPI_BIAS | fa.FFK_EPI_PRELU | fa.FFK_EPI_BN
    if in_range:
        flags |= fa.FFK_EPI_PRELU_LE1 | fa.FFK_EPI_IN_RANGE
        assert gpu_lib.ffk_requant_in_range(P.ctypes.data, 64, 27, flags) == 1
    if rgb8:
        lut = np.empty((3, 256), np.int8)
        assert gpu_lib.ffk_make_rgb8_lut(inv.ctypes.data, lut.ctypes.data) == 0
        got_x, got_bn = run_conv(gpu_lib, imgs, w, 1, 1, params=P, flags=flags | fa.FFK_IN_RGB8,
                                 in_lut=lut, want_bn=True, x_even=True)
    else:
        got_x, got_bn = run_conv(gpu_lib, faces, w, 1, 1, params=P, flags=flags, in_inv=inv,
                                 want_bn=True, x_even=True)
    q = oracle.quant_input(faces, inv)
    exp_x = oracle.fused_epilogue(oracle.conv_i32(q, w, 1, 1), ws=ws, bias=bias, prelu=slope, inv_pc=winv)
    assert 0.05 < np.mean(np.abs(exp_x) < 127)
    assert np.array_equal(got_x, exp_x[:, ::2, ::2])
    exp_bn = oracle.bn_prelu_requant(exp_x, in_scale_pc=bsin, bn_scale=bns, bn_offset=bno, inv_pc=binv)
    assert np.array_equal(got_bn, exp_bn)


STEM_MODES = ["none", "prelu", "prelu_bn"]
STEM_FORMS = ["general", "in_range", "fma"]
STEM_CASES = [(m, f, xe, 3) for m in STEM_MODES for f in STEM_FORMS for xe in (False, True)] + \
             [("prelu_bn", "fma", False, 23), ("prelu_bn", "fma", True, 23), ("none", "general", False, 23)]


@pytest.mark.parametrize("mode,form,x_even,B", STEM_CASES)
def test_stem_epilogue_forms(gpu_lib, oracle, mode, form, x_even, B):
    """The input layer's int8 epilogue variants (no activation / PReLU /
    PReLU + BN second output; the general, in-range and one-fma-tail
    requant) with X at every pixel and at its even pixels; at 23 faces the
    persistent workgroups walk several tiles, so the flush offsets step per
    tile."""
    r = rng(1700 + B + 3 * STEM_FORMS.index(form) + STEM_MODES.index(mode) + 9 * x_even)
    rp = rng(1691)                               # parameters: the same in every case
    w = r.integers(-128, 128, size=(64, 3, 3, 3), dtype=np.int8)
    inv_in = np.array([127.0, 126.9, 127.3], np.float32)
    faces = r.uniform(-1.0, 1.0, size=(B, 112, 112, 3)).astype(F32)
    ws, bias, winv = _unsaturated_params(rp, 64, 27)
    rows = dict(ws=ws, bias=bias, inv=winv)
    ekw = dict(ws=ws, bias=bias, inv_pc=winv)
    flags = fa.FFK_EPI_BIAS
    slope = rp.uniform(0.05, 0.3, 64).astype(F32)
    if "prelu" in mode:
        rows["slope"] = slope
        ekw["prelu"] = slope
        flags |= fa.FFK_EPI_PRELU | (0 if form == "general" else fa.FFK_EPI_PRELU_LE1)
    bsin = rp.uniform(1e-3, 5e-2, 64).astype(F32)
    bns = rp.uniform(0.5, 1.5, 64).astype(F32)
    bno = rp.normal(0, 0.05, 64).astype(F32)
    binv = (1.0 / rp.uniform(0.01, 0.1, 64)).astype(F32)
    bn = "bn" in mode
    if bn:
        rows.update(bn_sin=bsin, bn_s=bns, bn_o=bno, bn_inv=binv)
        flags |= fa.FFK_EPI_BN
    P = params_block(64, **rows)
    if form != "general":
        assert gpu_lib.ffk_requant_in_range(P.ctypes.data, 64, 27, flags) == 1
        flags |= fa.FFK_EPI_IN_RANGE
    if form == "fma":
        assert gpu_lib.ffk_requant_fma_ok(P.ctypes.data, 64, 27, flags) == 1
        flags |= fa.FFK_EPI_FMA_TAIL
    got_x, got_bn = run_conv(gpu_lib, faces, w, 1, 1, params=P, flags=flags, in_inv=inv_in, want_bn=bn,
                             x_even=x_even)
    q = oracle.quant_input(faces, inv_in)
    exp_x = oracle.fused_epilogue(oracle.conv_i32(q, w, 1, 1), **ekw)
    assert 0.05 < np.mean(np.abs(exp_x) < 127)
    assert np.array_equal(got_x, exp_x[:, ::2, ::2] if x_even else exp_x)
    if bn:
        exp_bn = oracle.bn_prelu_requant(exp_x, in_scale_pc=bsin, bn_scale=bns, bn_offset=bno, inv_pc=binv)
        assert np.array_equal(got_bn, exp_bn)


@pytest.mark.parametrize("B", [2, 341])
def test_x_even_winograd(gpu_lib, oracle, B):
    """The Winograd path keeps pixel (0, 0) of each 2x2 output block, also at
    341 faces of 112x112 (a ragged last tile)."""
    r = rng(960 + B)
    H = 112 if B > 2 else 56
    x = r.integers(-128, 128, size=(B, H, H, 64), dtype=np.int8)
    w = r.integers(-128, 128, size=(64, 64, 3, 3), dtype=np.int8)
    ws, bias, inv = _unsaturated_params(r, 64, 576)
    add = r.integers(-128, 128, size=(B, H, H, 64), dtype=np.int8)
    adds = r.uniform(1e-3, 5e-2, 64).astype(F32)
    bsin = r.uniform(1e-3, 5e-2, 64).astype(F32)
    bns = r.uniform(0.5, 1.5, 64).astype(F32)
    bno = r.normal(0, 0.05, 64).astype(F32)
    binv = (1.0 / r.uniform(0.01, 0.1, 64)).astype(F32)
    P = params_block(64, ws=ws, bias=bias, inv=inv, adds=adds, bn_sin=bsin, bn_s=bns, bn_o=bno, bn_inv=binv)
    flags = fa.FFK_EPI_BIAS | fa.FFK_EPI_ADD | fa.FFK_EPI_BN
    got_x, got_bn = run_conv(gpu_lib, x, w, 1, 1, params=P, flags=flags, add=add, want_bn=True,
                             winograd=True, x_even=True)
    idx = sorted({0, B // 2, B - 1})
    exp_x = oracle.fused_epilogue(oracle.conv_i32(x[idx], w, 1, 1), ws=ws, bias=bias, inv_pc=inv,
                                  add_src=add[idx], add_scale_pc=adds)
    assert np.array_equal(got_x[idx], exp_x[:, ::2, ::2])
    exp_bn = oracle.bn_prelu_requant(exp_x, in_scale_pc=bsin, bn_scale=bns, bn_offset=bno, inv_pc=binv)
    assert np.array_equal(got_bn[idx], exp_bn)


@pytest.mark.parametrize("B", ["small", "big"])
@pytest.mark.parametrize("cin,cout,Hc", SHORTCUT_S1)
def test_shortcut_stride1_over_compact_x(gpu_lib, oracle, cin, cout, Hc, B):
    """A 1x1 stride-1 conv over the even pixels of X equals the 1x1 stride-2
    conv over the whole X (the oracle's), int32 for int32."""
    r = rng(970 + cin + cout + Hc)
    B = 2 if B == "small" else _direct_batch(gpu_lib, cin, cout, 1, 1, Hc)
    full = r.integers(-128, 128, size=(B, 2 * Hc, 2 * Hc, cin), dtype=np.int8)
    w = r.integers(-128, 128, size=(cout, cin, 1, 1), dtype=np.int8)
    full[-1, 0] = -128
    w[0] = -128
    got = run_conv(gpu_lib, np.ascontiguousarray(full[:, ::2, ::2]), w, 1, 0, raw=True)
    idx = sorted({0, B // 2, B - 1})
    assert np.array_equal(got[idx], oracle.conv_i32(full[idx], w, 2, 0))


# ---- FFK_EPI_IN_RANGE: the requant without the x86 out-of-range case ----
RANGE_MODES = ["none", "prelu_le1", "add_bn", "prelu_bn_le1"]


@pytest.mark.parametrize("split", [True, False, "direct"], ids=["splitk", "wholek", "direct"])
@pytest.mark.parametrize("mode", RANGE_MODES)
@pytest.mark.parametrize("cin,cout,k,s,H", EPI_SHAPES)
def test_in_range_epilogue(gpu_lib, oracle, mode, cin, cout, k, s, H, split):
    """With parameters the host check accepts (ffk_requant_in_range), the
    in-range epilogue gives the oracle's int8 values, ties and negative zero
    included."""
    if split is True and (cin, cout, k, s, H) not in SPLIT_SHAPES:
        pytest.skip("no split-K variant for this geometry")
    r = rng(1100 + cin + cout + H + RANGE_MODES.index(mode))
    if split == "direct":
        B = _direct_batch(gpu_lib, cin, cout, k, s, H)
        idx = sorted({0, B // 2, B - 1})
        split = False
    else:
        B = 1 if split else 2
        idx = list(range(B))
    x = r.integers(-128, 128, size=(B, H, H, cin), dtype=np.int8)
    w = r.integers(-128, 128, size=(cout, cin, k, k), dtype=np.int8)
    Ho = (H + 2 * (k // 2) - k) // s + 1
    ws, bias, inv = _unsaturated_params(r, cout, k * k * cin)
    ws[0], bias[0], inv[0] = 0.5, 0.0, 1.0 / 64        # exact .5 ties after scaling
    ws[4], bias[4] = -1e-3, -0.0
    rows = dict(ws=ws, bias=bias, inv=inv)
    ekw = dict(ws=ws, bias=bias, inv_pc=inv)
    flags = fa.FFK_EPI_BIAS
    add = None
    if "prelu" in mode:
        slope = r.uniform(0, 0.3, cout).astype(F32)
        slope[7:10] = [1.0, 0.0, -0.5]
        rows["slope"] = slope; ekw["prelu"] = slope
        flags |= fa.FFK_EPI_PRELU | fa.FFK_EPI_PRELU_LE1
    if "add" in mode:
        add = r.integers(-128, 128, size=(B, Ho, Ho, cout), dtype=np.int8)
        adds = r.uniform(1e-3, 5e-2, cout).astype(F32)
        rows["adds"] = adds; ekw.update(add_src=add[idx], add_scale_pc=adds); flags |= fa.FFK_EPI_ADD
    bn = "bn" in mode
    if bn:
        bsin = r.uniform(1e-3, 5e-2, cout).astype(F32)
        bns = r.uniform(0.5, 1.5, cout).astype(F32)
        bno = r.normal(0, 0.05, cout).astype(F32)
        binv = (1.0 / r.uniform(0.01, 0.1, cout)).astype(F32)
        rows.update(bn_sin=bsin, bn_s=bns, bn_o=bno, bn_inv=binv)
        flags |= fa.FFK_EPI_BN
    P = params_block(cout, **rows)
    assert gpu_lib.ffk_requant_in_range(P.ctypes.data, cout, k * k * cin, flags) == 1
    got_x, got_bn = run_conv(gpu_lib, x, w, s, k // 2, params=P, flags=flags | fa.FFK_EPI_IN_RANGE,
                             add=add, want_bn=bn, split=split)
    exp_x = oracle.fused_epilogue(oracle.conv_i32(x[idx], w, s, k // 2), **ekw)
    assert 0.05 < np.mean(np.abs(exp_x) < 127)
    assert np.array_equal(got_x[idx], exp_x)
    if bn:
        exp_bn = oracle.bn_prelu_requant(exp_x, in_scale_pc=bsin, bn_scale=bns, bn_offset=bno, inv_pc=binv)
        assert np.array_equal(got_bn[idx], exp_bn)


@pytest.mark.parametrize("mode", ["raw", "add_bn"])
def test_patch_64_wide_tiles(gpu_lib, oracle, mode):
    """The 64->64 3x3 layer at 56x56 takes 512x64 tiles (8 waves, waves 0-3
    loading the weights) from 84 faces on; 91 faces leave a ragged last tile.
    Bit-exact against the oracle on the first, middle and last image."""
    B = 91
    assert _variant(gpu_lib, 64, 64, 3, 1, 56, B) == "patch"
    r = rng(1400 + len(mode))
    x = r.integers(-128, 128, size=(B, 56, 56, 64), dtype=np.int8)
    w = r.integers(-128, 128, size=(64, 64, 3, 3), dtype=np.int8)
    x[B - 1, -1] = -128
    idx = [0, B // 2, B - 1]
    if mode == "raw":
        got = run_conv(gpu_lib, x, w, 1, 1, raw=True)
        assert np.array_equal(got[idx], oracle.conv_i32(x[idx], w, 1, 1))
        return
    ws, bias, inv = _unsaturated_params(r, 64, 576)
    add = r.integers(-128, 128, size=(B, 56, 56, 64), dtype=np.int8)
    adds = r.uniform(1e-3, 5e-2, 64).astype(F32)
    bsin = r.uniform(1e-3, 5e-2, 64).astype(F32)
    bns = r.uniform(0.5, 1.5, 64).astype(F32)
    bno = r.normal(0, 0.05, 64).astype(F32)
    binv = (1.0 / r.uniform(0.01, 0.1, 64)).astype(F32)
    P = params_block(64, ws=ws, bias=bias, inv=inv, adds=adds, bn_sin=bsin, bn_s=bns, bn_o=bno, bn_inv=binv)
    flags = fa.FFK_EPI_BIAS | fa.FFK_EPI_ADD | fa.FFK_EPI_BN | fa.FFK_EPI_IN_RANGE
    gx, gb = run_conv(gpu_lib, x, w, 1, 1, params=P, flags=flags, add=add, want_bn=True)
    exp_x = oracle.fused_epilogue(oracle.conv_i32(x[idx], w, 1, 1), ws=ws, bias=bias, inv_pc=inv,
                                  add_src=add[idx], add_scale_pc=adds)
    assert np.array_equal(gx[idx], exp_x)
    assert np.array_equal(gb[idx], oracle.bn_prelu_requant(exp_x, in_scale_pc=bsin, bn_scale=bns,
                                                           bn_offset=bno, inv_pc=binv))


# ---- a stride-2 conv and its 1x1 shortcut as one launch ----
S2_PAIRS = [(64, 64, 112, 64), (128, 128, 56, 64), (256, 256, 28, 128)]


def _pair_desc(lib, keep, B, cin, cout, k, s, pad, H, x, w, P, flags, out, out_bn=None, add=None):
    d = fa.ffk_conv_desc()
    d.batch, d.cin, d.cout, d.kh, d.kw = B, cin, cout, k, k
    d.stride, d.pad, d.hin, d.win = s, pad, H, H
    for arr, field in ((x, "in_"), (gpu_util.pack_conv(lib, w), "w"), (P, "params")):
        dv = gpu_util.Dev(lib, host=arr); keep.append(dv)
        setattr(d, field, dv.ptr)
    if flags & fa.FFK_EPI_BN:
        dl = gpu_util.Dev(lib, host=gpu_util.make_bn_lut(lib, P)); keep.append(dl)
        d.bn_lut = dl.ptr
    d.out, d.out_bn, d.add_src = out, out_bn, add
    d.flags = flags
    d.in_scale = 1.0
    return d


@pytest.mark.parametrize("bn", [True, False], ids=["bn", "nobn"])
@pytest.mark.parametrize("fast", [True, False], ids=["inrange", "general"])
@pytest.mark.parametrize("cin,cout,H,cx", S2_PAIRS)
def test_s2_shortcut_pair_equals_two_launches(gpu_lib, cin, cout, H, cx, fast, bn):
    """ffk_conv_s2_shortcut: a block's 3x3 stride-2 conv and the 1x1 shortcut
    whose epilogue adds its output (over the compact block input), as one
    launch, give ffk_conv's X and BN(X) of the two launches bit for bit, at a
    ragged batch of the large-tile kernel, on the in-range and the general
    epilogue forms; forms and batches it does not serve return 0 and launch
    nothing."""
    lib = gpu_lib
    r = rng(1300 + cin + H + cx + 2 * fast + bn)
    B = _direct_batch(lib, cin, cout, 3, 2, H)
    Ho = H // 2
    x = r.integers(-128, 128, size=(B, H, H, cin), dtype=np.int8)
    w = r.integers(-128, 128, size=(cout, cin, 3, 3), dtype=np.int8)
    xc = r.integers(-128, 128, size=(B, Ho, Ho, cx), dtype=np.int8)
    w2 = r.integers(-128, 128, size=(cout, cx, 1, 1), dtype=np.int8)
    x[-1, -1, -1] = -128
    w2[3] = 127
    ws, bias, inv = _unsaturated_params(r, cout, 9 * cin)
    ws[0], bias[0], inv[0] = 0.5, 0.0, 1.0 / 64          # exact .5 ties
    P1 = params_block(cout, ws=ws, bias=bias, inv=inv)
    ws2, bias2, inv2 = _unsaturated_params(r, cout, cx)
    rows2 = dict(ws=ws2, bias=bias2, inv=inv2, adds=r.uniform(1e-3, 5e-2, cout).astype(F32))
    if bn:
        rows2.update(bn_sin=r.uniform(1e-3, 5e-2, cout).astype(F32), bn_s=r.uniform(0.5, 1.5, cout).astype(F32),
                     bn_o=r.normal(0, 0.05, cout).astype(F32), bn_inv=(1.0 / r.uniform(0.01, 0.1, cout)).astype(F32))
    P2 = params_block(cout, **rows2)
    f1 = fa.FFK_EPI_BIAS
    f2 = fa.FFK_EPI_BIAS | fa.FFK_EPI_ADD | (fa.FFK_EPI_BN if bn else 0)
    if fast:
        assert lib.ffk_requant_in_range(P1.ctypes.data, cout, 9 * cin, f1) == 1
        assert lib.ffk_requant_in_range(P2.ctypes.data, cout, cx, f2) == 1
        f1 |= fa.FFK_EPI_IN_RANGE
        f2 |= fa.FFK_EPI_IN_RANGE

    # two launches
    R, _ = run_conv(lib, x, w, 2, 1, params=P1, flags=f1, split=False)
    X_exp, BN_exp = run_conv(lib, xc, w2, 1, 0, params=P2, flags=f2, add=R, want_bn=bn, split=False)

    # one launch
    keep = []
    n = B * Ho * Ho * cout
    dR, dX = gpu_util.Dev(lib, nbytes=n), gpu_util.Dev(lib, nbytes=n)
    dBN = gpu_util.Dev(lib, nbytes=n) if bn else None
    keep += [dR, dX] + ([dBN] if bn else [])
    c = _pair_desc(lib, keep, B, cin, cout, 3, 2, 1, H, x, w, P1, f1, dR.ptr)
    sc = _pair_desc(lib, keep, B, cx, cout, 1, 1, 0, Ho, xc, w2, P2, f2, dX.ptr,
                    out_bn=dBN.ptr if bn else None, add=dR.ptr)
    assert lib.ffk_conv_variant(C.byref(c)) == b"phase"
    gpu_util.check(lib, lib.ffk_zero(dX.ptr, n, None))
    assert lib.ffk_conv_s2_shortcut(C.byref(c), C.byref(sc), None) == 1
    gpu_util.check(lib, lib.ffk_stream_sync(None))
    assert np.array_equal(dX.get(np.int8, (B, Ho, Ho, cout)), X_exp)
    if bn:
        assert np.array_equal(dBN.get(np.int8, (B, Ho, Ho, cout)), BN_exp)

    # not served: the stage-4 pair (two launches measured faster), a PReLU on the conv, a residual other than the conv's
    # output, a batch the large tiles do not take (when the layer has one)
    c.flags = f1 | fa.FFK_EPI_PRELU
    assert lib.ffk_conv_s2_shortcut(C.byref(c), C.byref(sc), None) == 0
    c.flags = f1
    sc.add_src = dX.ptr
    assert lib.ffk_conv_s2_shortcut(C.byref(c), C.byref(sc), None) == 0
    sc.add_src = dR.ptr
    c.batch = sc.batch = 1
    if lib.ffk_conv_variant(C.byref(c)) != b"phase":
        assert lib.ffk_conv_s2_shortcut(C.byref(c), C.byref(sc), None) == 0
    c4 = fa.ffk_conv_desc.from_buffer_copy(c)
    s4 = fa.ffk_conv_desc.from_buffer_copy(sc)
    c4.cin = c4.cout = s4.cout = 512
    c4.hin = c4.win = 14
    s4.cin, s4.hin, s4.win = 256, 7, 7
    c4.batch = s4.batch = 1024
    assert lib.ffk_conv_s2_shortcut(C.byref(c4), C.byref(s4), None) == 0


@pytest.mark.parametrize("cin,cout,H,cx", S2_PAIRS)
def test_s2_shortcut_pair_x_even(gpu_lib, cin, cout, H, cx):
    """The fused stride-2 pair with the shortcut's X stored at its even
    pixels only (FFK_OUT_X_EVEN, a compact [B, Ho/2, Ho/2, Cout] tensor) and
    BN(X) everywhere: X equals the even pixels of the two launches' X, BN(X)
    the two launches' BN(X), bit for bit, at a ragged batch; every X byte
    outside the compact tensor is left alone."""
    lib = gpu_lib
    r = rng(1400 + cin + H)
    B = _direct_batch(lib, cin, cout, 3, 2, H)
    Ho = H // 2
    x = r.integers(-128, 128, size=(B, H, H, cin), dtype=np.int8)
    w = r.integers(-128, 128, size=(cout, cin, 3, 3), dtype=np.int8)
    xc = r.integers(-128, 128, size=(B, Ho, Ho, cx), dtype=np.int8)
    w2 = r.integers(-128, 128, size=(cout, cx, 1, 1), dtype=np.int8)
    ws, bias, inv = _unsaturated_params(r, cout, 9 * cin)
    P1 = params_block(cout, ws=ws, bias=bias, inv=inv)
    ws2, bias2, inv2 = _unsaturated_params(r, cout, cx)
    P2 = params_block(cout, ws=ws2, bias=bias2, inv=inv2, adds=r.uniform(1e-3, 5e-2, cout).astype(F32),
                      bn_sin=r.uniform(1e-3, 5e-2, cout).astype(F32), bn_s=r.uniform(0.5, 1.5, cout).astype(F32),
                      bn_o=r.normal(0, 0.05, cout).astype(F32), bn_inv=(1.0 / r.uniform(0.01, 0.1, cout)).astype(F32))
    f1 = fa.FFK_EPI_BIAS | fa.FFK_EPI_IN_RANGE
    f2 = fa.FFK_EPI_BIAS | fa.FFK_EPI_ADD | fa.FFK_EPI_BN | fa.FFK_EPI_IN_RANGE
    assert lib.ffk_requant_in_range(P1.ctypes.data, cout, 9 * cin, f1) == 1
    assert lib.ffk_requant_in_range(P2.ctypes.data, cout, cx, f2) == 1

    R, _ = run_conv(lib, x, w, 2, 1, params=P1, flags=f1, split=False)
    X_exp, BN_exp = run_conv(lib, xc, w2, 1, 0, params=P2, flags=f2, add=R, want_bn=True, split=False)

    keep = []
    n = B * Ho * Ho * cout
    ne = B * (Ho // 2) * (Ho // 2) * cout
    dR, dBN = gpu_util.Dev(lib, nbytes=n), gpu_util.Dev(lib, nbytes=n)
    guard = np.full(ne + 4096, 0x5A, np.uint8)              # a guard region past the tensor
    dX = gpu_util.Dev(lib, host=guard)
    keep += [dR, dX, dBN]
    c = _pair_desc(lib, keep, B, cin, cout, 3, 2, 1, H, x, w, P1, f1, dR.ptr)
    sc = _pair_desc(lib, keep, B, cx, cout, 1, 1, 0, Ho, xc, w2, P2, f2 | fa.FFK_OUT_X_EVEN, dX.ptr,
                    out_bn=dBN.ptr, add=dR.ptr)
    assert lib.ffk_conv_variant(C.byref(c)) == b"phase"
    assert lib.ffk_conv_s2_shortcut(C.byref(c), C.byref(sc), None) == 1
    gpu_util.check(lib, lib.ffk_stream_sync(None))
    got = dX.get(np.int8, (ne + 4096,))
    assert np.array_equal(got[:ne].reshape(B, Ho // 2, Ho // 2, cout), X_exp[:, ::2, ::2, :])
    assert (got[ne:].view(np.uint8) == 0x5A).all()
    assert np.array_equal(dBN.get(np.int8, (B, Ho, Ho, cout)), BN_exp)


# ---- FFK_EPI_FMA_TAIL: the requant's last two roundings as one fma ----
FMA_MODES = ["none", "prelu_le1", "prelu_bn_le1", "bn_only"]


@pytest.mark.parametrize("split", [True, False, "direct"], ids=["splitk", "wholek", "direct"])
@pytest.mark.parametrize("mode", FMA_MODES)
@pytest.mark.parametrize("cin,cout,k,s,H", EPI_SHAPES)
def test_fma_tail_epilogue(gpu_lib, oracle, mode, cin, cout, k, s, H, split):
    """With parameters the host proof accepts (ffk_requant_fma_ok), the
    one-rounding tail gives the oracle's int8 values on every kernel variant,
    exact .5 ties and negative zero included."""
    if split is True and (cin, cout, k, s, H) not in SPLIT_SHAPES:
        pytest.skip("no split-K variant for this geometry")
    r = rng(1550 + cin + cout + H + FMA_MODES.index(mode))
    rp = rng(1510 + cin + cout + H + FMA_MODES.index(mode))   # parameters: the same for every batch
    if split == "direct":
        B = _direct_batch(gpu_lib, cin, cout, k, s, H)
        idx = sorted({0, B // 2, B - 1})
        split = False
    else:
        B = 1 if split else 2
        idx = list(range(B))
    x = r.integers(-128, 128, size=(B, H, H, cin), dtype=np.int8)
    w = r.integers(-128, 128, size=(cout, cin, k, k), dtype=np.int8)
    ws, bias, inv = _unsaturated_params(rp, cout, k * k * cin)
    ws[0], bias[0], inv[0] = 0.5, 0.0, 1.0 / 64        # exact .5 ties after scaling
    ws[4], bias[4] = -1e-3, -0.0
    rows = dict(ws=ws, bias=bias, inv=inv)
    ekw = dict(ws=ws, bias=bias, inv_pc=inv)
    flags = fa.FFK_EPI_BIAS
    if "prelu" in mode:
        slope = rp.uniform(0.05, 0.3, cout).astype(F32)
        slope[7:9] = [1.0, 0.0]
        rows["slope"] = slope; ekw["prelu"] = slope
        flags |= fa.FFK_EPI_PRELU | fa.FFK_EPI_PRELU_LE1
    bn = "bn" in mode
    if bn:
        bsin = r.uniform(1e-3, 5e-2, cout).astype(F32)
        bns = r.uniform(0.5, 1.5, cout).astype(F32)
        bno = r.normal(0, 0.05, cout).astype(F32)
        binv = (1.0 / r.uniform(0.01, 0.1, cout)).astype(F32)
        rows.update(bn_sin=bsin, bn_s=bns, bn_o=bno, bn_inv=binv)
        flags |= fa.FFK_EPI_BN
    P = params_block(cout, **rows)
    assert gpu_lib.ffk_requant_fma_ok(P.ctypes.data, cout, k * k * cin, flags) == 1
    got_x, got_bn = run_conv(gpu_lib, x, w, s, k // 2, params=P,
                             flags=flags | fa.FFK_EPI_IN_RANGE | fa.FFK_EPI_FMA_TAIL, want_bn=bn, split=split)
    exp_x = oracle.fused_epilogue(oracle.conv_i32(x[idx], w, s, k // 2), **ekw)
    assert 0.05 < np.mean(np.abs(exp_x) < 127)
    assert np.array_equal(got_x[idx], exp_x)
    if bn:
        exp_bn = oracle.bn_prelu_requant(exp_x, in_scale_pc=bsin, bn_scale=bns, bn_offset=bno, inv_pc=binv)
        assert np.array_equal(got_bn[idx], exp_bn)


def test_fma_tail_window_is_real(gpu_lib, oracle):
    """Where the proof rejects, the flag would change results: channel 0 of a
    1x1 layer has accumulators -1, 0 and 1 and a weight scale and inv that put
    f*inv inside the one window where the two tails differ.  Without the flag
    the kernel gives the reference's -1 / 0 / 1, with it (forced, against the
    proof) 0 / 0 / 0; every other channel is unaffected."""
    lib = gpu_lib
    r = rng(1600)
    B, H, C_ = 1, 56, 64
    x = r.integers(-3, 4, size=(B, H, H, C_), dtype=np.int8)
    x[..., 0] = r.integers(-1, 2, size=(B, H, H), dtype=np.int8)
    w = r.integers(-2, 3, size=(C_, C_, 1, 1), dtype=np.int8)
    w[0] = 0
    w[0, 0] = 1                                          # channel 0: acc = x[..., 0]
    ws = r.uniform(1e-2, 5e-2, C_).astype(F32)
    inv = r.uniform(5, 20, C_).astype(F32)
    bias = r.normal(0, 0.1, C_).astype(F32)
    ws[0], inv[0], bias[0] = 0.1515151411294937, 3.3, 0.0
    P = params_block(C_, ws=ws, bias=bias, inv=inv)
    flags = fa.FFK_EPI_BIAS
    assert lib.ffk_requant_fma_ok(P.ctypes.data, C_, C_, flags) == 0
    exp = oracle.fused_epilogue(oracle.conv_i32(x, w, 1, 0), ws=ws, bias=bias, inv_pc=inv)
    assert set(np.unique(exp[..., 0])) == {-1, 0, 1}
    plain, _ = run_conv(lib, x, w, 1, 0, params=P, flags=flags | fa.FFK_EPI_IN_RANGE, split=False)
    forced, _ = run_conv(lib, x, w, 1, 0, params=P, flags=flags | fa.FFK_EPI_IN_RANGE | fa.FFK_EPI_FMA_TAIL,
                         split=False)
    assert np.array_equal(plain, exp)
    assert (forced[..., 0] == 0).all()
    assert np.array_equal(forced[..., 1:], exp[..., 1:])


MAP_CASES = [  # (C, pixels, bn, prelu): ragged pixel counts, and more passes than the grid has workgroups
    (64, 1, True, False), (128, 37, False, True), (256, 1001, True, True), (512, 49, False, False),
    (64, 3 * 2048 * 64 + 5, True, True),
]


@pytest.mark.parametrize("C_,pix,bn,prelu", MAP_CASES)
def test_standalone_map_kernel(gpu_lib, oracle, C_, pix, bn, prelu):
    """A stand-alone BN / PReLU through its per-channel table on the device
    equals the oracle's bn_prelu_requant (itself pinned to the reference's
    bn_prelu_requant_int8) on every element, special parameters included."""
    lib = gpu_lib
    r = rng(1700 + C_ + pix)
    x = r.integers(-128, 128, size=(pix, C_), dtype=np.int8)
    x[0, :] = np.arange(C_) % 256 - 128                  # every value in some channel
    s_in = r.uniform(1e-3, 5e-2, C_).astype(F32)
    bns = r.uniform(0.5, 1.5, C_).astype(F32)
    bno = r.normal(0, 0.05, C_).astype(F32)
    slope = r.uniform(0.0, 0.3, C_).astype(F32)
    inv = (1.0 / r.uniform(0.01, 0.1, C_)).astype(F32)
    s_in[0], bns[1], slope[2], inv[3], bno[4] = np.float32(3e-45), np.nan, -0.5, 3e38, -0.0
    lut = np.empty((C_, 256), np.int8)
    gpu_util.check(lib, lib.ffk_make_map_lut(s_in.ctypes.data, bns.ctypes.data if bn else None,
                                             bno.ctypes.data if bn else None,
                                             slope.ctypes.data if prelu else None, inv.ctypes.data,
                                             C_, lut.ctypes.data))
    d_in, d_lut = gpu_util.Dev(lib, host=x), gpu_util.Dev(lib, host=lut)
    d_out = gpu_util.Dev(lib, nbytes=x.nbytes)
    gpu_util.check(lib, lib.ffk_map_i8(d_in.ptr, d_out.ptr, pix, C_, d_lut.ptr, None))
    gpu_util.check(lib, lib.ffk_stream_sync(None))
    got = d_out.get(np.int8, x.shape)
    exp = oracle.bn_prelu_requant(x, in_scale_pc=s_in, bn_scale=bns if bn else None,
                                  bn_offset=bno if bn else None, prelu=slope if prelu else None,
                                  inv_pc=inv)
    assert np.array_equal(got, exp)


@pytest.mark.parametrize("n,scales", [(16, (0.013, 0.021, 0.03)), (65536 * 16, (0.5, 0.5, 1.0)),
                                      (4 * 1024 * 256 * 16 + 48, (3e38, 3e38, 1e-30))])
def test_standalone_add_kernel(gpu_lib, oracle, n, scales):
    """A stand-alone Add through its pair table on the device equals the
    oracle's add_requant (pinned to the reference's add_requant_int8); the
    largest case takes more passes than the grid has workgroups."""
    lib = gpu_lib
    r = rng(1800 + n)
    a = r.integers(-128, 128, size=n, dtype=np.int8)
    b = r.integers(-128, 128, size=n, dtype=np.int8)
    if n >= 65536:                                       # every pair once
        a[:65536] = np.repeat(np.arange(-128, 128, dtype=np.int8), 256)
        b[:65536] = np.tile(np.arange(-128, 128, dtype=np.int8), 256)
    lut = np.empty(65536, np.int8)
    gpu_util.check(lib, lib.ffk_make_add_lut(*scales, lut.ctypes.data))
    da, db, dl = gpu_util.Dev(lib, host=a), gpu_util.Dev(lib, host=b), gpu_util.Dev(lib, host=lut)
    do = gpu_util.Dev(lib, nbytes=n)
    gpu_util.check(lib, lib.ffk_add_i8(da.ptr, db.ptr, do.ptr, n, dl.ptr, None))
    gpu_util.check(lib, lib.ffk_stream_sync(None))
    assert np.array_equal(do.get(np.int8, n), oracle.add_requant(a, scales[0], b, scales[1], scales[2]))


GENERIC_CASES = [  # (cin, cout, kh, kw, stride, pad, H, W, B): no tuned kernel for any of them
    (96, 64, 3, 3, 1, 1, 15, 13, 2),      # channel count, non-square image
    (64, 64, 3, 3, 1, 0, 9, 9, 3),        # no padding
    (17, 40, 5, 5, 2, 2, 23, 23, 2),      # odd channels, 5x5 stride 2, a partial channel tile
    (256, 130, 1, 1, 1, 0, 7, 7, 5),      # 1x1, ragged output channels
    (64, 72, 7, 1, 1, 3, 12, 12, 1),      # 7x1 kernel
    (128, 64, 3, 3, 3, 1, 20, 20, 3),     # stride 3
]


def _generic_variant(lib, cin, cout, kh, kw, s, pad, H, W, B):
    d = fa.ffk_conv_desc()
    d.batch, d.cin, d.cout, d.kh, d.kw = B, cin, cout, kh, kw
    d.stride, d.pad, d.hin, d.win = s, pad, H, W
    return lib.ffk_conv_variant(C.byref(d))


@pytest.mark.parametrize("cin,cout,kh,kw,s,pad,H,W,B", GENERIC_CASES)
def test_generic_conv_int32_accumulators(gpu_lib, oracle, cin, cout, kh, kw, s, pad, H, W, B):
    """A geometry without a tuned kernel runs on the generic implicit GEMM:
    int32 accumulators equal the oracle's convolution (pinned to brute force
    on these shapes), extreme values included."""
    assert _generic_variant(gpu_lib, cin, cout, kh, kw, s, pad, H, W, B) == b"generic"
    r = rng(1900 + cin + cout + kh * 7 + kw + s)
    x = r.integers(-128, 128, size=(B, H, W, cin), dtype=np.int8)
    w = r.integers(-128, 128, size=(cout, cin, kh, kw), dtype=np.int8)
    x[0, 0] = -128
    w[0] = -128
    got = run_conv(gpu_lib, x, w, s, pad, raw=True)
    assert np.array_equal(got, oracle.conv_i32(x, w, s, pad))


@pytest.mark.parametrize("mode", ["prelu", "add_bn", "prelu_bn_even", "inscale_prelu_le1"])
@pytest.mark.parametrize("case", [0, 2, 3])
def test_generic_conv_epilogue(gpu_lib, oracle, mode, case):
    """The generic kernel's epilogue (the tuned kernels' general form per
    element: in-scale, ws, bias, residual, PReLU, round half away with the
    x86 out-of-range case; X at even pixels; BN(X) through the table) equals
    the oracle's fused epilogue and BN requant, special parameters included.
    The shorter-form flags change nothing there."""
    cin, cout, kh, kw, s, pad, H, W, B = GENERIC_CASES[case]
    r = rng(2000 + case * 10 + len(mode))
    x = r.integers(-128, 128, size=(B, H, W, cin), dtype=np.int8)
    w = r.integers(-128, 128, size=(cout, cin, kh, kw), dtype=np.int8)
    Ho, Wo = (H + 2 * pad - kh) // s + 1, (W + 2 * pad - kw) // s + 1
    ws, bias, inv = _special_params(r, cout)
    rows = dict(ws=ws, bias=bias, inv=inv)
    ekw = dict(ws=ws, bias=bias, inv_pc=inv)
    flags = fa.FFK_EPI_BIAS
    add = None
    in_scale = 1.0
    if "prelu" in mode:
        slope = r.uniform(0, 0.3, cout).astype(F32)
        slope[7] = -0.5
        rows["slope"] = slope; ekw["prelu"] = slope; flags |= fa.FFK_EPI_PRELU
    if "le1" in mode:
        flags |= fa.FFK_EPI_PRELU_LE1 | fa.FFK_EPI_IN_RANGE
    if "inscale" in mode:
        in_scale = 0.0173
        ekw["in_scale"] = in_scale; flags |= fa.FFK_EPI_INSCALE
    if "add" in mode:
        add = r.integers(-128, 128, size=(B, Ho, Wo, cout), dtype=np.int8)
        adds = r.uniform(1e-3, 5e-2, cout).astype(F32)
        rows["adds"] = adds; ekw.update(add_src=add, add_scale_pc=adds); flags |= fa.FFK_EPI_ADD
    want_bn = "bn" in mode
    if want_bn:
        bsin = r.uniform(1e-3, 5e-2, cout).astype(F32)
        bns = r.uniform(0.5, 1.5, cout).astype(F32)
        bno = r.normal(0, 0.05, cout).astype(F32)
        binv = (1.0 / r.uniform(0.01, 0.1, cout)).astype(F32)
        rows.update(bn_sin=bsin, bn_s=bns, bn_o=bno, bn_inv=binv)
        flags |= fa.FFK_EPI_BN
    x_even = "even" in mode and Ho % 2 == 0 and Wo % 2 == 0
    exp_x = oracle.fused_epilogue(oracle.conv_i32(x, w, s, pad), **ekw)
    got_x, got_bn = run_conv(gpu_lib, x, w, s, pad, params=params_block(cout, **rows), flags=flags,
                             add=add, want_bn=want_bn, in_scale=in_scale, x_even=x_even)
    assert np.array_equal(got_x, exp_x[:, ::2, ::2] if x_even else exp_x)
    if want_bn:
        exp_bn = oracle.bn_prelu_requant(exp_x, in_scale_pc=bsin, bn_scale=bns, bn_offset=bno, inv_pc=binv)
        assert np.array_equal(got_bn, exp_bn)


GENERIC_WIDE_CASES = [  # batches large enough for 128-pixel tiles (at least 256 workgroups)
    (96, 72, 3, 3, 1, 1, 28, 28, 48),     # 128x128 tiles, 16-byte channel runs, ragged channels
    (40, 64, 3, 3, 1, 1, 28, 28, 48),     # 128x64 tiles, 8-byte channel runs
]


@pytest.mark.parametrize("case", range(len(GENERIC_WIDE_CASES)))
def test_generic_conv_wide_tiles(gpu_lib, oracle, case):
    """The generic kernel's 128-wide tiles: int32 accumulators and the fused
    PReLU + residual + BN epilogue equal the oracle's."""
    cin, cout, kh, kw, s, pad, H, W, B = GENERIC_WIDE_CASES[case]
    assert _generic_variant(gpu_lib, cin, cout, kh, kw, s, pad, H, W, B) == b"generic"
    r = rng(2150 + case)
    x = r.integers(-128, 128, size=(B, H, W, cin), dtype=np.int8)
    w = r.integers(-128, 128, size=(cout, cin, kh, kw), dtype=np.int8)
    acc = oracle.conv_i32(x, w, s, pad)
    assert np.array_equal(run_conv(gpu_lib, x, w, s, pad, raw=True), acc)
    Ho, Wo = (H + 2 * pad - kh) // s + 1, (W + 2 * pad - kw) // s + 1
    ws = r.uniform(1e-4, 1e-3, cout).astype(F32)
    bias = r.normal(0, 0.1, cout).astype(F32)
    inv = (1.0 / r.uniform(0.01, 0.05, cout)).astype(F32)
    slope = r.uniform(0, 0.3, cout).astype(F32)
    add = r.integers(-128, 128, size=(B, Ho, Wo, cout), dtype=np.int8)
    adds = r.uniform(1e-3, 5e-2, cout).astype(F32)
    bsin = r.uniform(1e-3, 5e-2, cout).astype(F32)
    bns = r.uniform(0.5, 1.5, cout).astype(F32)
    bno = r.normal(0, 0.05, cout).astype(F32)
    binv = (1.0 / r.uniform(0.01, 0.1, cout)).astype(F32)
    flags = fa.FFK_EPI_BIAS | fa.FFK_EPI_PRELU | fa.FFK_EPI_ADD | fa.FFK_EPI_BN
    prm = params_block(cout, ws=ws, bias=bias, inv=inv, slope=slope, adds=adds, bn_sin=bsin, bn_s=bns, bn_o=bno,
                       bn_inv=binv)
    got_x, got_bn = run_conv(gpu_lib, x, w, s, pad, params=prm, flags=flags, add=add, want_bn=True)
    exp_x = oracle.fused_epilogue(acc, ws=ws, bias=bias, inv_pc=inv, prelu=slope, add_src=add, add_scale_pc=adds)
    assert np.array_equal(got_x, exp_x)
    assert np.array_equal(got_bn, oracle.bn_prelu_requant(exp_x, in_scale_pc=bsin, bn_scale=bns, bn_offset=bno,
                                                          inv_pc=binv))


SLICE_CASES = [  # (kind, cin, cout, kh, kw, stride, pad, H, W): images per 2 GiB launch slice
    ("tuned", 64, 64, 3, 3, 1, 1, 56, 56),          # 200,704 bytes per image: 10,699 per slice
    ("generic", 16, 16, 1, 1, 1, 0, 512, 512),      # 4 MiB per image: 511 per slice
]


@pytest.mark.parametrize("case", SLICE_CASES, ids=[c[0] for c in SLICE_CASES])
def test_conv_batch_slices_at_2gib(gpu_lib, oracle, case):
    """A batch whose int8 tensors reach 2 GiB runs as several launches over
    consecutive image ranges (32-bit buffer offsets): the images at both ends
    and on both sides of the slice boundary, with a residual input and the BN
    second output, equal the oracle's."""
    kind, cin, cout, kh, kw, s, pad, H, W = case
    Ho, Wo = (H + 2 * pad - kh) // s + 1, (W + 2 * pad - kw) // s + 1
    img = max(H * W * cin, Ho * Wo * cout)
    per = 0x7FFFFFFF // img                                # images per launch slice
    B = per + 2
    r = rng(2300 + cin)
    block = r.integers(-128, 128, size=(4, H, W, cin), dtype=np.int8)
    x = np.empty((B, H, W, cin), np.int8)
    for i in range(0, B, 4):
        x[i:i + 4] = block[:min(4, B - i)]
    add = np.empty((B, Ho, Wo, cout), np.int8)
    ablock = r.integers(-128, 128, size=(4, Ho, Wo, cout), dtype=np.int8)
    for i in range(0, B, 4):
        add[i:i + 4] = ablock[:min(4, B - i)]
    picks = [0, per - 1, per, B - 1]
    for i in picks[1:]:                                  # fresh content around the boundary
        x[i] = r.integers(-128, 128, size=(H, W, cin), dtype=np.int8)
        add[i] = r.integers(-128, 128, size=(Ho, Wo, cout), dtype=np.int8)
    w = r.integers(-128, 128, size=(cout, cin, kh, kw), dtype=np.int8)
    d = fa.ffk_conv_desc()
    d.batch, d.cin, d.cout, d.kh, d.kw = B, cin, cout, kh, kw
    d.stride, d.pad, d.hin, d.win = s, pad, H, W
    assert (gpu_lib.ffk_conv_variant(C.byref(d)) == b"generic") == (kind == "generic")
    ws = r.uniform(1e-4, 1e-3, cout).astype(F32)
    bias = r.normal(0, 0.1, cout).astype(F32)
    inv = (1.0 / r.uniform(0.01, 0.05, cout)).astype(F32)
    slope = r.uniform(0, 0.3, cout).astype(F32)
    adds = r.uniform(1e-3, 5e-2, cout).astype(F32)
    bsin = r.uniform(1e-3, 5e-2, cout).astype(F32)
    bns = r.uniform(0.5, 1.5, cout).astype(F32)
    bno = r.normal(0, 0.05, cout).astype(F32)
    binv = (1.0 / r.uniform(0.01, 0.1, cout)).astype(F32)
    flags = fa.FFK_EPI_BIAS | fa.FFK_EPI_PRELU | fa.FFK_EPI_ADD | fa.FFK_EPI_BN
    prm = params_block(cout, ws=ws, bias=bias, inv=inv, slope=slope, adds=adds, bn_sin=bsin, bn_s=bns, bn_o=bno,
                       bn_inv=binv)
    got_x, got_bn = run_conv(gpu_lib, x, w, s, pad, params=prm, flags=flags, add=add, want_bn=True, split=False)
    xs = x[picks]
    acc = oracle.conv_i32(xs, w, s, pad)
    exp_x = oracle.fused_epilogue(acc, ws=ws, bias=bias, inv_pc=inv, prelu=slope, add_src=add[picks],
                                  add_scale_pc=adds)
    assert np.array_equal(got_x[picks], exp_x)
    assert np.array_equal(got_bn[picks], oracle.bn_prelu_requant(exp_x, in_scale_pc=bsin, bn_scale=bns,
                                                                 bn_offset=bno, inv_pc=binv))


@pytest.mark.parametrize("rgb8", [False, True], ids=["fp32", "rgb8"])
def test_generic_input_layer(gpu_lib, oracle, rgb8):
    """A 3-channel input layer without a tuned kernel (5x5 stride 2, 32
    channels): the faces are quantized on load (fp32, the reference's
    lrintf semantics incl. ties and out-of-range values) or mapped through
    the uint8 table, then the same int32 accumulators as the oracle's."""
    r = rng(2100)
    B = 2
    w = r.integers(-128, 128, size=(32, 3, 5, 5), dtype=np.int8)
    inv = np.array([127.0, 126.9, 127.3], F32)
    if rgb8:
        imgs = r.integers(0, 256, size=(B, 112, 112, 3), dtype=np.uint8)
        lut = np.empty((3, 256), np.int8)
        assert gpu_lib.ffk_make_rgb8_lut(inv.ctypes.data, lut.ctypes.data) == 0
        got = run_conv(gpu_lib, imgs, w, 2, 2, raw=True, in_lut=lut, flags=fa.FFK_IN_RGB8)
        q = oracle.quant_input((imgs.astype(F32) - 127.5) / 127.5, inv)
    else:
        x = r.uniform(-1, 1, size=(B, 112, 112, 3)).astype(F32)
        x[0, 0, :4, 0] = [0.5 / 127, 1.5 / 127, 1e10, np.nan]
        x[0, 1, :2, 1] = [-2.5 / 126.9, np.inf]
        got = run_conv(gpu_lib, x, w, 2, 2, raw=True, in_inv=inv)
        q = oracle.quant_input(x, inv)
    assert np.array_equal(got, oracle.conv_i32(q, w, 2, 2))
