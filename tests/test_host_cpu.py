"""Host-side checks that need no GPU: the C ABI library loads and exports
every entry point the headers declare, weight packing, plan coverage."""
import ctypes as C
import os
import re

import numpy as np
import pytest

import fastface_amd as fa
from fastface_amd import synth

INCLUDE = os.path.join(fa.REPO_ROOT, "include")


def _declared_functions():
    names = set()
    for h in os.listdir(INCLUDE):
        if not h.endswith(".h"):
            continue
        src = open(os.path.join(INCLUDE, h)).read()
        src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
        for m in re.finditer(r"\b((?:fastface|ffk)_[a-z0-9_]+)\s*\(", src):
            names.add(m.group(1))
    return names


def test_library_exports_every_declared_symbol():
    lib = fa.load()
    declared = _declared_functions()
    assert len(declared) >= 35
    missing = [n for n in declared if not hasattr(lib, n)]
    assert not missing, missing
    bound = {n for n, _, _ in fa.EXPORTS}
    assert declared == bound, declared ^ bound


def test_conv_weight_packing_layout():
    lib = fa.load()
    r = np.random.default_rng(0)
    for cout, cin, k in [(64, 3, 3), (128, 64, 3), (256, 128, 1)]:
        w = r.integers(-128, 128, size=(cout, cin, k, k), dtype=np.int8)
        n = lib.ffk_conv_packed_bytes(cin, cout, k, k)
        packed = np.empty(n, np.int8)
        assert lib.ffk_pack_conv_weights(w.ctypes.data, cout, cin, k, k, packed.ctypes.data) == 0
        ktot = k * k * cin
        steps = -(-ktot // 64)
        assert n == steps * cout * 64
        # reduction index k = (kh*KW + kw)*Cin + ci, zero padded to 64-steps
        wk = np.zeros((cout, steps * 64), np.int8)
        wk[:, :ktot] = w.transpose(0, 2, 3, 1).reshape(cout, ktot)
        exp = wk.reshape(cout, steps, 64).transpose(1, 0, 2).reshape(-1)
        assert np.array_equal(packed, exp)


def test_fc_weight_packing_layout():
    lib = fa.load()
    r = np.random.default_rng(1)
    W = r.integers(-128, 128, size=(8, 256), dtype=np.int8)
    packed = np.empty(lib.ffk_fc_packed_bytes(8, 256), np.int8)
    assert lib.ffk_pack_fc_weights(W.ctypes.data, 8, 256, packed.ctypes.data) == 0
    assert np.array_equal(packed, W.reshape(8, 4, 64).transpose(1, 0, 2).reshape(-1))
    assert lib.ffk_pack_fc_weights(W.ctypes.data, 8, 100, packed.ctypes.data) != 0


def test_bn_table_matches_oracle_bn_requant(oracle):
    """The BN second output is a table over the 256 int8 values; every entry
    equals the (reference-pinned) BN requant of that value."""
    lib = fa.load()
    r = np.random.default_rng(3)
    C_ = 96
    s_in = r.uniform(1e-3, 5e-2, C_).astype(np.float32)
    s_in[0], s_in[1] = np.float32(3e-45), np.float32(1.2e-38)      # denormal / tiny
    bns = r.uniform(0.5, 1.5, C_).astype(np.float32)
    bns[2] = np.nan
    bno = r.normal(0, 0.05, C_).astype(np.float32)
    bno[3] = -0.0
    inv = (1.0 / r.uniform(0.01, 0.1, C_)).astype(np.float32)
    inv[4], inv[5] = 1e9, 3e38
    lut = np.empty((C_, 256), np.int8)
    assert lib.ffk_make_bn_lut(s_in.ctypes.data, bns.ctypes.data, bno.ctypes.data,
                               inv.ctypes.data, C_, lut.ctypes.data) == 0
    q = np.arange(-128, 128, dtype=np.int8).reshape(256, 1).repeat(C_, axis=1)
    exp = oracle.bn_prelu_requant(q, in_scale_pc=s_in, bn_scale=bns, bn_offset=bno, inv_pc=inv)
    assert np.array_equal(lut.T, exp)


def _map_params(r, C_):
    """Per-channel parameters of a stand-alone BN / PReLU with the delicate
    values: denormal and tiny scales, NaN, -0, huge inverses, negative and
    > 1 slopes, exact .5 ties (q * 0.5 * 1.0)."""
    s_in = r.uniform(1e-3, 5e-2, C_).astype(np.float32)
    s_in[0], s_in[1], s_in[8] = np.float32(3e-45), np.float32(1.2e-38), 0.5
    bns = r.uniform(0.5, 1.5, C_).astype(np.float32)
    bns[2], bns[8] = np.nan, 1.0
    bno = r.normal(0, 0.05, C_).astype(np.float32)
    bno[3], bno[8] = -0.0, 0.0
    slope = r.uniform(0.0, 0.3, C_).astype(np.float32)
    slope[4], slope[5], slope[6], slope[8] = -0.7, 2.5, np.nan, 1.0
    inv = (1.0 / r.uniform(0.01, 0.1, C_)).astype(np.float32)
    inv[4], inv[5], inv[7], inv[8] = 1e9, 3e38, 1e30, 1.0
    return s_in, bns, bno, slope, inv


MAP_FORMS = [(True, False), (False, True), (True, True), (False, False)]   # (bn, prelu)


def _make_map_lut(lib, s_in, bns, bno, slope, inv, bn, prelu):
    C_ = s_in.size
    lut = np.empty((C_, 256), np.int8)
    assert lib.ffk_make_map_lut(s_in.ctypes.data, bns.ctypes.data if bn else None,
                                bno.ctypes.data if bn else None, slope.ctypes.data if prelu else None,
                                inv.ctypes.data, C_, lut.ctypes.data) == 0
    return lut


@pytest.mark.parametrize("bn,prelu", MAP_FORMS)
def test_map_table_matches_oracle(oracle, bn, prelu):
    """A stand-alone BN / PReLU is a per-channel table over the 256 int8
    values: every entry equals the oracle's bn_prelu_requant of that value."""
    lib = fa.load()
    C_ = 72
    s_in, bns, bno, slope, inv = _map_params(np.random.default_rng(31), C_)
    lut = _make_map_lut(lib, s_in, bns, bno, slope, inv, bn, prelu)
    q = np.arange(-128, 128, dtype=np.int8).reshape(256, 1).repeat(C_, axis=1)
    exp = oracle.bn_prelu_requant(q, in_scale_pc=s_in, bn_scale=bns if bn else None,
                                  bn_offset=bno if bn else None, prelu=slope if prelu else None,
                                  inv_pc=inv)
    assert np.array_equal(lut.T, exp)
    assert lib.ffk_make_map_lut(s_in.ctypes.data, bns.ctypes.data, None, None, inv.ctypes.data,
                                C_, lut.ctypes.data) != 0


@pytest.mark.parametrize("bn,prelu", MAP_FORMS)
@pytest.mark.parametrize("per_channel", [True, False])
def test_map_table_matches_reference(ref, bn, prelu, per_channel):
    """The same tables against the reference's own bn_prelu_requant_int8,
    with per-channel scales and with the scalar in-scale and 1/(s + 1e-9f)
    inverse the reference falls back to (libfastface.c:401-424)."""
    lib = fa.load()
    C_ = 72
    s_in, bns, bno, slope, inv = _map_params(np.random.default_rng(32), C_)
    kw = dict(bn_scale=bns if bn else None, bn_offset=bno if bn else None,
              prelu=slope if prelu else None)
    if per_channel:
        kw.update(in_scale_pc=s_in, inv_pc=inv)
    else:
        s, out_s = np.float32(0.0213), np.float32(0.0371)
        s_in = np.full(C_, s, np.float32)
        inv = np.full(C_, np.float32(1.0) / (out_s + np.float32(1e-9)), np.float32)
        kw.update(in_scale=float(s), out_scale=float(out_s))
    lut = _make_map_lut(lib, s_in, bns, bno, slope, inv, bn, prelu)
    q = np.arange(-128, 128, dtype=np.int8).reshape(256, 1).repeat(C_, axis=1)
    assert np.array_equal(lut.T, ref.bn_prelu_requant(q, **kw))


ADD_SCALES = [  # (a_scale, b_scale, out_scale)
    (0.013, 0.021, 0.03),            # the residual sum's usual range
    (0.5, 0.5, 1.0),                 # exact halves: round-half-even ties
    (1.0, -1.0, 0.5),                # saturation both ways
    (3e38, 3e38, 1e-30),             # inf and NaN sums, then lrintf's out-of-range long
    (2.0 ** 20, 1.0, 2.0 ** -12),    # values in [2^31, 2^63): the int cast keeps 32 bits
    (np.nan, 0.01, 0.02),
    (1e-40, -2e-39, 1e-38),          # denormal scales
]


def _add_table(lib, sa, sb, so):
    lut = np.empty(65536, np.int8)
    assert lib.ffk_make_add_lut(sa, sb, so, lut.ctypes.data) == 0
    return lut.reshape(256, 256)


def _all_pairs():
    v = np.arange(-128, 128, dtype=np.int8)
    return np.repeat(v, 256), np.tile(v, 256)


@pytest.mark.parametrize("sa,sb,so", ADD_SCALES)
def test_add_table_matches_oracle(oracle, sa, sb, so):
    """A stand-alone Add is one 256 x 256 table (its scales are per tensor):
    every entry equals the oracle's add_requant of that pair."""
    lib = fa.load()
    a, b = _all_pairs()
    exp = oracle.add_requant(a, sa, b, sb, so).reshape(256, 256)
    assert np.array_equal(_add_table(lib, sa, sb, so), exp)


@pytest.mark.parametrize("sa,sb,so", ADD_SCALES)
def test_add_table_matches_reference(ref, sa, sb, so):
    lib = fa.load()
    a, b = _all_pairs()
    exp = ref.add_requant(a, sa, b, sb, so).reshape(256, 256)
    assert np.array_equal(_add_table(lib, sa, sb, so), exp)


def test_eltwise_launch_argument_checks():
    """The launchers reject what their kernels assume away, before touching
    the device (pointers are never dereferenced on these paths)."""
    lib = fa.load()
    p = C.c_void_p(4096)
    assert lib.ffk_map_i8(p, p, 10, 96, p, None) == -1           # channels not a multiple of 64
    assert lib.ffk_map_i8(C.c_void_p(4100), p, 10, 64, p, None) == -1   # misaligned
    assert lib.ffk_map_i8(None, p, 10, 64, p, None) == -1
    assert lib.ffk_add_i8(p, p, p, 24, p, None) == -1            # not a multiple of 16 bytes
    assert lib.ffk_add_i8(p, C.c_void_p(4104), p, 32, p, None) == -1
    assert lib.ffk_map_i8(p, p, 0, 64, p, None) == 0             # nothing to do
    assert lib.ffk_add_i8(p, p, p, 0, p, None) == 0


def test_every_iresnet_conv_has_a_kernel():
    lib = fa.load()
    H = 112
    seen = 0
    cur = (3, 112)
    blk = cur
    ops = synth.iresnet_schedule()
    for i, op in enumerate(ops):
        if op["type"] == synth.OP_CONV:
            src = blk if (i > 0 and ops[i - 1]["type"] == synth.OP_SAVE_ID) else cur
            assert lib.ffk_conv_supported(op["Cin"], op["Cout"], op["k"], op["k"], op["s"],
                                          op["p"], src[1], src[1]) == 1, op
            cur = (op["Cout"], (src[1] + 2 * op["p"] - op["k"]) // op["s"] + 1)
            seen += 1
        elif op["type"] == synth.OP_BLOCK_START:
            blk = cur
    assert seen == 53
    # the 1x1 shortcuts over a block input stored at its even pixels (stride 1)
    for cin, cout, hc in [(64, 64, 56), (64, 128, 28), (128, 256, 14), (256, 512, 7)]:
        assert lib.ffk_conv_supported(cin, cout, 1, 1, 1, 0, hc, hc) == 1
    assert lib.ffk_conv_supported(64, 64, 3, 3, 1, 0, H, H) == 0      # pad must be k/2
    assert lib.ffk_conv_supported(96, 64, 3, 3, 1, 1, H, H) == 0


def test_create_without_gpu_returns_null(synth_ffw4):
    lib = fa.load()
    if lib.ffk_device_count() > 0:
        pytest.skip("a GPU is visible")
    old = os.getcwd()
    os.chdir(fa.REPO_ROOT)
    try:
        assert lib.fastface_create(synth_ffw4.encode()) is None
    finally:
        os.chdir(old)


def test_split_workspace_only_for_small_batches():
    """Small batches of the 3x3 layers take the split-K path (a workspace is
    asked for); large batches and the stem never do."""
    lib = fa.load()
    d = fa.ffk_conv_desc()

    def need(cin, cout, k, s, H, B):
        d.batch, d.cin, d.cout, d.kh, d.kw = B, cin, cout, k, k
        d.stride, d.pad, d.hin, d.win = s, k // 2, H, H
        return lib.ffk_conv_workspace_bytes(C.byref(d))
    for cin, cout, s, H in [(128, 128, 2, 56), (128, 128, 1, 28), (128, 256, 1, 28),
                            (256, 256, 2, 28), (256, 256, 1, 14), (256, 512, 1, 14),
                            (512, 512, 1, 7), (512, 512, 2, 14)]:
        n = need(cin, cout, 3, s, H, 1)
        ho = (H - 1) // s + 1
        tiles = -(-ho * ho // 64) * (cout // 64)
        assert n > tiles * 64 * 64 * 4, (cin, cout, s, H)
        assert need(cin, cout, 3, s, H, 64) == 0
        assert need(cin, cout, 3, s, H, 1024) == 0
    assert need(3, 64, 3, 1, 112, 1) == 0
    assert need(64, 64, 3, 1, 56, 1) == 0             # short K chains never split
    assert need(64, 128, 3, 1, 56, 1) == 0
    assert need(64, 64, 1, 2, 112, 1) == 0            # 1x1: one K stage, nothing to split
    assert need(96, 64, 3, 1, 112, 1) == 0            # no tuned kernel: the generic one, no split
    assert lib.ffk_conv_workspace_bytes(None) == 0


def test_noalloc_scratch_covers_every_workspace():
    """ffk_conv_noalloc's device array holds the workspace of every layer the
    library runs, at any batch: the split-K grids are capped at the array's
    size (small batches), larger batches and the Winograd and generic paths
    need none; so the no-allocation entry point serves every layer."""
    lib = fa.load()
    d = fa.ffk_conv_desc()
    layers, cur, blk = set(), (3, 112), (3, 112)        # (cin, cout, k, stride, input size)
    ops = synth.iresnet_schedule()
    for i, op in enumerate(ops):
        if op["type"] == synth.OP_CONV:
            src = blk if ops[i - 1]["type"] == synth.OP_SAVE_ID else cur
            layers.add((op["Cin"], op["Cout"], op["k"], op["s"], src[1]))
            cur = (op["Cout"], (src[1] + 2 * op["p"] - op["k"]) // op["s"] + 1)
        elif op["type"] == synth.OP_BLOCK_START:
            blk = cur
    layers |= {(64, 64, 1, 1, 56), (64, 128, 1, 1, 28), (128, 256, 1, 1, 14), (256, 512, 1, 1, 7)}
    sizes = set()
    for cin, cout, k, s, hin in sorted(layers):
        for B in list(range(1, 33)) + [64, 256, 1024]:
            for wino in (0, fa.FFK_ALGO_WINOGRAD):
                d.batch, d.cin, d.cout, d.kh, d.kw = B, cin, cout, k, k
                d.stride, d.pad, d.hin, d.win, d.flags = s, k // 2, hin, hin, wino
                n = lib.ffk_conv_workspace_bytes(C.byref(d))
                sizes.add(n)
                assert n <= fa.FFK_NOALLOC_SCRATCH_BYTES, (cin, cout, k, s, hin, B, wino, n)
    assert max(sizes) > fa.FFK_NOALLOC_SCRATCH_BYTES // 2          # the array is not oversized


def test_generic_geometries_are_runnable():
    """Geometries outside the tuned table run on the generic kernel (variant
    "generic", no workspace, one workgroup per output tile: 128 channels
    wide above 64 output channels, 128 pixels high where that still gives
    256 workgroups, except on the 3-channel input layer); invalid geometries
    are refused before any launch."""
    lib = fa.load()
    d = fa.ffk_conv_desc()

    def desc(cin, cout, kh, kw, s, pad, H, W, B):
        d.batch, d.cin, d.cout, d.kh, d.kw = B, cin, cout, kh, kw
        d.stride, d.pad, d.hin, d.win = s, pad, H, W
        return C.byref(d)
    for g in [(96, 64, 3, 3, 1, 1, 15, 13), (17, 40, 5, 5, 2, 2, 23, 23), (64, 72, 7, 1, 1, 3, 12, 12),
              (3, 64, 5, 5, 1, 2, 112, 112), (64, 64, 3, 3, 1, 0, 56, 56)]:
        assert lib.ffk_conv_runnable(*g) == 1 and lib.ffk_conv_supported(*g) == 0, g
        cin, cout, kh, kw, s, pad, H, W = g
        ho, wo = (H + 2 * pad - kh) // s + 1, (W + 2 * pad - kw) // s + 1
        for B in (3, 64):
            assert lib.ffk_conv_variant(desc(*g, B)) == b"generic"
            M = B * ho * wo
            bn = 128 if cout > 64 else 64
            tn = -(-cout // bn)
            bm = 128 if cin != 3 and -(-M // 128) * tn >= 256 else 64
            assert lib.ffk_conv_grid(desc(*g, B)) == -(-M // bm) * tn, (g, B)
            assert lib.ffk_conv_workspace_bytes(desc(*g, B)) == 0
    assert lib.ffk_conv_runnable(64, 64, 3, 3, 1, 1, 56, 56) == 1          # tuned
    for bad in [(0, 64, 3, 3, 1, 1, 8, 8), (64, 64, 3, 3, 0, 1, 8, 8), (64, 64, 3, 3, 1, -1, 8, 8),
                (64, 64, 9, 9, 1, 0, 8, 8), (64, 64, 3, 3, 1, 1, 0, 8)]:
        assert lib.ffk_conv_runnable(*bad) == 0, bad
        assert lib.ffk_conv_variant(desc(*bad, 1)) is None
        d.in_ = d.w = d.params = d.out = 4096                     # (never dereferenced)
        d.flags = 0
        assert lib.ffk_conv(desc(*bad, 1), None) == -1


def test_conv_variant_policy():
    """Which kernel variant a layer runs at a batch (host-side launch policy)."""
    lib = fa.load()
    d = fa.ffk_conv_desc()

    def variant(cin, cout, k, s, H, B, ws=0, flags=0):
        d.batch, d.cin, d.cout, d.kh, d.kw = B, cin, cout, k, k
        d.stride, d.pad, d.hin, d.win = s, k // 2, H, H
        d.workspace, d.workspace_bytes = (4096, ws) if ws else (None, 0)
        d.flags = flags
        v = lib.ffk_conv_variant(C.byref(d))
        return v.decode() if v else None
    assert variant(3, 64, 3, 1, 112, 1) == "stem"
    assert variant(256, 256, 3, 1, 14, 1024) == "patch"          # 3x3 stride 1
    assert variant(256, 256, 3, 2, 28, 1024) == "phase"           # 3x3 stride 2
    assert variant(256, 256, 3, 1, 14, 64) == "patch_kg"           # small grid: K-groups
    assert variant(256, 256, 3, 1, 14, 1, ws=1 << 30) == "splitk"  # tiny grid: K split 3 ways
    assert variant(256, 256, 3, 1, 14, 1) == "tile64"             # no workspace: whole-K 64x64 tiles
    assert variant(64, 64, 3, 1, 56, 1) == "tile64"               # no split: 49 small tiles, not 13
    assert variant(64, 64, 3, 1, 56, 8) == "tile64"               # 392 small tiles
    assert variant(64, 64, 3, 1, 56, 16) == "patch"               # 784: the patch tiles
    assert variant(64, 64, 3, 1, 112, 4) == "patch"               # one 64-channel run
    # a split grid too large for the layer's own split (9) takes 3 ranges
    d.batch, d.cin, d.cout, d.kh, d.kw, d.stride, d.pad, d.hin, d.win = 8, 512, 512, 3, 3, 2, 1, 14, 14
    d.workspace, d.workspace_bytes, d.flags = 4096, 1 << 30, 0
    assert lib.ffk_conv_variant(C.byref(d)) == b"splitk" and lib.ffk_conv_grid(C.byref(d)) == 7 * 8 * 3
    d.batch = 1
    assert lib.ffk_conv_grid(C.byref(d)) == 1 * 8 * 9
    assert variant(96, 64, 3, 1, 112, 1) == "generic"             # no tuned kernel
    assert lib.ffk_conv_variant(None) is None
    # The large tiles where there are at least as many as CUs (512->512 @7 at
    # 512 faces: 392), the 128x128 K-group tiles below (at 256 faces: 196).
    # FFK_SHARED_GPU (one half of a split chain): the two halves' grids count
    # together (196 each at 256 faces), not where even they do not (at 64 faces)
    assert variant(512, 512, 3, 1, 7, 512) == "patch"
    assert variant(512, 512, 3, 1, 7, 256) == "patch_kg"
    assert variant(512, 512, 3, 1, 7, 256, flags=fa.FFK_SHARED_GPU) == "patch"
    assert variant(512, 512, 3, 1, 7, 64, flags=fa.FFK_SHARED_GPU) == "patch_kg"


def test_rgb8_table_matches_sdk_normalization_and_reference_quant(oracle):
    """lut[c][x] == the reference's input quantization of the fp32 pixel the
    SDKs feed it: numpy float32 (x - 127.5) / 127.5 (fastface.py:10)."""
    lib = fa.load()
    x = np.arange(256, dtype=np.uint8)
    norm = (x.astype(np.float32) - 127.5) / 127.5            # numpy float32 semantics
    assert norm.dtype == np.float32
    for inv in ([127.0, 127.0, 127.0], [127.00001, 126.5, 3.0e9], [1e-3, 0.5, 254.99]):
        inv = np.asarray(inv, np.float32)
        lut = np.empty((3, 256), np.int8)
        assert lib.ffk_make_rgb8_lut(inv.ctypes.data, lut.ctypes.data) == 0
        faces = np.repeat(norm[:, None], 3, axis=1)           # [256, 3]: pixel value per channel
        exp = oracle.quant_input(faces, inv)                  # [256, 3]
        assert np.array_equal(lut.T, exp), inv
    assert lib.ffk_make_rgb8_lut(None, lut.ctypes.data) != 0


def test_prelu_le1_condition():
    """ffk_prelu_le1_ok: the plan takes PReLU as max(f, f*slope) only when
    every slope is at most 1 and the pre-activation cannot reach -inf."""
    import numpy as np
    import fastface_amd as fa
    lib = fa.load()
    C = 8
    P = np.zeros((fa.FFK_NPARAM, C), np.float32)
    P[fa.FFK_P_WS] = 1e-3
    P[fa.FFK_P_BIAS] = 0.1
    P[fa.FFK_P_SLOPE] = np.linspace(-1, 1, C)
    ok = lambda q, k=2304, add=1: lib.ffk_prelu_le1_ok(np.ascontiguousarray(q).ctypes.data, C, k, add)
    assert ok(P) == 1
    q = P.copy(); q[fa.FFK_P_SLOPE, 3] = np.float32(1.0000001)
    assert ok(q) == 0
    q = P.copy(); q[fa.FFK_P_SLOPE, 0] = np.nan
    assert ok(q) == 0
    q = P.copy(); q[fa.FFK_P_WS, 5] = np.inf
    assert ok(q) == 0
    q = P.copy(); q[fa.FFK_P_WS, 5] = 1e32        # 2304*16384*1e32 overflows fp32
    assert ok(q) == 0
    q = P.copy(); q[fa.FFK_P_ADDSCALE, 1] = np.nan
    assert ok(q) == 0 and ok(q, add=0) == 1        # the residual scale counts only with an add


def test_winograd_weight_packing(oracle):
    """ffk_pack_winograd_weights: the int8 limbs recombine to the restated
    reference transform U = G' g G'^T (64*u1 + u0, u0 in [0, 63])."""
    import numpy as np
    import fastface_amd as fa
    from conftest import rng
    lib = fa.load()
    r = rng(61)
    w = r.integers(-128, 128, size=(64, 64, 3, 3), dtype=np.int8)
    w[0] = -128
    w[1, :, 0, :] = -128; w[1, :, 1, :] = 127; w[1, :, 2, :] = -128
    n = lib.ffk_winograd_packed_bytes(64, 64)
    assert n == 16 * 64 * 2 * 64
    packed = np.empty(n, np.int8)
    assert lib.ffk_pack_winograd_weights(w.ctypes.data, 64, 64, packed.ctypes.data) == 0
    p = packed.reshape(16, 64, 2, 64).astype(np.int32)
    u1, u0 = p[:, :, 0, :], p[:, :, 1, :]
    assert u0.min() >= 0 and u0.max() <= 63 and np.abs(u1).max() <= 18
    assert np.array_equal(64 * u1 + u0, oracle.winograd_weights(w).astype(np.int32))
    sup = lambda *g: lib.ffk_winograd_supported(*g)
    assert sup(64, 64, 3, 3, 1, 1, 56, 56) == 1 and sup(64, 64, 3, 3, 1, 1, 112, 112) == 1
    assert sup(64, 64, 3, 3, 2, 1, 112, 112) == 0 and sup(128, 128, 3, 3, 1, 1, 28, 28) == 0
    assert sup(64, 128, 3, 3, 1, 1, 56, 56) == 0 and sup(64, 64, 1, 1, 1, 0, 56, 56) == 0


def test_x_even_argument_checks():
    """FFK_OUT_X_EVEN needs an int8 X output of even height and width; the
    checks fail before anything touches a device (the pointers are never
    dereferenced)."""
    lib = fa.load()
    d = fa.ffk_conv_desc()
    d.batch, d.cin, d.cout, d.kh, d.kw, d.stride, d.pad, d.hin, d.win = 1, 512, 512, 3, 3, 1, 1, 7, 7
    d.in_, d.w, d.params, d.out = 4096, 8192, 12288, 16384
    d.flags = fa.FFK_EPI_BIAS | fa.FFK_OUT_X_EVEN
    assert lib.ffk_conv(C.byref(d), None) == -1                    # 7x7 output
    assert "even" in fa.last_error()
    d.cin = d.cout = 256
    d.hin = d.win = 14                                             # 14x14 output
    d.out, d.out_i32 = None, 16384                                 # raw int32 output
    assert lib.ffk_conv(C.byref(d), None) == -1
    d.out_i32, d.out_bn, d.bn_lut = None, 16384, 20480             # BN output only, no X
    d.flags |= fa.FFK_EPI_BN
    assert lib.ffk_conv(C.byref(d), None) == -1


def test_requant_in_range_condition():
    """ffk_requant_in_range: FFK_EPI_IN_RANGE only where every requant value
    is provably finite and below 2^31 - 128 (then the x86 out-of-range case,
    NaN or |r| >= 2^31 -> -128, cannot occur)."""
    lib = fa.load()
    C_ = 4
    P = np.zeros((fa.FFK_NPARAM, C_), np.float32)
    P[fa.FFK_P_WS] = 1e-3
    P[fa.FFK_P_BIAS] = 0.1
    P[fa.FFK_P_INV] = 20.0
    P[fa.FFK_P_SLOPE] = 0.25
    P[fa.FFK_P_ADDSCALE] = 0.05
    K = 2304
    PR, AD = fa.FFK_EPI_PRELU, fa.FFK_EPI_ADD
    ok = lambda q, flags=PR, k=K: lib.ffk_requant_in_range(np.ascontiguousarray(q).ctypes.data, C_, k, flags)
    assert ok(P) == 1 and ok(P, AD) == 1 and ok(P, 0) == 1
    # the bound: K*128^2*ws*inv just below / above 2^31 - 128
    acc_max = K * 128 * 128
    Q = P.copy(); Q[fa.FFK_P_BIAS] = 0; Q[fa.FFK_P_WS] = 1.0
    Q[fa.FFK_P_INV, 2] = np.float32(2147483520.0 / acc_max * 0.9999)
    assert ok(Q, 0) == 1
    Q[fa.FFK_P_INV, 2] = np.float32(2147483520.0 / acc_max * 1.0001)
    assert ok(Q, 0) == 0
    Q = P.copy(); Q[fa.FFK_P_INV, 1] = 3.0e38          # requant overflow
    assert ok(Q) == 0
    Q = P.copy(); Q[fa.FFK_P_WS, 0] = np.nan
    assert ok(Q) == 0
    Q = P.copy(); Q[fa.FFK_P_SLOPE, 3] = np.inf         # only checked with PReLU
    assert ok(Q, PR) == 0 and ok(Q, 0) == 1
    Q = P.copy(); Q[fa.FFK_P_ADDSCALE, 3] = np.inf      # only checked with the residual
    assert ok(Q, AD) == 0 and ok(Q, 0) == 1
    Q = P.copy(); Q[fa.FFK_P_SLOPE] = 1e4               # a slope above 1 scales the bound
    assert ok(Q, PR) == 0 and ok(Q, 0) == 1
    assert ok(P, PR | fa.FFK_EPI_INSCALE) == 0          # the in-scale path always checks
    assert ok(P, PR, 0) == 0


def test_scale_paths_follow_the_working_directory():
    """FastFace(cwd=...) opens the files fastface_create would open with `cwd`
    as the working directory (libfastface.c:236-240): a relative $OPSC2_PATH
    is taken relative to `cwd`, an absolute one as it is."""
    from fastface_amd.api import scale_paths
    cwd = "/data/run"
    assert scale_paths(cwd, {}) == ("/data/run/models/op_scales.bin",
                                     "/data/run/models/op_scales_v2.bin")
    assert scale_paths(cwd, {"OPSC2_PATH": "alt/v2.bin"})[1] == "/data/run/alt/v2.bin"
    assert scale_paths(cwd, {"OPSC2_PATH": "/abs/v2.bin"})[1] == "/abs/v2.bin"
    assert scale_paths(cwd, {"OPSC2_PATH": ""})[1] == "/data/run/models/op_scales_v2.bin"


# FFK_EPI_FMA_TAIL: the requant's last two roundings RN(RN(f*inv) + h),
# h = copysign(0.5, f), taken as one, RN(f*inv + h) (an fma).  Exact
# emulations of the pre-requant value f(acc) and of both tails over every
# accumulator of a channel (numpy float32 arithmetic is IEEE single; f*inv is
# exact in float64, and so is f*inv + h wherever |f*inv| >= 2^-5, the only
# place where the rounding can move the truncated result).
def _f_pre(acc, ws, bias, slope, prelu):
    f = (acc.astype(np.float32) * np.float32(ws)).astype(np.float32)
    f = (f + np.float32(bias)).astype(np.float32)
    if prelu:
        f = np.where(f < 0, (f * np.float32(slope)).astype(np.float32), f)
    return f


def _tail_reference(f, inv):
    t = (f * np.float32(inv)).astype(np.float32)
    r = (t + np.copysign(np.float32(0.5), t)).astype(np.float32)
    return np.clip(np.trunc(r), -128, 127)


def _tail_fma(f, inv):
    s = f.astype(np.float64) * float(np.float32(inv)) + np.copysign(0.5, f.astype(np.float64))
    return np.clip(np.trunc(s.astype(np.float32)), -128, 127)


def _fma_ok(lib, ws, bias, inv, slope, K, prelu=True, flags=0):
    P = np.zeros((fa.FFK_NPARAM, 1), np.float32)
    P[fa.FFK_P_WS], P[fa.FFK_P_BIAS], P[fa.FFK_P_INV], P[fa.FFK_P_SLOPE] = ws, bias, inv, slope
    fl = fa.FFK_EPI_BIAS | (fa.FFK_EPI_PRELU if prelu else 0) | flags
    return lib.ffk_requant_fma_ok(P.ctypes.data, 1, K, fl)


def test_fma_tail_proof_equals_brute_force():
    """ffk_requant_fma_ok accepts a channel exactly when no accumulator in
    [-K*128^2, K*128^2] gives another int8 with the one-rounding tail: every
    accumulator of 1024-deep channels whose PReLU branch is dense near
    f*inv = -1/2 (small slopes; the layers where the proof rejects), and of
    shallow channels with natural parameters."""
    lib = fa.load()
    K = 1024
    acc = np.arange(-K * 16384, K * 16384 + 1, dtype=np.int64)
    seen = {True: 0, False: 0}
    for ws, slope, target in [(2.6e-7, 2.2e-4, 15.0e6), (2.6e-7, 2.2e-4, 15.15e6), (2.6e-7, 2.2e-4, 15.3e6),
                              (1e-7, 5e-4, 16.16e6), (2e-7, 3e-4, 9e6), (2e-7, 3e-4, 9.09e6)]:
        inv = float(np.float32(0.5 / (target * ws * slope)))
        f = _f_pre(acc, ws, 0.01, slope, True)
        differs = bool((_tail_reference(f, inv) != _tail_fma(f, inv)).any())
        seen[differs] += 1
        assert _fma_ok(lib, ws, 0.01, inv, slope, K) == (0 if differs else 1), (ws, slope, inv)
    assert seen[True] >= 2 and seen[False] >= 2          # both outcomes are exercised
    r = np.random.default_rng(5)
    for _ in range(40):
        k = int(r.integers(1, 10))
        prelu = bool(r.integers(0, 2))
        ws = float(r.uniform(1e-4, 1e-2) * (1 if r.random() < 0.8 else -1))
        bias, inv, slope = float(r.normal(0, 0.1)), float(r.uniform(1, 100)), float(10 ** r.uniform(-4, -0.5))
        a = np.arange(-k * 16384, k * 16384 + 1, dtype=np.int64)
        f = _f_pre(a, ws, bias, slope, prelu)
        differs = bool((_tail_reference(f, inv) != _tail_fma(f, inv)).any())
        assert _fma_ok(lib, ws, bias, inv, slope, k, prelu) == (0 if differs else 1)


def test_fma_tail_proof_rejects_the_window():
    """The one place the two tails differ: f*inv strictly between
    1/2 - 2^-25 - 2^-26 and 1/2 - 2^-25, where the reference's first
    rounding lands on 1/2 - 2^-25 and its second rounds the tie up to 1.
    Here f = ws at accumulator 1 (and -ws at -1) puts f*inv inside it."""
    lib = fa.load()
    ws, inv = 0.1515151411294937, float(np.float32(3.3))
    p = float(np.float32(ws)) * inv
    assert 0.5 - 2.0 ** -25 - 2.0 ** -26 < p < 0.5 - 2.0 ** -25
    f = _f_pre(np.array([1, -1]), ws, 0.0, 0.0, False)
    assert list(_tail_reference(f, inv)) == [1, -1] and list(_tail_fma(f, inv)) == [0, 0]
    assert _fma_ok(lib, ws, 0.0, inv, 0.0, 1, prelu=False) == 0
    # the same channel whose values never reach the window: accepted
    assert _fma_ok(lib, ws, 0.25, inv, 0.0, 1, prelu=False) == 1
    f = _f_pre(np.arange(-16384, 16385), ws, 0.25, 0.0, False)
    assert (_tail_reference(f, inv) == _tail_fma(f, inv)).all()


def test_fma_tail_proof_preconditions():
    """Only in-range launches without a residual or an in-scale qualify;
    a zero weight scale (a constant channel) and a negative one are
    decided like any other."""
    lib = fa.load()
    assert _fma_ok(lib, 1e-3, 0.1, 20.0, 0.25, 2304) == 1
    assert _fma_ok(lib, 1e-3, 0.1, 20.0, 0.25, 2304, flags=fa.FFK_EPI_ADD) == 0
    assert _fma_ok(lib, 1e-3, 0.1, 20.0, 0.25, 2304, flags=fa.FFK_EPI_INSCALE) == 0
    assert _fma_ok(lib, 1e-3, 0.1, 3.0e38, 0.25, 2304) == 0           # not in range
    assert _fma_ok(lib, 1e-3, 0.1, 20.0, -0.25, 2304) == 0            # negative slope
    assert _fma_ok(lib, 0.0, 0.0072, 1e9, 0.075, 576) == 1            # constant channel
    assert _fma_ok(lib, 0.0, 0.1515151411294937 / 1.0, float(np.float32(3.3)), 0.0, 576, prelu=False) == 0
    assert _fma_ok(lib, -1e-3, 0.1, 20.0, 0.25, 2304) == 1
