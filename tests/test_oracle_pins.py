"""Pins the CPU oracle (oracle/ff_oracle.c) before anything is compared with it.

Each oracle function is checked against (a) the reference's own function
compiled from its sources (oracle/_ref, AVX-VNNI host), on seeded inputs and
on special cases chosen so that a plausible slip -- a dropped FMA, RNE
instead of half-away rounding, a saturating float->int conversion, flushed
denormals, a transposed weight index -- changes the output, and (b) closed
forms / brute force where the mathematics fixes the answer.
"""
import os

import numpy as np
import pytest

from conftest import rng

F32 = np.float32


def _specials_epilogue(C, r):
    """Per-channel parameter sets that land on the delicate cases."""
    ws = r.uniform(1e-3, 1e-2, C).astype(F32)
    bias = r.normal(0, 0.1, C).astype(F32)
    inv = (1.0 / r.uniform(0.01, 0.1, C)).astype(F32)
    ws[0], bias[0], inv[0] = 0.5, 0.0, 1.0          # acc odd -> exact .5 ties
    ws[1], bias[1], inv[1] = 1.0, 0.0, 0.5          # ties through inv
    ws[2], inv[2] = 1e-3, 3.0e38                    # |t| >= 2^31 and inf -> INT32_MIN -> -128
    ws[3] = np.float32(1.4e-44)                     # denormal weight scale
    inv[3] = np.float32(1e30)
    ws[4] = np.nan                                  # NaN -> -128
    ws[5], bias[5] = -1.0, -0.0                     # -0 handling
    inv[6] = 1e9                                    # 1/(denormal + 1e-9): real OPSC2 case
    ws[7], bias[7], inv[7] = 2.0 ** -20, 0.0, 2.0 ** 20   # exact products, sign of zero
    return ws, bias, inv


@pytest.mark.parametrize("prelu,add,add_pc,inv_pc,bn", [
    (False, False, False, True, False),
    (True, False, False, True, False),
    (False, True, True, True, False),
    (False, True, False, True, False),
    (True, False, False, False, False),
    (False, False, False, True, True),
])
def test_epilogue_vs_reference(oracle, ref, prelu, add, add_pc, inv_pc, bn):
    r = rng(11)
    C, P = 64, 3000
    acc = r.integers(-2_000_000, 2_000_000, size=(P, C), dtype=np.int32)
    acc[:, 0] = r.integers(-600, 600, size=P) | 1     # odd
    acc[::7] = 0
    ws, bias, inv = _specials_epilogue(C, r)
    kw = dict(ws=ws, bias=bias, inv_pc=inv if inv_pc else None, out_scale=0.037)
    if prelu:
        slope = r.uniform(0, 0.3, C).astype(F32)
        slope[8] = -1.0
        kw["prelu"] = slope
    if add:
        kw["add_src"] = r.integers(-128, 128, size=(P, C), dtype=np.int8)
        kw["add_scale"] = 0.021
        if add_pc:
            kw["add_scale_pc"] = r.uniform(1e-3, 5e-2, C).astype(F32)
    if bn:
        kw["bn_scale"] = r.uniform(0.5, 1.5, C).astype(F32)
        kw["bn_offset"] = r.normal(0, 0.05, C).astype(F32)
    got = oracle.fused_epilogue(acc, **kw)
    exp = ref.fused_epilogue(acc, **kw)
    assert np.array_equal(got, exp)
    # the special channels really hit their cases
    assert (exp[:, 2] == -128).any() and (exp[:, 4] == -128).all()


def test_epilogue_rounding_is_half_away_in_fp32(oracle):
    """t + copysign(0.5, t) is rounded to fp32 before truncation, so the fp32
    just below 0.5 rounds up to 1 (an exact round-half-away would give 0)."""
    below_half = np.nextafter(F32(0.5), F32(0))
    acc = np.array([[1], [3], [-3], [5], [-1], [0]], np.int32).repeat(8, axis=1)
    ws = np.full(8, 0.5, F32)
    inv = np.full(8, 1.0, F32)
    q = oracle.fused_epilogue(acc, ws=ws, bias=np.zeros(8, F32), inv_pc=inv)[:, 0]
    assert list(q) == [1, 2, -2, 3, -1, 0]
    acc1 = np.ones((1, 8), np.int32)
    q = oracle.fused_epilogue(acc1, ws=np.full(8, below_half, F32), bias=np.zeros(8, F32),
                              inv_pc=inv)
    assert q[0, 0] == 1


def test_cvtt_matches_x86_integer_indefinite(oracle):
    assert oracle.cvtt(2147483520.0) == 2147483520
    assert oracle.cvtt(2147483648.0) == -2147483648
    assert oracle.cvtt(-2147483648.0) == -2147483648
    assert oracle.cvtt(float("nan")) == -2147483648
    assert oracle.cvtt(-7.9) == -7


@pytest.mark.parametrize("use_pc,prelu", [(True, False), (False, False), (True, True)])
def test_bn_requant_vs_reference(oracle, ref, use_pc, prelu):
    r = rng(12)
    C, P = 128, 2000
    x = r.integers(-128, 128, size=(P, C), dtype=np.int8)
    s_in = r.uniform(1e-3, 5e-2, C).astype(F32)
    s_in[0] = np.float32(3e-45)            # denormal forward scale (present in OPSC2)
    bns = r.uniform(0.5, 1.5, C).astype(F32)
    bno = r.normal(0, 0.05, C).astype(F32)
    inv = (1.0 / r.uniform(0.01, 0.1, C)).astype(F32)
    inv[1] = 1e9
    kw = dict(in_scale=0.02, in_scale_pc=s_in if use_pc else None, bn_scale=bns, bn_offset=bno,
              inv_pc=inv, out_scale=0.05)
    if prelu:
        kw["prelu"] = r.uniform(0, 0.3, C).astype(F32)
    assert np.array_equal(oracle.bn_prelu_requant(x, **kw), ref.bn_prelu_requant(x, **kw))


def test_input_quant_vs_reference(oracle, ref):
    r = rng(13)
    x = r.uniform(-1, 1, size=(4096, 3)).astype(F32)
    x[:8, 0] = [0.5 / 127, 1.5 / 127, -2.5 / 127, 1e10, -1e10, np.inf, -np.inf, np.nan]
    x[8:12, 1] = [3e9, -3e9, 2.5, -2.5]
    inv = np.array([127.0, 127.00001, 1.0], F32)
    assert np.array_equal(oracle.quant_input(x, inv), ref.quant_input(x, inv))


def test_add_requant_vs_reference(oracle, ref):
    r = rng(14)
    a = r.integers(-128, 128, 5000, dtype=np.int8)
    b = r.integers(-128, 128, 5000, dtype=np.int8)
    assert np.array_equal(oracle.add_requant(a, 0.013, b, 0.021, 0.03),
                          ref.add_requant(a, 0.013, b, 0.021, 0.03))


CONV_SHAPES = [  # (Cin, Cout, k, stride, H)
    (3, 64, 3, 1, 20), (64, 64, 3, 1, 9), (64, 64, 3, 2, 10), (64, 64, 1, 2, 10),
    (64, 128, 3, 1, 7), (128, 128, 3, 2, 8), (256, 256, 3, 1, 5), (256, 512, 1, 2, 6),
]


@pytest.mark.parametrize("cin,cout,k,s,H", CONV_SHAPES)
def test_conv_i32_vs_reference(oracle, ref, cin, cout, k, s, H):
    r = rng(15 + cin + cout + k + s)
    x = r.integers(-128, 128, size=(2, H, H, cin), dtype=np.int8)
    w = r.integers(-128, 128, size=(cout, cin, k, k), dtype=np.int8)
    pad = k // 2
    assert np.array_equal(oracle.conv_i32(x, w, s, pad), ref.conv_i32(x, w, s, pad))


def test_conv_i32_brute_force(oracle):
    """Definition of convolution on a tiny case, including extreme values."""
    r = rng(16)
    x = r.integers(-128, 128, size=(2, 5, 4, 64), dtype=np.int8)
    x[0, 0, 0, :] = -128
    w = r.integers(-128, 128, size=(3, 64, 3, 3), dtype=np.int8)
    w[0] = -128
    for s in (1, 2):
        got = oracle.conv_i32(x, w, s, 1)
        xp = np.pad(x.astype(np.int64), ((0, 0), (1, 1), (1, 1), (0, 0)))
        Ho, Wo = (5 + 2 - 3) // s + 1, (4 + 2 - 3) // s + 1
        exp = np.zeros((2, Ho, Wo, 3), np.int64)
        for oh in range(Ho):
            for ow in range(Wo):
                patch = xp[:, oh * s:oh * s + 3, ow * s:ow * s + 3, :]      # [B,3,3,Cin]
                exp[:, oh, ow, :] = np.einsum("bhwc,ochw->bo", patch, w.astype(np.int64))
        assert np.array_equal(got, exp)


def _conv_brute(x, w, s, pad):
    B, H, W, _ = x.shape
    cout, _, kh, kw = w.shape
    xp = np.pad(x.astype(np.int64), ((0, 0), (pad, pad), (pad, pad), (0, 0)))
    Ho, Wo = (H + 2 * pad - kh) // s + 1, (W + 2 * pad - kw) // s + 1
    exp = np.zeros((B, Ho, Wo, cout), np.int64)
    for oh in range(Ho):
        for ow in range(Wo):
            patch = xp[:, oh * s:oh * s + kh, ow * s:ow * s + kw, :]
            exp[:, oh, ow, :] = np.einsum("bhwc,ochw->bo", patch, w.astype(np.int64))
    return exp


# geometries outside the IResNet table (the generic GPU kernel's cases):
# (cin, cout, kh, kw, stride, pad, H, W)
ODD_GEOMETRIES = [(96, 64, 3, 3, 1, 1, 7, 6), (17, 40, 5, 5, 2, 2, 9, 9), (64, 72, 7, 1, 1, 3, 8, 8),
                  (128, 64, 3, 3, 3, 1, 10, 10), (3, 32, 5, 5, 2, 0, 11, 11)]


@pytest.mark.parametrize("cin,cout,kh,kw,s,pad,H,W", ODD_GEOMETRIES)
def test_conv_i32_other_geometries(oracle, cin, cout, kh, kw, s, pad, H, W):
    """The oracle's convolution on shapes no tuned kernel has (channel counts,
    kernel sizes, non-square kernels, strides, paddings): the definition by
    brute force."""
    r = rng(17 + cin + kh * 3 + kw + s)
    x = r.integers(-128, 128, size=(2, H, W, cin), dtype=np.int8)
    w = r.integers(-128, 128, size=(cout, cin, kh, kw), dtype=np.int8)
    x[0, 0, 0, :] = -128
    w[0] = -128
    assert np.array_equal(oracle.conv_i32(x, w, s, pad), _conv_brute(x, w, s, pad))


@pytest.mark.parametrize("cin,cout,kh,kw,s,pad,H,W", [g for g in ODD_GEOMETRIES if g[2] == g[3]])
def test_conv_i32_other_geometries_vs_reference(oracle, ref, cin, cout, kh, kw, s, pad, H, W):
    """The same shapes (square kernels: the reference's packer takes one
    kernel size per axis as given) against the reference's im2col + VNNI."""
    r = rng(18 + cin + kh + s)
    x = r.integers(-128, 128, size=(2, H, W, cin), dtype=np.int8)
    w = r.integers(-128, 128, size=(cout, cin, kh, kw), dtype=np.int8)
    assert np.array_equal(oracle.conv_i32(x, w, s, pad), ref.conv_i32(x, w, s, pad))


def test_forward_vs_reference_embed_generic_geometries(oracle, ref):
    """Whole network with three convs of geometries no tuned kernel has (synth
    `iresnet_schedule(generic=True)`: a 5x5 stem, a 5x5 stage-3 conv, a 1x1
    stage-4 conv adding the residual): oracle interpreter == reference
    fastface_embed, bit for bit."""
    from fastface_amd import synth
    ffw = synth.synthetic_generic_path()
    faces = np.concatenate([synth.faces_uniform(1, 0), synth.faces_normal_clipped(1, 2)])
    m = oracle.load_model(ffw, synth.OPSC_PATH, synth.OPSC2_PATH)
    try:
        emb, _ = oracle.forward(m, faces)
    finally:
        oracle.free_model(m)
    assert np.array_equal(emb, ref.embed(ffw, faces, cwd=synth.REPO_ROOT))


WINO_SHAPES = [(64, 64, 56, 1), (64, 64, 112, 1), (16, 8, 6, 2)]


@pytest.mark.parametrize("cin,cout,H,B", WINO_SHAPES)
def test_winograd_f23_vs_reference(oracle, ref, cin, cout, H, B):
    """Integer Winograd F(2,3) (kernels/winograd_int8_ref.c): weight transform
    and tile conv bit-exact with the reference's own scalar code."""
    r = rng(900 + cin + H)
    x = r.integers(-128, 128, size=(B, H, H, cin), dtype=np.int8)
    w = r.integers(-128, 128, size=(cout, cin, 3, 3), dtype=np.int8)
    x[0, :2] = -128
    w[0] = -128
    w[1] = 127
    u = oracle.winograd_weights(w)
    assert np.array_equal(u, ref.winograd_weights(w))
    assert np.array_equal(oracle.conv_winograd(x, u), ref.conv_winograd(x, u))


def test_winograd_f23_is_four_times_direct(oracle):
    """Closed form, independent of the reference: with G' = 2G the F(2,3)
    output is exactly 4x the 3x3 s1 p1 convolution (brute force), and the
    transformed weights stay inside int16 at the int8 extremes."""
    r = rng(77)
    x = r.integers(-128, 128, size=(2, 8, 10, 24), dtype=np.int8)
    w = r.integers(-128, 128, size=(12, 24, 3, 3), dtype=np.int8)
    x[1] = -128
    w[3] = -128
    w[4, :, 1, :] = 127
    u = oracle.winograd_weights(w)
    assert np.abs(u.astype(np.int32)).max() <= 1152      # 4*2*... bound: |2a|+|a+b+c| combos
    B, H, W, Cin = x.shape
    xp = np.pad(x.astype(np.int64), ((0, 0), (1, 1), (1, 1), (0, 0)))
    direct = np.zeros((B, H, W, w.shape[0]), np.int64)
    for kh in range(3):
        for kw in range(3):
            direct += np.einsum("bhwc,oc->bhwo", xp[:, kh:kh + H, kw:kw + W, :],
                                w[:, :, kh, kw].astype(np.int64))
    assert np.array_equal(oracle.conv_winograd(x, u).astype(np.int64), 4 * direct)
    # one transform cell by hand: u[0] = G'[0] g G'[0]^T = 4 * g[0][0]
    assert np.array_equal(u[0], 4 * w[:, :, 0, 0].astype(np.int16))


def test_fc_vs_reference_and_closed_form(oracle, ref):
    r = rng(17)
    K, N = 25088, 64
    a = r.integers(-128, 128, K, dtype=np.int8)
    W = r.integers(-127, 128, size=(N, K), dtype=np.int8)
    ws = r.uniform(1e-7, 1e-5, N).astype(F32)
    bias = r.normal(0, 0.05, N).astype(F32)
    got = oracle.fc(a, W, ws, bias)
    assert np.array_equal(got, ref.fc(a, W, ws, bias))
    dot = W.astype(np.int64) @ a.astype(np.int64)
    exp = (dot.astype(np.float32).astype(np.float64) * ws.astype(np.float64) +
           bias.astype(np.float64)).astype(np.float32)     # fma: one rounding of the exact value
    assert np.array_equal(got, exp)


def test_schedule_matches_committed_opsc2():
    """The synthetic FFW4's op list has the channel pattern the committed
    OPSC2 records for the real w600k_r50 model (0 for marker ops)."""
    from fastface_amd import synth
    ops = synth.iresnet_schedule()
    _, per_op = synth.read_opsc2()
    assert len(ops) == len(per_op) == 177
    for op, sc in zip(ops, per_op):
        n = 0 if sc is None else len(sc)
        t = op["type"]
        if t == synth.OP_CONV:
            assert n == op["Cout"]
        elif t in (synth.OP_BN, synth.OP_PRELU):
            assert n == op["C"]
        elif t in (synth.OP_SAVE_ID, synth.OP_BLOCK_START):
            assert n == 0
        elif t == synth.OP_FLATTEN:
            assert n == 25088
        elif t == synth.OP_GEMM:
            assert n == 512


def test_forward_vs_reference_embed(oracle, ref, oracle_model, synth_ffw4):
    """Whole network: oracle interpreter == reference fastface_embed, bit-exact,
    on the reference's own real-face input fixture and a synthetic face."""
    from fastface_amd import synth
    gold_in = np.fromfile(os.path.join(os.path.dirname(__file__), "golden", "golden_input.bin"),
                          dtype=np.float32).reshape(1, 112, 112, 3)
    faces = np.concatenate([gold_in, synth.faces_uniform(1, 0)])
    emb, _ = oracle.forward(oracle_model, faces)
    emb_ref = ref.embed(synth_ffw4, faces, cwd=synth.REPO_ROOT)
    assert np.array_equal(emb, emb_ref)


# (FFW version, OPSC2 present): the formats below FFW4, and FFW4 without
# OPSC2, which the reference runs on per-tensor scales
OTHER_FORMATS = [(3, True), (3, False), (2, True), (2, False), (4, False)]


def ref_embed_without_opsc2(ref, ffw, faces, cwd=None):
    """The reference's fastface_embed with no OPSC2 file to load ($OPSC2_PATH
    naming a missing file: libfastface.c:238-240 then keeps the per-tensor
    OPSC scales); `cwd` holds models/op_scales.bin (default: the repo's)."""
    from fastface_amd import synth
    cwd = cwd or synth.REPO_ROOT
    old = os.environ.get("OPSC2_PATH")
    os.environ["OPSC2_PATH"] = os.path.join(cwd, "models", "no_such_op_scales_v2.bin")
    try:
        return ref.embed(ffw, faces, cwd=cwd)
    finally:
        if old is None:
            del os.environ["OPSC2_PATH"]
        else:
            os.environ["OPSC2_PATH"] = old


@pytest.mark.parametrize("version,with_opsc2", OTHER_FORMATS,
                         ids=["ffw3", "ffw3-noopsc2", "ffw2", "ffw2-noopsc2", "ffw4-noopsc2"])
def test_forward_vs_reference_embed_other_formats(oracle, ref, version, with_opsc2):
    """Whole network on the formats the loader also accepts: FFW3 (the FFW4
    layout) and FFW2 (no conv bias), which the reference runs on per-tensor
    scales, with an in-scale on every conv and the activation scale on the FC
    (libfastface.c:335-343,356-422; kernels/ffw2_loader.c:96-125); and FFW4
    without OPSC2.  Oracle interpreter == reference fastface_embed, bit for
    bit.  Below FFW4 the reference never reads OPSC2, so its presence
    changes nothing."""
    from fastface_amd import synth
    ffw = synth.synthetic_ffw4_path(3, version=version)
    faces = np.concatenate([synth.faces_uniform(1, 0), synth.faces_normal_clipped(1, 2)])
    m = oracle.load_model(ffw, synth.OPSC_PATH, synth.OPSC2_PATH if with_opsc2 else None)
    try:
        emb, acts = oracle.forward(m, faces, dump_ops=[3, 90])
    finally:
        oracle.free_model(m)
    emb_ref = ref.embed(ffw, faces, cwd=synth.REPO_ROOT) if with_opsc2 else \
        ref_embed_without_opsc2(ref, ffw, faces)
    assert np.array_equal(emb, emb_ref)
    if version < 4:
        assert np.array_equal(emb, ref_embed_without_opsc2(ref, ffw, faces) if with_opsc2 else
                              ref.embed(ffw, faces, cwd=synth.REPO_ROOT))
    # the model is not degenerate: its activations spread over the int8 range
    for a in acts.values():
        assert a.astype(np.float32).std() > 5 and (a == 0).mean() < 0.2


@pytest.mark.parametrize("with_opsc2", [True, False], ids=["opsc2", "noopsc2"])
def test_forward_vs_reference_embed_standalone_ops(oracle, ref, with_opsc2):
    """Whole network with elementwise ops that no conv absorbs (synth
    `iresnet_schedule(standalone=True)`: stand-alone PReLU, BN after PReLU,
    BN after an Add, an Add after a BN, a second BN; libfastface.c:401-434),
    on its own OPSC / OPSC2 files.  Oracle interpreter == reference
    fastface_embed, bit for bit, and the inserted ops' outputs are not
    degenerate."""
    from fastface_amd import synth
    d = synth.synthetic_standalone_dir()
    ffw = os.path.join(d, "model.ffw4")
    faces = np.concatenate([synth.faces_uniform(1, 0), synth.faces_normal_clipped(1, 2)])
    m = oracle.load_model(ffw, os.path.join(d, "models", "op_scales.bin"),
                          os.path.join(d, "models", "op_scales_v2.bin") if with_opsc2 else None)
    try:
        emb, acts = oracle.forward(m, faces, dump_ops=[53, 55, 70, 71, 74, 179, 180])
    finally:
        oracle.free_model(m)
    emb_ref = ref.embed(ffw, faces, cwd=d) if with_opsc2 else ref_embed_without_opsc2(ref, ffw, faces, cwd=d)
    assert np.array_equal(emb, emb_ref)
    if with_opsc2:
        for op, a in acts.items():
            a = a.astype(np.float32)
            assert a.std() > 5 and (a == 0).mean() < 0.2 and (np.abs(a) >= 127).mean() < 0.2, op


def test_forward_vs_reference_embed_hostile_parameters(oracle, ref):
    """Whole network with parameter values no shorter epilogue form survives
    (synth `hostile_channels`: a NaN weight scale in the input layer, +-3e38
    biases whose requant values overflow, a PReLU slope of 1.5): oracle
    interpreter == reference fastface_embed, bit for bit, and the
    overflowing channel is the x86 out-of-range -128 everywhere."""
    from fastface_amd import synth
    ffw = synth.synthetic_hostile_path()
    faces = np.concatenate([synth.faces_uniform(1, 0), synth.faces_normal_clipped(1, 2)])
    m = oracle.load_model(ffw, synth.OPSC_PATH, synth.OPSC2_PATH)
    try:
        emb, acts = oracle.forward(m, faces, dump_ops=[1])
    finally:
        oracle.free_model(m)
    assert np.array_equal(emb, ref.embed(ffw, faces, cwd=synth.REPO_ROOT))
    assert (acts[1][..., 0] == -128).all()


def test_synthetic_formats_share_their_weights():
    """FFW3 / FFW2 variants hold the FFW4 model's int8 weights (the same
    draws); FFW2 lacks exactly the 53 conv biases."""
    from fastface_amd import synth
    sizes = {v: os.path.getsize(synth.synthetic_ffw4_path(3, version=v)) for v in (4, 3, 2)}
    couts = sum(op["Cout"] for op in synth.iresnet_schedule() if op["type"] == synth.OP_CONV)
    assert sizes[3] == sizes[4] and sizes[4] - sizes[2] == 4 * couts
    with open(synth.synthetic_ffw4_path(3, version=4), "rb") as f4, \
            open(synth.synthetic_ffw4_path(3, version=3), "rb") as f3:
        a, b = f4.read(), f3.read()
    assert a[:4] == b"FFW4" and b[:4] == b"FFW3"
    stem_w = 8 + 1 + 12
    assert a[stem_w:stem_w + 64 * 27] == b[stem_w:stem_w + 64 * 27]


def test_forward_batch_invariance(oracle, oracle_model):
    from fastface_amd import synth
    faces = synth.faces_normal_clipped(3, 2)
    emb3, _ = oracle.forward(oracle_model, faces)
    for i in range(3):
        e1, _ = oracle.forward(oracle_model, faces[i:i + 1])
        assert np.array_equal(e1[0], emb3[i])


def test_input_quant_per_tensor_vs_reference(oracle, ref):
    """The OPSC-only input path (no OPSC2): one scale for all channels,
    inv = 1/(s + 1e-9f) computed in fp32 inside the function, then lrintf and
    the clamp (kernels/int8_epilogue.c:218-227).  Scales include the committed
    1/127, a denormal (inv = 1/1e-9 rounded) and zero."""
    r = rng(18)
    x = r.uniform(-1, 1, 5000).astype(F32)
    x[:10] = [0.5 / 127, 1.5 / 127, -2.5 / 127, 1e10, -1e10, np.inf, -np.inf, np.nan, 3e9, -0.0]
    for scale in (1.0 / 127, 0.0371, float(np.float32(1e-45)), 0.0, 2.0):
        got = oracle.quant_input_pt(x, scale)
        assert np.array_equal(got, ref.quant_input_pt(x, scale)), scale
    # closed form on the in-range values: round half to even of RN(x * inv)
    inv = np.float32(1.0) / (np.float32(1.0 / 127) + np.float32(1e-9))
    v = x[10:] * inv
    assert np.array_equal(oracle.quant_input_pt(x[10:], 1.0 / 127),
                          np.clip(np.rint(v), -128, 127).astype(np.int8))


@pytest.mark.parametrize("prelu,add,bn", [(False, False, False), (True, False, False),
                                          (False, True, False), (True, True, True)])
def test_epilogue_in_scale_vs_reference(oracle, ref, prelu, add, bn):
    """The FFW2/FFW3 branch of the epilogue, f = RN(RN(acc * in_scale) * ws)
    (+ bias): in_scale != 1, including a denormal and a scale whose products
    round, against the reference's fused_epilogue_int8 on the same inputs."""
    r = rng(19)
    C, P = 64, 2000
    acc = r.integers(-3_000_000, 3_000_000, size=(P, C), dtype=np.int32)
    acc[:, 0] = r.integers(-600, 600, size=P) | 1
    ws, bias, inv = _specials_epilogue(C, r)
    for in_scale in (0.0173, 3.3, float(np.float32(2.0 ** -130)), 1.0 / 3.0):
        kw = dict(ws=ws, bias=bias, inv_pc=inv, out_scale=0.037, in_scale=in_scale)
        if prelu:
            kw["prelu"] = r.uniform(0, 0.3, C).astype(F32)
        if add:
            kw["add_src"] = r.integers(-128, 128, size=(P, C), dtype=np.int8)
            kw["add_scale"] = 0.021
            kw["add_scale_pc"] = r.uniform(1e-3, 5e-2, C).astype(F32)
        if bn:
            kw["bn_scale"] = r.uniform(0.5, 1.5, C).astype(F32)
            kw["bn_offset"] = r.normal(0, 0.05, C).astype(F32)
        got = oracle.fused_epilogue(acc, **kw)
        assert np.array_equal(got, ref.fused_epilogue(acc, **kw)), in_scale
    # a dropped in-scale multiply would not pass: the scale changes the output
    base = oracle.fused_epilogue(acc, ws=ws, bias=bias, inv_pc=inv, in_scale=1.0)
    assert not np.array_equal(oracle.fused_epilogue(acc, ws=ws, bias=bias, inv_pc=inv,
                                                    in_scale=0.0173), base)


def _round_f32_exact(fr):
    """The fp32 value nearest the exact rational fr, ties to even (one
    rounding, with no double-rounding through float64)."""
    from fractions import Fraction
    c = np.float32(float(fr))
    cands = [np.nextafter(c, F32(-np.inf)), c, np.nextafter(c, F32(np.inf))]
    best = min(cands, key=lambda v: (abs(Fraction(float(v)) - fr),
                                     int(np.array(v, F32).view(np.uint32)) & 1))
    return F32(best)


def test_fc_a_scale_vs_reference_and_closed_form(oracle, ref):
    """FC with A_scale != 1 (FFW2/FFW3 models): out = fma(RN(RN(dot) * a_scale),
    ws, bias) (gemm_int8_matvec.c:78-79, libfastface.c:441-455), against the
    reference's matvec and against the exact closed form (exact int dot,
    fp32 roundings, one rounding of the exact fma)."""
    from fractions import Fraction
    r = rng(20)
    K, N = 25088, 48
    a = r.integers(-128, 128, K, dtype=np.int8)
    a[:64] = -128
    W = r.integers(-127, 128, size=(N, K), dtype=np.int8)
    W[0, :] = -127
    ws = r.uniform(1e-5, 1e-3, N).astype(F32)
    bias = r.normal(0, 0.05, N).astype(F32)
    for a_scale in (0.0213, 7.0, 1.0 / 3.0):
        got = oracle.fc(a, W, ws, bias, a_scale=a_scale)
        assert np.array_equal(got, ref.fc(a, W, ws, bias, a_scale=a_scale)), a_scale
        dot = W.astype(np.int64) @ a.astype(np.int64)
        t = dot.astype(F32) * F32(a_scale)                       # two fp32 roundings
        exp = np.array([_round_f32_exact(Fraction(float(t[n])) * Fraction(float(ws[n])) +
                                         Fraction(float(bias[n]))) for n in range(N)], F32)
        assert np.array_equal(got, exp), a_scale
