"""End-to-end parity of the fastface.h API on the GPU against the oracle
interpreter (itself bit-exact with the reference's fastface_embed).

Weights: the synthetic FFW4 (the reference's real w600k_r50_ffw4.bin is not
distributed); scales: the committed OPSC / OPSC2.
"""
import ctypes as C
import os

import numpy as np
import pytest

import fastface_amd as fa
from fastface_amd import synth
from gpu_util import Dev, check

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


@pytest.fixture(scope="module")
def ff(gpu_lib, synth_ffw4):
    f = fa.FastFace(synth_ffw4, cwd=synth.REPO_ROOT)
    yield f
    f.close()


def _cos(a, b):
    return float(np.dot(a, b) / (np.linalg.norm(a) * np.linalg.norm(b)))


def test_b1_config1(ff, oracle, oracle_model):
    x = synth.faces_uniform(1, 0)
    got = ff.embed(x[0])
    exp, _ = oracle.forward(oracle_model, x)
    assert np.array_equal(got, exp[0])


def test_reference_golden_input_face(ff, oracle, oracle_model):
    x = np.fromfile(os.path.join(GOLDEN, "golden_input.bin"), np.float32).reshape(1, 112, 112, 3)
    exp, _ = oracle.forward(oracle_model, x)
    assert np.array_equal(ff.embed(x[0]), exp[0])


def test_b8_config3(ff, oracle, oracle_model):
    x = synth.faces_normal_clipped(8, 2)
    got = ff.embed_batch(x)
    exp, _ = oracle.forward(oracle_model, x)
    for i in range(8):
        assert _cos(got[i], exp[i]) >= 0.9999
        assert np.abs(got[i] - exp[i]).max() <= 1e-3
    assert np.array_equal(got, exp)


def test_batch_equals_single(ff):
    x = synth.faces_uniform(6, 21)
    batch = ff.embed_batch(x)
    for i in range(6):
        assert np.array_equal(batch[i], ff.embed(x[i]))


def test_rgb8_input_equals_sdk_normalized_fp32(ff):
    """uint8 RGB faces through the input table give bit-for-bit the embeddings
    of the fp32 faces the reference SDK builds from them, in both orders of
    capture (rgb8 and fp32 chains of one batch size coexist)."""
    r = np.random.default_rng(31)
    imgs = r.integers(0, 256, size=(3, 112, 112, 3), dtype=np.uint8)
    imgs[0, :8] = 0
    imgs[0, 8:16] = 255
    faces = (imgs.astype(np.float32) - 127.5) / 127.5
    got = ff.embed_batch_rgb8(imgs)
    exp = ff.embed_batch(faces)
    assert np.array_equal(got, exp)
    assert np.array_equal(ff.embed_batch_rgb8(imgs[:1])[0], ff.embed(faces[0]))
    assert np.array_equal(ff.embed_batch_rgb8(imgs), got)


@pytest.mark.parametrize("B", [2, 23])
def test_rgb8_stem_kernel_vs_oracle(gpu_lib, oracle, B):
    """The input layer alone: uint8 pixels -> table -> int32 accumulators,
    against the oracle's quantization of the SDK-normalized pixels (at 23
    faces workgroups walk several tiles and reuse patch rows)."""
    from gpu_util import run_conv
    r = np.random.default_rng(32)
    imgs = r.integers(0, 256, size=(B, 112, 112, 3), dtype=np.uint8)
    w = r.integers(-128, 128, size=(64, 3, 3, 3), dtype=np.int8)
    inv = np.array([127.0, 126.9, 127.3], np.float32)
    lut = np.empty((3, 256), np.int8)
    assert gpu_lib.ffk_make_rgb8_lut(inv.ctypes.data, lut.ctypes.data) == 0
    got = run_conv(gpu_lib, imgs, w, 1, 1, raw=True, in_lut=lut, flags=fa.FFK_IN_RGB8)
    q = oracle.quant_input((imgs.astype(np.float32) - 127.5) / 127.5, inv)
    assert np.array_equal(got, oracle.conv_i32(q, w, 1, 1))


def test_graph_replays_and_batch_switching(ff):
    x = synth.faces_uniform(5, 22)
    first = ff.embed_batch(x)
    for b in (1, 5, 2, 5, 3):
        out = ff.embed_batch(x[:b])
        assert np.array_equal(out, first[:b])


def test_per_layer_int8_activations(gpu_lib, synth_ffw4, oracle, oracle_model):
    """Every intermediate int8 tensor (after each fused Conv and each BN) is
    bit-exact with the reference interpreter's activation at that op."""
    f = fa.FastFace(synth_ffw4, cwd=synth.REPO_ROOT)
    try:
        assert gpu_lib.fastface_debug_keep_tensors(f.ff, 1) == 0
        x = synth.faces_uniform(2, 23)
        got_emb = f.embed_batch(x)
        exp_emb, dumps = oracle.forward(oracle_model, x, dump_ops=set(range(177)))
        assert len(dumps) >= 70
        for op, t in sorted(dumps.items()):
            buf = np.empty(t.size, np.int8)
            n = gpu_lib.fastface_debug_read(f.ff, op, 2, buf.ctypes.data, buf.nbytes)
            assert n == t.size, "op %d: read %d" % (op, n)
            assert np.array_equal(buf.reshape(t.shape), t), "op %d differs" % op
        assert np.array_equal(got_emb, exp_emb)
        # back to the serving plan (stage outputs stored at their even pixels)
        assert gpu_lib.fastface_debug_keep_tensors(f.ff, 0) == 0
        assert np.array_equal(f.embed_batch(x), exp_emb)
    finally:
        f.close()


@pytest.mark.parametrize("version,with_opsc2", [(3, True), (3, False), (2, True), (4, False)],
                         ids=["ffw3", "ffw3-noopsc2", "ffw2", "ffw4-noopsc2"])
def test_other_formats_end_to_end(gpu_lib, oracle, version, with_opsc2):
    """The formats the loader accepts besides FFW4 with OPSC2: FFW3 and FFW2
    models (per-tensor scales, an in-scale on every conv, the activation scale
    on the FC; FFW2 without conv bias: libfastface.c:335-343,356-422,
    kernels/ffw2_loader.c:96-125) and FFW4 without OPSC2.  Embeddings equal
    the oracle's (itself equal to the reference's fastface_embed on these
    models) at b=1 and on faces of both halves of a split batch of 50; every
    intermediate int8 tensor equals the oracle's at 2 faces; below FFW4 every
    conv launches with the in-scale epilogue."""
    ffw = synth.synthetic_ffw4_path(3, version=version)
    opsc2 = synth.OPSC2_PATH if with_opsc2 else os.path.join(synth.REPO_ROOT, "models", "no_such_v2.bin")
    m = oracle.load_model(ffw, synth.OPSC_PATH, synth.OPSC2_PATH if with_opsc2 else None)
    f = fa.FastFace(ffw, scale_files=(synth.OPSC_PATH, opsc2))
    try:
        info = fa.fastface_step_info()
        n_insc = sum(1 for s in range(gpu_lib.fastface_num_steps(f.ff))
                     if gpu_lib.fastface_get_step(f.ff, s, C.byref(info)) == 0
                     and info.kind == 1 and info.flags & fa.FFK_EPI_INSCALE)
        assert n_insc == (53 if version < 4 else 0)
        x = synth.faces_uniform(50, 60 + version)
        batch = f.embed_batch(x)                        # two halves of 25 faces
        idx = [0, 24, 25, 49]
        exp, _ = oracle.forward(m, x[idx])
        assert np.array_equal(batch[idx], exp)
        assert np.array_equal(f.embed(x[0]), exp[0])
        assert gpu_lib.fastface_debug_keep_tensors(f.ff, 1) == 0
        exp2, dumps = oracle.forward(m, x[:2], dump_ops=set(range(177)))
        assert np.array_equal(f.embed_batch(x[:2]), exp2)
        for op, t in sorted(dumps.items()):
            buf = np.empty(t.size, np.int8)
            assert gpu_lib.fastface_debug_read(f.ff, op, 2, buf.ctypes.data, buf.nbytes) == t.size, op
            assert np.array_equal(buf.reshape(t.shape), t), "op %d differs" % op
    finally:
        f.close()
        oracle.free_model(m)


@pytest.mark.parametrize("with_opsc2", [True, False], ids=["opsc2", "noopsc2"])
def test_standalone_elementwise_ops_end_to_end(gpu_lib, oracle, with_opsc2):
    """A model with elementwise ops that no conv absorbs (synth
    `iresnet_schedule(standalone=True)`: a PReLU after a residual Add, whose
    output is a block input that a 1x1 stride-2 shortcut reads, a BN after
    that PReLU, an Add after a BN, a BN after that Add, a second BN and a
    PReLU after the last one;
    libfastface.c:401-434).  The plan runs them as table steps (five maps, one
    Add); embeddings equal the oracle's (itself equal to the reference's
    fastface_embed on this model) at b=1 and on faces of both halves of a split
    batch; every intermediate int8 tensor equals the oracle's at 2 faces."""
    d = synth.synthetic_standalone_dir()
    ffw = os.path.join(d, "model.ffw4")
    opsc = os.path.join(d, "models", "op_scales.bin")
    opsc2 = os.path.join(d, "models", "op_scales_v2.bin" if with_opsc2 else "no_such_v2.bin")
    m = oracle.load_model(ffw, opsc, opsc2 if with_opsc2 else None)
    f = fa.FastFace(ffw, scale_files=(opsc, opsc2))
    try:
        info = fa.fastface_step_info()
        kinds = []
        for s in range(gpu_lib.fastface_num_steps(f.ff)):
            assert gpu_lib.fastface_get_step(f.ff, s, C.byref(info)) == 0
            kinds.append(info.kind)
        assert kinds.count(3) == 5 and kinds.count(4) == 1 and kinds.count(1) == 53
        x = synth.faces_uniform(50, 70)
        batch = f.embed_batch(x)                        # two halves of 25 faces
        idx = [0, 24, 25, 49]
        exp, _ = oracle.forward(m, x[idx])
        assert np.array_equal(batch[idx], exp)
        assert np.array_equal(f.embed(x[0]), exp[0])
        assert gpu_lib.fastface_debug_keep_tensors(f.ff, 1) == 0
        exp2, dumps = oracle.forward(m, x[:2], dump_ops=set(range(183)))
        assert np.array_equal(f.embed_batch(x[:2]), exp2)
        for op in (53, 55, 70, 71, 74, 179, 180):      # the inserted ops, the BNs after them
            assert op in dumps
        for op, t in sorted(dumps.items()):
            buf = np.empty(t.size, np.int8)
            assert gpu_lib.fastface_debug_read(f.ff, op, 2, buf.ctypes.data, buf.nbytes) == t.size, op
            assert np.array_equal(buf.reshape(t.shape), t), "op %d differs" % op
    finally:
        f.close()
        oracle.free_model(m)


def test_generic_geometries_end_to_end(gpu_lib, oracle):
    """A model with three convs of geometries no tuned kernel has (synth
    `iresnet_schedule(generic=True)`: a 5x5 input layer, a 5x5 stage-3 conv
    with its PReLU, a 1x1 stage-4 conv adding the residual and storing BN of
    the sum): they run on the generic kernel, the rest as before.
    Embeddings equal the oracle's (itself equal to the reference's
    fastface_embed on this model) at b=1 and on faces of both halves of a
    split batch; every intermediate int8 tensor equals the oracle's at 2
    faces."""
    ffw = synth.synthetic_generic_path()
    m = oracle.load_model(ffw, synth.OPSC_PATH, synth.OPSC2_PATH)
    f = fa.FastFace(ffw, cwd=synth.REPO_ROOT)
    try:
        info = fa.fastface_step_info()
        generic = []
        for s in range(gpu_lib.fastface_num_steps(f.ff)):
            assert gpu_lib.fastface_get_step(f.ff, s, C.byref(info)) == 0
            if info.kind == 1 and not gpu_lib.ffk_conv_supported(info.cin, info.cout, info.kh, info.kw,
                                                                  info.stride, info.pad, info.hin, info.win):
                generic.append((info.cin, info.cout, info.kh))
        assert generic == [(3, 64, 5), (256, 256, 5), (512, 512, 1)]
        x = synth.faces_uniform(50, 80)
        batch = f.embed_batch(x)                        # two halves of 25 faces
        idx = [0, 24, 25, 49]
        exp, _ = oracle.forward(m, x[idx])
        assert np.array_equal(batch[idx], exp)
        assert np.array_equal(f.embed(x[0]), exp[0])
        assert gpu_lib.fastface_debug_keep_tensors(f.ff, 1) == 0
        exp2, dumps = oracle.forward(m, x[:2], dump_ops=set(range(177)))
        assert np.array_equal(f.embed_batch(x[:2]), exp2)
        for op, t in sorted(dumps.items()):
            buf = np.empty(t.size, np.int8)
            assert gpu_lib.fastface_debug_read(f.ff, op, 2, buf.ctypes.data, buf.nbytes) == t.size, op
            assert np.array_equal(buf.reshape(t.shape), t), "op %d differs" % op
    finally:
        f.close()
        oracle.free_model(m)


def test_hostile_parameters_end_to_end(gpu_lib, oracle):
    """A model whose parameters defeat the shorter epilogue forms in a few
    layers (synth `hostile_channels`: a NaN weight scale in the input layer,
    +-3e38 biases whose requant values overflow, a PReLU slope of 1.5): the
    plan gives exactly those launches the general forms (no FFK_EPI_IN_RANGE
    where a value can leave the int32 range or is NaN, no FFK_EPI_PRELU_LE1
    there or for the slope above 1) and every other launch its shorter
    forms.  Embeddings
    equal the oracle's (itself equal to the reference's fastface_embed on
    this model) at b=1 and on faces of both halves of a split batch; every
    intermediate int8 tensor equals the oracle's at 2 faces."""
    ffw = synth.synthetic_hostile_path()
    special = synth.hostile_channels(synth.iresnet_schedule())
    m = oracle.load_model(ffw, synth.OPSC_PATH, synth.OPSC2_PATH)
    f = fa.FastFace(ffw, cwd=synth.REPO_ROOT)
    try:
        info = fa.fastface_step_info()
        no_range, no_le1 = [], []
        for s in range(gpu_lib.fastface_num_steps(f.ff)):
            assert gpu_lib.fastface_get_step(f.ff, s, C.byref(info)) == 0
            if info.kind != 1:
                continue
            if not info.flags & fa.FFK_EPI_IN_RANGE:
                no_range.append(info.op_first)
            if info.flags & fa.FFK_EPI_PRELU and not info.flags & fa.FFK_EPI_PRELU_LE1:
                no_le1.append(info.op_first)
        ops = synth.iresnet_schedule()
        convs = sorted(i for i, v in special.items() if v[0] != "slope")
        assert sorted(no_range) == convs                  # the NaN scale and the +-3e38 biases
        # PReLU as a max needs finite, bounded parameters and slopes <= 1
        assert sorted(no_le1) == sorted([i for i in convs if ops[i + 1]["type"] == synth.OP_PRELU] +
                                        [i - 1 for i, v in special.items() if v[0] == "slope"])
        x = synth.faces_uniform(50, 90)
        batch = f.embed_batch(x)                        # two halves of 25 faces
        idx = [0, 24, 25, 49]
        exp, _ = oracle.forward(m, x[idx])
        assert np.array_equal(batch[idx], exp)
        assert np.array_equal(f.embed(x[0]), exp[0])
        assert gpu_lib.fastface_debug_keep_tensors(f.ff, 1) == 0
        exp2, dumps = oracle.forward(m, x[:2], dump_ops=set(range(177)))
        assert np.array_equal(f.embed_batch(x[:2]), exp2)
        for op, t in sorted(dumps.items()):
            buf = np.empty(t.size, np.int8)
            assert gpu_lib.fastface_debug_read(f.ff, op, 2, buf.ctypes.data, buf.nbytes) == t.size, op
            assert np.array_equal(buf.reshape(t.shape), t), "op %d differs" % op
    finally:
        f.close()
        oracle.free_model(m)


def test_stage_outputs_stored_at_even_pixels(ff, gpu_lib):
    """The stem's output X and each stage's last X are read only by the next
    stage's 1x1 stride-2 shortcut: the plan stores them at their even pixels
    and runs those shortcuts at stride 1 over the compact tensors."""
    info = fa.fastface_step_info()
    writers, shortcuts = [], []
    for s in range(gpu_lib.fastface_num_steps(ff.ff)):
        assert gpu_lib.fastface_get_step(ff.ff, s, C.byref(info)) == 0
        if info.kind != 1:
            continue
        if info.flags & fa.FFK_OUT_X_EVEN:
            writers.append((info.cout, info.hout))
            assert info.stores_x and info.flags & fa.FFK_EPI_BN
        if info.kh == 1:
            shortcuts.append((info.cin, info.cout, info.stride, info.hin, info.hout))
    assert writers == [(64, 112), (64, 56), (128, 28), (256, 14)]
    # every conv of the synthetic model has requant values provably in range;
    # 19 launches without a residual also take the one-rounding tail
    n_fma = 0
    for s in range(gpu_lib.fastface_num_steps(ff.ff)):
        assert gpu_lib.fastface_get_step(ff.ff, s, C.byref(info)) == 0
        assert info.kind != 1 or info.flags & fa.FFK_EPI_IN_RANGE, s
        if info.kind == 1 and info.flags & fa.FFK_EPI_FMA_TAIL:
            assert not info.flags & (fa.FFK_EPI_ADD | fa.FFK_EPI_INSCALE)
            n_fma += 1
    assert n_fma == 19
    assert shortcuts == [(64, 64, 1, 56, 56), (64, 128, 1, 28, 28), (128, 256, 1, 14, 14),
                         (256, 512, 1, 7, 7)]


def test_device_resident_api(ff, gpu_lib):
    x = synth.faces_uniform(4, 24)
    exp = ff.embed_batch(x)
    din = Dev(gpu_lib, host=x)
    dout = Dev(gpu_lib, nbytes=4 * 512 * 4)
    assert gpu_lib.fastface_embed_batch_device(ff.ff, din.ptr, 4, dout.ptr, None) == 0
    check(gpu_lib, gpu_lib.ffk_stream_sync(gpu_lib.fastface_stream(ff.ff)))
    assert np.array_equal(dout.get(np.float32, (4, 512)), exp)


def test_api_errors(ff, gpu_lib):
    out = np.empty(512, np.float32)
    x = np.zeros(37632, np.float32)
    assert gpu_lib.fastface_embed(None, x.ctypes.data, out.ctypes.data) != 0
    assert gpu_lib.fastface_embed(ff.ff, None, out.ctypes.data) != 0
    assert gpu_lib.fastface_embed(ff.ff, x.ctypes.data, None) != 0
    assert gpu_lib.fastface_embed_batch(ff.ff, x.ctypes.data, -1, out.ctypes.data) != 0
    assert gpu_lib.fastface_create(b"/nonexistent.ffw4") is None


@pytest.mark.parametrize("B", [256, 1024])
def test_large_batch_properties(ff, oracle, oracle_model, B):
    """BASELINE configs 4/5 sizes: batch rows equal single-face results and the
    oracle on sampled faces (the reference is batch-invariant)."""
    x = synth.faces_uniform(B, 30 + B)
    got = ff.embed_batch(x)
    assert np.isfinite(got).all()
    idx = [0, B // 3, B - 1]
    exp, _ = oracle.forward(oracle_model, x[idx])
    for j, i in enumerate(idx):
        assert np.array_equal(got[i], exp[j]), "face %d" % i
        assert np.array_equal(got[i], ff.embed(x[i]))


@pytest.mark.skipif(not os.path.exists(os.path.join(synth.REPO_ROOT, "models", "w600k_r50_ffw4.bin")),
                    reason="the reference's real weights blob is not distributed")
def test_reference_regression_with_real_weights(gpu_lib):
    """tests/run_regression.py of the reference: bit-exact vs golden_int8_emb.bin,
    cos >= 0.98 vs the ORT fp32 embedding."""
    f = fa.FastFace(os.path.join(synth.REPO_ROOT, "models", "w600k_r50_ffw4.bin"), cwd=synth.REPO_ROOT)
    x = np.fromfile(os.path.join(GOLDEN, "golden_input.bin"), np.float32)
    got = f.embed(x)
    f.close()
    assert np.array_equal(got, np.fromfile(os.path.join(GOLDEN, "golden_int8_emb.bin"), np.float32))
    assert _cos(got, np.fromfile(os.path.join(GOLDEN, "golden_ort_fp32_emb.bin"), np.float32)) >= 0.98


def test_winograd_stage1_network(gpu_lib, synth_ffw4, oracle, oracle_model):
    """fastface_set_conv_algo(WINOGRAD_F23): the five 64-channel 3x3
    stride-1 layers (4 at 56x56, 1 at 112x112) run as integer Winograd; every
    intermediate int8 tensor and the embeddings stay bit-exact with the
    oracle interpreter, and switching back restores the direct path."""
    f = fa.FastFace(synth_ffw4, cwd=synth.REPO_ROOT)
    try:
        x = synth.faces_uniform(3, 31)
        direct = f.embed_batch(x)
        assert gpu_lib.fastface_set_conv_algo(f.ff, 1) == 5
        info = fa.fastface_step_info()
        wino = [s for s in range(gpu_lib.fastface_num_steps(f.ff))
                if gpu_lib.fastface_get_step(f.ff, s, C.byref(info)) == 0
                and info.flags & fa.FFK_ALGO_WINOGRAD]
        assert len(wino) == 5
        assert gpu_lib.fastface_debug_keep_tensors(f.ff, 1) == 0
        got = f.embed_batch(x)
        exp, dumps = oracle.forward(oracle_model, x, dump_ops=set(range(177)))
        for op, t in sorted(dumps.items()):
            buf = np.empty(t.size, np.int8)
            assert gpu_lib.fastface_debug_read(f.ff, op, 3, buf.ctypes.data, buf.nbytes) == t.size
            assert np.array_equal(buf.reshape(t.shape), t), "op %d differs" % op
        assert np.array_equal(got, exp) and np.array_equal(got, direct)
        assert gpu_lib.fastface_debug_keep_tensors(f.ff, 0) == 0
        assert np.array_equal(f.embed(x[1]), exp[1])          # b=1, Winograd, graph
        assert gpu_lib.fastface_set_conv_algo(f.ff, 0) == 0
        assert np.array_equal(f.embed_batch(x), exp)
        assert gpu_lib.fastface_set_conv_algo(f.ff, 7) == -1
    finally:
        f.close()


def test_general_epilogue_forms(gpu_lib, synth_ffw4, oracle, oracle_model):
    """fastface_set_epilogue_forms(1): every conv launches with the general
    epilogue forms (compare/select PReLU, the x86 out-of-range emulation)
    instead of the shorter ones the plan proved value-identical.  The
    embeddings stay bit-exact with the oracle at b=1, 3 faces and a split
    batch of 101; the step flags show the change; switching back restores
    the plan's forms."""
    f = fa.FastFace(synth_ffw4, cwd=synth.REPO_ROOT)
    try:
        fast = fa.FFK_EPI_PRELU_LE1 | fa.FFK_EPI_IN_RANGE
        info = fa.fastface_step_info()
        n = gpu_lib.fastface_num_steps(f.ff)

        def n_fast():
            return sum(1 for s in range(n) if gpu_lib.fastface_get_step(f.ff, s, C.byref(info)) == 0
                       and info.kind == 1 and info.flags & fast)
        n_convs = n_fast()
        assert n_convs == n - 1                       # every conv of the synthetic model qualifies
        x = synth.faces_uniform(101, 33)
        shorter = f.embed_batch(x)
        assert gpu_lib.fastface_set_epilogue_forms(f.ff, 1) == n_convs
        assert n_fast() == 0
        exp, _ = oracle.forward(oracle_model, x[:3])
        assert np.array_equal(f.embed(x[0]), exp[0])
        assert np.array_equal(f.embed_batch(x[:3]), exp)
        assert np.array_equal(f.embed_batch(x), shorter)
        assert gpu_lib.fastface_set_epilogue_forms(f.ff, 0) == n_convs
        assert n_fast() == n_convs
        assert np.array_equal(f.embed_batch(x), shorter)
        assert gpu_lib.fastface_set_epilogue_forms(f.ff, 2) == -1
    finally:
        f.close()


def test_shortcut_fusion(gpu_lib, synth_ffw4, oracle, oracle_model):
    """fastface_set_shortcut_fusion: each stage's stride-2 conv and 1x1
    shortcut run as one launch (the default) or as two.  The plan has the
    four pairs of IResNet-50; embeddings are bit-identical either way at 701
    faces (two halves of 350 and 351, where stages 1-3 take the large tiles
    and so fuse) and at 9 faces (where only stage 1 does), and equal the
    oracle's on faces of both halves."""
    f = fa.FastFace(synth_ffw4, cwd=synth.REPO_ROOT)
    try:
        x = synth.faces_uniform(701, 35)
        fused = f.embed_batch(x)
        small = f.embed_batch(x[:9])
        assert gpu_lib.fastface_set_shortcut_fusion(f.ff, 0) == 4
        assert np.array_equal(f.embed_batch(x), fused)
        assert np.array_equal(f.embed_batch(x[:9]), small)
        assert gpu_lib.fastface_set_shortcut_fusion(f.ff, 1) == 4
        assert np.array_equal(f.embed_batch(x), fused)
        idx = [0, 349, 350, 700]
        exp, _ = oracle.forward(oracle_model, x[idx])
        assert np.array_equal(fused[idx], exp)
        assert gpu_lib.fastface_set_shortcut_fusion(f.ff, 2) == -1
    finally:
        f.close()


def test_streamed_host_batch_equals_one_shot(ff, gpu_lib):
    """Host batches stream in chunks (copy of one chunk during the compute of
    the previous): 600 fp32 faces as 256 + 344, 2100 as 256 + 768 + 768 + 308
    (three launch chains), 2100 uint8 faces as 4 x 512 + 52.  Embeddings equal
    the device-resident one-shot path's and the single-face path's; a small
    batch afterwards still reads its own buffers."""
    for B in (600, 2100):
        x = synth.faces_uniform(B, 41)
        got = ff.embed_batch(x)
        din, dout = Dev(gpu_lib, host=x), Dev(gpu_lib, nbytes=B * 512 * 4)
        assert gpu_lib.fastface_embed_batch_device(ff.ff, din.ptr, B, dout.ptr, None) == 0
        check(gpu_lib, gpu_lib.ffk_stream_sync(gpu_lib.fastface_stream(ff.ff)))
        assert np.array_equal(got, dout.get(np.float32, (B, 512)))
        for i in (0, 255, 256, 1023, 1024, 1791, 1792, B - 1):
            if i < B:
                assert np.array_equal(ff.embed(x[i]), got[i]), (B, i)
        din.free(); dout.free()
    x = synth.faces_uniform(600, 41)
    got = ff.embed_batch(x)
    B8 = 2100
    imgs = np.random.default_rng(42).integers(0, 256, size=(B8, 112, 112, 3), dtype=np.uint8)
    got8 = ff.embed_batch_rgb8(imgs)
    d8, dout8 = Dev(gpu_lib, host=imgs), Dev(gpu_lib, nbytes=B8 * 512 * 4)
    assert gpu_lib.fastface_embed_batch_rgb8_device(ff.ff, d8.ptr, B8, dout8.ptr, None) == 0
    check(gpu_lib, gpu_lib.ffk_stream_sync(gpu_lib.fastface_stream(ff.ff)))
    assert np.array_equal(got8, dout8.get(np.float32, (B8, 512)))
    assert np.array_equal(ff.embed_batch_rgb8(imgs[2047:2049]), got8[2047:2049])
    assert np.array_equal(ff.embed_batch(x[:3]), got[:3])


def test_split_chain_equals_unsplit_halves(gpu_lib, synth_ffw4):
    """Batches of 24 faces or more run as two halves, each on its own stream
    inside one captured graph (fork and join), each half in its own region
    of every activation buffer, both with the FFK_SHARED_GPU tiling.  Every
    embedding of every face equals the one-chain result of 16-face batches
    (faces are independent) for 25, 49, 101, 129, 256, 384 and 1025 faces
    (halves of 12-513, each with its own workspace), captured and then
    replayed;
    1024 uint8 faces against 16-face batches; the Winograd stage-1 path split
    against direct.  (Regression: halves that shared buffer regions corrupted
    faces from B/4 on, because a buffer holds tensors of different sizes at
    different layers and the halves run different layers at once.)"""
    f = fa.FastFace(synth_ffw4, cwd=synth.REPO_ROOT)
    try:
        stream = gpu_lib.fastface_stream(f.ff)

        def pieces(fn, a):
            return np.concatenate([fn(a[i:i + 16]) for i in range(0, len(a), 16)])

        for B in (25, 49, 101, 129, 256, 384, 1025):
            x = synth.faces_uniform(B, 61 + B)
            exp = pieces(f.embed_batch, x)
            din, dout = Dev(gpu_lib, host=x), Dev(gpu_lib, nbytes=B * 512 * 4)
            for rep in range(2):                  # capture, then replay
                assert gpu_lib.fastface_embed_batch_device(f.ff, din.ptr, B, dout.ptr, None) == 0
                check(gpu_lib, gpu_lib.ffk_stream_sync(stream))
                got = dout.get(np.float32, (B, 512))
                bad = [i for i in range(B) if not np.array_equal(got[i], exp[i])]
                assert not bad, "B=%d replay %d: faces %s differ" % (B, rep, bad[:16])
            assert np.array_equal(f.embed_batch(x), exp), B     # host path
        imgs = np.random.default_rng(62).integers(0, 256, size=(1024, 112, 112, 3), dtype=np.uint8)
        d8, dout = Dev(gpu_lib, host=imgs), Dev(gpu_lib, nbytes=1024 * 512 * 4)
        assert gpu_lib.fastface_embed_batch_rgb8_device(f.ff, d8.ptr, 1024, dout.ptr, None) == 0
        check(gpu_lib, gpu_lib.ffk_stream_sync(stream))
        assert np.array_equal(dout.get(np.float32, (1024, 512)), pieces(f.embed_batch_rgb8, imgs))
        x = synth.faces_uniform(1024, 64)
        din = Dev(gpu_lib, host=x)
        assert gpu_lib.fastface_embed_batch_device(f.ff, din.ptr, 1024, dout.ptr, None) == 0
        check(gpu_lib, gpu_lib.ffk_stream_sync(stream))
        direct = dout.get(np.float32, (1024, 512))
        assert gpu_lib.fastface_set_conv_algo(f.ff, 1) == 5
        assert gpu_lib.fastface_embed_batch_device(f.ff, din.ptr, 1024, dout.ptr, None) == 0
        check(gpu_lib, gpu_lib.ffk_stream_sync(stream))
        assert np.array_equal(dout.get(np.float32, (1024, 512)), direct)
    finally:
        f.close()


def test_concurrent_contexts(gpu_lib, synth_ffw4):
    """One context per thread (fastface.h): two contexts embedding on two
    threads at once -- each with its own stream, buffers and captured chains
    -- give the embeddings one context gives alone (the reference Go SDK's
    concurrent-instances test)."""
    import threading
    xs = [synth.faces_uniform(5, 50), synth.faces_uniform(3, 51)]
    ctxs = [fa.FastFace(synth_ffw4, cwd=synth.REPO_ROOT) for _ in range(2)]
    try:
        exp = [ctxs[0].embed_batch(x) for x in xs]
        out, errs = [[], []], []

        def work(i):
            try:
                for _ in range(6):
                    out[i].append(ctxs[i].embed_batch(xs[i]))
                    out[i].append(ctxs[i].embed(xs[i][0])[None])
            except Exception as e:          # reported below, in the main thread
                errs.append(e)
        th = [threading.Thread(target=work, args=(i,)) for i in range(2)]
        for t in th:
            t.start()
        for t in th:
            t.join(timeout=60)
        assert not errs and not any(t.is_alive() for t in th)
        for i in range(2):
            for k, got in enumerate(out[i]):
                want = exp[i] if k % 2 == 0 else exp[i][:1]
                assert np.array_equal(got, want), (i, k)
    finally:
        for c in ctxs:
            c.close()


def test_concurrent_contexts_streamed(gpu_lib, synth_ffw4):
    """Two contexts streaming host batches of 600 fp32 faces on two threads
    at once: each call goes through its context's pinned staging buffers and
    copy threads; the embeddings equal one context's alone, call after call,
    and a context destroyed after streaming stops its copy threads."""
    import threading
    xs = [synth.faces_uniform(600, 52), synth.faces_uniform(600, 53)]
    ctxs = [fa.FastFace(synth_ffw4, cwd=synth.REPO_ROOT) for _ in range(2)]
    try:
        exp = [ctxs[0].embed_batch(x) for x in xs]
        out, errs = [[], []], []

        def work(i):
            try:
                for _ in range(3):
                    out[i].append(ctxs[i].embed_batch(xs[i]))
            except Exception as e:          # reported below, in the main thread
                errs.append(e)
        th = [threading.Thread(target=work, args=(i,)) for i in range(2)]
        for t in th:
            t.start()
        for t in th:
            t.join(timeout=120)
        assert not errs and not any(t.is_alive() for t in th)
        for i in range(2):
            for got in out[i]:
                assert np.array_equal(got, exp[i]), i
    finally:
        for c in ctxs:
            c.close()


def test_device_calls_on_caller_streams_are_ordered(gpu_lib, synth_ffw4, oracle, oracle_model):
    """Device calls on two caller streams, interleaved with host calls on the
    context stream and with no host wait in between, never overlap on the
    context's I/O descriptor, activation buffers or split-K workspace: each
    call's embeddings equal the oracle's.  One face takes the split-K kernels
    (arrival counters in the workspace); an overlap would leave a counter
    wrong and corrupt every later small batch, so the sequence repeats."""
    f = fa.FastFace(synth_ffw4, cwd=synth.REPO_ROOT)
    streams = [C.c_void_p(), C.c_void_p()]
    for s in streams:
        check(gpu_lib, gpu_lib.ffk_stream_create(C.byref(s)))
    try:
        x = synth.faces_uniform(4, 61)
        exp, _ = oracle.forward(oracle_model, x)
        din = [Dev(gpu_lib, host=x[i:i + 1]) for i in range(3)]
        din3 = Dev(gpu_lib, host=x[:3])
        outs = []
        for rep in range(4):
            o = [Dev(gpu_lib, nbytes=512 * 4) for _ in range(3)]
            o3 = Dev(gpu_lib, nbytes=3 * 512 * 4)
            s1, s2 = streams[rep % 2], streams[1 - rep % 2]
            assert gpu_lib.fastface_embed_batch_device(f.ff, din[0].ptr, 1, o[0].ptr, s1) == 0
            host1 = f.embed(x[3])                                   # context stream, b=1
            assert gpu_lib.fastface_embed_batch_device(f.ff, din3.ptr, 3, o3.ptr, s2) == 0
            assert gpu_lib.fastface_embed_batch_device(f.ff, din[1].ptr, 1, o[1].ptr, s1) == 0
            # same I/O pointers as the previous call, another stream
            assert gpu_lib.fastface_embed_batch_device(f.ff, din[1].ptr, 1, o[1].ptr, s2) == 0
            assert gpu_lib.fastface_embed_batch_device(f.ff, din[2].ptr, 1, o[2].ptr, None) == 0
            outs.append((o, o3, host1))
        for s in streams:
            check(gpu_lib, gpu_lib.ffk_stream_sync(s))
        check(gpu_lib, gpu_lib.ffk_stream_sync(gpu_lib.fastface_stream(f.ff)))
        for rep, (o, o3, host1) in enumerate(outs):
            assert np.array_equal(host1, exp[3]), rep
            for i in range(3):
                assert np.array_equal(o[i].get(np.float32, (512,)), exp[i]), (rep, i)
            assert np.array_equal(o3.get(np.float32, (3, 512)), exp[:3]), rep
        assert np.array_equal(f.embed(x[0]), exp[0])
    finally:
        for s in streams:
            gpu_lib.ffk_stream_destroy(s)
        f.close()


def test_reference_c_caller_unchanged(gpu_lib, synth_ffw4, oracle, oracle_model, tmp_path):
    """The reference's own C-API client, test_libfastface.c (reference
    Makefile:72-73), compiled unchanged against include/fastface.h and linked to
    libfastface_amd.so (oracle/Makefile `ref`), run in a directory laid out as
    it expects: models/w600k_r50_ffw4.bin (here the synthetic FFW4),
    models/op_scales{,_v2}.bin and tests/golden_input.bin.  Its printed
    emb[0..4] must equal the oracle's embedding of that face (its own %g
    formatting of the same floats)."""
    import subprocess
    exe = os.path.join(synth.REPO_ROOT, "oracle", "_ref", "test_libfastface")
    if not os.path.exists(exe):
        pytest.skip("oracle/_ref/test_libfastface not built (needs /root/reference at build time)")
    (tmp_path / "models").mkdir()
    (tmp_path / "tests").mkdir()
    os.symlink(synth_ffw4, tmp_path / "models" / "w600k_r50_ffw4.bin")
    os.symlink(synth.OPSC_PATH, tmp_path / "models" / "op_scales.bin")
    os.symlink(synth.OPSC2_PATH, tmp_path / "models" / "op_scales_v2.bin")
    os.symlink(os.path.join(GOLDEN, "golden_input.bin"), tmp_path / "tests" / "golden_input.bin")
    env = {k: v for k, v in os.environ.items() if k != "OPSC2_PATH"}
    r = subprocess.run([exe], cwd=str(tmp_path), capture_output=True, text=True, timeout=120, env=env)
    assert r.returncode == 0, r.stderr
    x = np.fromfile(os.path.join(GOLDEN, "golden_input.bin"), np.float32).reshape(1, 112, 112, 3)
    exp, _ = oracle.forward(oracle_model, x)
    line = [l for l in r.stdout.splitlines() if l.startswith("emb[0..4] = ")]
    assert line, r.stdout
    want = "emb[0..4] = " + " ".join("%g" % float(v) for v in exp[0, :5])
    assert line[0] == want
