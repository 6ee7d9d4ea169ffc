"""The model loader and launch planner (ff_model.c, ff_plan.c) on valid,
truncated and corrupt weight and scale files, run under AddressSanitizer and
UndefinedBehaviorSanitizer (fastface_amd/csrc/host/ff_loader_check.c, built
by `make -C fastface_amd/csrc san`; CPU only).

Acceptance rules follow the reference (kernels/ffw2_loader.c:96-155,
libfastface.c:133-204,235-240): a weights file with a bad magic, an unknown
op type or missing bytes, and an OPSC file that is missing, malformed or has
another op count, make create fail (NULL); an OPSC2 file that is missing,
malformed or has another op count is dropped and the per-tensor OPSC scales
are used (the reference degrades the same way; unlike it, a mid-file OPSC2
error drops the whole file rather than keeping the tables read so far).
The reference reads its mmapped file without bounds checks, so truncation
has no reference behaviour to match: here it is an error.
"""
import os
import struct
import subprocess

import numpy as np
import pytest

from fastface_amd import synth

ROOT = synth.REPO_ROOT
CSRC = os.path.join(ROOT, "fastface_amd", "csrc")
EXE = os.path.join(CSRC, "_build", "san", "ff_loader_check")
LIB = os.path.join(ROOT, "fastface_amd", "lib", "libfastface_amd.so")


@pytest.fixture(scope="module")
def checker():
    if not os.path.exists(LIB):
        pytest.skip("library not built")
    subprocess.run(["make", "-s", "-C", CSRC, "san"], check=True, capture_output=True)
    return EXE


def run(exe, ffw, opsc=synth.OPSC_PATH, opsc2=synth.OPSC2_PATH):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([exe, ffw, opsc, opsc2 or "-"], capture_output=True, text=True, env=env,
                       timeout=120)
    assert r.returncode == 0, "sanitizer or crash:\n" + r.stderr[-3000:]
    assert "runtime error" not in r.stderr and "AddressSanitizer" not in r.stderr, r.stderr[-3000:]
    out = {}
    for line in r.stdout.splitlines():
        t = line.split()
        for k, v in zip(t[0::2], t[1::2]):
            out.setdefault(k, v)
    return out


def op_offsets(blob):
    """Byte offset of every op record of an FFW3/FFW4 blob (the layout
    kernels/ffw2_loader.c:96-155 parses), and the end offset."""
    n = struct.unpack_from("<I", blob, 4)[0]
    off, offs = 8, []
    for _ in range(n):
        offs.append(off)
        t = blob[off]
        off += 1
        if t == synth.OP_CONV:
            cin, cout, kh, kw = struct.unpack_from("<4H", blob, off)
            off += 12 + cout * cin * kh * kw + 8 * cout
        elif t in (synth.OP_BN,):
            c = struct.unpack_from("<H", blob, off)[0]
            off += 2 + 8 * c
        elif t == synth.OP_PRELU:
            c = struct.unpack_from("<H", blob, off)[0]
            off += 2 + 4 * c
        elif t == synth.OP_GEMM:
            N, K = struct.unpack_from("<2I", blob, off)
            off += 8 + N * K + 8 * N
    return offs, off


@pytest.fixture(scope="module")
def blob(synth_ffw4):
    with open(synth_ffw4, "rb") as f:
        return f.read()


def write(tmp_path, name, data):
    p = tmp_path / name
    p.write_bytes(bytes(data))
    return str(p)


def test_valid_model_loads_and_plans(checker, synth_ffw4):
    o = run(checker, synth_ffw4)
    assert o["load"] == "0" and o["version"] == "4" and o["ops"] == "177" and o["v2"] == "1"
    assert o["plan"] == "0" and o["steps"] == "54"
    o = run(checker, synth_ffw4, opsc2=None)            # OPSC only: per-tensor scales
    assert o["load"] == "0" and o["v2"] == "0" and o["plan"] == "0"


def test_fused_pairs_never_write_what_they_read(checker, synth_ffw4):
    """A stage's stride-2 conv and its 1x1 shortcut may run as one launch
    (ff_plan_pair); the shortcut's outputs must then take no buffer the
    launch still reads: the conv's input, the shortcut's input, the conv's
    output.  The buffer plan releases the pair's inputs only after it; a
    regression would be a data race on the GPU, so it is checked here."""
    o = run(checker, synth_ffw4)
    assert o["pairs"] == "4" and o["overlaps"] == "0"


def test_fma_tail_launches(checker, synth_ffw4):
    """The plan proves the one-rounding requant tail (ffk_requant_fma_ok) on
    19 of the synthetic FFW4's 29 in-range launches without a residual (the
    other ten have a channel whose small PReLU slope makes every float near
    f*inv = -1/2 reachable); none of an FFW3 model (in-scale on every conv)."""
    o = run(checker, synth_ffw4)
    assert o["in_range"] == "53" and o["fma_tail"] == "19" and o["fma_bad"] == "0"
    o = run(checker, synth.synthetic_ffw4_path(3, version=3))
    assert o["fma_tail"] == "0" and o["fma_bad"] == "0"


def test_layout_walk_matches_file(blob):
    offs, end = op_offsets(blob)
    assert len(offs) == 177 and end == len(blob)


def test_truncated_weights_fail(checker, blob, tmp_path):
    offs, end = op_offsets(blob)
    gemm = [o for o in offs if blob[o] == synth.OP_GEMM][0]
    cuts = [0, 3, 7, 8, offs[0] + 5, offs[0] + 20, offs[5] + 1, gemm + 6, gemm + 5000, end - 1]
    for cut in cuts:
        o = run(checker, write(tmp_path, "t%d.ffw" % cut, blob[:cut]))
        assert o["load"] != "0", cut


def test_corrupt_weights_fail(checker, blob, tmp_path):
    offs, _ = op_offsets(blob)
    bad_magic = bytearray(blob)
    bad_magic[:4] = b"FFWX"
    bad_op = bytearray(blob)
    bad_op[offs[5]] = 99                                  # unknown op type
    zero_ops = bytearray(blob)
    struct.pack_into("<I", zero_ops, 4, 0)
    many_ops = bytearray(blob)
    struct.pack_into("<I", many_ops, 4, 0x7FFFFFFF)
    big_conv = bytearray(blob)
    struct.pack_into("<H", big_conv, offs[0] + 3, 0xFFFF)  # Cout of the stem
    gemm = [o for o in offs if blob[o] == synth.OP_GEMM][0]
    big_gemm = bytearray(blob)
    struct.pack_into("<2I", big_gemm, gemm + 1, 0xFFFFFFFF, 0xFFFFFFFF)
    for name, data in [("magic", bad_magic), ("op", bad_op), ("zero", zero_ops),
                       ("many", many_ops), ("conv", big_conv), ("gemm", big_gemm)]:
        o = run(checker, write(tmp_path, name + ".ffw", data))
        assert o["load"] != "0", name


def test_opsc_errors_fail(checker, synth_ffw4, tmp_path):
    with open(synth.OPSC_PATH, "rb") as f:
        opsc = f.read()
    n = struct.unpack_from("<I", opsc, 4)[0]
    assert n == 177
    fewer = bytearray(opsc[:12 + 176 * 4])
    struct.pack_into("<I", fewer, 4, 176)                # n_ops mismatch
    cases = {"missing": str(tmp_path / "nope.bin"),
             "magic": write(tmp_path, "m.bin", b"OPSX" + opsc[4:]),
             "truncated": write(tmp_path, "t.bin", opsc[:100]),
             "mismatch": write(tmp_path, "n.bin", fewer),
             "empty": write(tmp_path, "e.bin", b"")}
    for name, path in cases.items():
        o = run(checker, synth_ffw4, opsc=path)
        assert o["load"] != "0", name


def test_opsc2_errors_degrade_to_per_tensor(checker, synth_ffw4, tmp_path):
    with open(synth.OPSC2_PATH, "rb") as f:
        v2 = f.read()
    mism = bytearray(v2)
    struct.pack_into("<I", mism, 5, 176)
    huge = bytearray(v2)
    struct.pack_into("<I", huge, 9, 0xFFFFFFFF)           # input channel count
    cases = {"missing": str(tmp_path / "nope2.bin"),
             "magic": write(tmp_path, "m2.bin", b"OPSCX" + v2[5:]),
             "mismatch": write(tmp_path, "n2.bin", mism),
             "truncated_mid": write(tmp_path, "t2.bin", v2[:len(v2) // 2]),
             "truncated_end": write(tmp_path, "u2.bin", v2[:-1]),
             "huge_in": write(tmp_path, "h2.bin", huge)}
    for name, path in cases.items():
        o = run(checker, synth_ffw4, opsc2=path)
        assert o["load"] == "0" and o["v2"] == "0" and o["plan"] == "0", name


def test_unsupported_op_sequence_fails_plan(checker, tmp_path):
    """A PReLU on the fp32 input faces (no conv before it; only the stem conv
    reads them, quantizing on the fly) is a valid file the planner rejects
    with a message: create fails instead of running it otherwise."""
    ffw = b"FFW4" + struct.pack("<I", 1) + bytes([synth.OP_PRELU]) + struct.pack("<H", 3) + \
        np.full(3, 0.25, np.float32).tobytes()
    opsc = b"OPSC" + struct.pack("<I", 1) + np.float32(1 / 127).tobytes() + \
        np.float32(0.05).tobytes()
    o = run(checker, write(tmp_path, "p.ffw", ffw), opsc=write(tmp_path, "p.bin", opsc), opsc2=None)
    assert o["load"] == "0" and o["plan"] != "0"


def test_weight_arena_equals_independent_packing(checker, synth_ffw4, blob, oracle, tmp_path):
    """The plan's weight arena (filled by packing jobs on several threads)
    equals the same contents built independently here with numpy from the
    FFW4 file: every conv's weights in reduction order k = (kh*KW + kw)*Cin +
    ci cut into [K/64][Cout][64], the FC's columns moved from the reference's
    NCHW flatten order to NHWC and cut the same way, each BN table the
    oracle's BN requant of the 256 int8 values, each Winograd region the
    packer's output for that conv."""
    import fastface_amd as fa
    lib = fa.load()
    dump = str(tmp_path / "arena")
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0")
    r = subprocess.run([checker, synth_ffw4, synth.OPSC_PATH, synth.OPSC2_PATH, dump],
                       capture_output=True, text=True, env=env, timeout=120)
    assert r.returncode == 0, r.stderr[-2000:]
    arena = np.fromfile(dump + ".bin", np.int8)
    params = np.fromfile(dump + ".params.bin", np.float32)
    offs, _ = op_offsets(blob)

    def conv_w(op):
        cin, cout, kh, kw = struct.unpack_from("<4H", blob, offs[op] + 1)
        w = np.frombuffer(blob, np.int8, cout * cin * kh * kw, offs[op] + 13)
        return w.reshape(cout, cin, kh, kw)

    seen = set()
    for line in open(dump + ".txt"):
        kind, op, off, n, *rest = line.split()
        op, off, n = int(op), int(off), int(n)
        got = arena[off:off + n]
        seen.add(kind)
        if kind == "conv":
            w = conv_w(op)
            cout, cin, kh, kw = w.shape
            K = kh * kw * cin
            steps = -(-K // 64)
            wk = np.zeros((cout, steps * 64), np.int8)
            wk[:, :K] = w.transpose(0, 2, 3, 1).reshape(cout, K)
            exp = wk.reshape(cout, steps, 64).transpose(1, 0, 2).reshape(-1)
        elif kind == "wino":
            w = conv_w(op)
            exp = np.empty(n, np.int8)
            assert lib.ffk_pack_winograd_weights(np.ascontiguousarray(w).ctypes.data, w.shape[0], w.shape[1],
                                                 exp.ctypes.data) == 0
        elif kind == "fc":
            N, K = struct.unpack_from("<2I", blob, offs[op] + 1)
            W = np.frombuffer(blob, np.int8, N * K, offs[op] + 9).reshape(N, 512, K // 512)
            Wn = W.transpose(0, 2, 1).reshape(N, K)              # column c*HW + hw -> hw*C + c
            exp = Wn.reshape(N, K // 64, 64).transpose(1, 0, 2).reshape(-1)
        else:                                                    # bn: table from the step's BN rows
            C_, p_off = n // 256, int(rest[0])
            rows = params[p_off:p_off + fa.FFK_NPARAM * C_].reshape(fa.FFK_NPARAM, C_)
            q = np.arange(-128, 128, dtype=np.int8).reshape(256, 1).repeat(C_, axis=1)
            exp = oracle.bn_prelu_requant(q, in_scale_pc=rows[fa.FFK_P_BN_SIN], bn_scale=rows[fa.FFK_P_BN_S],
                                          bn_offset=rows[fa.FFK_P_BN_O], inv_pc=rows[fa.FFK_P_BN_INV]).T.reshape(-1)
        assert np.array_equal(got, exp), (kind, op)
    assert seen == {"conv", "wino", "bn", "fc"}


def test_launch_lists_without_a_gpu(checker, synth_ffw4):
    """The chain's launch list at b=1, 8, 256 and 1024 faces (two halves from
    24), from the plan and the library's host-side launch choice: 53 convs +
    the FC per chain or half, every conv with a kernel variant and (but the
    persistent input layer) a workgroup count; small batches take the
    split-K / small-grid variants, 512-face halves the large tiles."""
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0")
    r = subprocess.run([checker, synth_ffw4, synth.OPSC_PATH, synth.OPSC2_PATH, "-", "--launches",
                        "1", "8", "256", "1024"], capture_output=True, text=True, env=env, timeout=120)
    assert r.returncode == 0, r.stderr[-2000:]
    chains = {}
    for line in r.stdout.splitlines():
        t = line.split()
        if t[0] == "launch":
            chains.setdefault(t[1], []).append(t)
    assert sorted(chains) == sorted(["1", "8", "256/h0", "256/h1", "1024/h0", "1024/h1"])
    for tag, launches in chains.items():
        assert len(launches) == 54, tag
        for t in launches:
            if t[3] == "fc":
                assert t[4] == ("matvec" if tag in ("1", "8") else "gemm"), t
                continue
            assert t[4] != "none", t
            assert int(t[5]) > 0 or t[4] == "stem", t
    variants = lambda tag: {t[4] for t in chains[tag]}
    assert "splitk" in variants("1") and "splitk" not in variants("1024/h0")
    assert "patch_kg" not in variants("1024/h0") and "patch" in variants("1024/h0")


def test_standalone_ops_plan_and_tables(checker, oracle, tmp_path):
    """The model with stand-alone elementwise ops (synth
    `iresnet_schedule(standalone=True)`) plans under the sanitizers with and
    without OPSC2: 53 convs + 5 table maps + 1 table Add + the FC, each map or
    Add in every chain's launch list at its tensor's pixel count; each map's
    table is the oracle's bn_prelu_requant of the 256 int8 values with the
    step's rows, whose BN / PReLU rows are the file's; the Add's table is
    the oracle's add_requant of every pair with the per-tensor scales the
    reference passes (libfastface.c:429-434: the current scale, the saved
    tensor's, the op's own)."""
    import fastface_amd as fa
    d = synth.synthetic_standalone_dir()
    ffw = os.path.join(d, "model.ffw4")
    opsc, opsc2 = os.path.join(d, "models", "op_scales.bin"), os.path.join(d, "models", "op_scales_v2.bin")
    with open(ffw, "rb") as f:
        blob = f.read()
    offs, _ = op_offsets(blob)
    _, sc = synth.read_opsc(opsc)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0")
    for v2 in (opsc2, "-"):
        dump = str(tmp_path / ("arena" + ("2" if v2 != "-" else "")))
        r = subprocess.run([checker, ffw, opsc, v2, dump], capture_output=True, text=True, env=env,
                           timeout=120)
        assert r.returncode == 0, r.stderr[-2000:]
        assert "plan 0 steps 60 " in r.stdout, r.stdout
        arena = np.fromfile(dump + ".bin", np.int8)
        params = np.fromfile(dump + ".params.bin", np.float32)
        maps = []
        for line in open(dump + ".txt"):
            kind, op, off, n, *rest = line.split()
            if kind not in ("map", "add"):
                continue
            op, off, n, p_off = int(op), int(off), int(n), int(rest[0])
            got = arena[off:off + n]
            if kind == "add":
                assert op == 71 and n == 65536
                a_s, b_s, o_s = params[p_off:p_off + 3]
                assert (a_s, b_s, o_s) == (sc[68], sc[68], sc[71])
                v = np.arange(-128, 128, dtype=np.int8)
                exp = oracle.add_requant(np.repeat(v, 256), a_s, np.tile(v, 256), b_s, o_s)
                assert np.array_equal(got, exp)
                continue
            maps.append(op)
            C_ = n // 256
            rows = params[p_off:p_off + fa.FFK_NPARAM * C_].reshape(fa.FFK_NPARAM, C_)
            t = blob[offs[op]]
            file_vals = np.frombuffer(blob, np.float32, (2 if t == synth.OP_BN else 1) * C_, offs[op] + 3)
            if t == synth.OP_BN:
                assert np.array_equal(rows[fa.FFK_P_BN_S], file_vals[:C_])
                assert np.array_equal(rows[fa.FFK_P_BN_O], file_vals[C_:])
            else:
                assert np.array_equal(rows[fa.FFK_P_SLOPE], file_vals)
            q = np.arange(-128, 128, dtype=np.int8).reshape(256, 1).repeat(C_, axis=1)
            bn = t == synth.OP_BN
            exp = oracle.bn_prelu_requant(q, in_scale_pc=rows[fa.FFK_P_BN_SIN],
                                          bn_scale=rows[fa.FFK_P_BN_S] if bn else None,
                                          bn_offset=rows[fa.FFK_P_BN_O] if bn else None,
                                          prelu=None if bn else rows[fa.FFK_P_SLOPE],
                                          inv_pc=rows[fa.FFK_P_BN_INV]).T.reshape(-1)
            assert np.array_equal(got, exp), op
        assert maps == [53, 55, 74, 179, 180]
    r = subprocess.run([checker, ffw, opsc, opsc2, "-", "--launches", "1", "50"], capture_output=True,
                       text=True, env=env, timeout=120)
    assert r.returncode == 0, r.stderr[-2000:]
    chains = {}
    for line in r.stdout.splitlines():
        t = line.split()
        if t[0] == "launch":
            chains.setdefault(t[1], []).append(t)
    assert sorted(chains) == ["1", "50/h0", "50/h1"]
    for tag, launches in chains.items():
        faces = 1 if tag == "1" else 25
        assert len(launches) == 60
        tables = [(t[3], int(t[4]), int(t[5])) for t in launches if t[3] in ("map", "add")]
        assert tables == [("map", 128, 784 * faces), ("map", 128, 784 * faces), ("add", 256, 196 * faces),
                          ("map", 256, 196 * faces), ("map", 512, 49 * faces), ("map", 512, 49 * faces)]



def _tiny_model(tmp_path, name, ops):
    """A small FFW4 of `ops` (synth op dicts) with OPSC / OPSC2 files whose
    entries are flat 0.02 scales of each op's channel count."""
    per_op, sc, c = [], [], 3
    for op in ops:
        if op["type"] == synth.OP_CONV:
            c = op["Cout"]
        n = op.get("C", c)
        has = op["type"] in (synth.OP_CONV, synth.OP_BN, synth.OP_PRELU)
        per_op.append(np.full(n, 0.02, np.float32) if has else None)
        sc.append(0.02 if has else 0.0)
    opsc2 = (np.full(3, 1 / 127, np.float32), per_op)
    ffw = str(tmp_path / (name + ".ffw4"))
    synth.write_synthetic_ffw4(ffw, seed=1, ops=ops, opsc2=opsc2)
    opsc, opsc2p = str(tmp_path / (name + "_opsc.bin")), str(tmp_path / (name + "_opsc2.bin"))
    synth.write_opsc(opsc, 1 / 127, sc)
    synth.write_opsc2(opsc2p, *opsc2)
    return ffw, opsc, opsc2p


def test_standalone_op_rejections(checker, tmp_path):
    """Op sequences the plan refuses even with stand-alone ops supported, each
    a valid file: the plan fails with its message (under the sanitizers), and
    create would return NULL."""
    conv = lambda ci, co, s=1: dict(type=synth.OP_CONV, Cin=ci, Cout=co, k=3, s=s, p=1)
    cases = {
        "prelu_size": ([conv(3, 64), dict(type=synth.OP_PRELU, C=64), dict(type=synth.OP_BN, C=64),
                        dict(type=synth.OP_PRELU, C=32)], "PReLU size != channels"),
        "add_shapes": ([conv(3, 64), dict(type=synth.OP_PRELU, C=64), dict(type=synth.OP_SAVE_ID),
                        dict(type=synth.OP_BN, C=64), conv(64, 64, 2), dict(type=synth.OP_PRELU, C=64),
                        dict(type=synth.OP_BN, C=64), dict(type=synth.OP_ADD)],
                       "Add operands differ in shape"),
        "map_channels": ([conv(3, 96), dict(type=synth.OP_PRELU, C=96), dict(type=synth.OP_BN, C=96),
                          dict(type=synth.OP_BN, C=96)], "multiple of 64 channels"),
        "input_op": ([dict(type=synth.OP_BN, C=3), conv(3, 64), dict(type=synth.OP_PRELU, C=64)],
                     "input faces"),
        "add_no_slot": ([conv(3, 64), dict(type=synth.OP_PRELU, C=64), dict(type=synth.OP_BN, C=64),
                         dict(type=synth.OP_ADD)], "Add before any SAVE_ID"),
    }
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0")
    for name, (ops, msg) in cases.items():
        ffw, opsc, opsc2 = _tiny_model(tmp_path, name, ops)
        r = subprocess.run([checker, ffw, opsc, opsc2], capture_output=True, text=True, env=env, timeout=120)
        assert r.returncode == 0, r.stderr[-2000:]
        assert "runtime error" not in r.stderr and "AddressSanitizer" not in r.stderr, r.stderr[-2000:]
        assert "load 0 " in r.stdout and "plan -1 " in r.stdout and msg in r.stdout, (name, r.stdout)
