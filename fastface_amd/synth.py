"""Synthetic FFW4 weights and seeded synthetic faces.

The reference's real weights (`models/w600k_r50_ffw4.bin`) are not
distributed with it, so tests and the bench run on a synthetic FFW4 with the
same 177-op IResNet-50 schedule and byte layout that the reference's writer
emits (prepare_weights_v3.py:280-307; loader kernels/ffw2_loader.c:71-159):

    "FFW4" u32 n_ops, then per op: u8 type + payload
      CONV  (1): 6 x u16 [Cin, Cout, Kh, Kw, stride, pad], i8[Cout*Cin*Kh*Kw]
                 (OIHW), f32[Cout] weight scales, f32[Cout] bias
      BN    (2): u16 n, f32[n] scale, f32[n] offset
      PRELU (3): u16 n, f32[n] slope
      GEMM  (5): u32 N, u32 K, i8[N*K], f32[N] scales, f32[N] bias
      ADD (4), FLATTEN (6), SAVE_ID (7), BLOCK_START (8): no payload

Schedule (op index order):
    CONV stem 3->64 3x3 s1, PRELU
    per block of stages [3, 4, 14, 3] at 64/128/256/512 channels:
      BLOCK_START, BN(Cin), CONV c1 3x3 s1 Cin->C, PRELU,
      first block of a stage: CONV c2 3x3 s2, SAVE_ID, CONV ds 1x1 s2 Cin->C, ADD
      other blocks:           CONV c2 3x3 s1, ADD
      SAVE_ID unless last block of the stage
    BN(512), FLATTEN, GEMM 25088->512

Values follow the recipe: int8 weights uniform in [-127, 127], per-channel
fp32 scales, bias N(0, 0.05), PReLU slopes U(0, 0.3), seeded numpy PCG64.
Weight scales are sized from the committed OPSC2 output scales so that the
activations stay inside the int8 range rather than saturating.
"""
from __future__ import annotations

import os
import struct

import numpy as np

OP_CONV, OP_BN, OP_PRELU, OP_ADD, OP_GEMM, OP_FLATTEN, OP_SAVE_ID, OP_BLOCK_START = range(1, 9)

STAGES = ((3, 64), (4, 128), (14, 256), (3, 512))
INPUT_HW = 112
INPUT_C = 3
EMB_N = 512
FACE_FLOATS = INPUT_HW * INPUT_HW * INPUT_C

_HERE = os.path.dirname(os.path.abspath(__file__))
REPO_ROOT = os.path.dirname(_HERE)
OPSC_PATH = os.path.join(REPO_ROOT, "models", "op_scales.bin")
OPSC2_PATH = os.path.join(REPO_ROOT, "models", "op_scales_v2.bin")


def iresnet_schedule(stages=STAGES, standalone=False, generic=False):
    """List of op dicts in FFW4 order (types and conv geometry only).

    standalone=True inserts elementwise ops that no conv absorbs (each marked
    with `extra`, how its scale entries are made): a PReLU after the last
    residual Add of stage 2; in stage 3's second block, after its Add, a
    SAVE_ID, a BN (the conv's second output) and an Add of the two (an Add
    after no conv), so that the next block's leading BN reads an Add's
    output; and a second BN and a PReLU after the final BN.  The reference's
    interpreter runs them one by one (libfastface.c:401-434).

    generic=True changes three convs to geometries without a tuned kernel,
    keeping every tensor's shape (so the committed scale files still apply):
    the stem and stage 3's fifth block's first conv as 5x5 pad 2, and stage
    4's second block's second conv (the one adding the residual) as 1x1."""
    ops = [dict(type=OP_CONV, Cin=3, Cout=64, k=5 if generic else 3, s=1, p=2 if generic else 1),
           dict(type=OP_PRELU, C=64)]
    cin = 64
    for si, (nblocks, c) in enumerate(stages):
        for bi in range(nblocks):
            ops.append(dict(type=OP_BLOCK_START))
            ops.append(dict(type=OP_BN, C=cin))
            k1 = 5 if generic and si == 2 and bi == 4 else 3
            ops.append(dict(type=OP_CONV, Cin=cin, Cout=c, k=k1, s=1, p=k1 // 2))
            ops.append(dict(type=OP_PRELU, C=c))
            if bi == 0:
                ops.append(dict(type=OP_CONV, Cin=c, Cout=c, k=3, s=2, p=1))
                ops.append(dict(type=OP_SAVE_ID))
                ops.append(dict(type=OP_CONV, Cin=cin, Cout=c, k=1, s=2, p=0))
                ops.append(dict(type=OP_ADD))
            else:
                k2 = 1 if generic and si == 3 and bi == 1 else 3
                ops.append(dict(type=OP_CONV, Cin=c, Cout=c, k=k2, s=1, p=k2 // 2))
                ops.append(dict(type=OP_ADD))
            if standalone and si == 1 and bi == nblocks - 1:
                ops.append(dict(type=OP_PRELU, C=c, extra="copy"))
            if standalone and si == 2 and bi == 1:
                ops += [dict(type=OP_SAVE_ID, extra="none"), dict(type=OP_BN, C=c, extra="copy"),
                        dict(type=OP_ADD, extra="sum")]
            if bi != nblocks - 1:
                ops.append(dict(type=OP_SAVE_ID))
            cin = c
    ops.append(dict(type=OP_BN, C=cin))
    if standalone:
        ops += [dict(type=OP_BN, C=cin, extra="copy"), dict(type=OP_PRELU, C=cin, extra="copy")]
    ops.append(dict(type=OP_FLATTEN))
    ops.append(dict(type=OP_GEMM, N=EMB_N, K=cin * 7 * 7))
    return ops


def read_opsc2(path=OPSC2_PATH):
    """(input_scales, [per-op forward scale arrays or None])."""
    with open(path, "rb") as f:
        d = f.read()
    assert d[:5] == b"OPSC2"
    off = 5
    n_ops, n_in = struct.unpack_from("<II", d, off)
    off += 8
    in_s = np.frombuffer(d, np.float32, n_in, off).copy()
    off += 4 * n_in
    per_op = []
    for _ in range(n_ops):
        (c,) = struct.unpack_from("<I", d, off)
        off += 4
        per_op.append(np.frombuffer(d, np.float32, c, off).copy() if c else None)
        off += 4 * c
    return in_s, per_op


def read_opsc(path=OPSC_PATH):
    """(input_scale, per-op scales) of an OPSC file (libfastface.c:116-129;
    a scale <= 0 means "keep the current one")."""
    with open(path, "rb") as f:
        d = f.read()
    assert d[:4] == b"OPSC"
    (n,) = struct.unpack_from("<I", d, 4)
    in_s = float(np.frombuffer(d, np.float32, 1, 8)[0])
    return in_s, np.frombuffer(d, np.float32, n, 12).copy()


def write_opsc(path, input_scale, scales):
    """OPSC file (libfastface.c:116-129): "OPSC", u32 n, f32 input scale,
    f32[n] per-op scales."""
    with open(path, "wb") as f:
        f.write(b"OPSC")
        f.write(struct.pack("<I", len(scales)))
        f.write(np.float32(input_scale).tobytes())
        f.write(np.asarray(scales, np.float32).tobytes())


def write_opsc2(path, input_scales, per_op):
    """OPSC2 file (libfastface.c:133-204): "OPSC2", u32 n_ops, u32 n_in,
    f32[n_in], then per op u32 c and f32[c] (c = 0: no entry)."""
    with open(path, "wb") as f:
        f.write(b"OPSC2")
        f.write(struct.pack("<II", len(per_op), len(input_scales)))
        f.write(np.asarray(input_scales, np.float32).tobytes())
        for a in per_op:
            if a is None:
                f.write(struct.pack("<I", 0))
            else:
                f.write(struct.pack("<I", len(a)))
                f.write(np.asarray(a, np.float32).tobytes())


def standalone_scales(ops):
    """OPSC and OPSC2 contents for a schedule with inserted ops: every op of
    the plain schedule keeps its entries from the committed files, in order;
    an inserted op copies the latest positive per-tensor scale and the latest
    per-channel entry ("copy": the BN keeps the current per-tensor scale, as
    the model's BNs do), has none ("none"), or, for the Add, twice the
    current per-tensor scale and no per-channel entry ("sum")."""
    in_s, sc = read_opsc()
    in_pc, per_op = read_opsc2()
    new_sc, new_pc = [], []
    j = 0
    for op in ops:
        kind = op.get("extra")
        if kind is None:
            new_sc.append(float(sc[j]))
            new_pc.append(per_op[j])
            j += 1
            continue
        last_sc = next(v for v in reversed(new_sc) if v > 0)
        last_pc = next(v for v in reversed(new_pc) if v is not None)
        if kind == "copy":
            new_sc.append(0.0 if op["type"] == OP_BN else last_sc)
            new_pc.append(last_pc.copy())
        elif kind == "sum":
            new_sc.append(2.0 * last_sc)
            new_pc.append(None)
        else:
            new_sc.append(0.0)
            new_pc.append(None)
    assert j == len(sc)
    return (in_s, np.asarray(new_sc, np.float32)), (in_pc, new_pc)


def _per_tensor_scales(ops, opsc):
    """The per-tensor scales the reference's interpreter tracks for models
    below FFW4 (libfastface.c:349-440 with version < 4): for every op, the
    scale of the tensor it reads (a shortcut conv reads the block input's)
    and the scale its output is requantized to (a conv's fused PReLU / Add
    decides it).  Returns two lists indexed by op (None where unused)."""
    in_s, sc = opsc
    n = len(ops)
    a_in, out = [None] * n, [None] * n
    A = blk = in_s
    i = 0
    while i < n:
        t = ops[i]["type"]
        nxt = sc[i] if sc[i] > 0 else A
        if t == OP_CONV:
            a_in[i] = blk if i > 0 and ops[i - 1]["type"] == OP_SAVE_ID else A
            eff = nxt
            if i + 1 < n and ops[i + 1]["type"] in (OP_PRELU, OP_ADD):
                eff = sc[i + 1] if sc[i + 1] > 0 else nxt
                out[i] = eff
                A = eff
                i += 2
                continue
            out[i] = eff
            A = eff
        elif t == OP_BN:
            a_in[i], out[i] = A, nxt
            A = nxt
        elif t == OP_BLOCK_START:
            blk = A
        elif t == OP_GEMM:
            a_in[i] = A
        i += 1
    return a_in, out


def _fill_scales(ops, opsc2):
    """Per-op forward activation scales the interpreter tracks (the producer's
    OPSC2 entry, libfastface.c:395-396,410-411)."""
    in_s, per_op = opsc2
    cur = in_s
    out = []
    for i, op in enumerate(ops):
        out.append(cur)
        if per_op[i] is not None and op["type"] in (OP_CONV, OP_PRELU, OP_ADD, OP_BN):
            cur = per_op[i]
    return out


def hostile_channels(ops):
    """Parameter values that no shorter epilogue form survives, for
    `write_synthetic_ffw4(hostile=True)`: {op index: (field, channel, value)}.
    The input layer's channel 0 gets a NaN weight scale, the first 256-channel
    conv with a PReLU a bias of 3e38 on channel 1 (its requant value
    overflows: the x86 out-of-range case), the first 512-channel conv that
    adds a residual a bias of -3e38 on channel 3, and the first 128-channel
    conv's PReLU a slope of 1.5 on channel 2 (PReLU is then no max)."""
    out = {0: ("scales", 0, np.float32(np.nan))}
    conv = lambda i, c, nxt: (ops[i]["type"] == OP_CONV and ops[i]["Cout"] == c and
                              ops[i + 1]["type"] == nxt)
    i256 = next(i for i in range(len(ops) - 1) if conv(i, 256, OP_PRELU))
    i512 = next(i for i in range(len(ops) - 1) if conv(i, 512, OP_ADD))
    i128 = next(i for i in range(len(ops) - 1) if conv(i, 128, OP_PRELU))
    out[i256] = ("bias", 1, np.float32(3e38))
    out[i512] = ("bias", 3, np.float32(-3e38))
    out[i128 + 1] = ("slope", 2, np.float32(1.5))
    return out


def write_synthetic_ffw4(path, seed=3, act_sigma=40.0, gain=0.35, opsc2_path=OPSC2_PATH, version=4,
                         ops=None, opsc2=None, hostile=False):
    """Write a synthetic FFW4 file (about 43.7 MB) and return its path.

    version 3 or 2 writes the same network as an FFW3 / FFW2 file
    (kernels/ffw2_loader.c:96-125: the FFW4 layout under another magic;
    FFW2 without the conv bias).  The reference runs those on per-tensor
    scales (libfastface.c:335-343,356-422: the OPSC file's, an in-scale on
    every conv, the activation scale on the FC), so their weight, BN and FC
    scales are sized from the OPSC per-tensor scales instead of the OPSC2
    per-channel ones.  The random draws are the same for every version: the
    int8 weights, biases and slopes are identical.  `ops` / `opsc2`: another
    schedule and its OPSC2 contents (FFW4 only).  hostile: the values of
    `hostile_channels` written into a few convs and one PReLU."""
    assert version in (2, 3, 4)
    assert ops is None or version == 4
    rng = np.random.default_rng(seed)
    ops = ops if ops is not None else iresnet_schedule()
    opsc2 = opsc2 if opsc2 is not None else read_opsc2(opsc2_path)
    special = hostile_channels(ops) if hostile else {}
    _, per_op = opsc2
    track = _fill_scales(ops, opsc2)
    pt_in, pt_out = _per_tensor_scales(ops, read_opsc()) if version < 4 else (None, None)
    n = len(ops)
    tmp = path + ".tmp%d" % os.getpid()
    with open(tmp, "wb") as f:
        f.write(b"FFW%d" % version)
        f.write(struct.pack("<I", n))
        for i, op in enumerate(ops):
            t = op["type"]
            f.write(struct.pack("<B", t))
            if t == OP_CONV:
                cin, cout, k = op["Cin"], op["Cout"], op["k"]
                w = rng.integers(-127, 128, size=(cout, cin, k, k), dtype=np.int8)
                # requant target of this conv: the fused PReLU/Add's scale if any
                eff = i + 1 if ops[i + 1]["type"] in (OP_PRELU, OP_ADD) else i
                s_out = per_op[eff] if per_op[eff] is not None else np.full(cout, 0.02, np.float32)
                kreal = cin * k * k
                if version < 4:         # f = acc * in_scale * ws, requantized by 1/out_scale
                    s_out = np.full(cout, pt_out[i] / pt_in[i])
                # keeps the int8 output spread close to the input's
                base = s_out.astype(np.float64) * gain / (np.sqrt(kreal) * 73.6)
                jitter = rng.uniform(0.5, 1.5, size=cout)
                scales = (base * jitter).astype(np.float32)
                bias = rng.normal(0.0, 0.05, size=cout).astype(np.float32)
                if i in special:
                    field, ch, v = special[i]
                    (scales if field == "scales" else bias)[ch] = v
                f.write(struct.pack("<6H", cin, cout, k, k, op["s"], op["p"]))
                f.write(w.tobytes())
                f.write(scales.tobytes())
                if version >= 3:
                    f.write(bias.tobytes())
            elif t == OP_BN:
                c = op["C"]
                s_in = track[i].astype(np.float64)
                s_bn = per_op[i].astype(np.float64) if per_op[i] is not None else s_in
                if version < 4:
                    s_in, s_bn = np.full(c, pt_in[i]), np.full(c, pt_out[i])
                ratio = np.clip(s_bn / np.maximum(s_in, 1e-30), 1e-3, 1e3)
                scale = (ratio * rng.uniform(0.5, 1.5, size=c)).astype(np.float32)
                offset = rng.normal(0.0, 0.05, size=c).astype(np.float32)
                f.write(struct.pack("<H", c))
                f.write(scale.tobytes())
                f.write(offset.tobytes())
            elif t == OP_PRELU:
                c = op["C"]
                slope = rng.uniform(0.0, 0.3, size=c).astype(np.float32)
                if i in special:
                    slope[special[i][1]] = special[i][2]
                f.write(struct.pack("<H", c))
                f.write(slope.tobytes())
            elif t == OP_GEMM:
                nn, kk = op["N"], op["K"]
                w = rng.integers(-127, 128, size=(nn, kk), dtype=np.int8)
                scales = rng.uniform(0.5, 1.5, size=nn) / (np.sqrt(kk) * 73.6 * act_sigma)
                if version < 4:         # out = dot * A_scale * ws + bias
                    scales = scales / pt_in[i]
                scales = scales.astype(np.float32)
                bias = rng.normal(0.0, 0.05, size=nn).astype(np.float32)
                f.write(struct.pack("<II", nn, kk))
                f.write(w.tobytes())
                f.write(scales.tobytes())
                f.write(bias.tobytes())
    os.replace(tmp, path)
    return path


def synthetic_ffw4_path(seed=3, cache_dir=None, version=4):
    """Path of the cached synthetic model for `seed` (FFW4, or with
    version 3 / 2 the FFW3 / FFW2 file), generated on first use."""
    cache_dir = cache_dir or os.environ.get("FASTFACE_CACHE", "/tmp/fastface_cache")
    os.makedirs(cache_dir, exist_ok=True)
    name = "synthetic_r50_seed%d.ffw4" % seed if version == 4 else \
        "synthetic_r50_seed%d_v%d.ffw" % (seed, version)
    path = os.path.join(cache_dir, name)
    if not os.path.exists(path):
        write_synthetic_ffw4(path, seed=seed, version=version)
    return path


def synthetic_hostile_path(seed=7, cache_dir=None):
    """Path of a synthetic FFW4 with `hostile_channels` (the committed scale
    files apply to it), generated on first use."""
    cache_dir = cache_dir or os.environ.get("FASTFACE_CACHE", "/tmp/fastface_cache")
    os.makedirs(cache_dir, exist_ok=True)
    path = os.path.join(cache_dir, "synthetic_r50_hostile_seed%d.ffw4" % seed)
    if not os.path.exists(path):
        write_synthetic_ffw4(path, seed=seed, hostile=True)
    return path


def synthetic_generic_path(seed=6, cache_dir=None):
    """Path of a synthetic FFW4 of `iresnet_schedule(generic=True)` (the
    committed scale files apply to it), generated on first use."""
    cache_dir = cache_dir or os.environ.get("FASTFACE_CACHE", "/tmp/fastface_cache")
    os.makedirs(cache_dir, exist_ok=True)
    path = os.path.join(cache_dir, "synthetic_r50_generic_seed%d.ffw4" % seed)
    if not os.path.exists(path):
        write_synthetic_ffw4(path, seed=seed, ops=iresnet_schedule(generic=True))
    return path


def synthetic_standalone_dir(seed=5, cache_dir=None):
    """Directory holding a synthetic FFW4 of `iresnet_schedule(standalone=True)`
    (model.ffw4) with its own models/op_scales.bin and models/op_scales_v2.bin
    (`standalone_scales`), generated on first use."""
    cache_dir = cache_dir or os.environ.get("FASTFACE_CACHE", "/tmp/fastface_cache")
    d = os.path.join(cache_dir, "standalone_seed%d" % seed)
    ffw = os.path.join(d, "model.ffw4")
    if not os.path.exists(ffw):
        os.makedirs(os.path.join(d, "models"), exist_ok=True)
        ops = iresnet_schedule(standalone=True)
        (in_s, sc), (in_pc, per_op) = standalone_scales(ops)
        write_opsc(os.path.join(d, "models", "op_scales.bin"), in_s, sc)
        write_opsc2(os.path.join(d, "models", "op_scales_v2.bin"), in_pc, per_op)
        write_synthetic_ffw4(ffw, seed=seed, ops=ops, opsc2=(in_pc, per_op))
    return d


def faces_uniform(batch, seed):
    """`batch` faces [B,112,112,3] fp32, uniform in [-1, 1]."""
    rng = np.random.default_rng(seed)
    return rng.uniform(-1.0, 1.0, size=(batch, INPUT_HW, INPUT_HW, INPUT_C)).astype(np.float32)


def faces_normal_clipped(batch, seed, sigma=0.5):
    """`batch` faces, N(0, sigma) clipped to [-1, 1]."""
    rng = np.random.default_rng(seed)
    x = rng.normal(0.0, sigma, size=(batch, INPUT_HW, INPUT_HW, INPUT_C))
    return np.clip(x, -1.0, 1.0).astype(np.float32)
