"""Single-layer microbenchmark of the int8 conv kernels through the C ABI.

    python fastface_amd/layerbench.py --cin 256 --cout 256 --k 3 --stride 1 --hin 14 \
        --batch 64 --iters 200 [--epi prelu|add_bn|none|raw]

Defaults are BASELINE config 2 (N=64, 14x14, 256->256, 3x3 s1 p1, PReLU
epilogue).  Inputs are seeded random int8; prints one JSON line with the
mean launch time (HIP events on the launch stream) and int8 TOP/s.  Also the
workload rocprofv3 counter runs use, since it launches only the layer asked
for.
"""
import argparse
import ctypes as C
import json
import os
import sys

import numpy as np

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
import fastface_amd as fa  # noqa: E402


def time_layer(lib, cin=256, cout=256, k=3, stride=1, hin=14, batch=64, iters=200, epi="prelu",
               winograd=False, no_split=False, graph_reps=0, epis=None, x_even=False):
    """Mean launch time of one conv layer (HIP events on the launch stream)
    over `iters` launches after 3 warm-up launches; frees what it allocates.
    Inputs: seeded int8 U[-127,127] activations and weights (seed 1), ws
    U[1e-3,1e-2], bias N(0,0.1), PReLU slope 0.25.
    epi: prelu | prelu_le1 | prelu_le1_bn | add_bn | none | raw; an "_rng"
    suffix adds FFK_EPI_IN_RANGE (the parameters here satisfy
    ffk_requant_in_range); a "_planned" suffix (prelu_planned, ...) takes
    the shorter forms the launch plan would prove for these parameters
    (PReLU as a max, in range, the one-fma tail).  x_even: X stored at its even pixels only
    (FFK_OUT_X_EVEN, as the network stores the stem's and each stage's last X).
    graph_reps > 0: the `iters` launches are captured in one hipGraph (epis,
    if given, cycles the epilogue form per launch) and the graph is replayed
    graph_reps times between the events: the per-launch time then excludes
    the host's launch gaps, as a kernel trace's durations do."""
    pad = k // 2
    ho = (hin + 2 * pad - k) // stride + 1
    if not lib.ffk_conv_runnable(cin, cout, k, k, stride, pad, hin, hin):
        raise ValueError("invalid layer geometry")
    r = np.random.default_rng(1)
    if cin == 3:        # the input layer reads fp32 faces in [-1, 1]
        x = r.uniform(-1, 1, size=(batch, hin, hin, cin)).astype(np.float32)
    else:
        x = r.integers(-127, 128, size=(batch, hin, hin, cin), dtype=np.int8)
    w = r.integers(-127, 128, size=(cout, cin, k, k), dtype=np.int8)
    if winograd:
        packed = np.empty(lib.ffk_winograd_packed_bytes(cin, cout), np.int8)
        lib.ffk_pack_winograd_weights(w.ctypes.data, cout, cin, packed.ctypes.data)
    else:
        packed = np.empty(lib.ffk_conv_packed_bytes(cin, cout, k, k), np.int8)
        lib.ffk_pack_conv_weights(w.ctypes.data, cout, cin, k, k, packed.ctypes.data)
    P = np.zeros((fa.FFK_NPARAM, cout), np.float32)
    P[fa.FFK_P_WS] = r.uniform(1e-3, 1e-2, cout)
    P[fa.FFK_P_BIAS] = r.normal(0, 0.1, cout)
    P[fa.FFK_P_SLOPE] = 0.25
    P[fa.FFK_P_ADDSCALE] = 0.02
    P[fa.FFK_P_INV] = 1.0 / 40.0
    P[fa.FFK_P_BN_SIN] = 0.02
    P[fa.FFK_P_BN_S] = 1.0
    P[fa.FFK_P_BN_INV] = 50.0
    held = []

    def dev(arr=None, nbytes=None):
        n = arr.nbytes if arr is not None else nbytes
        p = lib.ffk_malloc(n)
        if not p:
            raise MemoryError(fa.last_error())
        held.append(p)
        if arr is not None:
            lib.ffk_memcpy_h2d(p, arr.ctypes.data, n, None)
        return p
    n_out = batch * ho * ho * cout
    forms = list(epis) if epis else [epi]
    epi = forms[0]
    d = fa.ffk_conv_desc()
    d.batch, d.cin, d.cout, d.kh, d.kw = batch, cin, cout, k, k
    d.stride, d.pad, d.hin, d.win = stride, pad, hin, hin
    d.in_ = dev(x)
    if cin == 3:
        d.in_inv = dev(np.array([127.0, 127.0, 127.0, 0.0], np.float32))
    d.w = dev(packed)
    d.params = dev(P)
    d.flags = fa.FFK_EPI_BIAS | (fa.FFK_ALGO_WINOGRAD if winograd else 0)
    if epi == "raw":
        d.out_i32 = dev(nbytes=n_out * 4)
    else:
        d.out = dev(nbytes=n_out)
    if any(f.startswith("add") for f in forms):
        d.add_src = dev(r.integers(-127, 128, size=n_out, dtype=np.int8))
    if any("bn" in f for f in forms):
        d.out_bn = dev(nbytes=n_out)
        lut = np.empty((cout, 256), np.int8)
        rows = [np.ascontiguousarray(P[i]) for i in (fa.FFK_P_BN_SIN, fa.FFK_P_BN_S,
                                                       fa.FFK_P_BN_O, fa.FFK_P_BN_INV)]
        lib.ffk_make_bn_lut(rows[0].ctypes.data, rows[1].ctypes.data, rows[2].ctypes.data,
                            rows[3].ctypes.data, cout, lut.ctypes.data)
        d.bn_lut = dev(lut)

    def form_flags(f):
        fl = d.flags & (fa.FFK_EPI_BIAS | fa.FFK_ALGO_WINOGRAD)
        if f.startswith("prelu"):
            fl |= fa.FFK_EPI_PRELU
        if f.startswith("prelu_le1"):
            fl |= fa.FFK_EPI_PRELU_LE1
        if f.startswith("add"):
            fl |= fa.FFK_EPI_ADD
        if "bn" in f:
            fl |= fa.FFK_EPI_BN
        if x_even:
            fl |= fa.FFK_OUT_X_EVEN
        if f.endswith("_rng"):
            fl |= fa.FFK_EPI_IN_RANGE
            assert lib.ffk_requant_in_range(P.ctypes.data, cout, k * k * cin, fl) == 1
        if f.endswith("_planned"):      # the forms the planner proves for these parameters
            if fl & fa.FFK_EPI_PRELU and lib.ffk_prelu_le1_ok(P.ctypes.data, cout, k * k * cin,
                                                             1 if fl & fa.FFK_EPI_ADD else 0):
                fl |= fa.FFK_EPI_PRELU_LE1
            if lib.ffk_requant_in_range(P.ctypes.data, cout, k * k * cin, fl):
                fl |= fa.FFK_EPI_IN_RANGE
                if lib.ffk_requant_fma_ok(P.ctypes.data, cout, k * k * cin, fl):
                    fl |= fa.FFK_EPI_FMA_TAIL
        return fl
    d.flags = form_flags(epi)
    ws_bytes = 0 if no_split else lib.ffk_conv_workspace_bytes(C.byref(d))
    if ws_bytes:
        d.workspace, d.workspace_bytes = dev(nbytes=ws_bytes), ws_bytes
        assert lib.ffk_zero(d.workspace, ws_bytes, None) == 0, fa.last_error()
    stream = C.c_void_p()
    e0, e1 = C.c_void_p(), C.c_void_p()
    lib.ffk_stream_create(C.byref(stream))
    lib.ffk_event_create(C.byref(e0))
    lib.ffk_event_create(C.byref(e1))
    g = C.c_void_p()
    ms = C.c_float()
    try:
        variant = lib.ffk_conv_variant(C.byref(d))
        descs = []
        for f in forms:
            df = fa.ffk_conv_desc.from_buffer_copy(d)
            df.flags = form_flags(f)
            if not f.startswith("add"):
                df.add_src = None
            if "bn" not in f:
                df.out_bn, df.bn_lut = None, None
            descs.append(df)
        for i in range(3):
            assert lib.ffk_conv(C.byref(descs[i % len(descs)]), stream) == 0, fa.last_error()
        if graph_reps > 0:
            assert lib.ffk_graph_begin(stream) == 0, fa.last_error()
            for i in range(iters):
                assert lib.ffk_conv(C.byref(descs[i % len(descs)]), stream) == 0, fa.last_error()
            assert lib.ffk_graph_end(stream, C.byref(g)) == 0, fa.last_error()
            assert lib.ffk_graph_launch(g, stream) == 0, fa.last_error()          # warm
            lib.ffk_event_record(e0, stream)
            for _ in range(graph_reps):
                lib.ffk_graph_launch(g, stream)
            lib.ffk_event_record(e1, stream)
        else:
            lib.ffk_event_record(e0, stream)
            for i in range(iters):
                lib.ffk_conv(C.byref(descs[i % len(descs)]), stream)
            lib.ffk_event_record(e1, stream)
        assert lib.ffk_event_elapsed_ms(e0, e1, C.byref(ms)) == 0, fa.last_error()
    finally:
        lib.ffk_stream_sync(stream)
        if g.value:
            lib.ffk_graph_destroy(g)
        lib.ffk_event_destroy(e0)
        lib.ffk_event_destroy(e1)
        lib.ffk_stream_destroy(stream)
        for p in held:
            lib.ffk_free(p)
    per = ms.value / (iters * max(graph_reps, 1))
    ops = 2.0 * batch * ho * ho * cout * k * k * cin
    return {"layer": "%d->%d k%d s%d @%d" % (cin, cout, k, stride, hin), "batch": batch,
            "epi": "/".join(forms), "graph": graph_reps > 0,
            "kernel": variant.decode() if variant else None, "split_ws_bytes": ws_bytes,
            "ms_per_launch": round(per, 5), "int8_tops": round(ops / (per * 1e-3) / 1e12, 2),
            "frac_of_peak": round(ops / (per * 1e-3) / 5e15, 4)}


def time_pair(lib, cin=64, cout=64, hin=112, cx=64, batch=1024, iters=10, fused=True):
    """Mean time of a stage's stride-2 pair: the 3x3 stride-2 conv (bias, in-range
    form) and the 1x1 shortcut over the compact block input (cx channels,
    residual + BN, in-range form) whose residual is the conv's output, as one
    launch (ffk_conv_s2_shortcut) or, fused=False, as two ffk_conv launches.
    Seeded data as in time_layer; HIP events on the launch stream."""
    ho = hin // 2
    r = np.random.default_rng(1)
    x = r.integers(-127, 128, size=(batch, hin, hin, cin), dtype=np.int8)
    xc = r.integers(-127, 128, size=(batch, ho, ho, cx), dtype=np.int8)
    held = []

    def dev(arr=None, nbytes=None):
        n = arr.nbytes if arr is not None else nbytes
        p = lib.ffk_malloc(n)
        if not p:
            raise MemoryError(fa.last_error())
        held.append(p)
        if arr is not None:
            lib.ffk_memcpy_h2d(p, arr.ctypes.data, n, None)
        return p

    def desc(ci, k, s, h, inp, flags):
        w = r.integers(-127, 128, size=(cout, ci, k, k), dtype=np.int8)
        packed = np.empty(lib.ffk_conv_packed_bytes(ci, cout, k, k), np.int8)
        lib.ffk_pack_conv_weights(w.ctypes.data, cout, ci, k, k, packed.ctypes.data)
        P = np.zeros((fa.FFK_NPARAM, cout), np.float32)
        P[fa.FFK_P_WS] = r.uniform(1e-3, 1e-2, cout)
        P[fa.FFK_P_BIAS] = r.normal(0, 0.1, cout)
        P[fa.FFK_P_ADDSCALE] = 0.02
        P[fa.FFK_P_INV] = 1.0 / 40.0
        P[fa.FFK_P_BN_SIN], P[fa.FFK_P_BN_S], P[fa.FFK_P_BN_INV] = 0.02, 1.0, 50.0
        assert lib.ffk_requant_in_range(P.ctypes.data, cout, k * k * ci, flags) == 1
        d = fa.ffk_conv_desc()
        d.batch, d.cin, d.cout, d.kh, d.kw = batch, ci, cout, k, k
        d.stride, d.pad, d.hin, d.win = s, k // 2, h, h
        d.in_, d.w, d.params = inp, dev(packed), dev(P)
        d.flags = flags | fa.FFK_EPI_IN_RANGE
        if flags & fa.FFK_EPI_BN:
            lut = np.empty((cout, 256), np.int8)
            rows = [np.ascontiguousarray(P[i]) for i in (fa.FFK_P_BN_SIN, fa.FFK_P_BN_S,
                                                           fa.FFK_P_BN_O, fa.FFK_P_BN_INV)]
            lib.ffk_make_bn_lut(rows[0].ctypes.data, rows[1].ctypes.data, rows[2].ctypes.data,
                                rows[3].ctypes.data, cout, lut.ctypes.data)
            d.bn_lut = dev(lut)
        return d
    n_out = batch * ho * ho * cout
    c = desc(cin, 3, 2, hin, dev(x), fa.FFK_EPI_BIAS)
    c.out = dev(nbytes=n_out)
    sc = desc(cx, 1, 1, ho, dev(xc), fa.FFK_EPI_BIAS | fa.FFK_EPI_ADD | fa.FFK_EPI_BN)
    sc.add_src, sc.out, sc.out_bn = c.out, dev(nbytes=n_out), dev(nbytes=n_out)
    stream = C.c_void_p()
    e0, e1 = C.c_void_p(), C.c_void_p()
    lib.ffk_stream_create(C.byref(stream))
    lib.ffk_event_create(C.byref(e0))
    lib.ffk_event_create(C.byref(e1))
    ms = C.c_float()

    def run():
        if fused:
            assert lib.ffk_conv_s2_shortcut(C.byref(c), C.byref(sc), stream) == 1, "pair not served"
        else:
            assert lib.ffk_conv(C.byref(c), stream) == 0, fa.last_error()
            assert lib.ffk_conv(C.byref(sc), stream) == 0, fa.last_error()
    try:
        for _ in range(3):
            run()
        lib.ffk_event_record(e0, stream)
        for _ in range(iters):
            run()
        lib.ffk_event_record(e1, stream)
        assert lib.ffk_event_elapsed_ms(e0, e1, C.byref(ms)) == 0, fa.last_error()
    finally:
        lib.ffk_stream_sync(stream)
        lib.ffk_event_destroy(e0)
        lib.ffk_event_destroy(e1)
        lib.ffk_stream_destroy(stream)
        for p in held:
            lib.ffk_free(p)
    return {"pair": "%d->%d k3 s2 @%d + %d->%d k1 shortcut" % (cin, cout, hin, cx, cout), "batch": batch,
            "fused": fused, "ms": round(ms.value / iters, 5)}


def time_eltwise(lib, op="map", channels=256, hin=14, batch=1024, iters=20):
    """Mean launch time of a stand-alone BN / PReLU (`op` "map": the
    per-channel table kernel) or Add ("add": the pair table kernel) over
    batch x hin x hin pixels of `channels` int8 channels (HIP events on the
    launch stream; seeded int8 data and tables).  Reports the HBM rate of
    the algorithmic bytes (2 or 3 per element) against 8 TB/s."""
    r = np.random.default_rng(11)
    n = batch * hin * hin * channels
    held = []

    def dev(arr=None, nbytes=None):
        m = arr.nbytes if arr is not None else nbytes
        p = lib.ffk_malloc(m)
        if not p:
            raise MemoryError(fa.last_error())
        held.append(p)
        if arr is not None:
            lib.ffk_memcpy_h2d(p, arr.ctypes.data, m, None)
        return p
    a = dev(r.integers(-128, 128, size=n, dtype=np.int8))
    out = dev(nbytes=n)
    if op == "map":
        lut = dev(r.integers(-128, 128, size=channels * 256, dtype=np.int8))
        run = lambda s: lib.ffk_map_i8(a, out, batch * hin * hin, channels, lut, s)
        per_elem = 2
    else:
        b = dev(r.integers(-128, 128, size=n, dtype=np.int8))
        lut = dev(r.integers(-128, 128, size=65536, dtype=np.int8))
        run = lambda s: lib.ffk_add_i8(a, b, out, n, lut, s)
        per_elem = 3
    stream, e0, e1, ms = C.c_void_p(), C.c_void_p(), C.c_void_p(), C.c_float()
    lib.ffk_stream_create(C.byref(stream))
    lib.ffk_event_create(C.byref(e0))
    lib.ffk_event_create(C.byref(e1))
    try:
        for _ in range(3):
            assert run(stream) == 0, fa.last_error()
        lib.ffk_event_record(e0, stream)
        for _ in range(iters):
            run(stream)
        lib.ffk_event_record(e1, stream)
        assert lib.ffk_event_elapsed_ms(e0, e1, C.byref(ms)) == 0, fa.last_error()
    finally:
        lib.ffk_stream_sync(stream)
        lib.ffk_event_destroy(e0)
        lib.ffk_event_destroy(e1)
        lib.ffk_stream_destroy(stream)
        for p in held:
            lib.ffk_free(p)
    per = ms.value / iters
    gbs = per_elem * n / (per * 1e-3) / 1e9
    return {"op": op, "channels": channels, "pixels": batch * hin * hin, "bytes": per_elem * n,
            "ms_per_launch": round(per, 5), "hbm_gbs": round(gbs, 1), "frac_of_hbm": round(gbs / 8000.0, 4)}


def time_fc(lib, batch=1, iters=50, path=0):
    """Mean launch time of the FC head 25088 -> 512 at `batch` faces (the
    path and split-K workspace ffk_fc chooses, or with path 1 / 2 the matvec
    / MFMA GEMM path; HIP events on the launch stream); seeded int8
    activations and weights.  Frees what it allocates."""
    N, K = 512, 25088
    r = np.random.default_rng(7)
    a = r.integers(-128, 128, size=(batch, K), dtype=np.int8)
    W = r.integers(-127, 128, size=(N, K), dtype=np.int8)
    packed = np.empty(lib.ffk_fc_packed_bytes(N, K), np.int8)
    lib.ffk_pack_fc_weights(W.ctypes.data, N, K, packed.ctypes.data)
    ws = r.uniform(1e-5, 1e-3, N).astype(np.float32)
    bias = r.normal(0, 0.05, N).astype(np.float32)
    held = []

    def dev(arr=None, nbytes=None):
        n = arr.nbytes if arr is not None else nbytes
        p = lib.ffk_malloc(n)
        if not p:
            raise MemoryError(fa.last_error())
        held.append(p)
        if arr is not None:
            lib.ffk_memcpy_h2d(p, arr.ctypes.data, n, None)
        return p
    d = fa.ffk_fc_desc()
    d.batch, d.n, d.k = batch, N, K
    d.a, d.w, d.ws, d.bias = dev(a), dev(packed), dev(ws), dev(bias)
    d.out = dev(nbytes=batch * N * 4)
    d.a_scale = 1.0
    d.path = path
    n_ws = lib.ffk_fc_workspace_bytes(C.byref(d))
    if n_ws:
        d.workspace, d.workspace_bytes = dev(nbytes=n_ws), n_ws
        assert lib.ffk_zero(d.workspace, n_ws, None) == 0, fa.last_error()
    stream, e0, e1, ms = C.c_void_p(), C.c_void_p(), C.c_void_p(), C.c_float()
    lib.ffk_stream_create(C.byref(stream))
    lib.ffk_event_create(C.byref(e0))
    lib.ffk_event_create(C.byref(e1))
    try:
        for _ in range(3):
            assert lib.ffk_fc(C.byref(d), stream) == 0, fa.last_error()
        lib.ffk_event_record(e0, stream)
        for _ in range(iters):
            lib.ffk_fc(C.byref(d), stream)
        lib.ffk_event_record(e1, stream)
        assert lib.ffk_event_elapsed_ms(e0, e1, C.byref(ms)) == 0, fa.last_error()
    finally:
        lib.ffk_stream_sync(stream)
        lib.ffk_event_destroy(e0)
        lib.ffk_event_destroy(e1)
        lib.ffk_stream_destroy(stream)
        for p in held:
            lib.ffk_free(p)
    per = ms.value / iters
    return {"layer": "fc 25088->512", "batch": batch, "split_ws_bytes": n_ws,
            "path": {1: "matvec", 2: "gemm"}.get(path, "matvec" if batch <= 16 else "gemm"),
            "ms_per_launch": round(per, 5),
            "weight_gbs": round(N * K / (per * 1e-3) / 1e9, 1),
            "int8_tops": round(2.0 * batch * N * K / (per * 1e-3) / 1e12, 2)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--cin", type=int, default=256)
    ap.add_argument("--cout", type=int, default=256)
    ap.add_argument("--k", type=int, default=3)
    ap.add_argument("--stride", type=int, default=1)
    ap.add_argument("--hin", type=int, default=14)
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--iters", type=int, default=200)
    ap.add_argument("--epi", default="prelu",
                    choices=["prelu", "prelu_le1", "add_bn", "none", "raw", "prelu_le1_rng", "add_bn_rng",
                             "none_rng", "prelu_le1_bn", "prelu_le1_bn_rng", "prelu_planned",
                             "prelu_bn_planned", "none_planned"])
    ap.add_argument("--x-even", action="store_true",
                    help="store X at its even pixels only (the network's stem and stage-last convs)")
    ap.add_argument("--winograd", action="store_true",
                    help="64-channel 3x3 stride-1 layers: the integer Winograd F(2,3) path")
    ap.add_argument("--no-split", action="store_true",
                    help="give no split-K workspace (small batches then use the whole-K tiling)")
    ap.add_argument("--fc", action="store_true",
                    help="instead: the FC head 25088 -> 512 at --batch faces")
    ap.add_argument("--fc-path", type=int, default=0, choices=[0, 1, 2],
                    help="with --fc: 0 the library's choice, 1 the matvec, 2 the MFMA GEMM")
    ap.add_argument("--pair-cx", type=int, default=0,
                    help="instead: the stride-2 conv (--cin/--cout/--hin, k3 s2) and its 1x1 shortcut "
                         "over this many compact input channels, as one launch")
    ap.add_argument("--unfused", action="store_true", help="with --pair-cx: as two launches")
    ap.add_argument("--eltwise", choices=["map", "add"],
                    help="instead: a stand-alone BN / PReLU (map) or Add over --batch x --hin x --hin "
                         "pixels of --cout channels")
    ap.add_argument("--copy-mb", type=int, default=0,
                    help="instead: device-to-device copies of this many MiB (the calibration "
                         "workload for rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    a = ap.parse_args()
    lib = fa.load()
    if lib.ffk_device_count() <= 0:
        raise RuntimeError("no HIP device")
    if a.copy_mb:
        n = a.copy_mb << 20
        src, dst = lib.ffk_malloc(n), lib.ffk_malloc(n)
        for _ in range(a.iters):
            assert lib.ffk_memcpy_d2d(dst, src, n, None) == 0, fa.last_error()
        lib.ffk_stream_sync(None)
        print(json.dumps({"copy_bytes": n, "iters": a.iters}), flush=True)
        return
    if a.fc:
        print(json.dumps(time_fc(lib, a.batch, a.iters, a.fc_path)), flush=True)
        return
    if a.eltwise:
        print(json.dumps(time_eltwise(lib, a.eltwise, a.cout, a.hin, a.batch, a.iters)), flush=True)
        return
    if a.pair_cx:
        print(json.dumps(time_pair(lib, a.cin, a.cout, a.hin, a.pair_cx, a.batch, a.iters,
                                   fused=not a.unfused)), flush=True)
        return
    try:
        res = time_layer(lib, a.cin, a.cout, a.k, a.stride, a.hin, a.batch, a.iters, a.epi,
                         winograd=a.winograd, no_split=a.no_split, x_even=a.x_even)
    except ValueError as e:
        raise SystemExit(str(e))
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
