"""Headline benchmark: INT8 IResNet-50 (ArcFace) faces/s at B=1024 on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--batch 1024]

A step is one forward pass of the whole network (stem .. FC head, one
captured hipGraph) over a batch of synthetic faces already resident in HBM.
Prints ONE JSON line.  Besides the headline value it reports the b=1 latency,
the roofline position of the dominant kernel (the 26 convolutions
256->256 3x3 s1 at 14x14, timed live with HIP events on the stream they run
on) and the reference CPU path timed on this host's cores.
"""
import argparse
import ctypes as C
import json
import os
import re
import statistics
import subprocess
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "faces/sec at B=1024 INT8 IResNet-50 (1 GPU); b=1 latency ms; % int8 MFMA peak"
PEAK_INT8_TOPS = 5000.0          # MI355X dense int8, 5.0 POP/s
PEAK_HBM_GBS = 8000.0
# the instantiation that runs the 26 dominant convs at B=1024 (rocprofv3 name)
DOMINANT_KERNEL = "conv3_patch_kernel<256, 256, 14, 14, 4, 2, 2, 2, 4>"


def log(msg):
    print("[bench] " + msg, file=sys.stderr, flush=True)


def check(lib, rc, what):
    if rc != 0:
        import fastface_amd
        raise RuntimeError("%s failed (%d): %s" % (what, rc, fastface_amd.last_error()))


def host_cpu():
    """CPU model, family/model/stepping, physical cores, SMT state and the
    VNNI flags of this host (from /proc/cpuinfo)."""
    model, cores, logical, ident, flags = "?", set(), 0, {}, set()
    try:
        phys = None
        for line in open("/proc/cpuinfo"):
            k, _, v = line.partition(":")
            k, v = k.strip(), v.strip()
            if k == "processor":
                logical += 1
            elif k == "model name":
                model = v
            elif k in ("cpu family", "model", "stepping", "vendor_id") and k not in ident:
                ident[k] = v
            elif k == "flags" and not flags:
                flags = set(v.split())
            elif k == "physical id":
                phys = v
            elif k == "core id":
                cores.add((phys, v))
    except OSError:
        pass
    n = len(cores) or logical
    return {"model": model, "vendor": ident.get("vendor_id"), "family": ident.get("cpu family"),
            "model_number": ident.get("model"), "stepping": ident.get("stepping"),
            "physical_cores": n, "logical_cpus": logical, "smt": logical > n,
            "avx_vnni": "avx_vnni" in flags, "avx512_vnni": "avx512_vnni" in flags}


def _ref_best(exe, args, threads, env):
    """Run one of the reference's binaries in its built-in bench mode; returns
    (faces/s, ms/face) of its best trial or None."""
    env = dict(env, OMP_NUM_THREADS=str(threads))
    r = subprocess.run([exe] + args + ["--threads", str(threads)], cwd=ROOT, env=env,
                       capture_output=True, text=True, timeout=600)
    m = re.search(r"Best:\s*([\d.]+) ms/batch = ([\d.]+) ms/face\s*\(([\d.]+) face/s\)", r.stdout)
    if r.returncode == 0 and m:
        return float(m.group(3)), float(m.group(2))
    m = re.search(r"Best:\s*([\d.]+) ms/inference\s*\(([\d.]+) face/s\)", r.stdout)
    if r.returncode == 0 and m:
        return float(m.group(2)), float(m.group(1))
    log("reference binary %s failed (rc %d): %s" % (exe, r.returncode, r.stderr[-300:]))
    return None


def cpu_baseline(ffw, runs=5, cooldown=1.0):
    """The reference's own CPU binaries (oracle/_ref, built from its sources)
    on this host.  `value`: fastface_int8_batched --batch 8 on all (up to 16)
    cores, its built-in bench (5 trials x 30 passes, best;
    arcface_forward_int8.c:549-562).  Also: the same on its default 8 threads,
    and the reference's stable protocol for b=1 (bench_stable_int8_ffw4.py:7-13:
    repeated runs of fastface_int8 with a cooldown between them, median of
    the runs' best) with `runs` runs and `cooldown` seconds instead of its 20
    and 3 s, so that the default bench stays within minutes, on 8 threads and
    on all physical cores (at most 16: the GPU box's CPU share per GPU).
    About 40 s of CPU work.  Falls back to the C restatement when the host lacks AVX-VNNI
    (the reference build would SIGILL)."""
    from oracle.oracle import host_has_avx_vnni
    cpu = host_cpu()
    cores = min(16, cpu["physical_cores"] or os.cpu_count() or 1)
    exe = os.path.join(ROOT, "oracle", "_ref", "fastface_int8_batched")
    exe1 = os.path.join(ROOT, "oracle", "_ref", "fastface_int8")
    cc = os.path.join(ROOT, "oracle", "_ref", "compiler.txt")
    compiler = open(cc).read().strip() if os.path.exists(cc) else None
    env = dict(os.environ, OMP_PROC_BIND="close", OMP_PLACES="cores")
    if os.path.exists(exe) and host_has_avx_vnni():
        log("cpu baseline: reference fastface_int8_batched --batch 8, %d threads" % cores)
        best = _ref_best(exe, [ffw, "--batch", "8"], cores, env)
        if best:
            rec = {"value": best[0], "unit": "faces/s", "cores": cores, "kind": "reference",
                   "sample": "reference fastface_int8_batched, B=8 synthetic faces, best of 5x30 "
                             "passes (%.2f ms/face); synthetic FFW4 + committed OPSC2" % best[1],
                   "host": cpu, "compiler": compiler,
                   "build_flags": "-O3 -march=x86-64-v3 -mavx2 -mfma -mavxvnni -fopenmp (Makefile:32-37, "
                                  "CFLAGS_ARCH override)"}
            b8 = _ref_best(exe, [ffw, "--batch", "8"], 8, env)
            if b8:
                rec["value_8_threads"] = b8[0]
            if os.path.exists(exe1):
                # b=1 on the reference's default 8 threads and on all physical
                # cores (BASELINE.md's two thread counts)
                for threads, tag in ((8, "8_threads"), (cores, "all_cores")):
                    b1 = []
                    for i in range(runs):
                        if i:
                            time.sleep(cooldown)
                        r1 = _ref_best(exe1, [ffw], threads, env)
                        if r1:
                            b1.append(r1[1])
                    if b1:
                        log("cpu baseline: reference fastface_int8 b=1, %d threads: median of %d runs %.3f ms"
                            % (threads, len(b1), statistics.median(b1)))
                        rec["b1_ms_" + tag] = min(b1)
                        rec["b1_stable_" + tag] = {
                            "threads": threads, "runs": len(b1), "cooldown_s": cooldown,
                            "median_ms": round(statistics.median(b1), 3),
                            "min_ms": round(min(b1), 3), "max_ms": round(max(b1), 3),
                            "protocol": "bench_stable_int8_ffw4.py:7-13 (median of runs, each the binary's "
                                        "best of 5x30), %d runs / %.1f s cooldown%s"
                                        % (len(b1), cooldown, "" if (len(b1), cooldown) == (20, 3.0)
                                           else " instead of 20 / 3 s")}
            return rec
    from fastface_amd import synth
    from oracle.oracle import Oracle
    log("cpu baseline: C restatement (oracle), B=4")
    orc = Oracle()
    m = orc.load_model(ffw, synth.OPSC_PATH, synth.OPSC2_PATH)
    x = synth.faces_uniform(4, 99)
    t0 = time.perf_counter()
    orc.forward(m, x)
    dt = time.perf_counter() - t0
    orc.free_model(m)
    return {"value": 4 / dt, "unit": "faces/s", "cores": cores, "kind": "port",
            "sample": "oracle/ff_oracle.c forward of 4 synthetic faces", "host": cpu, "compiler": compiler}


def profiler_preloaded():
    """True when a rocprofv3 tool library is loaded into this process (its
    preload or its ROCPROF* settings in the environment)."""
    return ("rocprof" in os.environ.get("LD_PRELOAD", "")
            or any(k.startswith("ROCPROF") for k in os.environ))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--batch", type=int, default=1024)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--profile-reps", type=int, default=3)
    ap.add_argument("--b1024-only", action="store_true",
                    help="time only the B=%d chain, its per-step profile, the dominant-kernel "
                         "timing and the Winograd leg (the rocprofv3 kernel-statistics run: b=1, "
                         "B=8, the config-2 layer, the host-buffer rates, the switched-chain legs "
                         "and the cold-start leg are left out; implied when a profiler is "
                         "preloaded)" % 1024)
    ap.add_argument("--cpu-runs", type=int, default=5,
                    help="runs of the reference's b=1 binary in its stable protocol (reference: 20)")
    ap.add_argument("--cpu-cooldown", type=float, default=1.0,
                    help="seconds between those runs (reference: 3)")
    ap.add_argument("--no-general-epilogue", action="store_true",
                    help="skip the B=1024 legs with every conv on the general epilogue forms "
                         "and with the stride-2 convs and shortcuts unfused (--b1024-only skips "
                         "them too)")
    ap.add_argument("--no-winograd", action="store_true",
                    help="skip the config-5 run of the stage-1 layers as Winograd F(2,3)")
    args = ap.parse_args()
    # Under the rocprofv3 kernel tracer the default run once ended with a host
    # segmentation fault inside the tracer at the first launch of the B=8
    # graph (the same run completes without the tracer).  A traced run
    # therefore takes only the B=1024 legs.
    profiled = profiler_preloaded()
    if profiled and not args.b1024_only:
        log("profiler preloaded: running the B=1024 legs only (as --b1024-only)")
        args.b1024_only = True
    if args.gpus != 1:
        print("bench.py: this build measures one GPU only (the path is per-face data "
              "parallel: N GPUs would each run their own context on a slice of the batch, "
              "with no exchange inside the forward pass).", file=sys.stderr)
        sys.exit(2)

    import fastface_amd
    from fastface_amd import synth

    lib = fastface_amd.load()
    if lib.ffk_device_count() <= 0:
        raise RuntimeError("no HIP device")
    B, K, W = args.batch, args.steps, args.warmup
    ffw = synth.synthetic_ffw4_path(3)
    log("weights %s" % ffw)
    # cold start (the reference's ~180 ms, README.md:91): the first
    # fastface_create of the process (HIP runtime and code objects come up,
    # the FFW4/OPSC files are read, weights packed and uploaded)
    t_create = time.perf_counter()
    ff = fastface_amd.FastFace(ffw, cwd=ROOT)
    first_create_ms = (time.perf_counter() - t_create) * 1e3
    check(lib, lib.fastface_reserve(ff.ff, B), "reserve")
    stream = lib.fastface_stream(ff.ff)

    # inputs resident in HBM before timing (uniform faces)
    x = synth.faces_uniform(B, 5)
    d_in = lib.ffk_malloc(x.nbytes)
    d_out = lib.ffk_malloc(B * 512 * 4)
    check(lib, lib.ffk_memcpy_h2d(d_in, x.ctypes.data, x.nbytes, stream), "upload")
    check(lib, lib.ffk_stream_sync(stream), "sync")

    def step():
        check(lib, lib.fastface_embed_batch_device(ff.ff, d_in, B, d_out, stream), "embed")

    log("warmup %d x B=%d" % (W, B))
    for _ in range(max(W, 1)):
        step()
    check(lib, lib.ffk_stream_sync(stream), "sync")
    # one HIP event between consecutive graph launches: the whole timed region
    # and each step's duration (median / p10 / p90)
    evs = [C.c_void_p() for _ in range(K + 1)]
    for e in evs:
        check(lib, lib.ffk_event_create(C.byref(e)), "event")
    ev0, ev1 = evs[0], evs[K]
    log("timing %d steps" % K)
    t0 = time.perf_counter()
    for i in range(K):
        check(lib, lib.ffk_event_record(evs[i], stream), "record")
        step()
    check(lib, lib.ffk_event_record(evs[K], stream), "record")
    check(lib, lib.ffk_stream_sync(stream), "sync")
    wall = time.perf_counter() - t0
    ms = C.c_float()
    check(lib, lib.ffk_event_elapsed_ms(ev0, ev1, C.byref(ms)), "elapsed")
    ms_per_step = ms.value / K
    faces_per_s = B * K / (ms.value / 1e3)
    per_step = []
    for i in range(K):
        check(lib, lib.ffk_event_elapsed_ms(evs[i], evs[i + 1], C.byref(ms)), "elapsed")
        per_step.append(ms.value)
    p10, p50, p90 = (float(np.percentile(per_step, q)) for q in (10, 50, 90))
    log("%.3f ms/step (median %.3f, p10 %.3f, p90 %.3f), %.0f faces/s (wall %.3f s)"
        % (ms_per_step, p50, p10, p90, faces_per_s, wall))
    out = np.empty((B, 512), np.float32)
    check(lib, lib.ffk_memcpy_d2h(out.ctypes.data, d_out, out.nbytes, stream), "download")
    check(lib, lib.ffk_stream_sync(stream), "sync")
    assert np.isfinite(out).all()
    out_direct = out.copy()          # embeddings of x on the direct path

    # per-launch durations of every step of the chain (events between launches)
    n_steps = lib.fastface_num_steps(ff.ff)
    step_ms = np.zeros(n_steps, np.float32)
    x1 = np.ascontiguousarray(x[:1])
    e1 = np.empty(512, np.float32)
    check(lib, lib.fastface_embed_batch(ff.ff, x.ctypes.data, B, out.ctypes.data), "embed host")
    rc = lib.fastface_profile_steps(ff.ff, B, args.profile_reps, step_ms.ctypes.data)
    if rc != n_steps:
        raise RuntimeError("profile_steps failed: %s" % fastface_amd.last_error())
    info = fastface_amd.fastface_step_info()
    steps = []
    for s in range(n_steps):
        check(lib, lib.fastface_get_step(ff.ff, s, C.byref(info)), "step info")
        steps.append(dict(kind=info.kind, cin=info.cin, cout=info.cout, k=info.kh, s=info.stride,
                          hin=info.hin, hout=info.hout, ops=info.ops_per_face,
                          act=info.act_bytes_per_face, wbytes=info.weight_bytes,
                          ms=float(step_ms[s])))
    by_shape = {}
    for st in steps:
        key = "fc" if st["kind"] == 2 else "%d->%d k%d s%d @%d" % (st["cin"], st["cout"], st["k"],
                                                                    st["s"], st["hin"])
        e = by_shape.setdefault(key, [0, 0.0, st["ops"] * B])
        e[0] += 1
        e[1] += st["ms"]
    for key, (n, tms, ops) in sorted(by_shape.items(), key=lambda kv: -kv[1][1]):
        log("B=%d %-22s x%-2d %8.3f ms total  %7.4f ms each  %6.1f TOP/s" %
            (B, key, n, tms, tms / n, ops / (tms / n * 1e-3) / 1e12))
    dom = [st for st in steps if st["kind"] == 1 and st["cin"] == 256 and st["cout"] == 256
           and st["k"] == 3 and st["s"] == 1]
    # in-chain figure: HIP events between the eager launches of the per-step
    # profile, so it includes the host's launch gap before each launch
    dom_chain_ms = statistics.mean(st["ms"] for st in dom)
    dom_ops = dom[0]["ops"] * B
    # roofline figure: the same kernel at the same batch in the network's two
    # epilogue forms (13 x PReLU max form, 13 x residual + BN second output,
    # both in range), 26 launches captured in one hipGraph and replayed
    # between HIP events on the launch stream -- kernel time without launch
    # gaps, the quantity a kernel trace reports as the launch duration
    from fastface_amd.layerbench import time_layer
    dom_g = time_layer(lib, 256, 256, 3, 1, 14, batch=B, iters=26, graph_reps=20,
                       epis=["prelu_le1_rng", "add_bn_rng"])
    if dom_g["kernel"] != "patch":
        raise RuntimeError("the dominant layer did not take the patch kernel: %s" % dom_g["kernel"])
    dom_ms = dom_g["ms_per_launch"]
    dom_tops = dom_ops / (dom_ms * 1e-3) / 1e12
    total_ops = sum(st["ops"] for st in steps) * B
    chain_tops = total_ops / (ms_per_step * 1e-3) / 1e12
    fc = [st for st in steps if st["kind"] == 2][0]
    stages = {}
    for st in steps:
        if st["kind"] != 1:
            continue
        key = "stage%d" % {112: 1, 56: 1, 28: 2, 14: 3, 7: 4}[st["hout"]] if st["cin"] != 3 else "stem"
        d = stages.setdefault(key, [0.0, 0.0, 0.0])
        d[0] += st["ops"] * B
        d[1] += st["ms"]
        d[2] += st["act"] * B + st["wbytes"]
    stage_util = {k: round(v[0] / (v[1] * 1e-3) / 1e12 / PEAK_INT8_TOPS, 4) for k, v in stages.items()}
    # algorithmic HBM rate of each stage (activation bytes in + out + residual +
    # BN output, plus weights): the epilogue-bound stem / stage 1 against 8 TB/s
    stage_gbs = {k: round(v[2] / (v[1] * 1e-3) / 1e9, 1) for k, v in stages.items()}
    log("dominant conv 256x256x3x3@14: %.4f ms/launch, %.1f TOP/s (%.1f%% of peak) from a graph of "
        "26 launches; %.4f ms per launch in the eager per-step chain profile"
        % (dom_ms, dom_tops, 100 * dom_tops / PEAK_INT8_TOPS, dom_chain_ms))

    traffic = None
    tf = os.path.join(ROOT, "profiles", "traffic_conv256_b1024.json")
    if os.path.exists(tf):
        with open(tf) as f:
            tj = json.load(f)
        if DOMINANT_KERNEL in tj.get("kernel", ""):      # counters of this very kernel only
            traffic = tj.get("bytes_per_launch")

    b1_ms = b1_dev_ms = b1_fc_ms = b8_ms_face = b256_faces_s = host_fp32 = host_rgb8 = dev_rgb8 = cfg2 = None
    if not args.b1024_only:
        # b=1 latency: host buffers in, host buffers out (fastface_embed), and the
        # device-only chain
        lat = []
        for i in range(60):
            t = time.perf_counter()
            check(lib, lib.fastface_embed(ff.ff, x1.ctypes.data, e1.ctypes.data), "embed b1")
            lat.append((time.perf_counter() - t) * 1e3)
        lat = sorted(lat[10:])
        b1_ms = statistics.median(lat)
        check(lib, lib.fastface_embed_batch_device(ff.ff, d_in, 1, d_out, stream), "b1 dev")
        check(lib, lib.ffk_stream_sync(stream), "sync")
        check(lib, lib.ffk_event_record(ev0, stream), "record")
        for _ in range(50):
            check(lib, lib.fastface_embed_batch_device(ff.ff, d_in, 1, d_out, stream), "b1 dev")
        check(lib, lib.ffk_event_record(ev1, stream), "record")
        check(lib, lib.ffk_event_elapsed_ms(ev0, ev1, C.byref(ms)), "elapsed")
        b1_dev_ms = ms.value / 50
        log("b=1: %.3f ms host-to-host median, %.3f ms device chain" % (b1_ms, b1_dev_ms))
        b1_steps = np.zeros(n_steps, np.float32)
        if lib.fastface_profile_steps(ff.ff, 1, 20, b1_steps.ctypes.data) == n_steps:
            for s in np.argsort(-b1_steps)[:8]:
                st = steps[s]
                log("b=1 step %2d: %.4f ms  conv %d->%d k%d s%d @%d" % (s, b1_steps[s], st["cin"],
                    st["cout"], st["k"], st["s"], st["hin"]))
            log("b=1 sum of step times %.4f ms" % float(b1_steps.sum()))
            fc_steps = [s for s in range(n_steps) if steps[s]["kind"] == 2]
            if fc_steps:
                b1_fc_ms = float(b1_steps[fc_steps[0]])
                log("b=1 FC head: %.4f ms, %.0f GB/s of weights" % (b1_fc_ms, steps[fc_steps[0]]["wbytes"]
                                                                    / (b1_fc_ms * 1e-3) / 1e9))

        # B=8 (the reference README's batched operating point),
        # device-resident chain, ms per face
        check(lib, lib.fastface_embed_batch_device(ff.ff, d_in, 8, d_out, stream), "b8 dev")
        check(lib, lib.ffk_stream_sync(stream), "sync")
        check(lib, lib.ffk_event_record(ev0, stream), "record")
        for _ in range(50):
            check(lib, lib.fastface_embed_batch_device(ff.ff, d_in, 8, d_out, stream), "b8 dev")
        check(lib, lib.ffk_event_record(ev1, stream), "record")
        check(lib, lib.ffk_event_elapsed_ms(ev0, ev1, C.byref(ms)), "elapsed")
        b8_ms_face = ms.value / 50 / 8
        log("B=8: %.4f ms/face (%.3f ms per batch), device chain" % (b8_ms_face, b8_ms_face * 8))

        # B=256 throughput (the synthetic FFW4 is the config's
        # seed-3 random-init model), device-resident chain
        for _ in range(3):
            check(lib, lib.fastface_embed_batch_device(ff.ff, d_in, 256, d_out, stream), "b256 dev")
        check(lib, lib.ffk_stream_sync(stream), "sync")
        check(lib, lib.ffk_event_record(ev0, stream), "record")
        for _ in range(20):
            check(lib, lib.fastface_embed_batch_device(ff.ff, d_in, 256, d_out, stream), "b256 dev")
        check(lib, lib.ffk_event_record(ev1, stream), "record")
        check(lib, lib.ffk_event_elapsed_ms(ev0, ev1, C.byref(ms)), "elapsed")
        b256_faces_s = 256 * 20 / (ms.value * 1e-3)
        log("B=256: %.3f ms per batch, %.0f faces/s, device chain" % (ms.value / 20, b256_faces_s))

        # the single 256->256 3x3 layer microbench at N=64
        from fastface_amd.layerbench import time_layer
        cfg2 = time_layer(lib, 256, 256, 3, 1, 14, batch=64, iters=200, epi="prelu")
        log("config 2 layer (N=64, 14x14, 256->256, PReLU): %.4f ms, %.1f TOP/s (%.1f%% of peak), %s"
            % (cfg2["ms_per_launch"], cfg2["int8_tops"], 100 * cfg2["frac_of_peak"], cfg2["kernel"]))

        # Host-buffer (PCIe-inclusive) rates of the boundary: fp32 faces and the
        # uint8 RGB entry point (a quarter of the input bytes).  Reported beside
        # `value`, never as it.  Pageable numpy buffers, as a caller would pass.
        imgs = np.random.default_rng(5).integers(0, 256, size=(B, 112, 112, 3), dtype=np.uint8)

        def host_rate(fn, arr, reps=3):
            fn(ff.ff, arr.ctypes.data, B, out.ctypes.data)           # capture / warm
            t = time.perf_counter()
            for _ in range(reps):
                check(lib, fn(ff.ff, arr.ctypes.data, B, out.ctypes.data), "host embed")
            return B * reps / (time.perf_counter() - t)
        host_fp32 = host_rate(lib.fastface_embed_batch, x)
        host_rgb8 = host_rate(lib.fastface_embed_batch_rgb8, imgs)
        d_img = lib.ffk_malloc(imgs.nbytes)
        check(lib, lib.ffk_memcpy_h2d(d_img, imgs.ctypes.data, imgs.nbytes, stream), "upload rgb8")
        check(lib, lib.fastface_embed_batch_rgb8_device(ff.ff, d_img, B, d_out, stream), "rgb8 dev")
        check(lib, lib.ffk_stream_sync(stream), "sync")
        check(lib, lib.ffk_event_record(ev0, stream), "record")
        for _ in range(K):
            check(lib, lib.fastface_embed_batch_rgb8_device(ff.ff, d_img, B, d_out, stream), "rgb8 dev")
        check(lib, lib.ffk_event_record(ev1, stream), "record")
        check(lib, lib.ffk_event_elapsed_ms(ev0, ev1, C.byref(ms)), "elapsed")
        dev_rgb8 = B * K / (ms.value / 1e3)
        lib.ffk_free(d_img)
        log("B=%d host buffers: fp32 %.0f faces/s, uint8 RGB %.0f faces/s; uint8 RGB resident %.0f faces/s"
            % (B, host_fp32, host_rgb8, dev_rgb8))

    # BASELINE config 5 also runs the stage-1 64-channel 3x3 stride-1 convs as
    # integer Winograd F(2,3): same batch, same timing; the embeddings must be
    # bit-identical to the direct path's
    wino = None
    if not args.no_winograd:
        n_w = lib.fastface_set_conv_algo(ff.ff, 1)
        if n_w <= 0:
            raise RuntimeError("fastface_set_conv_algo failed (%d)" % n_w)
        for _ in range(3):
            step()
        check(lib, lib.ffk_stream_sync(stream), "sync")
        kw = max(K // 4, 5)
        check(lib, lib.ffk_event_record(ev0, stream), "record")
        for _ in range(kw):
            step()
        check(lib, lib.ffk_event_record(ev1, stream), "record")
        check(lib, lib.ffk_event_elapsed_ms(ev0, ev1, C.byref(ms)), "elapsed")
        w_ms = ms.value / kw
        out_w = np.empty((B, 512), np.float32)
        check(lib, lib.ffk_memcpy_d2h(out_w.ctypes.data, d_out, out_w.nbytes, stream), "download")
        check(lib, lib.ffk_stream_sync(stream), "sync")
        same = bool(np.array_equal(out_w, out_direct))
        w_steps = np.zeros(n_steps, np.float32)
        if lib.fastface_profile_steps(ff.ff, B, args.profile_reps, w_steps.ctypes.data) != n_steps:
            raise RuntimeError("profile_steps failed: %s" % fastface_amd.last_error())
        layers = {}
        for s_ in range(n_steps):
            check(lib, lib.fastface_get_step(ff.ff, s_, C.byref(info)), "step info")
            if not info.flags & fastface_amd.FFK_ALGO_WINOGRAD:
                continue
            key = "64->64 k3 s1 @%d" % info.hin
            e = layers.setdefault(key, {"n": 0, "winograd_ms": 0.0, "direct_ms": 0.0,
                                        "ops": info.ops_per_face * B})
            e["n"] += 1
            e["winograd_ms"] += float(w_steps[s_])
            e["direct_ms"] += steps[s_]["ms"]
        for key, e in layers.items():
            n = e.pop("n")
            ops = e.pop("ops")
            e.update(count=n, winograd_ms=round(e["winograd_ms"] / n, 4),
                     direct_ms=round(e["direct_ms"] / n, 4))
            e["winograd_frac_of_int8_peak"] = round(ops / (e["winograd_ms"] * 1e-3) / 1e12 / PEAK_INT8_TOPS, 4)
            log("B=%d %s x%d: Winograd F(2,3) %.4f ms, direct %.4f ms" % (B, key, n, e["winograd_ms"],
                                                                         e["direct_ms"]))
        wino = {"layers": n_w, "faces_s": round(B / (w_ms * 1e-3), 1), "ms_per_step": round(w_ms, 4),
                "embeddings_equal_direct": same, "per_layer": layers}
        log("B=%d Winograd stage 1: %.3f ms/step, %.0f faces/s, embeddings %s the direct path's"
            % (B, w_ms, wino["faces_s"], "equal to" if same else "DIFFERENT FROM"))
        if not same:
            raise RuntimeError("Winograd embeddings differ from the direct path")
        check(lib, lib.fastface_set_conv_algo(ff.ff, 0), "algo direct")

    # The B=1024 chain with a context switch flipped: throughput, and the
    # embeddings, which must stay bit-identical to the default chain's.
    def switched_leg(setter, value, restore, what):
        n_l = setter(ff.ff, value)
        if n_l < 0:
            raise RuntimeError("%s: switch failed (%d)" % (what, n_l))
        for _ in range(3):
            step()
        check(lib, lib.ffk_stream_sync(stream), "sync")
        kg = max(K // 4, 5)
        check(lib, lib.ffk_event_record(ev0, stream), "record")
        for _ in range(kg):
            step()
        check(lib, lib.ffk_event_record(ev1, stream), "record")
        check(lib, lib.ffk_event_elapsed_ms(ev0, ev1, C.byref(ms)), "elapsed")
        l_ms = ms.value / kg
        out_l = np.empty((B, 512), np.float32)
        check(lib, lib.ffk_memcpy_d2h(out_l.ctypes.data, d_out, out_l.nbytes, stream), "download")
        check(lib, lib.ffk_stream_sync(stream), "sync")
        same = bool(np.array_equal(out_l, out_direct))
        log("B=%d %s (%d): %.3f ms/step, %.0f faces/s, embeddings %s"
            % (B, what, n_l, l_ms, B / (l_ms * 1e-3), "equal to the default chain's" if same else "DIFFERENT"))
        if not same:
            raise RuntimeError("%s: embeddings differ from the default chain's" % what)
        if setter(ff.ff, restore) < 0:          # (returns a count)
            raise RuntimeError("%s: restoring failed: %s" % (what, fastface_amd.last_error()))
        return n_l, round(B / (l_ms * 1e-3), 1), round(l_ms, 4)

    # every conv on the general epilogue forms (the reference's compare/select
    # PReLU and cvttps2dq emulation, which a model whose parameters do not
    # prove the shorter forms runs)
    general = None
    # each stage's stride-2 conv and 1x1 shortcut as two launches instead of one
    separate = None
    if not args.no_general_epilogue and not args.b1024_only:
        n_g, f_g, m_g = switched_leg(lib.fastface_set_epilogue_forms, 1, 0, "general epilogue forms")
        general = {"launches": n_g, "faces_s": f_g, "ms_per_step": m_g, "embeddings_equal_fast_forms": True}
        n_p, f_p, m_p = switched_leg(lib.fastface_set_shortcut_fusion, 0, 1, "stride-2 convs and shortcuts unfused")
        separate = {"pairs": n_p, "faces_s": f_p, "ms_per_step": m_p, "embeddings_equal_fused": True}

    # a second context in the same process: create, first b=1 embed (captures
    # its launch chain), destroy
    cold = {"first_create_ms": round(first_create_ms, 1)}
    if not args.b1024_only:
        t_c = time.perf_counter()
        ff2 = fastface_amd.FastFace(ffw, cwd=ROOT)
        create_ms = (time.perf_counter() - t_c) * 1e3
        t_e = time.perf_counter()
        ff2.embed(x1[0] if x1.ndim == 4 else x1)
        first_embed_ms = (time.perf_counter() - t_e) * 1e3
        ff2.close()
        cold.update(create_ms=round(create_ms, 1), first_embed_ms=round(first_embed_ms, 2))
        log("cold start: first create %.1f ms, create %.1f ms, first embed %.2f ms"
            % (first_create_ms, create_ms, first_embed_ms))
    cold["note"] = ("first_create: the process's first fastface_create (HIP runtime start-up "
                    "included); create: a second context; first_embed: its first b=1 embed "
                    "(launch chain captured)")

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(ffw, runs=args.cpu_runs, cooldown=args.cpu_cooldown)
        log("cpu baseline: %.1f %s (%s)" % (cpu["value"], cpu["unit"], cpu["kind"]))

    ff.close()

    def rnd(v, n):
        return None if v is None else round(v, n)
    rec = {
        "metric": METRIC,
        "value": round(faces_per_s, 1),
        "unit": "faces/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(ms_per_step, 4),
        "ms_per_step_median": round(p50, 4),
        "ms_per_step_p10": round(p10, 4),
        "ms_per_step_p90": round(p90, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded uniform faces; synthetic FFW4 weights, committed OPSC/OPSC2 scales)",
        "config": {"workload": "ArcFace IResNet-50 INT8 forward, B=%d (BASELINE config 5), "
                               "inputs resident in HBM, one hipGraph per step" % B,
                   "global_batch": B, "input": "112x112x3 fp32 NHWC", "parallelism": "single GPU"},
        "b1_latency_ms": rnd(b1_ms, 4),
        "host_fp32_faces_s": rnd(host_fp32, 1),
        "host_rgb8_faces_s": rnd(host_rgb8, 1),
        "rgb8_resident_faces_s": rnd(dev_rgb8, 1),
        "b1_device_ms": rnd(b1_dev_ms, 4),
        "b1_fc_ms": rnd(b1_fc_ms, 4),
        "b8_ms_per_face": rnd(b8_ms_face, 5),
        "b256_faces_s": rnd(b256_faces_s, 1),
        "config2_layer": cfg2,
        "chain_int8_tops": round(chain_tops, 2),
        "chain_frac_of_int8_peak": round(chain_tops / PEAK_INT8_TOPS, 4),
        "stage_frac_of_int8_peak": stage_util,
        "stage_hbm_gbs": stage_gbs,
        "fc_ms": round(fc["ms"], 4),
        "fc_hbm_gbs": round((fc["wbytes"] + fc["act"] * B) / (fc["ms"] * 1e-3) / 1e9, 1),
        "roofline": {"bound": "mfma", "kernel": DOMINANT_KERNEL,
                     "achieved": round(dom_tops, 2), "peak": PEAK_INT8_TOPS, "unit": "TOP/s",
                     "frac": round(dom_tops / PEAK_INT8_TOPS, 4), "traffic": traffic,
                     "launch_ms": round(dom_ms, 5), "ops_per_launch": dom_ops,
                     "launch_ms_in_eager_chain": round(dom_chain_ms, 5),
                     "timing": "26 launches (13 PReLU, 13 residual+BN) in one hipGraph, 20 replays "
                               "between HIP events on the launch stream"},
        "stage1_winograd": wino,
        "general_epilogue": general,
        "unfused_shortcuts": separate,
        "cold_start": cold,
        "profiler_preloaded": profiled,
        "cpu_baseline": cpu,
    }
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
