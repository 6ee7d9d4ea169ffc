"""fastface_amd -- MI355X-native INT8 IResNet-50 (ArcFace) face embedding.

The product is the C library `lib/libfastface_amd.so` (C99 host code +
gfx950 HIP kernels) exporting the reference's `fastface.h` API and the
kernel-level `fastface_kernels.h` ABI.  This package only loads it with
ctypes; there is no Python or CPU compute path -- if the library is missing
or no GPU is present, loading fails loudly.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
REPO_ROOT = os.path.dirname(HERE)
LIB_PATH = os.environ.get("FASTFACE_LIB") or os.path.join(HERE, "lib", "libfastface_amd.so")
CSRC = os.path.join(HERE, "csrc")

FASTFACE_INPUT_N = 37632
FASTFACE_OUTPUT_N = 512

# fastface_kernels.h
FFK_EPI_PRELU, FFK_EPI_ADD, FFK_EPI_BN, FFK_EPI_BIAS, FFK_EPI_INSCALE = 1, 2, 4, 8, 16
FFK_IN_RGB8 = 0x20
FFK_EPI_PRELU_LE1 = 0x40
FFK_ALGO_WINOGRAD = 0x80
FFK_OUT_X_EVEN = 0x100
FFK_EPI_IN_RANGE = 0x200
FFK_EPI_FMA_TAIL = 0x800
FFK_SHARED_GPU = 0x400
FFK_NOALLOC_SCRATCH_BYTES = 2048 + 320 * 64 * 64 * 4
(FFK_P_WS, FFK_P_BIAS, FFK_P_SLOPE, FFK_P_ADDSCALE, FFK_P_INV, FFK_P_BN_SIN, FFK_P_BN_S,
 FFK_P_BN_O, FFK_P_BN_INV, FFK_NPARAM) = range(10)

_p = C.c_void_p


class ffk_io(C.Structure):
    _fields_ = [("in_", _p), ("out", _p)]


class ffk_conv_desc(C.Structure):
    _fields_ = [("batch", C.c_int), ("cin", C.c_int), ("cout", C.c_int), ("kh", C.c_int),
                ("kw", C.c_int), ("stride", C.c_int), ("pad", C.c_int), ("hin", C.c_int),
                ("win", C.c_int), ("in_", _p), ("in_inv", _p), ("io", _p), ("w", _p),
                ("params", _p), ("add_src", _p), ("bn_lut", _p), ("out", _p), ("out_bn", _p),
                ("out_i32", _p),
                ("flags", C.c_int), ("in_scale", C.c_float),
                ("workspace", _p), ("workspace_bytes", C.c_size_t), ("in_lut", _p)]


class ffk_fc_desc(C.Structure):
    _fields_ = [("batch", C.c_int), ("n", C.c_int), ("k", C.c_int), ("a", _p), ("w", _p),
                ("ws", _p), ("bias", _p), ("a_scale", C.c_float), ("out", _p), ("io", _p),
                ("path", C.c_int), ("workspace", _p), ("workspace_bytes", C.c_size_t)]


class fastface_step_info(C.Structure):
    _fields_ = [("kind", C.c_int), ("op_first", C.c_int), ("op_last", C.c_int),
                ("cin", C.c_int), ("cout", C.c_int), ("kh", C.c_int), ("kw", C.c_int),
                ("stride", C.c_int), ("pad", C.c_int), ("hin", C.c_int), ("win", C.c_int),
                ("hout", C.c_int), ("wout", C.c_int), ("flags", C.c_int), ("stores_x", C.c_int),
                ("ops_per_face", C.c_double), ("act_bytes_per_face", C.c_double),
                ("weight_bytes", C.c_double)]


# (name, restype, argtypes) of every exported symbol declared in include/*.h
EXPORTS = [
    # fastface.h
    ("fastface_create", _p, [C.c_char_p]),
    ("fastface_create_with_scales", _p, [C.c_char_p, C.c_char_p, C.c_char_p]),
    ("fastface_embed", C.c_int, [_p, _p, _p]),
    ("fastface_destroy", None, [_p]),
    ("fastface_embed_batch", C.c_int, [_p, _p, C.c_int, _p]),
    ("fastface_embed_batch_device", C.c_int, [_p, _p, C.c_int, _p, _p]),
    ("fastface_embed_batch_rgb8", C.c_int, [_p, _p, C.c_int, _p]),
    ("fastface_embed_batch_rgb8_device", C.c_int, [_p, _p, C.c_int, _p, _p]),
    ("fastface_reserve", C.c_int, [_p, C.c_int]),
    ("fastface_stream", _p, [_p]),
    ("fastface_set_conv_algo", C.c_int, [_p, C.c_int]),
    ("fastface_set_epilogue_forms", C.c_int, [_p, C.c_int]),
    ("fastface_set_shortcut_fusion", C.c_int, [_p, C.c_int]),
    ("fastface_num_steps", C.c_int, [_p]),
    ("fastface_get_step", C.c_int, [_p, C.c_int, C.POINTER(fastface_step_info)]),
    ("fastface_profile_steps", C.c_int, [_p, C.c_int, C.c_int, _p]),
    ("fastface_debug_keep_tensors", C.c_int, [_p, C.c_int]),
    ("fastface_debug_read", C.c_longlong, [_p, C.c_int, C.c_int, _p, C.c_size_t]),
    # fastface_kernels.h
    ("ffk_last_error", C.c_char_p, []),
    ("ffk_device_count", C.c_int, []),
    ("ffk_malloc", _p, [C.c_size_t]),
    ("ffk_free", C.c_int, [_p]),
    ("ffk_host_alloc", _p, [C.c_size_t]),
    ("ffk_host_free", C.c_int, [_p]),
    ("ffk_memcpy_h2d", C.c_int, [_p, _p, C.c_size_t, _p]),
    ("ffk_memcpy_d2h", C.c_int, [_p, _p, C.c_size_t, _p]),
    ("ffk_memcpy_d2d", C.c_int, [_p, _p, C.c_size_t, _p]),
    ("ffk_zero", C.c_int, [_p, C.c_size_t, _p]),
    ("ffk_stream_create", C.c_int, [C.POINTER(_p)]),
    ("ffk_stream_destroy", C.c_int, [_p]),
    ("ffk_stream_sync", C.c_int, [_p]),
    ("ffk_event_create", C.c_int, [C.POINTER(_p)]),
    ("ffk_event_destroy", C.c_int, [_p]),
    ("ffk_event_record", C.c_int, [_p, _p]),
    ("ffk_event_sync", C.c_int, [_p]),
    ("ffk_stream_wait_event", C.c_int, [_p, _p]),
    ("ffk_event_elapsed_ms", C.c_int, [_p, _p, C.POINTER(C.c_float)]),
    ("ffk_graph_begin", C.c_int, [_p]),
    ("ffk_graph_end", C.c_int, [_p, C.POINTER(_p)]),
    ("ffk_graph_launch", C.c_int, [_p, _p]),
    ("ffk_graph_destroy", C.c_int, [_p]),
    ("ffk_conv_supported", C.c_int, [C.c_int] * 8),
    ("ffk_conv_runnable", C.c_int, [C.c_int] * 8),
    ("ffk_prelu_le1_ok", C.c_int, [_p, C.c_int, C.c_int, C.c_int]),
    ("ffk_requant_in_range", C.c_int, [_p, C.c_int, C.c_int, C.c_int]),
    ("ffk_requant_fma_ok", C.c_int, [_p, C.c_int, C.c_int, C.c_int]),
    ("ffk_conv_packed_bytes", C.c_size_t, [C.c_int] * 4),
    ("ffk_pack_conv_weights", C.c_int, [_p, C.c_int, C.c_int, C.c_int, C.c_int, _p]),
    ("ffk_conv_workspace_bytes", C.c_size_t, [C.POINTER(ffk_conv_desc)]),
    ("ffk_conv", C.c_int, [C.POINTER(ffk_conv_desc), _p]),
    ("ffk_conv_noalloc", C.c_int, [C.POINTER(ffk_conv_desc), _p]),
    ("ffk_conv_s2_shortcut", C.c_int, [C.POINTER(ffk_conv_desc), C.POINTER(ffk_conv_desc), _p]),
    ("ffk_conv_variant", C.c_char_p, [C.POINTER(ffk_conv_desc)]),
    ("ffk_conv_grid", C.c_int, [C.POINTER(ffk_conv_desc)]),
    ("ffk_winograd_supported", C.c_int, [C.c_int] * 8),
    ("ffk_winograd_packed_bytes", C.c_size_t, [C.c_int, C.c_int]),
    ("ffk_pack_winograd_weights", C.c_int, [_p, C.c_int, C.c_int, _p]),
    ("ffk_make_bn_lut", C.c_int, [_p, _p, _p, _p, C.c_int, _p]),
    ("ffk_make_rgb8_lut", C.c_int, [_p, _p]),
    ("ffk_make_map_lut", C.c_int, [_p, _p, _p, _p, _p, C.c_int, _p]),
    ("ffk_make_add_lut", C.c_int, [C.c_float, C.c_float, C.c_float, _p]),
    ("ffk_map_i8", C.c_int, [_p, _p, C.c_longlong, C.c_int, _p, _p]),
    ("ffk_add_i8", C.c_int, [_p, _p, _p, C.c_longlong, _p, _p]),
    ("ffk_fc_packed_bytes", C.c_size_t, [C.c_int, C.c_int]),
    ("ffk_pack_fc_weights", C.c_int, [_p, C.c_int, C.c_int, _p]),
    ("ffk_pack_fc_row", C.c_int, [_p, C.c_int, C.c_int, C.c_int, _p]),
    ("ffk_fc", C.c_int, [C.POINTER(ffk_fc_desc), _p]),
    ("ffk_fc_workspace_bytes", C.c_size_t, [C.POINTER(ffk_fc_desc)]),
    ("ffk_selftest_mfma", C.c_int, []),
]

_lib = None


def build(verbose=False):
    """Compile the library in-tree (hipcc --offload-arch=gfx950 + gcc)."""
    import subprocess
    jobs = str(min(8, os.cpu_count() or 4))
    subprocess.run(["make", "-C", CSRC, "-j", jobs] + ([] if verbose else ["-s"]), check=True)


def load():
    """Load libfastface_amd.so (raises if it is not built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError("fastface_amd: %s is not built (run __graft_entry__.build())" % LIB_PATH)
    lib = C.CDLL(LIB_PATH)
    for name, res, args in EXPORTS:
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def last_error():
    return load().ffk_last_error().decode(errors="replace")


from .api import FastFace  # noqa: E402,F401
