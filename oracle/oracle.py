"""ctypes bindings for the CPU oracle (liboracle.so) and for the reference's
own int8 path compiled from its sources (_ref/libfastface_ref.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the product package.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_DIR = os.path.join(HERE, "_ref")
REF_SO = os.path.join(REF_DIR, "libfastface_ref.so")

_p = C.c_void_p
_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")


def build():
    subprocess.run(["make", "-s", "-C", HERE, "all"], check=True)


def _opt(a, dtype):
    """numpy array -> pointer, None -> NULL."""
    if a is None:
        return None
    a = np.ascontiguousarray(a, dtype=dtype)
    return a.ctypes.data_as(_p), a


class Oracle:
    def __init__(self, path=ORACLE_SO):
        if not os.path.exists(path):
            build()
        L = self.lib = C.CDLL(path)
        L.orc_cvtt_x86.argtypes = [C.c_float]
        L.orc_cvtt_x86.restype = C.c_int32
        L.orc_quant_input_pc.argtypes = [_f32p, C.c_int, C.c_int, _f32p, _i8p]
        L.orc_conv_i32.argtypes = [_i8p, C.c_int, C.c_int, C.c_int, C.c_int, _i8p,
                                   C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                   C.c_int, C.c_int, _i32p]
        _i16p = np.ctypeslib.ndpointer(np.int16, flags="C_CONTIGUOUS")
        L.orc_winograd_f23_weights.argtypes = [_i8p, C.c_int, C.c_int, _i16p]
        L.orc_conv_winograd_f23.argtypes = [_i8p, C.c_int, C.c_int, C.c_int, C.c_int, _i16p,
                                            C.c_int, _i32p]
        L.orc_fused_epilogue.argtypes = [_i32p, C.c_int, C.c_int, C.c_float, _p, _p, _p,
                                         _p, _p, _p, C.c_float, _p, _p, C.c_float, _i8p]
        L.orc_bn_prelu_requant.argtypes = [_i8p, C.c_float, _p, _p, _p, _p, _p,
                                           C.c_float, _i8p, C.c_int, C.c_int]
        L.orc_add_requant.argtypes = [_i8p, C.c_float, _i8p, C.c_float, _i8p,
                                      C.c_float, C.c_int]
        L.orc_quant_input_pt.argtypes = [_f32p, C.c_int, C.c_float, _i8p]
        L.orc_fc.argtypes = [_i8p, _i8p, _f32p, _f32p, C.c_float, _f32p, C.c_int, C.c_int]
        L.orc_model_load.argtypes = [C.c_char_p, C.c_char_p, C.c_char_p]
        L.orc_model_load.restype = _p
        L.orc_model_free.argtypes = [_p]
        L.orc_model_n_ops.argtypes = [_p]
        L.orc_model_version.argtypes = [_p]
        self._dump_t = C.CFUNCTYPE(None, _p, C.c_int, C.POINTER(C.c_int8),
                                   C.c_int, C.c_int, C.c_int, C.c_int)
        L.orc_forward.argtypes = [_p, _f32p, C.c_int, _f32p, self._dump_t, _p]
        L.orc_forward.restype = C.c_int

    # ---- kernels ----
    def cvtt(self, r):
        return self.lib.orc_cvtt_x86(r)

    def quant_input(self, x, inv_pc):
        x = np.ascontiguousarray(x, np.float32)
        C_ = x.shape[-1]
        out = np.empty(x.shape, np.int8)
        self.lib.orc_quant_input_pc(x.reshape(-1), x.size // C_, C_,
                                    np.ascontiguousarray(inv_pc, np.float32), out.reshape(-1))
        return out

    def quant_input_pt(self, x, scale):
        """Per-tensor input quantization (the OPSC-only path)."""
        x = np.ascontiguousarray(x, np.float32).reshape(-1)
        out = np.empty(x.size, np.int8)
        self.lib.orc_quant_input_pt(x, x.size, scale, out)
        return out

    def conv_i32(self, x, w_oihw, stride, pad):
        """x [B,H,W,Cin] int8, w [Cout,Cin,KH,KW] int8 -> int32 [B,Ho,Wo,Cout]."""
        x = np.ascontiguousarray(x, np.int8)
        w = np.ascontiguousarray(w_oihw, np.int8)
        B, H, W, Cin = x.shape
        Cout, _, KH, KW = w.shape
        Ho = (H + 2 * pad - KH) // stride + 1
        Wo = (W + 2 * pad - KW) // stride + 1
        out = np.empty((B, Ho, Wo, Cout), np.int32)
        self.lib.orc_conv_i32(x.reshape(-1), B, H, W, Cin, w.reshape(-1), Cout, KH, KW,
                              stride, pad, Ho, Wo, out.reshape(-1))
        return out

    def winograd_weights(self, w_oihw):
        """[Cout,Cin,3,3] int8 -> u = G' g G'^T, int16 [16, Cout, Cin]."""
        w = np.ascontiguousarray(w_oihw, np.int8)
        Cout, Cin = w.shape[:2]
        u = np.empty((16, Cout, Cin), np.int16)
        self.lib.orc_winograd_f23_weights(w.reshape(-1), Cout, Cin, u.reshape(-1))
        return u

    def conv_winograd(self, x, u):
        """x [B,H,W,Cin] int8 (H, W even), u from winograd_weights -> int32
        [B,H,W,Cout] = 4 x the 3x3 s1 p1 convolution."""
        x = np.ascontiguousarray(x, np.int8)
        B, H, W, Cin = x.shape
        Cout = u.shape[1]
        out = np.empty((B, H, W, Cout), np.int32)
        self.lib.orc_conv_winograd_f23(x.reshape(-1), B, H, W, Cin,
                                       np.ascontiguousarray(u, np.int16).reshape(-1), Cout,
                                       out.reshape(-1))
        return out

    def fused_epilogue(self, acc, ws, bias=None, in_scale=1.0, bn_scale=None,
                       bn_offset=None, prelu=None, add_src=None, add_scale=0.0,
                       add_scale_pc=None, inv_pc=None, out_scale=1.0):
        acc = np.ascontiguousarray(acc, np.int32)
        Cout = acc.shape[-1]
        keep = []

        def P(a, dt=np.float32):
            r = _opt(a, dt)
            if r is None:
                return None
            keep.append(r[1])
            return r[0]
        out = np.empty(acc.shape, np.int8)
        self.lib.orc_fused_epilogue(acc.reshape(-1), acc.size // Cout, Cout, in_scale,
                                    P(ws), P(bias), P(bn_scale), P(bn_offset), P(prelu),
                                    P(add_src, np.int8), add_scale, P(add_scale_pc),
                                    P(inv_pc), out_scale, out.reshape(-1))
        return out

    def bn_prelu_requant(self, x, in_scale=1.0, in_scale_pc=None, bn_scale=None,
                         bn_offset=None, prelu=None, inv_pc=None, out_scale=1.0):
        x = np.ascontiguousarray(x, np.int8)
        C_ = x.shape[-1]
        keep = []

        def P(a):
            r = _opt(a, np.float32)
            if r is None:
                return None
            keep.append(r[1])
            return r[0]
        out = np.empty(x.shape, np.int8)
        self.lib.orc_bn_prelu_requant(x.reshape(-1), in_scale, P(in_scale_pc), P(bn_scale),
                                      P(bn_offset), P(prelu), P(inv_pc), out_scale,
                                      out.reshape(-1), x.size // C_, C_)
        return out

    def add_requant(self, a, a_scale, b, b_scale, out_scale):
        a = np.ascontiguousarray(a, np.int8).reshape(-1)
        b = np.ascontiguousarray(b, np.int8).reshape(-1)
        out = np.empty_like(a)
        self.lib.orc_add_requant(a, a_scale, b, b_scale, out, out_scale, a.size)
        return out

    def fc(self, a, W, ws, bias, a_scale=1.0):
        a = np.ascontiguousarray(a, np.int8).reshape(-1)
        W = np.ascontiguousarray(W, np.int8)
        N, K = W.shape
        out = np.empty(N, np.float32)
        self.lib.orc_fc(a, W, np.ascontiguousarray(ws, np.float32),
                        np.ascontiguousarray(bias, np.float32), a_scale, out, N, K)
        return out

    # ---- model ----
    def load_model(self, ffw, opsc, opsc2):
        m = self.lib.orc_model_load(ffw.encode(), opsc.encode(),
                                    opsc2.encode() if opsc2 else None)
        if not m:
            raise RuntimeError("oracle: model load failed: %s" % ffw)
        return m

    def free_model(self, m):
        self.lib.orc_model_free(m)

    def forward(self, model, faces, dump_ops=None):
        """faces [B,112,112,3] fp32 -> ([B,512] fp32, {op_idx: int8 NHWC})."""
        faces = np.ascontiguousarray(faces, np.float32)
        B = faces.shape[0]
        out = np.empty((B, 512), np.float32)
        dumps = {}

        def cb(user, op_idx, ptr, b, h, w, c):
            if dump_ops is None or op_idx in dump_ops:
                n = b * h * w * c
                dumps[op_idx] = np.ctypeslib.as_array(ptr, shape=(n,)).copy().reshape(b, h, w, c)
        fn = self._dump_t(cb) if dump_ops is not None else self._dump_t()
        rc = self.lib.orc_forward(model, faces.reshape(-1), B, out.reshape(-1), fn, None)
        if rc != 0:
            raise RuntimeError("oracle forward failed rc=%d" % rc)
        return out, dumps


def host_has_avx_vnni():
    try:
        with open("/proc/cpuinfo") as f:
            return "avx_vnni" in f.read()
    except OSError:
        return False


class Ref:
    """The reference's shipped int8 functions, compiled from its sources
    (oracle/Makefile `ref`).  Needs an AVX-VNNI host."""

    def __init__(self, path=REF_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        L = self.lib = C.CDLL(path)
        L.fused_epilogue_int8.argtypes = [_i32p, C.c_int, C.c_int, C.c_float, _p, _p, _p, _p,
                                          _p, _p, C.c_float, _p, _p, C.c_float, _i8p]
        L.bn_prelu_requant_int8.argtypes = [_i8p, C.c_float, _p, _p, _p, _p, _p, C.c_float,
                                            _i8p, C.c_int, C.c_int]
        L.quantize_fp32_nhwc_to_int8_per_channel.argtypes = [_f32p, C.c_int, C.c_int, _f32p, _i8p]
        L.quantize_fp32_nhwc_to_int8.argtypes = [_f32p, C.c_int, C.c_float, _i8p]
        L.add_requant_int8.argtypes = [_i8p, C.c_float, _i8p, C.c_float, _i8p, C.c_float, C.c_int]
        L.pack_conv_weight_nhwc.argtypes = [_i8p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                            _i8p, _i8p, _i32p]
        L.fastface_conv2d_i8_nhwc_batched.argtypes = [_i8p, C.c_int, C.c_int, C.c_int, C.c_int,
                                                      C.c_int, C.c_int, C.c_int, C.c_int,
                                                      C.c_int, _i8p, _i32p, C.c_int, C.c_int,
                                                      _i32p, _u8p]
        L.fastface_gemm_i8_matvec_vnni.argtypes = [_u8p, _i8p, _i32p, _f32p, _f32p, C.c_float,
                                                   _f32p, C.c_int, C.c_int]
        _i16p = np.ctypeslib.ndpointer(np.int16, flags="C_CONTIGUOUS")
        L.winograd_int8_transform_weights_ref.argtypes = [_i8p, C.c_int, C.c_int, _i16p]
        L.fastface_conv2d_i8_winograd_f23_ref.argtypes = [_i8p, C.c_int, C.c_int, C.c_int,
                                                          C.c_int, _i16p, _i32p]
        L.fastface_create.argtypes = [C.c_char_p]
        L.fastface_create.restype = _p
        L.fastface_embed.argtypes = [_p, _f32p, _f32p]
        L.fastface_embed.restype = C.c_int
        L.fastface_destroy.argtypes = [_p]

    def fused_epilogue(self, acc, ws, bias=None, in_scale=1.0, bn_scale=None,
                       bn_offset=None, prelu=None, add_src=None, add_scale=0.0,
                       add_scale_pc=None, inv_pc=None, out_scale=1.0):
        acc = np.ascontiguousarray(acc, np.int32)
        Cout = acc.shape[-1]
        keep = []

        def P(a, dt=np.float32):
            r = _opt(a, dt)
            if r is None:
                return None
            keep.append(r[1])
            return r[0]
        out = np.empty(acc.shape, np.int8)
        self.lib.fused_epilogue_int8(acc.reshape(-1), acc.size // Cout, Cout, in_scale, P(ws),
                                     P(bias), P(bn_scale), P(bn_offset), P(prelu),
                                     P(add_src, np.int8), add_scale, P(add_scale_pc),
                                     P(inv_pc), out_scale, out.reshape(-1))
        return out

    def bn_prelu_requant(self, x, in_scale=1.0, in_scale_pc=None, bn_scale=None,
                         bn_offset=None, prelu=None, inv_pc=None, out_scale=1.0):
        x = np.ascontiguousarray(x, np.int8)
        C_ = x.shape[-1]
        keep = []

        def P(a):
            r = _opt(a, np.float32)
            if r is None:
                return None
            keep.append(r[1])
            return r[0]
        out = np.empty(x.shape, np.int8)
        self.lib.bn_prelu_requant_int8(x.reshape(-1), in_scale, P(in_scale_pc), P(bn_scale),
                                       P(bn_offset), P(prelu), P(inv_pc), out_scale,
                                       out.reshape(-1), x.size // C_, C_)
        return out

    def quant_input(self, x, inv_pc):
        x = np.ascontiguousarray(x, np.float32)
        C_ = x.shape[-1]
        out = np.empty(x.shape, np.int8)
        self.lib.quantize_fp32_nhwc_to_int8_per_channel(
            x.reshape(-1), x.size // C_, C_, np.ascontiguousarray(inv_pc, np.float32),
            out.reshape(-1))
        return out

    def quant_input_pt(self, x, scale):
        x = np.ascontiguousarray(x, np.float32).reshape(-1)
        out = np.empty(x.size, np.int8)
        self.lib.quantize_fp32_nhwc_to_int8(x, x.size, C.c_float(scale), out)
        return out

    def add_requant(self, a, a_scale, b, b_scale, out_scale):
        a = np.ascontiguousarray(a, np.int8).reshape(-1)
        b = np.ascontiguousarray(b, np.int8).reshape(-1)
        out = np.empty_like(a)
        self.lib.add_requant_int8(a, a_scale, b, b_scale, out, out_scale, a.size)
        return out

    def conv_i32(self, x, w_oihw, stride, pad):
        x = np.ascontiguousarray(x, np.int8)
        w = np.ascontiguousarray(w_oihw, np.int8)
        B, H, W, Cin = x.shape
        Cout, _, KH, KW = w.shape
        Ho = (H + 2 * pad - KH) // stride + 1
        Wo = (W + 2 * pad - KW) // stride + 1
        Kp = (Cin * KH * KW + 3) & ~3
        wrow = np.empty(Kp * Cout + 64, np.int8)
        wpk = np.empty(Kp * Cout + 64, np.int8)
        cs = np.empty(Cout + 16, np.int32)
        self.lib.pack_conv_weight_nhwc(w.reshape(-1), Cout, Cin, KH, KW, Kp, wrow, wpk, cs)
        # the reference GEMM walks M in blocks of 4 rows (gemm_int8_v2.c:97),
        # so it reads and writes up to 3 rows past M: pad like its callers do
        M = B * Ho * Wo
        out = np.empty((M + 4) * Cout + 64, np.int32)
        scratch = np.full((M + 4) * Kp + 64, 128, np.uint8)
        self.lib.fastface_conv2d_i8_nhwc_batched(x.reshape(-1), B, Cin, H, W, Cout, KH, KW,
                                                 stride, pad, wpk, cs, Ho, Wo, out, scratch)
        return out[:B * Ho * Wo * Cout].reshape(B, Ho, Wo, Cout)

    def winograd_weights(self, w_oihw):
        w = np.ascontiguousarray(w_oihw, np.int8)
        Cout, Cin = w.shape[:2]
        u = np.empty((16, Cout, Cin), np.int16)
        self.lib.winograd_int8_transform_weights_ref(w.reshape(-1), Cout, Cin, u.reshape(-1))
        return u

    def conv_winograd(self, x, u):
        """One image at a time (the reference function is per image)."""
        x = np.ascontiguousarray(x, np.int8)
        B, H, W, Cin = x.shape
        Cout = u.shape[1]
        out = np.empty((B, H, W, Cout), np.int32)
        uu = np.ascontiguousarray(u, np.int16).reshape(-1)
        for b in range(B):
            o = np.empty(H * W * Cout, np.int32)
            self.lib.fastface_conv2d_i8_winograd_f23_ref(np.ascontiguousarray(x[b]).reshape(-1),
                                                         Cin, H, W, Cout, uu, o)
            out[b] = o.reshape(H, W, Cout)
        return out

    def fc(self, a, W, ws, bias, a_scale=1.0):
        a = np.ascontiguousarray(a, np.int8).reshape(-1)
        W = np.ascontiguousarray(W, np.int8)
        N, K = W.shape
        au = (a.view(np.uint8) ^ 0x80).astype(np.uint8)
        rs = W.astype(np.int32).sum(axis=1).astype(np.int32)
        out = np.empty(N, np.float32)
        self.lib.fastface_gemm_i8_matvec_vnni(au, W, rs, np.ascontiguousarray(ws, np.float32),
                                              np.ascontiguousarray(bias, np.float32), a_scale,
                                              out, N, K)
        return out

    def embed(self, ffw_path, faces, cwd):
        """fastface_create/embed/destroy (libfastface.c); cwd must hold
        models/op_scales.bin (the reference opens it CWD-relative)."""
        old = os.getcwd()
        os.chdir(cwd)
        try:
            ff = self.lib.fastface_create(ffw_path.encode())
            if not ff:
                raise RuntimeError("reference fastface_create failed")
            faces = np.ascontiguousarray(faces, np.float32).reshape(-1, 112 * 112 * 3)
            out = np.empty((faces.shape[0], 512), np.float32)
            for i in range(faces.shape[0]):
                o = np.empty(512, np.float32)
                if self.lib.fastface_embed(ff, np.ascontiguousarray(faces[i]), o) != 0:
                    raise RuntimeError("reference fastface_embed failed")
                out[i] = o
            self.lib.fastface_destroy(ff)
            return out
        finally:
            os.chdir(old)
