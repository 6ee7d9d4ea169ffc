"""In-process Python binding of the fastface.h C API.

Mirrors the reference SDK's `FastFace` class (fastface.py:41-162: embed,
embed_batch, cos_sim, close, context manager) but calls the C library
directly instead of piping frames to a `--server` subprocess.  Inputs are
HWC [112, 112, 3] fp32 faces in [-1, 1]; outputs raw (not L2-normalized)
512-d fp32 embeddings.
"""
from __future__ import annotations

import os
from typing import Sequence

import numpy as np

from . import FASTFACE_INPUT_N, FASTFACE_OUTPUT_N, load


def scale_paths(cwd: str, environ=None) -> tuple:
    """The OPSC and OPSC2 files fastface_create would open with `cwd` as the
    working directory (libfastface.c:236-240): models/op_scales.bin, and
    $OPSC2_PATH or models/op_scales_v2.bin, relative paths taken relative to
    `cwd`."""
    environ = os.environ if environ is None else environ
    opsc = os.path.join(cwd, "models", "op_scales.bin")
    env2 = environ.get("OPSC2_PATH")
    if env2:
        opsc2 = env2 if os.path.isabs(env2) else os.path.join(cwd, env2)
    else:
        opsc2 = os.path.join(cwd, "models", "op_scales_v2.bin")
    return opsc, opsc2


class FastFace:
    def __init__(self, weights: str = "models/w600k_r50_ffw4.bin", batch: int = 1,
                 cwd: str | None = None, scale_files: tuple | None = None):
        """`cwd`: directory holding models/op_scales.bin and
        models/op_scales_v2.bin (fastface_create opens them relative to the
        working directory, like the reference; with `cwd` they are named
        explicitly instead, so the process's working directory is left alone
        and contexts can be created on several threads).  `scale_files`:
        (OPSC path, OPSC2 path) named directly instead; an OPSC2 path that
        does not exist runs the model on the OPSC per-tensor scales, as the
        reference does without that file."""
        self.lib = load()
        self.batch = int(batch)
        w = os.path.abspath(weights).encode()
        if cwd or scale_files:
            opsc, opsc2 = scale_files if scale_files else scale_paths(cwd)
            self.ff = self.lib.fastface_create_with_scales(w, opsc.encode(), opsc2.encode())
        else:
            self.ff = self.lib.fastface_create(w)
        if not self.ff:
            raise RuntimeError("fastface_create failed for %s" % weights)
        if self.batch > 1:
            self.lib.fastface_reserve(self.ff, self.batch)

    def embed(self, arr: np.ndarray) -> np.ndarray:
        a = np.ascontiguousarray(arr, dtype=np.float32)
        if a.size != FASTFACE_INPUT_N:
            raise ValueError("arr must have %d elements, got %d" % (FASTFACE_INPUT_N, a.size))
        out = np.empty(FASTFACE_OUTPUT_N, np.float32)
        rc = self.lib.fastface_embed(self.ff, a.ctypes.data, out.ctypes.data)
        if rc != 0:
            raise RuntimeError("fastface_embed failed (%d)" % rc)
        return out

    def embed_batch(self, arrs: Sequence[np.ndarray] | np.ndarray) -> np.ndarray:
        a = np.ascontiguousarray(np.asarray(arrs, dtype=np.float32))
        b = a.size // FASTFACE_INPUT_N
        if a.size != b * FASTFACE_INPUT_N:
            raise ValueError("input is not a whole number of faces")
        out = np.empty((b, FASTFACE_OUTPUT_N), np.float32)
        rc = self.lib.fastface_embed_batch(self.ff, a.ctypes.data, b, out.ctypes.data)
        if rc != 0:
            raise RuntimeError("fastface_embed_batch failed (%d)" % rc)
        return out

    def embed_batch_rgb8(self, imgs: Sequence[np.ndarray] | np.ndarray) -> np.ndarray:
        """uint8 RGB faces, HWC [112, 112, 3] each: the embeddings of the
        fp32 faces (x - 127.5) / 127.5 that the reference SDK builds from them."""
        a = np.ascontiguousarray(np.asarray(imgs, dtype=np.uint8))
        b = a.size // FASTFACE_INPUT_N
        if a.size != b * FASTFACE_INPUT_N:
            raise ValueError("input is not a whole number of faces")
        out = np.empty((b, FASTFACE_OUTPUT_N), np.float32)
        rc = self.lib.fastface_embed_batch_rgb8(self.ff, a.ctypes.data, b, out.ctypes.data)
        if rc != 0:
            raise RuntimeError("fastface_embed_batch_rgb8 failed (%d)" % rc)
        return out

    @staticmethod
    def cos_sim(a: np.ndarray, b: np.ndarray) -> float:
        return float(np.dot(a, b) / (np.linalg.norm(a) * np.linalg.norm(b)))

    def close(self):
        if getattr(self, "ff", None):
            self.lib.fastface_destroy(self.ff)
            self.ff = None

    def __enter__(self):
        return self

    def __exit__(self, exc_type, exc, tb):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
