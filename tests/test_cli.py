"""The wire-compatible CLI replacements (fastface_amd/bin/fastface_int8 and
fastface_int8_batched): argument handling, exit codes and the --server frame
protocol of the reference's arcface_forward_int8{,_batched}.c, which its SDKs
(fastface.py, go/fastface) drive."""
import os
import subprocess

import numpy as np
import pytest

import fastface_amd as fa
from fastface_amd import synth

BIN = os.path.join(fa.HERE, "bin")
CLI = os.path.join(BIN, "fastface_int8")
CLI_B = os.path.join(BIN, "fastface_int8_batched")


def _run(args, stdin=b"", timeout=120):
    return subprocess.run(args, input=stdin, capture_output=True, cwd=synth.REPO_ROOT,
                          timeout=timeout)


def test_cli_binaries_built():
    assert os.access(CLI, os.X_OK) and os.access(CLI_B, os.X_OK)


@pytest.mark.parametrize("exe", [CLI, CLI_B])
def test_cli_load_failure_exits_1(exe):
    r = _run([exe, "/nonexistent/weights.ffw4", "--server", "--threads", "4"])
    assert r.returncode == 1
    assert r.stdout == b""                       # server mode: nothing but frames on stdout


@pytest.mark.gpu
def test_cli_server_frames_match_oracle(synth_ffw4, oracle, oracle_model):
    x = synth.faces_uniform(3, 41)
    exp, _ = oracle.forward(oracle_model, x)
    r = _run([CLI, synth_ffw4, "--server"], stdin=x.astype(np.float32).tobytes())
    assert r.returncode == 0, r.stderr.decode()[-500:]
    got = np.frombuffer(r.stdout, np.float32).reshape(-1, 512)
    assert got.shape == (3, 512)
    assert np.array_equal(got, exp)


@pytest.mark.gpu
def test_cli_batched_server_frames(synth_ffw4, oracle, oracle_model):
    x = synth.faces_uniform(8, 42)
    exp, _ = oracle.forward(oracle_model, x)
    r = _run([CLI_B, synth_ffw4, "--batch", "4", "--server"], stdin=x.tobytes())
    assert r.returncode == 0, r.stderr.decode()[-500:]
    assert np.array_equal(np.frombuffer(r.stdout, np.float32).reshape(8, 512), exp)


@pytest.mark.gpu
def test_cli_partial_frame_exits_4(synth_ffw4):
    x = synth.faces_uniform(1, 43)
    r = _run([CLI, synth_ffw4, "--server"], stdin=x.tobytes() + x.tobytes()[:400])
    assert r.returncode == 4
    assert len(r.stdout) == 512 * 4               # the whole frame was answered first


@pytest.mark.gpu
def test_cli_validate_mode(synth_ffw4, oracle, oracle_model, tmp_path):
    x = synth.faces_uniform(1, 44)
    exp, _ = oracle.forward(oracle_model, x)
    fin, fout = tmp_path / "in.bin", tmp_path / "out.bin"
    x.astype(np.float32).tofile(fin)
    r = _run([CLI, synth_ffw4, "--in", str(fin), "--out", str(fout)])
    assert r.returncode == 0, r.stderr.decode()[-500:]
    assert np.array_equal(np.fromfile(fout, np.float32), exp[0])
    r = _run([CLI, synth_ffw4, "--in", str(tmp_path / "missing.bin"), "--out", str(fout)])
    assert r.returncode == 2
