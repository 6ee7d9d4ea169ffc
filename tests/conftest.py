import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def oracle():
    from oracle.oracle import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def ref():
    """The reference's int8 functions compiled from its sources (oracle/_ref)."""
    from oracle.oracle import REF_SO, Ref, host_has_avx_vnni
    if not os.path.exists(REF_SO):
        pytest.skip("oracle/_ref not built (needs /root/reference at build time)")
    if not host_has_avx_vnni():
        pytest.skip("host CPU lacks AVX-VNNI: the reference build would SIGILL")
    return Ref()


@pytest.fixture(scope="session")
def synth_ffw4():
    from fastface_amd import synth
    return synth.synthetic_ffw4_path(3)


@pytest.fixture(scope="session")
def oracle_model(oracle, synth_ffw4):
    from fastface_amd import synth
    m = oracle.load_model(synth_ffw4, synth.OPSC_PATH, synth.OPSC2_PATH)
    yield m
    oracle.free_model(m)


@pytest.fixture(scope="session")
def gpu_lib():
    import fastface_amd
    lib = fastface_amd.load()
    if lib.ffk_device_count() <= 0:
        pytest.fail("no HIP device visible for a gpu-marked test")
    return lib


def rng(seed):
    return np.random.default_rng(seed)
