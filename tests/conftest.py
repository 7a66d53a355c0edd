"""Shared fixtures.  `gpu` tests need a gfx950 device and the built libinferox.so;
everything else runs on the CPU (oracle, host logic, library exports)."""
from __future__ import annotations

import os
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU and the built HIP library")
    config.addinivalue_line("markers", "slow: multi-GB synthetic models")


def _ensure_host_libs():
    """The oracle and the synth generator are plain gcc builds; make them if absent."""
    if not os.path.exists(os.path.join(ROOT, "oracle", "liboracle.so")):
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)
    from inferox_amd import build
    if not os.path.exists(os.path.join(ROOT, "inferox_amd", "lib", "libifx_synth.so")):
        build.build_synth()


_ensure_host_libs()


@pytest.fixture(scope="session")
def tmpdir_session(tmp_path_factory):
    return tmp_path_factory.mktemp("ifx")


@pytest.fixture(scope="session")
def tiny_path(tmpdir_session):
    from inferox_amd import synth
    path = str(tmpdir_session / "tiny.gguf")
    synth.write_llama(path, synth.TINY, seed=1234)
    return path


@pytest.fixture(scope="session")
def tiny_prompt():
    from inferox_amd import synth
    return synth.token_ids(16, synth.TINY.vocab, seed=4321)


def rel_l2(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))
