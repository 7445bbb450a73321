"""Test setup: the `gpu` marker, import paths and shared fixtures.

CPU tests (-m "not gpu") cover the oracle against hand-computed known answers, the host-side
logic and that libtpthip loads and exports its C ABI.  GPU tests (-m gpu) are the parity tests:
the HIP path through the C ABI against the oracle on the same seeded inputs.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "tpt-spark_amd"), os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and libtpthip's kernels")


@pytest.fixture(scope="session")
def ctx():
    import tpthip
    c = tpthip.Context(0)
    yield c
    c.close()


@pytest.fixture(scope="session")
def tiny_gguf(tmp_path_factory):
    from tpthip import synth
    path = str(tmp_path_factory.mktemp("models") / "tiny.gguf")
    synth.write_llama(path, synth.TINY, seed=7)
    return path
