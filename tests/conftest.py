"""Test configuration: the `gpu` marker and import paths.

Tests marked `gpu` need a HIP device and the in-tree library
(full-inference-engine_amd/fie_amd/_native/libfie_sampler.so, built by
`__graft_entry__.build()`); everything else runs on the CPU.
"""

import os
import sys

import pytest

_REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("full-inference-engine_amd", "oracle"):
    p = os.path.join(_REPO, sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X) and the built library")


@pytest.fixture(scope="session")
def oracle_lib():
    import oracle

    oracle.build()
    return oracle
