"""Test configuration: the `gpu` marker, and loaders for the oracle and the product library.

CPU tests (-m "not gpu") cover the oracle against the reference's golden vectors and that the C-ABI
library loads and exports every declared symbol. GPU tests (-m gpu) are the parity tests: the HIP
path through the C ABI against the oracle on the same seeded inputs.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle
    if not os.path.exists(oracle._LIB_PATH):
        oracle.build()
    return oracle


@pytest.fixture(scope="session")
def rbt_lib():
    from rabbit_amd import abi
    if not os.path.exists(abi.LIB_PATH):
        from rabbit_amd import build
        build.build()
    return abi.load()


@pytest.fixture(scope="session")
def ctx(rbt_lib):
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.zeros(1, device="cuda")  # initialise the device through torch first (one HIP runtime)
    import rabbit_amd
    c = rabbit_amd.Context(0)
    yield c
    c.close()
