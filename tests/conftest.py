import os
import sys
from pathlib import Path

import pytest

sys.path.insert(0, str(Path(__file__).resolve().parent))
sys.path.insert(0, str(Path(__file__).resolve().parents[1]))

import helpers  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and libsgq.so")


@pytest.fixture(scope="session")
def oracle():
    from oracle.oracle import Oracle

    return Oracle()


@pytest.fixture(scope="session")
def ref():
    from oracle.oracle import Reference, reference_available

    if not reference_available():
        pytest.skip("oracle/_ref not built (the reference checkout is only present in the dev container)")
    return Reference()


@pytest.fixture(scope="session")
def golden():
    return helpers.load_golden()


@pytest.fixture(scope="session")
def synth():
    return helpers.load_synth()


@pytest.fixture(scope="session")
def sgq():
    return helpers.load_sgq()


@pytest.fixture(scope="session")
def dev(sgq):
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    sgq.load_library()  # fails loudly when libsgq.so is missing
    d = torch.device("cuda:0")
    print(f"\n[gpu] {torch.cuda.get_device_name(d)} pid={os.getpid()}", flush=True)
    return d
