import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libcwen_gpu.so)")
    config.addinivalue_line("markers", "slow: full-size workload check")


@pytest.fixture(scope="session")
def oracle():
    from oracle.binding import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def ref():
    from oracle.binding import Reference, ref_lib_path
    if not ref_lib_path().exists():
        pytest.skip("reference checker build absent (needs the reference tree)")
    return Reference()


@pytest.fixture(scope="session")
def ref_avx2():
    from oracle.binding import Reference, ref_lib_path
    if not ref_lib_path("avx2").exists():
        pytest.skip("reference checker build absent (needs the reference tree)")
    return Reference("avx2")
