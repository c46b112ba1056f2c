import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: runs libtvara_capi.so kernels on an MI355X")


@pytest.fixture(scope="session")
def oracle():
    """The C restatement (oracle/liboracle.so), built on first use if missing."""
    lib = ROOT / "oracle" / "liboracle.so"
    if not lib.exists():
        subprocess.run(["make", "-C", str(ROOT / "oracle")], check=True, capture_output=True)
    from oracle import pyoracle

    return pyoracle


@pytest.fixture(scope="session")
def ref(oracle):
    """The reference's own code (oracle/_ref), when it was built where the reference is."""
    if not oracle.ref_available():
        pytest.skip("oracle/_ref not built (the reference tree is absent here)")
    return oracle


@pytest.fixture(scope="session")
def device():
    """libtvara_capi.so; a GPU test fails loudly when it is missing."""
    from tvara_amd import _capi

    _capi.lib()
    import tvara_amd.kv as kv

    return kv
