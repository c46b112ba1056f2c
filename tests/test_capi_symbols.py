"""libtvara_capi.so loads and exports every entry point declared in
include/tvara_capi.h (no device calls: CPU only)."""

import ctypes
import re
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def declared():
    text = (ROOT / "include" / "tvara_capi.h").read_text()
    return re.findall(r"TVARA_API\s+[\w\s\*]+?\b(tvara_\w+)\s*\(", text)


def test_header_declares_entry_points():
    names = declared()
    assert len(names) == len(set(names)) >= 40


def test_library_exports_every_declared_symbol():
    from tvara_amd import _capi, build

    if not build.LIBRARY.exists():
        build.build()
    lib = ctypes.CDLL(str(_capi.find_library()))
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, missing
    # the Python binding declares exactly the header's entry points
    assert sorted(_capi.SIGNATURES) == sorted(declared())


def test_no_cpu_fallback_in_product_package():
    # the product package never imports the oracle
    for path in (ROOT / "tvara_amd").rglob("*.py"):
        text = path.read_text()
        assert "import oracle" not in text and "from oracle" not in text, path
