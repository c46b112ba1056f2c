"""The library's HIP-free host code on the CPU (tests/native).

* libtvara_host.so links the library's own pool and tables (kv_ledger.cpp),
  prefix tree (radix.cpp), ledger and prefix-cache exports (ledger_capi.cpp)
  and error convention (abi.cpp) with a host-memory block store
  (tests/native/host_store.cpp).  Through the same Python classes as the GPU
  library it runs the restated known answers of tests/core/test_kv.cpp and
  test_radix.cpp, and random operation sequences compared after every step --
  results, error class and message, every node, retained counts and the whole
  pool state -- with the reference's own PagedCache and RadixCache compiled
  from their headers (oracle/_ref).
* ledger_faults is the same host code plus the GGUF reader under
  -fsanitize=address,undefined: audited random churn, an allocation-failure
  sweep over every mutating operation (each failed call must leave the pool,
  tables and tree unchanged), and the malformed-GGUF corpus.
"""

import shutil
import subprocess
import sys
from pathlib import Path

import pytest

import kv_cases
import radix_cases

ROOT = Path(__file__).resolve().parents[1]
NATIVE = ROOT / "tests" / "native"


@pytest.fixture(scope="session")
def host_build():
    if not shutil.which("g++") or not shutil.which("make"):
        pytest.skip("g++ / make not available")
    res = subprocess.run(["make", "-C", str(NATIVE)], capture_output=True, text=True)
    assert res.returncode == 0, res.stdout[-3000:] + res.stderr[-3000:]
    return NATIVE / "_build"


@pytest.fixture(scope="session")
def host_lib(host_build):
    from tvara_amd import _capi

    return _capi.bind_subset(host_build / "libtvara_host.so")


def _make(lib):
    from tvara_amd.kv import PagedCache

    return lambda *g: PagedCache(*g, lib=lib)


def _errors():
    from tvara_amd._capi import CacheExhausted, InvalidArgument

    return (InvalidArgument, CacheExhausted)


@pytest.mark.parametrize("case", kv_cases.CASES, ids=lambda f: f.__name__)
def test_ledger_known_answers(host_lib, case):
    case(_make(host_lib), _errors())


@pytest.mark.parametrize("geometry,seed", [((2, 2, 4, 4, 12), 1), ((1, 1, 2, 3, 9), 2), ((3, 1, 4, 5, 20), 3),
                                           ((1, 2, 8, 16, 6), 4)])
def test_ledger_matches_reference(ref, host_lib, geometry, seed):
    layers, kv_heads, dim, tpb, _ = geometry
    n = kv_cases.random_ops(_make(host_lib)(*geometry), ref.RefCache(*geometry), 300, seed, layers * kv_heads * dim,
                            tpb)
    assert n >= 1


def test_radix_known_answers(host_lib):
    from tvara_amd.radix import RadixCache

    radix_cases.known_answers(_make(host_lib)(1, 1, 1, 4, 64), RadixCache)


@pytest.mark.parametrize("geometry,seed,alphabet", [((1, 1, 2, 4, 24), 1, 3), ((2, 1, 2, 3, 40), 2, 4),
                                                    ((1, 2, 2, 2, 16), 3, 2), ((1, 1, 1, 5, 64), 4, 6),
                                                    ((1, 1, 2, 4, 48), 5, 3), ((1, 1, 1, 2, 96), 6, 2)])
def test_radix_matches_reference(ref, host_lib, geometry, seed, alphabet):
    # the prefix tree against the reference's RadixCache, node by node and
    # pool state by pool state (ids, split pins, eviction order, release order)
    from tvara_amd.radix import RadixCache

    layers, kv_heads, dim, _, _ = geometry
    hc, rc = _make(host_lib)(*geometry), ref.RefCache(*geometry)
    pairs = [(rc, ref.RefRadix(rc, "model/tokenizer/tenant")), (hc, RadixCache(hc, "model/tokenizer/tenant"))]
    assert radix_cases.random_ops(pairs, 600, seed, layers * kv_heads * dim, alphabet) > 10


def test_radix_long_churn_matches_reference(ref, host_lib):
    # enough evictions and inserts that the tree compacts its arena and token
    # store several times
    from tvara_amd.radix import RadixCache

    geometry = (1, 1, 1, 3, 200)
    hc, rc = _make(host_lib)(*geometry), ref.RefCache(*geometry)
    pairs = [(rc, ref.RefRadix(rc, "churn")), (hc, RadixCache(hc, "churn"))]
    assert radix_cases.random_ops(pairs, 2500, 11, 1, 8) > 100


def test_sanitized_churn_and_fault_injection(host_build):
    res = subprocess.run([str(host_build / "ledger_faults"), "all"], capture_output=True, text=True, timeout=600)
    assert res.returncode == 0, res.stdout[-3000:] + res.stderr[-5000:]
    assert "passed" in res.stdout
    assert "attach (snapshot publication):" in res.stdout and "reuse (import_sequence):" in res.stdout


def test_sanitized_gguf_reader(host_build, tmp_path, request):
    # every malformed file is rejected with the reference's message (or, for
    # the RoPE layout and an epsilon that rounds to zero in f32, accepted by
    # the parser and rejected later by the model loader's configuration
    # check), every fixture parses, and nothing trips the sanitizers
    sys.path.insert(0, str(ROOT / "tests"))
    import test_model_cpu as tm
    from tvara_amd import gguf_writer as gf

    cases = tm.malformed(tmp_path)
    good = [gf.LlamaSpec(matrix_type=t).write(tmp_path / f"good{t}.gguf") for t in (gf.T_F32, gf.T_Q8_0, gf.T_Q4_0)]
    files = [str(p) for _, p in cases] + [str(p) for p in good]
    res = subprocess.run([str(host_build / "ledger_faults"), "gguf", *files], capture_output=True, text=True,
                         timeout=300)
    assert res.returncode == 0, res.stderr[-5000:]
    lines = res.stdout.splitlines()
    assert len(lines) == len(files)
    assert all(line == "ok" for line in lines[len(cases):])
    ref_capi = ROOT / "oracle" / "_ref" / "libtvara_ref_capi.so"
    for (label, path), line in zip(cases, lines):
        if line == "ok":
            assert label in ("rope layout", "rope layout type", "epsilon underflows float"), label
            continue
        assert line.startswith("error: "), (label, line)
        if ref_capi.exists():
            assert line[len("error: "):] == tm.opened_error(path, str(ref_capi)), label


def test_truncate_batch_matches_single_truncations(host_lib):
    """tvara_kv_truncate_batch against a loop of tvara_kv_truncate on a twin
    cache: the same pool state after a valid batch, and after a batch whose
    third entry fails (a length past the sequence's end) the same state as
    the first two single calls, with the failure's class and the applied
    count reported."""
    import numpy as np

    from tvara_amd._capi import InvalidArgument

    geometry = (2, 1, 4, 4, 40)
    caches = [_make(host_lib)(*geometry) for _ in range(2)]
    ids = []
    for c in caches:
        base = c.create_sequence()
        for t in range(10):
            c.append(base, np.full(8, t, np.float32), np.full(8, -t, np.float32))
        seqs = [base] + [c.fork(base) for _ in range(3)]
        for j, s in enumerate(seqs[1:]):
            for t in range(j + 2):
                c.append(s, np.full(8, 100 + t, np.float32), np.full(8, 200 + t, np.float32))
        ids.append(seqs)
    assert ids[0] == ids[1]
    seqs = ids[0]
    lengths = [7, 12, 3, 9]
    assert caches[0].truncate_batch(seqs, lengths) == 4
    for s, n in zip(seqs, lengths):
        caches[1].truncate(s, n)
    assert caches[0].state() == caches[1].state()
    bad = [5, 4, 99, 1]
    with pytest.raises(InvalidArgument) as err:
        caches[0].truncate_batch(seqs, bad)
    assert caches[0].last_applied == 2
    for s, n in zip(seqs[:2], bad[:2]):
        caches[1].truncate(s, n)
    with pytest.raises(InvalidArgument) as err1:
        caches[1].truncate(seqs[2], bad[2])
    assert str(err.value) == str(err1.value)
    assert caches[0].state() == caches[1].state()
    assert caches[0].truncate_batch([], []) == 0
