"""Loading and comparing the golden fixtures written by tests/golden/make_golden.py."""

import hashlib
from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name):
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def state_arrays(state, prefix):
    """A cache state dict in the fixture's array form."""
    ids = sorted(state["tables"])
    return {
        f"{prefix}_refs": np.array(state["refs"], np.uint32),
        f"{prefix}_generations": np.array(state["generations"], np.uint32),
        f"{prefix}_free": np.array(state["free"], np.uint32),
        f"{prefix}_seq_ids": np.array(ids, np.uint64),
        f"{prefix}_lengths": np.array([state["tables"][s][0] for s in ids], np.uint32),
        f"{prefix}_sizes": np.array([len(state["tables"][s][1]) for s in ids], np.uint32),
        f"{prefix}_blocks": np.array([b for s in ids for b in state["tables"][s][1]], np.uint32).reshape(-1, 2),
    }


def check_stress(cache, unaligned, checksum):
    """Run the shared-prefix stress on `cache` and compare every recorded phase
    and every live block's checksum with the reference's fixture."""
    from tvara_amd import workloads

    w = workloads.kv_c3(unaligned=unaligned)
    g = load(w.name.replace("(", "").replace(")", "").replace("+", "_"))
    phases = {"fork", "step0", f"step{w.steps - 1}", "rollback"}
    seen = []

    def record(name, seqs):
        if name in phases:
            got = state_arrays(cache.state(), name)
            for k, v in got.items():
                assert np.array_equal(v, g[k]), (name, k)
            seen.append(name)

    seqs = workloads.run_kv_stress(cache, w, record)
    assert sorted(seen) == sorted(phases)
    live = sorted({h for s in seqs for h in cache.blocks(s)})
    assert np.array_equal(np.array(live, np.uint32).reshape(-1, 2), g["live"])
    assert [int(x) for x in g["checksums"]] == checksum(cache, live)


def q8_digest(blocks_canonical, tokens, kv_width, tokens_per_block=16):
    """sha256 over the K groups then the V groups of `tokens` tokens, in token
    order, from canonical single-layer Q8_0 block images."""
    gpr = kv_width // 32
    k, v = [], []
    for b, img in enumerate(blocks_canonical):
        img = np.asarray(img, np.uint8).reshape(2, tokens_per_block, gpr * 34)
        n = min(tokens_per_block, tokens - b * tokens_per_block)
        k.append(img[0, :n].reshape(-1))
        v.append(img[1, :n].reshape(-1))
    return hashlib.sha256(np.concatenate(k).tobytes() + np.concatenate(v).tobytes()).digest()
