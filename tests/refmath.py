"""Float64 brute-force attention used to pin the oracle independently of it.

Exact two-pass softmax with grouped-query heads, the semantics of the
reference's numpy model (python/tvara/reference/math.py:39-58) and of
grouped_attention (core/include/tvara/model.hpp:86-107), evaluated entirely
in float64.
"""

import numpy as np


def attention(q, keys, values, heads, kv_heads, dim):
    """q [heads*dim]; keys/values [positions, kv_heads*dim] -> [heads*dim]."""
    q = np.asarray(q, np.float64).reshape(heads, dim)
    k = np.asarray(keys, np.float64).reshape(-1, kv_heads, dim)
    v = np.asarray(values, np.float64).reshape(-1, kv_heads, dim)
    group = heads // kv_heads
    out = np.empty((heads, dim))
    for h in range(heads):
        kh = h // group
        s = k[:, kh, :] @ q[h] / np.sqrt(dim)
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ v[:, kh, :]
    return out.reshape(-1)


def close(a, b, tol):
    """|a-b| <= tol*(1+|b|) elementwise (tests/core/prefill_support.hpp:7-9)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return bool(np.all(np.abs(a - b) <= tol * (1 + np.abs(b))))


def max_rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b) / (1 + np.abs(b)))) if a.size else 0.0
