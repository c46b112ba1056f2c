"""ctypes access to the test oracle (liboracle.so, the C restatement) and, when
built, to the reference's own code compiled into oracle/_ref/libtvara_ref.so.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, never by the product package.

Both back ends expose the same Python surface (``Cache``), mirroring the
reference's PagedCache/BlockPool (core/include/tvara/kv.hpp) and
fused_paged_attention / fused_prompt_attention (core/include/tvara/attention.hpp),
so a test can drive the oracle, the reference and the HIP library through one
sequence of calls.
"""

from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_PATH = HERE / "liboracle.so"
REF_PATH = HERE / "_ref" / "libtvara_ref.so"

_fp = C.POINTER(C.c_float)
_sz = C.c_size_t
_u64 = C.c_uint64


class OracleError(RuntimeError):
    pass


class InvalidArgument(OracleError, ValueError):
    pass


class CacheExhausted(OracleError):
    pass


class LogicError(OracleError):
    pass


_ERRORS = {-2: InvalidArgument, -3: CacheExhausted, -4: LogicError}


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _ptr(a):
    return a.ctypes.data_as(_fp) if a is not None else None


class _Handle(C.Structure):
    _fields_ = [("id", _sz), ("generation", _u64)]


class _Geometry(C.Structure):
    _fields_ = [(n, _sz) for n in ("layers", "kv_heads", "head_dim", "tokens_per_block", "max_blocks")]


def _load_oracle():
    if not ORACLE_PATH.exists():
        raise FileNotFoundError(f"{ORACLE_PATH} is not built (run `make -C oracle`)")
    lib = C.CDLL(str(ORACLE_PATH))
    lib.tvo_last_error.restype = C.c_char_p
    lib.tvo_cache_create.restype = C.c_void_p
    lib.tvo_cache_create.argtypes = [C.POINTER(_Geometry)]
    lib.tvo_cache_destroy.argtypes = [C.c_void_p]
    lib.tvo_cache_clone.restype = C.c_void_p
    lib.tvo_cache_clone.argtypes = [C.c_void_p]
    lib.tvo_geometry_validate.argtypes = [C.POINTER(_Geometry)]
    lib.tvo_elements_per_block.restype = _sz
    lib.tvo_elements_per_block.argtypes = [C.POINTER(_Geometry)]
    lib.tvo_kv_offset.restype = _sz
    lib.tvo_kv_offset.argtypes = [C.POINTER(_Geometry), _sz, _sz, _sz]
    lib.tvo_pool_allocate.argtypes = [C.c_void_p, C.POINTER(_Handle)]
    for name in ("tvo_pool_retain", "tvo_pool_release"):
        getattr(lib, name).argtypes = [C.c_void_p, _Handle]
    lib.tvo_pool_references.argtypes = [C.c_void_p, _Handle, C.POINTER(_sz)]
    lib.tvo_pool_references_by_id.restype = _sz
    lib.tvo_pool_references_by_id.argtypes = [C.c_void_p, _sz]
    lib.tvo_pool_available.restype = _sz
    lib.tvo_pool_available.argtypes = [C.c_void_p]
    lib.tvo_pool_audit.argtypes = [C.c_void_p]
    lib.tvo_pool_data.argtypes = [C.c_void_p, _Handle, C.POINTER(_fp)]
    lib.tvo_create_sequence.restype = _u64
    lib.tvo_create_sequence.argtypes = [C.c_void_p]
    lib.tvo_sequence_length.argtypes = [C.c_void_p, _u64, C.POINTER(_sz)]
    lib.tvo_sequence_blocks.argtypes = [C.c_void_p, _u64, C.POINTER(_Handle), _sz, C.POINTER(_sz)]
    lib.tvo_physical_block.argtypes = [C.c_void_p, _u64, _sz, C.POINTER(_Handle)]
    lib.tvo_append.argtypes = [C.c_void_p, _u64, _fp, _fp]
    lib.tvo_read.argtypes = [C.c_void_p, _u64, _sz, _sz, C.c_int, _fp]
    lib.tvo_read_all.argtypes = [C.c_void_p, _u64, _sz, C.c_int, _fp, _sz]
    lib.tvo_drop.argtypes = [C.c_void_p, _u64]
    lib.tvo_fork.restype = _u64
    lib.tvo_fork.argtypes = [C.c_void_p, _u64]
    lib.tvo_truncate.argtypes = [C.c_void_p, _u64, _sz]
    lib.tvo_audit.argtypes = [C.c_void_p, C.POINTER(_sz), _sz]
    lib.tvo_import_sequence.restype = _u64
    lib.tvo_import_sequence.argtypes = [C.c_void_p, C.POINTER(_Handle), _sz, _sz, _sz]
    lib.tvo_pool_state.argtypes = [C.c_void_p, C.POINTER(_sz), C.POINTER(_u64), C.POINTER(_sz), C.POINTER(_sz)]
    lib.tvo_sequence_count.restype = _sz
    lib.tvo_sequence_count.argtypes = [C.c_void_p]
    lib.tvo_sequence_ids.argtypes = [C.c_void_p, C.POINTER(_u64), _sz]
    lib.tvo_checksum_words.restype = _u64
    lib.tvo_checksum_words.argtypes = [C.POINTER(C.c_uint32), _sz]
    lib.tvo_attention_dot.restype = C.c_double
    lib.tvo_attention_dot.argtypes = [_fp, _fp, _sz]
    lib.tvo_fused_paged_attention.argtypes = [C.c_void_p, _u64, _sz, _sz, _sz, _fp, _fp, _fp, _sz, _fp]
    lib.tvo_fused_prompt_attention.argtypes = [C.c_void_p, _u64, _sz, _sz, _sz, _sz, _sz, _fp, _fp]
    lib.tvo_set_dot_mode.argtypes = [C.c_int]
    lib.tvo_half_to_float.restype = C.c_float
    lib.tvo_half_to_float.argtypes = [C.c_uint16]
    lib.tvo_double_to_half.restype = C.c_uint16
    lib.tvo_double_to_half.argtypes = [C.c_double]
    lib.tvo_dequantize_q8_0.argtypes = [C.POINTER(C.c_uint8), _sz, _fp, _sz]
    lib.tvo_quantize_q8_0_block.argtypes = [_fp, C.POINTER(C.c_uint8)]
    lib.tvo_quantize_q8_0_block.restype = None
    lib.tvo_quantize_q8_0.argtypes = [_fp, _sz, C.POINTER(C.c_uint8)]
    lib.tvo_quantize_q8_0.restype = None
    return lib


_oracle = None


def oracle_lib():
    global _oracle
    if _oracle is None:
        _oracle = _load_oracle()
    return _oracle


def checksum_words(words: np.ndarray) -> int:
    w = np.ascontiguousarray(words).view(np.uint32)
    return int(oracle_lib().tvo_checksum_words(w.ctypes.data_as(C.POINTER(C.c_uint32)), w.size))


def half_to_float(h: int) -> float:
    return float(oracle_lib().tvo_half_to_float(h))


def double_to_half(x: float) -> int:
    return int(oracle_lib().tvo_double_to_half(x))


def dequantize_q8_0(raw: np.ndarray) -> np.ndarray:
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    out = np.empty(raw.size // 34 * 32, np.float32)
    rc = oracle_lib().tvo_dequantize_q8_0(raw.ctypes.data_as(C.POINTER(C.c_uint8)), raw.size, _ptr(out), out.size)
    if rc:
        raise _ERRORS.get(rc, OracleError)(oracle_lib().tvo_last_error().decode())
    return out


def quantize_q8_0(x: np.ndarray) -> np.ndarray:
    """Encode float32 values (length a multiple of 32) into 34-byte Q8_0 groups."""
    x = np.ascontiguousarray(_f32(x).reshape(-1, 32))
    out = np.empty((x.shape[0], 34), np.uint8)
    oracle_lib().tvo_quantize_q8_0(_ptr(x), x.shape[0], out.ctypes.data_as(C.POINTER(C.c_uint8)))
    return out.reshape(-1)


class Cache:
    """The oracle's PagedCache (kv.hpp:78-165) with its BlockPool (kv.hpp:36-75)."""

    def __init__(self, layers, kv_heads, head_dim, tokens_per_block, max_blocks, _ptr=None):
        self.lib = oracle_lib()
        self.geometry = (layers, kv_heads, head_dim, tokens_per_block, max_blocks)
        self._g = _Geometry(layers, kv_heads, head_dim, tokens_per_block, max_blocks)
        self.layers, self.kv_heads, self.head_dim, self.tokens_per_block, self.max_blocks = self.geometry
        self.kv_width = kv_heads * head_dim
        self.h = _ptr if _ptr is not None else self.lib.tvo_cache_create(C.byref(self._g))
        if not self.h:
            self._raise(-2)

    def __del__(self):
        if getattr(self, "h", None):
            self.lib.tvo_cache_destroy(self.h)
            self.h = None

    def _raise(self, rc):
        raise _ERRORS.get(rc, OracleError)(self.lib.tvo_last_error().decode())

    def _check(self, rc):
        if rc:
            self._raise(rc)

    def clone(self):
        return Cache(*self.geometry, _ptr=self.lib.tvo_cache_clone(self.h))

    @property
    def elements_per_block(self):
        return self.layers * 2 * self.tokens_per_block * self.kv_width

    def kv_offset(self, layer, kind, slot):
        v = self.lib.tvo_kv_offset(C.byref(self._g), layer, kind, slot)
        if v == (1 << 64) - 1:
            self._raise(-2)
        return v

    # pool
    def allocate(self):
        h = _Handle()
        self._check(self.lib.tvo_pool_allocate(self.h, C.byref(h)))
        return (h.id, h.generation)

    def retain(self, handle):
        self._check(self.lib.tvo_pool_retain(self.h, _Handle(*handle)))

    def release(self, handle):
        self._check(self.lib.tvo_pool_release(self.h, _Handle(*handle)))

    def references(self, handle):
        out = _sz()
        self._check(self.lib.tvo_pool_references(self.h, _Handle(*handle), C.byref(out)))
        return out.value

    def references_by_id(self, i):
        v = self.lib.tvo_pool_references_by_id(self.h, i)
        if v == (1 << 64) - 1:
            self._raise(-4)
        return v

    def available(self):
        return self.lib.tvo_pool_available(self.h)

    def block_data(self, handle):
        p = _fp()
        self._check(self.lib.tvo_pool_data(self.h, _Handle(*handle), C.byref(p)))
        return np.ctypeslib.as_array(p, shape=(self.elements_per_block,)).copy()

    def block_write(self, handle, offset, values):
        p = _fp()
        self._check(self.lib.tvo_pool_data(self.h, _Handle(*handle), C.byref(p)))
        arr = np.ctypeslib.as_array(p, shape=(self.elements_per_block,))
        values = _f32(values).reshape(-1)
        if offset + values.size > arr.size:
            raise InvalidArgument("write outside block")
        arr[offset : offset + values.size] = values

    # cache
    def create_sequence(self):
        s = self.lib.tvo_create_sequence(self.h)
        if not s:
            self._raise(-1)
        return s

    def length(self, seq):
        out = _sz()
        self._check(self.lib.tvo_sequence_length(self.h, seq, C.byref(out)))
        return out.value

    def blocks(self, seq):
        n = _sz()
        self._check(self.lib.tvo_sequence_blocks(self.h, seq, None, 0, C.byref(n)))
        arr = (_Handle * max(1, n.value))()
        self._check(self.lib.tvo_sequence_blocks(self.h, seq, arr, n.value, C.byref(n)))
        return [(arr[i].id, arr[i].generation) for i in range(n.value)]

    def physical_block(self, seq, position):
        h = _Handle()
        self._check(self.lib.tvo_physical_block(self.h, seq, position, C.byref(h)))
        return (h.id, h.generation)

    def append(self, seq, keys, values):
        k, v = _f32(keys).reshape(-1), _f32(values).reshape(-1)
        if k.size != self.layers * self.kv_width or v.size != k.size:
            raise InvalidArgument("invalid paged KV append dimensions")
        self._check(self.lib.tvo_append(self.h, seq, _ptr(k), _ptr(v)))

    def append_many(self, seq, keys, values):
        k = _f32(keys).reshape(-1, self.layers * self.kv_width)
        v = _f32(values).reshape(k.shape)
        for i in range(k.shape[0]):
            self._check(self.lib.tvo_append(self.h, seq, _ptr(k[i]), _ptr(v[i])))

    def append_batch(self, seqs, keys, values):
        w = self.layers * self.kv_width
        k = _f32(keys).reshape(-1, w)
        v = _f32(values).reshape(k.shape)
        for i, s in enumerate(seqs):
            self._check(self.lib.tvo_append(self.h, int(s), _ptr(k[i]), _ptr(v[i])))
        return len(seqs)

    def read(self, seq, layer, position, value=False):
        out = np.empty(self.kv_width, np.float32)
        self._check(self.lib.tvo_read(self.h, seq, layer, position, int(value), _ptr(out)))
        return out

    def read_all(self, seq, layer, value=False):
        n = self.length(seq)
        out = np.empty(max(1, n * self.kv_width), np.float32)
        self._check(self.lib.tvo_read_all(self.h, seq, layer, int(value), _ptr(out), out.size))
        return out[: n * self.kv_width]

    def drop(self, seq):
        self._check(self.lib.tvo_drop(self.h, seq))

    def fork(self, seq):
        s = self.lib.tvo_fork(self.h, seq)
        if not s:
            self._raise(-2 if "unknown" in self.lib.tvo_last_error().decode() else -1)
        return s

    def truncate(self, seq, length):
        self._check(self.lib.tvo_truncate(self.h, seq, length))

    def audit(self, external=None):
        if external is None:
            self._check(self.lib.tvo_audit(self.h, None, 0))
        else:
            ext = np.ascontiguousarray(external, dtype=np.uint64)
            self._check(self.lib.tvo_audit(self.h, ext.ctypes.data_as(C.POINTER(_sz)), ext.size))

    def import_sequence(self, blocks, source_length, length):
        arr = (_Handle * max(1, len(blocks)))(*[_Handle(*b) for b in blocks])
        s = self.lib.tvo_import_sequence(self.h, arr, len(blocks), source_length, length)
        if not s:
            msg = self.lib.tvo_last_error().decode()
            raise (InvalidArgument if ("prefix" in msg or "stale" in msg) else OracleError)(msg)
        return s

    def sequence_ids(self):
        n = self.lib.tvo_sequence_count(self.h)
        arr = np.zeros(max(1, n), np.uint64)
        self._check(self.lib.tvo_sequence_ids(self.h, arr.ctypes.data_as(C.POINTER(_u64)), n))
        return [int(x) for x in arr[:n]]

    def state(self):
        """Exact allocator and table state for bit-exact comparisons."""
        n = self.max_blocks
        refs = np.zeros(n, np.uint64)
        gens = np.zeros(n, np.uint64)
        free = np.zeros(n, np.uint64)
        count = _sz()
        self._check(
            self.lib.tvo_pool_state(
                self.h,
                refs.ctypes.data_as(C.POINTER(_sz)),
                gens.ctypes.data_as(C.POINTER(_u64)),
                free.ctypes.data_as(C.POINTER(_sz)),
                C.byref(count),
            )
        )
        tables = {s: (self.length(s), self.blocks(s)) for s in self.sequence_ids()}
        return {
            "refs": refs.tolist(),
            "generations": gens.tolist(),
            "free": free[: count.value].tolist(),
            "tables": tables,
        }

    # attention
    def fused_paged_attention(self, q, seq, layer, heads, context, tail_key=None, tail_value=None, visible=None):
        q = _f32(q).reshape(-1)
        out = np.empty(heads * self.head_dim, np.float32)
        tk = _f32(tail_key).reshape(-1) if tail_key is not None else None
        tv = _f32(tail_value).reshape(-1) if tail_value is not None else None
        vis = (1 << 64) - 1 if visible is None else visible
        self._check(
            self.lib.tvo_fused_paged_attention(self.h, seq, layer, heads, context, _ptr(q), _ptr(tk), _ptr(tv), vis,
                                               _ptr(out))
        )
        return out

    def fused_prompt_attention(self, queries, seq, layer, start, count, heads, context):
        q = _f32(queries).reshape(-1)
        out = np.empty(count * heads * self.head_dim, np.float32)
        self._check(
            self.lib.tvo_fused_prompt_attention(self.h, seq, layer, heads, context, start, count, _ptr(q), _ptr(out))
        )
        return out


# ----------------------------------------------------------------- reference

_ref = None


def ref_available() -> bool:
    return REF_PATH.exists()


def ref_lib():
    global _ref
    if _ref is None:
        if not REF_PATH.exists():
            raise FileNotFoundError(f"{REF_PATH} is not built (run `make -C oracle ref` where the reference is)")
        lib = C.CDLL(str(REF_PATH))
        lib.tvr_last_error.restype = C.c_char_p
        lib.tvr_cache_create.restype = C.c_void_p
        lib.tvr_cache_create.argtypes = [_sz] * 5
        lib.tvr_cache_destroy.argtypes = [C.c_void_p]
        lib.tvr_pool_allocate.argtypes = [C.c_void_p, C.POINTER(_u64), C.POINTER(_u64)]
        lib.tvr_pool_retain.argtypes = [C.c_void_p, _u64, _u64]
        lib.tvr_pool_release.argtypes = [C.c_void_p, _u64, _u64]
        lib.tvr_pool_references.argtypes = [C.c_void_p, _u64, _u64, C.POINTER(_sz)]
        lib.tvr_pool_available.restype = _sz
        lib.tvr_pool_available.argtypes = [C.c_void_p]
        lib.tvr_create_sequence.restype = _u64
        lib.tvr_create_sequence.argtypes = [C.c_void_p]
        lib.tvr_append.argtypes = [C.c_void_p, _u64, _fp, _fp]
        lib.tvr_append_many.argtypes = [C.c_void_p, _u64, _fp, _fp, _sz]
        lib.tvr_read_all.argtypes = [C.c_void_p, _u64, _sz, C.c_int, _fp, _sz]
        lib.tvr_read.argtypes = [C.c_void_p, _u64, _sz, _sz, C.c_int, _fp]
        lib.tvr_kv_offset.argtypes = [C.c_void_p, _sz, _sz, _sz, C.POINTER(_sz)]
        lib.tvr_drop.argtypes = [C.c_void_p, _u64]
        lib.tvr_fork.restype = _u64
        lib.tvr_fork.argtypes = [C.c_void_p, _u64]
        lib.tvr_truncate.argtypes = [C.c_void_p, _u64, _sz]
        lib.tvr_audit.argtypes = [C.c_void_p, C.POINTER(_sz), _sz]
        lib.tvr_import_blocks.restype = _u64
        lib.tvr_import_blocks.argtypes = [C.c_void_p, C.POINTER(_u64), C.POINTER(_u64), _sz, _sz, _sz]
        lib.tvr_import.restype = _u64
        lib.tvr_import.argtypes = [C.c_void_p, _u64, _sz]
        lib.tvr_sequence.argtypes = [C.c_void_p, _u64, C.POINTER(_sz), C.POINTER(_u64), C.POINTER(_u64), _sz,
                                     C.POINTER(_sz)]
        lib.tvr_pool_state.argtypes = [C.c_void_p, C.POINTER(_sz), C.POINTER(_u64), C.POINTER(_sz), C.POINTER(_sz),
                                       _u64]
        lib.tvr_block_data.argtypes = [C.c_void_p, _u64, _u64, _fp, _sz]
        lib.tvr_block_write.argtypes = [C.c_void_p, _u64, _u64, _sz, _fp, _sz]
        lib.tvr_fused_paged_attention.argtypes = [C.c_void_p, _u64, _sz, _sz, _sz, _fp, _fp, _fp, _sz, C.c_int, _fp]
        lib.tvr_fused_prompt_attention.argtypes = [C.c_void_p, _u64, _sz, _sz, _sz, _sz, _sz, _fp, _fp]
        lib.tvr_grouped_attention.argtypes = [_fp, _fp, _fp, _sz, _sz, _sz, _sz, _sz, _fp]
        lib.tvr_radix_create.restype = C.c_void_p
        lib.tvr_radix_create.argtypes = [C.c_void_p, C.c_char_p]
        lib.tvr_radix_destroy.argtypes = [C.c_void_p]
        lib.tvr_radix_insert.argtypes = [C.c_void_p, C.POINTER(C.c_int32), _sz, C.POINTER(_u64)]
        lib.tvr_radix_lookup.argtypes = [C.c_void_p, C.POINTER(C.c_int32), _sz, C.POINTER(_u64), C.POINTER(_sz)]
        lib.tvr_radix_attach.argtypes = [C.c_void_p, _u64, _u64]
        lib.tvr_radix_reuse.argtypes = [C.c_void_p, C.POINTER(C.c_int32), _sz, C.c_int, C.POINTER(_u64),
                                        C.POINTER(_sz)]
        for name in ("pin", "unpin", "touch"):
            getattr(lib, "tvr_radix_" + name).argtypes = [C.c_void_p, _u64]
        lib.tvr_radix_eviction_candidate.argtypes = [C.c_void_p, C.POINTER(_u64)]
        lib.tvr_radix_evict_one.argtypes = [C.c_void_p, C.POINTER(C.c_int)]
        lib.tvr_radix_reset.argtypes = [C.c_void_p]
        lib.tvr_radix_size.argtypes = [C.c_void_p, C.POINTER(_sz)]
        lib.tvr_radix_node.argtypes = [C.c_void_p, _u64, C.POINTER(_u64), C.POINTER(C.c_int32), _sz, C.POINTER(_sz),
                                       C.POINTER(_sz), C.POINTER(_u64), C.POINTER(_sz), C.POINTER(_sz),
                                       C.POINTER(_sz)]
        lib.tvr_radix_external_references.argtypes = [C.c_void_p, C.POINTER(_sz), _sz]
        lib.tvr_half_to_float.restype = C.c_float
        lib.tvr_half_to_float.argtypes = [C.c_uint16]
        lib.tvr_fused_batch.argtypes = [C.c_void_p, C.POINTER(_u64), _sz, _sz, _sz, _sz, _fp, _fp, C.c_int]
        lib.tvr_prompt_batch.argtypes = [C.c_void_p, _u64, _sz, _sz, _sz, _sz, _sz, _fp, _fp, _sz, C.c_int]
        lib.tvr_use_avx2.restype = C.c_int
        lib.tvr_host_triad.restype = C.c_double
        lib.tvr_host_triad.argtypes = [_sz, C.c_int, C.c_int]
        lib.tvr_dequantize_q8_0.argtypes = [C.POINTER(C.c_uint8), _sz, _fp, _sz]
        _ref = lib
    return _ref


class RefCache:
    """The reference's own PagedCache, through oracle/_ref/libtvara_ref.so."""

    def __init__(self, layers, kv_heads, head_dim, tokens_per_block, max_blocks):
        self.lib = ref_lib()
        self.geometry = (layers, kv_heads, head_dim, tokens_per_block, max_blocks)
        self.layers, self.kv_heads, self.head_dim, self.tokens_per_block, self.max_blocks = self.geometry
        self.kv_width = kv_heads * head_dim
        self.h = self.lib.tvr_cache_create(*self.geometry)
        if not self.h:
            raise InvalidArgument(self.lib.tvr_last_error().decode())
        self._seqs = set()

    def __del__(self):
        if getattr(self, "h", None):
            self.lib.tvr_cache_destroy(self.h)
            self.h = None

    @property
    def elements_per_block(self):
        return self.layers * 2 * self.tokens_per_block * self.kv_width

    def _check(self, rc):
        if rc:
            raise _ERRORS.get(rc, OracleError)(self.lib.tvr_last_error().decode())

    def allocate(self):
        i, g = _u64(), _u64()
        self._check(self.lib.tvr_pool_allocate(self.h, C.byref(i), C.byref(g)))
        return (i.value, g.value)

    def retain(self, handle):
        self._check(self.lib.tvr_pool_retain(self.h, *handle))

    def release(self, handle):
        self._check(self.lib.tvr_pool_release(self.h, *handle))

    def references(self, handle):
        out = _sz()
        self._check(self.lib.tvr_pool_references(self.h, handle[0], handle[1], C.byref(out)))
        return out.value

    def available(self):
        return self.lib.tvr_pool_available(self.h)

    def create_sequence(self):
        s = self.lib.tvr_create_sequence(self.h)
        if not s:
            raise OracleError(self.lib.tvr_last_error().decode())
        self._seqs.add(s)
        return s

    def append(self, seq, keys, values):
        k, v = _f32(keys).reshape(-1), _f32(values).reshape(-1)
        if k.size != self.layers * self.kv_width or v.size != k.size:
            raise InvalidArgument("invalid paged KV append dimensions")
        self._check(self.lib.tvr_append(self.h, seq, _ptr(k), _ptr(v)))

    def append_many(self, seq, keys, values):
        k = _f32(keys).reshape(-1, self.layers * self.kv_width)
        v = _f32(values).reshape(k.shape)
        self._check(self.lib.tvr_append_many(self.h, seq, _ptr(k), _ptr(v), k.shape[0]))

    def kv_offset(self, layer, kind, slot):
        out = _sz()
        self._check(self.lib.tvr_kv_offset(self.h, layer, kind, slot, C.byref(out)))
        return out.value

    def read(self, seq, layer, position, value=False):
        out = np.empty(self.kv_width, np.float32)
        self._check(self.lib.tvr_read(self.h, seq, layer, position, int(value), _ptr(out)))
        return out

    def append_batch(self, seqs, keys, values):
        w = self.layers * self.kv_width
        k = _f32(keys).reshape(-1, w)
        v = _f32(values).reshape(k.shape)
        for i, s in enumerate(seqs):
            self._check(self.lib.tvr_append(self.h, int(s), _ptr(k[i]), _ptr(v[i])))
        return len(seqs)

    def read_all(self, seq, layer, value=False):
        n = self.length(seq)
        out = np.empty(max(1, n * self.kv_width), np.float32)
        self._check(self.lib.tvr_read_all(self.h, seq, layer, int(value), _ptr(out), out.size))
        return out[: n * self.kv_width]

    def drop(self, seq):
        self._check(self.lib.tvr_drop(self.h, seq))
        self._seqs.discard(seq)

    def fork(self, seq):
        s = self.lib.tvr_fork(self.h, seq)
        if not s:
            raise InvalidArgument(self.lib.tvr_last_error().decode())
        self._seqs.add(s)
        return s

    def truncate(self, seq, length):
        self._check(self.lib.tvr_truncate(self.h, seq, length))

    def audit(self, external=None):
        ext = np.ascontiguousarray(external if external is not None else [], dtype=np.uint64)
        self._check(self.lib.tvr_audit(self.h, ext.ctypes.data_as(C.POINTER(_sz)), ext.size))

    def import_sequence(self, blocks, source_length, length):
        ids = np.ascontiguousarray([b[0] for b in blocks] or [0], dtype=np.uint64)
        gens = np.ascontiguousarray([b[1] for b in blocks] or [0], dtype=np.uint64)
        s = self.lib.tvr_import_blocks(self.h, ids.ctypes.data_as(C.POINTER(_u64)), gens.ctypes.data_as(C.POINTER(_u64)),
                                       len(blocks), source_length, length)
        if not s:
            raise InvalidArgument(self.lib.tvr_last_error().decode())
        self._seqs.add(s)
        return s

    def import_from(self, source_seq, length):
        s = self.lib.tvr_import(self.h, source_seq, length)
        if not s:
            raise InvalidArgument(self.lib.tvr_last_error().decode())
        self._seqs.add(s)
        return s

    def length(self, seq):
        return self._sequence(seq)[0]

    def blocks(self, seq):
        return self._sequence(seq)[1]

    def _sequence(self, seq):
        length, count = _sz(), _sz()
        self._check(self.lib.tvr_sequence(self.h, seq, C.byref(length), None, None, 0, C.byref(count)))
        ids = np.zeros(max(1, count.value), np.uint64)
        gens = np.zeros(max(1, count.value), np.uint64)
        self._check(
            self.lib.tvr_sequence(self.h, seq, C.byref(length), ids.ctypes.data_as(C.POINTER(_u64)),
                                  gens.ctypes.data_as(C.POINTER(_u64)), count.value, C.byref(count))
        )
        return length.value, [(int(ids[i]), int(gens[i])) for i in range(count.value)]

    def physical_block(self, seq, position):
        length, blocks = self._sequence(seq)
        if position >= length:
            raise InvalidArgument("KV position beyond sequence")
        return blocks[position // self.tokens_per_block]

    def sequence_ids(self):
        return sorted(self._seqs)

    def state(self, max_generation=1 << 20):
        n = self.max_blocks
        refs = np.zeros(n, np.uint64)
        gens = np.zeros(n, np.uint64)
        free = np.zeros(n, np.uint64)
        count = _sz()
        self._check(
            self.lib.tvr_pool_state(self.h, refs.ctypes.data_as(C.POINTER(_sz)), gens.ctypes.data_as(C.POINTER(_u64)),
                                    free.ctypes.data_as(C.POINTER(_sz)), C.byref(count), max_generation)
        )
        tables = {s: (self.length(s), self.blocks(s)) for s in self.sequence_ids()}
        return {"refs": refs.tolist(), "generations": gens.tolist(), "free": free[: count.value].tolist(),
                "tables": tables}

    def block_data(self, handle):
        out = np.empty(self.elements_per_block, np.float32)
        self._check(self.lib.tvr_block_data(self.h, handle[0], handle[1], _ptr(out), out.size))
        return out

    def block_write(self, handle, offset, values):
        v = _f32(values).reshape(-1)
        self._check(self.lib.tvr_block_write(self.h, handle[0], handle[1], offset, _ptr(v), v.size))

    def fused_paged_attention(self, q, seq, layer, heads, context, tail_key=None, tail_value=None, visible=None,
                              scalar=False):
        q = _f32(q).reshape(-1)
        out = np.empty(heads * self.head_dim, np.float32)
        tk = _f32(tail_key).reshape(-1) if tail_key is not None else None
        tv = _f32(tail_value).reshape(-1) if tail_value is not None else None
        vis = (1 << 64) - 1 if visible is None else visible
        self._check(self.lib.tvr_fused_paged_attention(self.h, seq, layer, heads, context, _ptr(q), _ptr(tk),
                                                       _ptr(tv), vis, int(scalar), _ptr(out)))
        return out

    def fused_batch(self, seqs, q, layer, heads, context, threads=1):
        """fused_paged_attention for every listed sequence on `threads`
        std::threads (the CPU-baseline runner of bench.py)."""
        seqs = np.ascontiguousarray(seqs, dtype=np.uint64)
        q = _f32(q).reshape(seqs.size, heads * self.head_dim)
        out = np.empty_like(q)
        self._check(self.lib.tvr_fused_batch(self.h, seqs.ctypes.data_as(C.POINTER(_u64)), seqs.size, layer, heads,
                                             context, _ptr(q), _ptr(out), threads))
        return out

    def prompt_batch(self, queries, seq, layer, start, count, heads, context, rows_per_unit, threads=1):
        """fused_prompt_attention over rows start .. start+count-1 in runs of
        rows_per_unit rows on `threads` std::threads."""
        q = _f32(queries).reshape(-1)
        out = np.empty(count * heads * self.head_dim, np.float32)
        self._check(self.lib.tvr_prompt_batch(self.h, seq, layer, heads, context, start, count, _ptr(q), _ptr(out),
                                              rows_per_unit, threads))
        return out

    def fused_prompt_attention(self, queries, seq, layer, start, count, heads, context):
        q = _f32(queries).reshape(-1)
        out = np.empty(count * heads * self.head_dim, np.float32)
        self._check(self.lib.tvr_fused_prompt_attention(self.h, seq, layer, heads, context, start, count, _ptr(q),
                                                        _ptr(out)))
        return out


def ref_grouped_attention(q, keys, values, positions, heads, kv_heads, head_dim, context):
    lib = ref_lib()
    q, k, v = _f32(q).reshape(-1), _f32(keys).reshape(-1), _f32(values).reshape(-1)
    out = np.empty(heads * head_dim, np.float32)
    rc = lib.tvr_grouped_attention(_ptr(q), _ptr(k), _ptr(v), positions, heads, kv_heads, head_dim, context, _ptr(out))
    if rc:
        raise _ERRORS.get(rc, OracleError)(lib.tvr_last_error().decode())
    return out


def ref_uses_avx2() -> bool:
    """Whether the reference's attention dot takes its AVX2 path on this host."""
    return bool(ref_lib().tvr_use_avx2())


def host_triad_gbs(doubles: int, threads: int, reps: int = 3) -> float:
    """STREAM-style triad bandwidth of the host (GB/s, best of reps)."""
    return ref_lib().tvr_host_triad(doubles, threads, reps) / 1e9


def ref_half_to_float(h: int) -> float:
    return float(ref_lib().tvr_half_to_float(h))


def ref_dequantize_q8_0(raw: np.ndarray) -> np.ndarray:
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    out = np.empty(raw.size // 34 * 32, np.float32)
    rc = ref_lib().tvr_dequantize_q8_0(raw.ctypes.data_as(C.POINTER(C.c_uint8)), raw.size, _ptr(out), out.size)
    if rc:
        raise _ERRORS.get(rc, OracleError)(ref_lib().tvr_last_error().decode())
    return out


class RefRadix:
    """The reference's RadixCache (core/include/tvara/radix.hpp:17-131) over a
    RefCache, through oracle/_ref/libtvara_ref.so; same methods and return
    values as tvara_amd.radix.RadixCache."""

    def __init__(self, cache, isolation):
        self.cache = cache
        self.lib = cache.lib
        self.h = self.lib.tvr_radix_create(cache.h, isolation.encode("utf-8"))
        if not self.h:
            raise InvalidArgument(self.lib.tvr_last_error().decode())

    def __del__(self):
        self.close()

    def close(self):
        if getattr(self, "h", None):
            self.lib.tvr_radix_destroy(self.h)
            self.h = None

    def _check(self, rc):
        if rc:
            raise _ERRORS.get(rc, OracleError)(self.lib.tvr_last_error().decode())

    @staticmethod
    def _tokens(tokens):
        t = np.ascontiguousarray(tokens, dtype=np.int32).reshape(-1)
        return t, t.ctypes.data_as(C.POINTER(C.c_int32))

    def size(self):
        n = _sz()
        self._check(self.lib.tvr_radix_size(self.h, C.byref(n)))
        return n.value

    def lookup(self, tokens):
        t, p = self._tokens(tokens)
        node, matched = _u64(), _sz()
        self._check(self.lib.tvr_radix_lookup(self.h, p, t.size, C.byref(node), C.byref(matched)))
        return node.value, matched.value

    def insert(self, tokens):
        t, p = self._tokens(tokens)
        node = _u64()
        self._check(self.lib.tvr_radix_insert(self.h, p, t.size, C.byref(node)))
        return node.value

    def attach(self, node, sequence):
        self._check(self.lib.tvr_radix_attach(self.h, node, sequence))

    def reuse(self, tokens, partial=False):
        t, p = self._tokens(tokens)
        seq, length = _u64(), _sz()
        self._check(self.lib.tvr_radix_reuse(self.h, p, t.size, int(partial), C.byref(seq), C.byref(length)))
        self.cache._seqs.add(seq.value)
        return seq.value, length.value

    def pin(self, node):
        self._check(self.lib.tvr_radix_pin(self.h, node))

    def unpin(self, node):
        self._check(self.lib.tvr_radix_unpin(self.h, node))

    def touch(self, node):
        self._check(self.lib.tvr_radix_touch(self.h, node))

    def eviction_candidate(self):
        node = _u64()
        self._check(self.lib.tvr_radix_eviction_candidate(self.h, C.byref(node)))
        return node.value or None

    def evict_one(self):
        e = C.c_int()
        self._check(self.lib.tvr_radix_evict_one(self.h, C.byref(e)))
        return bool(e.value)

    def reset(self):
        self._check(self.lib.tvr_radix_reset(self.h))

    def node(self, node_id):
        parent, elen, pins, acc, kvlen, kvb, ch = _u64(), _sz(), _sz(), _u64(), _sz(), _sz(), _sz()
        self._check(self.lib.tvr_radix_node(self.h, node_id, C.byref(parent), None, 0, C.byref(elen), C.byref(pins),
                                            C.byref(acc), C.byref(kvlen), C.byref(kvb), C.byref(ch)))
        edge = np.zeros(max(1, elen.value), np.int32)
        self._check(self.lib.tvr_radix_node(self.h, node_id, C.byref(parent), edge.ctypes.data_as(C.POINTER(C.c_int32)),
                                            elen.value, C.byref(elen), C.byref(pins), C.byref(acc), C.byref(kvlen),
                                            C.byref(kvb), C.byref(ch)))
        has_kv = kvb.value != (1 << 64) - 1
        return {"id": node_id, "parent": parent.value, "edge": [int(x) for x in edge[: elen.value]],
                "pins": pins.value, "accessed": acc.value, "kv_length": kvlen.value if has_kv else None,
                "kv_blocks": kvb.value if has_kv else None, "children": ch.value}

    def external_references(self):
        counts = np.zeros(self.cache.max_blocks, np.uint64)
        self._check(self.lib.tvr_radix_external_references(self.h, counts.ctypes.data_as(C.POINTER(_sz)),
                                                           counts.size))
        return [int(x) for x in counts]
