"""NativeModel over libtvara_capi's model-level exports (the Python ctypes
surface of python/tvara/native.py:26-218: open, metadata, sequences, logits),
plus the batch decode and truncate calls that NativeSpeculativeModel binds
(python/tvara/speculative.py:222-295).

The reference's own NativeModel runs unchanged on this library
(TVARA_LIBRARY=.../libtvara_capi.so): the 11 exports keep its signatures.
"""

from __future__ import annotations

import ctypes
import json
import threading
import weakref
from pathlib import Path

import numpy as np

from . import _capi


class NativeModel:
    def __init__(self, path, library=None, max_blocks=256, block_tokens=16):
        if (not isinstance(max_blocks, int) or not isinstance(block_tokens, int) or max_blocks <= 0
                or block_tokens <= 0):
            raise ValueError("Cache geometry must be positive integers")
        self._lock = threading.RLock()
        self._library = _capi.model_lib(library)
        lib = self._library
        self._handle = lib.tvara_model_open(str(Path(path).resolve()).encode("utf-8"), max_blocks, block_tokens)
        if not self._handle:
            self._raise_error()
        self._finalizer = weakref.finalize(self, lib.tvara_model_close, self._handle)
        self._max_blocks, self._block_tokens = max_blocks, block_tokens
        self.vocab_size = int(lib.tvara_model_vocab_size(self._handle))
        self.context_size = int(lib.tvara_model_context_size(self._handle))

    def _raise_error(self):
        message = self._library.tvara_last_error()
        raise RuntimeError(message.decode("utf-8", errors="replace") if message else "Native operation failed")

    def _check_open(self):
        if not self._handle:
            raise RuntimeError("Model is closed")

    def close(self):
        with self._lock:
            if self._handle:
                self._finalizer()
                self._handle = None

    def __enter__(self):
        self._check_open()
        return self

    def __exit__(self, *args):
        self.close()

    @property
    def metadata(self):
        with self._lock:
            self._check_open()
            raw = self._library.tvara_model_metadata(self._handle)
            if not raw:
                self._raise_error()
            return json.loads(raw.decode("utf-8"))

    def metadata_json(self):
        """The raw JSON text of tvara_model_metadata."""
        with self._lock:
            self._check_open()
            raw = self._library.tvara_model_metadata(self._handle)
            if not raw:
                self._raise_error()
            return raw.decode("utf-8")

    def new_sequence(self):
        with self._lock:
            self._check_open()
            sequence = self._library.tvara_sequence_create(self._handle)
            if not sequence:
                self._raise_error()
            return sequence

    def drop_sequence(self, sequence):
        with self._lock:
            if self._handle and self._library.tvara_sequence_drop(self._handle, sequence):
                self._raise_error()

    _new_sequence = new_sequence
    _drop_sequence = drop_sequence

    def _valid_token(self, token):
        return (not isinstance(token, (bool, np.bool_)) and isinstance(token, (int, np.integer))
                and 0 <= token < self.vocab_size)

    def logits(self, sequence, token):
        if not self._valid_token(token):
            raise ValueError("Invalid token ID")
        output = np.empty(self.vocab_size, dtype=np.float32)
        with self._lock:
            self._check_open()
            if self._library.tvara_sequence_decode(self._handle, sequence, int(token),
                                                   output.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                                                   len(output)):
                self._raise_error()
        return output

    def decode_batch(self, sequence, tokens):
        """Logits [len(tokens), vocab] of consecutive tokens; on failure the
        sequence is truncated back to its entry length."""
        toks = np.ascontiguousarray(tokens, dtype=np.uint32).reshape(-1)
        output = np.empty((toks.size, self.vocab_size), dtype=np.float32)
        with self._lock:
            self._check_open()
            if self._library.tvara_sequence_decode_batch(self._handle, sequence,
                                                         toks.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)),
                                                         toks.size,
                                                         output.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                                                         output.size):
                self._raise_error()
        return output

    def prefill(self, sequence, tokens):
        """Logits [vocab] of the last of `tokens`, decoded in order at the end
        of `sequence` (tvara_sequence_prefill: one pass per chunk); on failure
        the sequence is truncated back to its entry length.  A library without
        the export (the reference's) decodes token by token."""
        toks = np.ascontiguousarray(tokens, dtype=np.uint32).reshape(-1)
        if not toks.size:
            raise ValueError("empty prompt")
        fn = getattr(self._library, "tvara_sequence_prefill", None)
        if fn is None or fn.argtypes is None:  # not bound: a build of the reference's 11 exports
            with self._lock:
                for token in toks:
                    out = self.logits(sequence, int(token))
            return out
        output = np.empty(self.vocab_size, dtype=np.float32)
        with self._lock:
            self._check_open()
            if fn(self._handle, sequence, toks.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), toks.size,
                  output.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), output.size):
                self._raise_error()
        return output

    def decode_sequences(self, sequences, tokens):
        """One token for each of several distinct sequences in one pass
        (tvara_sequences_decode): logits [len(sequences), vocab]."""
        seqs = np.ascontiguousarray(sequences, dtype=np.uint64).reshape(-1)
        toks = np.ascontiguousarray(tokens, dtype=np.uint32).reshape(-1)
        if seqs.size != toks.size:
            raise ValueError("one token per sequence")
        output = np.empty((seqs.size, self.vocab_size), dtype=np.float32)
        with self._lock:
            self._check_open()
            if self._library.tvara_sequences_decode(self._handle, seqs.ctypes.data_as(ctypes.POINTER(ctypes.c_uint64)),
                                                    toks.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), seqs.size,
                                                    output.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                                                    output.size):
                self._raise_error()
        return output

    def cache(self):
        """The model's KV cache as a tvara_amd.kv.PagedCache (tvara_model_cache):
        fork, snapshots, retain / release, import and the prefix cache
        (tvara_amd.radix.RadixCache) work on the model's sequences."""
        from . import kv

        with self._lock:
            self._check_open()
            h = self._library.tvara_model_cache(self._handle)
            if not h:
                self._raise_error()
            md = self.metadata
            heads, kvh = md["llama.attention.head_count"], md["llama.attention.head_count_kv"]
            dim = md["llama.embedding_length"] // heads
            return kv.PagedCache.lent(h, md["llama.block_count"], kvh, dim, self._block_tokens, self._max_blocks,
                                      owner=self)

    def truncate(self, sequence, length):
        with self._lock:
            self._check_open()
            if self._library.tvara_sequence_truncate(self._handle, sequence, length):
                self._raise_error()
