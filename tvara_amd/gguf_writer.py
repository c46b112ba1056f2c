"""GGUF writer and synthetic Llama models (for the model-level tests and the
model benchmark).

Writes GGUF v3 (little-endian): header, metadata key/values, tensor infos,
padding to the alignment, then the tensor payloads at aligned offsets -- the
layout core/include/tvara/gguf.hpp:43-209 reads.  Synthetic weights are
random, seeded per tensor (numpy's PCG64 keyed by seed and tensor name); every
storage type the reference's model loader accepts (f32, f16, Q4_0, Q8_0, Q4_K;
model.hpp:119-134) can be chosen per tensor class.
"""

from __future__ import annotations

import struct
import zlib
from dataclasses import dataclass, field

import numpy as np

# GGUF metadata value types
U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
# tensor storage types
T_F32, T_F16, T_Q4_0, T_Q8_0, T_Q4_K = 0, 1, 2, 8, 12


def _str(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", U64: "<Q", I64: "<q",
           F64: "<d"}


def _value(vtype: int, value) -> bytes:
    if vtype == STR:
        return _str(value)
    if vtype == BOOL:
        return struct.pack("<B", 1 if value else 0)
    if vtype == ARR:
        etype, items = value
        out = struct.pack("<IQ", etype, len(items))
        return out + b"".join(_value(etype, v) for v in items)
    return struct.pack(_SCALAR[vtype], value)


class Lazy:
    """A payload of known size generated while the file is written."""

    def __init__(self, size, make):
        self.size, self.make = size, make

    def __call__(self):
        data = self.make()
        assert len(data) == self.size
        return data


def write_gguf(path, metadata, tensors, alignment=32, version=3):
    """metadata: list of (key, type, value); tensors: list of (name, dims,
    storage type, payload), dims fastest-first; a payload is bytes or a Lazy."""
    parts = [b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(metadata))]
    for key, vtype, value in metadata:
        parts.append(_str(key) + struct.pack("<I", vtype) + _value(vtype, value))
    offset = 0
    for name, dims, ttype, payload in tensors:
        size = payload.size if isinstance(payload, Lazy) else len(payload)
        parts.append(_str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
                     + struct.pack("<IQ", ttype, offset))
        offset += (size + alignment - 1) // alignment * alignment
    head = b"".join(parts)
    with open(path, "wb") as f:
        f.write(head + b"\0" * ((-len(head)) % alignment))
        for _, _, _, payload in tensors:
            data = payload() if isinstance(payload, Lazy) else payload
            f.write(data)
            f.write(b"\0" * ((-len(data)) % alignment))


def _payload_size(ttype, dims):
    n = int(np.prod(dims))
    return {T_F32: 4 * n, T_F16: 2 * n, T_Q8_0: n // 32 * 34, T_Q4_0: n // 32 * 18, T_Q4_K: n // 256 * 144}[ttype]


# ------------------------------------------------------------ payloads

def _f16_bits(x):
    return np.asarray(x, np.float16).view(np.uint16)


def _rng(seed, tag):
    return np.random.default_rng([seed, zlib.crc32(tag.encode())])


def payload(ttype, rows, cols, seed, tag, scale):
    """Random weights of shape [rows][cols] in storage type ttype."""
    n = rows * cols
    g = _rng(seed, tag)
    if ttype == T_F32:
        return (g.standard_normal(n, np.float32) * np.float32(scale)).astype("<f4").tobytes()
    if ttype == T_F16:
        return (g.standard_normal(n, np.float32) * np.float32(scale)).astype("<f2").tobytes()
    if ttype == T_Q8_0:
        groups = n // 32
        blk = np.empty((groups, 34), np.uint8)
        blk[:, 0:2] = _f16_bits(scale / 64.0 * (0.5 + g.random(groups))).astype("<u2").view(np.uint8).reshape(groups, 2)
        blk[:, 2:] = g.integers(-127, 128, (groups, 32), dtype=np.int8).view(np.uint8)
        return blk.tobytes()
    if ttype == T_Q4_0:
        groups = n // 32
        blk = np.empty((groups, 18), np.uint8)
        blk[:, 0:2] = _f16_bits(scale / 4.0 * (0.5 + g.random(groups))).astype("<u2").view(np.uint8).reshape(groups, 2)
        blk[:, 2:] = g.integers(0, 256, (groups, 16), dtype=np.uint8)
        return blk.tobytes()
    if ttype == T_Q4_K:
        supers = n // 256
        blk = np.empty((supers, 144), np.uint8)
        blk[:, 0:2] = _f16_bits(scale / 256.0 * (0.5 + g.random(supers))).astype("<u2").view(np.uint8).reshape(supers, 2)
        blk[:, 2:4] = _f16_bits(scale / 512.0 * (0.5 + g.random(supers))).astype("<u2").view(np.uint8).reshape(supers, 2)
        blk[:, 4:] = g.integers(0, 256, (supers, 140), dtype=np.uint8)
        return blk.tobytes()
    raise ValueError(ttype)


@dataclass
class LlamaSpec:
    vocab: int = 96
    hidden: int = 64
    intermediate: int = 128
    layers: int = 2
    heads: int = 4
    kv_heads: int = 2
    context: int = 64
    rms_epsilon: float = 1e-5
    rope_theta: float = 10000.0
    rope_layout: str | None = None        # None: key absent (interleaved)
    output: bool = True                   # an output.weight tensor (else the embedding is tied)
    matrix_type: int = T_F32              # projections and FFN
    embed_type: int = T_F32
    norm_type: int = T_F32
    seed: int = 7
    attn_norm_scale: float = 1.0          # multiplies the attention norms' weights
    extra: list = field(default_factory=list)  # more metadata (key, type, value)

    def metadata(self):
        m = [("general.architecture", STR, "llama"),
             ("general.name", STR, "synthetic \"tiny\" llama\\n\t"),
             ("tokenizer.ggml.tokens", ARR, (STR, [f"t{i}" for i in range(self.vocab)])),
             ("llama.embedding_length", U32, self.hidden),
             ("llama.feed_forward_length", U32, self.intermediate),
             ("llama.block_count", U32, self.layers),
             ("llama.attention.head_count", U32, self.heads),
             ("llama.attention.head_count_kv", U32, self.kv_heads),
             ("llama.context_length", U32, self.context),
             ("llama.attention.layer_norm_rms_epsilon", F32, self.rms_epsilon),
             ("llama.rope.freq_base", F32, self.rope_theta)]
        if self.rope_layout is not None:
            m.append(("tvara.rope.layout", STR, self.rope_layout))
        return m + list(self.extra)

    def tensors(self):
        h, i, v = self.hidden, self.intermediate, self.vocab
        kv = h // self.heads * self.kv_heads
        s = self.seed

        def norm(name):
            w = (1.0 + 0.1 * _rng(s, name).standard_normal(h)).astype(np.float32)
            if name.endswith("attn_norm.weight"):
                w = (w * np.float32(self.attn_norm_scale)).astype(np.float32)
            if self.norm_type == T_F16:
                return (name, [h], T_F16, w.astype("<f2").tobytes())
            return (name, [h], T_F32, w.astype("<f4").tobytes())

        def mat(name, rows, cols, ttype):
            return (name, [cols, rows], ttype,
                    Lazy(_payload_size(ttype, [cols, rows]), lambda: payload(ttype, rows, cols, s, name, 1.0 / np.sqrt(cols))))

        t = [mat("token_embd.weight", v, h, self.embed_type), norm("output_norm.weight")]
        if self.output:
            t.append(mat("output.weight", v, h, self.matrix_type))
        for layer in range(self.layers):
            p = f"blk.{layer}."
            t += [norm(p + "attn_norm.weight"), norm(p + "ffn_norm.weight"),
                  mat(p + "attn_q.weight", h, h, self.matrix_type), mat(p + "attn_k.weight", kv, h, self.matrix_type),
                  mat(p + "attn_v.weight", kv, h, self.matrix_type),
                  mat(p + "attn_output.weight", h, h, self.matrix_type),
                  mat(p + "ffn_gate.weight", i, h, self.matrix_type), mat(p + "ffn_up.weight", i, h, self.matrix_type),
                  mat(p + "ffn_down.weight", h, i, self.matrix_type)]
        return t

    def write(self, path):
        write_gguf(path, self.metadata(), self.tensors())
        return path


def tiny_random_llama(**kw):
    """The shape of the reference's arithmetic fixture, Hugging Face's
    tiny-random-LlamaForCausalLM (docs/reference-model.md:3-6: hidden 16, two
    layers; 4 / 4 heads, FFN 64, vocabulary 32,000), exported with the split
    RoPE layout as tools/convert_reference_gguf.py:47 writes it, with random
    f32 weights."""
    args = dict(vocab=32000, hidden=16, intermediate=64, layers=2, heads=4, kv_heads=4, context=2048,
                rms_epsilon=1e-6, rope_layout="split", seed=13)
    args.update(kw)
    return LlamaSpec(**args)


def llama32_1b(**kw):
    """The Llama-3.2-1B shape (16 layers, hidden 2048, 32 / 8 heads, FFN 8192,
    vocabulary 128,256, tied embedding) with random Q8_0 weights."""
    args = dict(vocab=128256, hidden=2048, intermediate=8192, layers=16, heads=32, kv_heads=8, context=8192,
                rope_theta=500000.0, output=False, matrix_type=T_Q8_0, embed_type=T_Q8_0, seed=11)
    args.update(kw)
    return LlamaSpec(**args)
