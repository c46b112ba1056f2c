"""Synthetic Llama GGUF files for the model-level tests.

Writes GGUF v3 (little-endian): header, metadata key/values, tensor infos,
padding to the alignment, then the tensor payloads at aligned offsets -- the
layout core/include/tvara/gguf.hpp:43-209 reads.  Weights are random and
seeded (tvara_amd.synth); every storage type the reference's model loader
accepts (f32, f16, Q4_0, Q8_0, Q4_K; model.hpp:119-134) can be chosen per
tensor class.
"""

from __future__ import annotations

import struct
from dataclasses import dataclass, field

import numpy as np

from tvara_amd import synth

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


def write_gguf(path, metadata, tensors, alignment=32, version=3):
    """metadata: list of (key, type, value); tensors: list of (name, dims,
    storage type, payload bytes), dims fastest-first."""
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(metadata))
    for key, vtype, value in metadata:
        head += _str(key) + struct.pack("<I", vtype) + _value(vtype, value)
    offset, infos = 0, []
    for name, dims, ttype, payload in tensors:
        infos.append(_str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
                     + struct.pack("<IQ", ttype, offset))
        offset += (len(payload) + alignment - 1) // alignment * alignment
    head += b"".join(infos)
    head += b"\0" * ((-len(head)) % alignment)
    body = b""
    for _, _, _, payload in tensors:
        body += payload + b"\0" * ((-len(payload)) % alignment)
    with open(path, "wb") as f:
        f.write(head + body)


# ------------------------------------------------------------ payloads

def _f16_bits(x):
    return np.asarray(x, np.float16).view(np.uint16)


def payload(ttype, rows, cols, seed, tag, scale):
    """Random weights of shape [rows][cols] in storage type ttype."""
    n = rows * cols
    if ttype == T_F32:
        return (synth.normal(seed, tag, n) * np.float32(scale)).astype("<f4").tobytes()
    if ttype == T_F16:
        return (synth.normal(seed, tag, n) * np.float32(scale)).astype("<f2").tobytes()
    u = synth.uniform(seed, tag + "/d", n // 32 + 1)
    if ttype == T_Q8_0:
        groups = n // 32
        d = _f16_bits(scale / 64.0 * (0.5 + u[:groups]))
        q = (synth.integers(seed, tag + "/q", n, 0, 255) - 127).astype(np.int8).reshape(groups, 32)
        blk = np.zeros((groups, 34), np.uint8)
        blk[:, 0:2] = d.astype("<u2").view(np.uint8).reshape(groups, 2)
        blk[:, 2:] = q.view(np.uint8)
        return blk.tobytes()
    if ttype == T_Q4_0:
        groups = n // 32
        d = _f16_bits(scale / 4.0 * (0.5 + u[:groups]))
        nib = synth.integers(seed, tag + "/q", groups * 16, 0, 255).astype(np.uint8).reshape(groups, 16)
        blk = np.zeros((groups, 18), np.uint8)
        blk[:, 0:2] = d.astype("<u2").view(np.uint8).reshape(groups, 2)
        blk[:, 2:] = nib
        return blk.tobytes()
    if ttype == T_Q4_K:
        supers = n // 256
        d = _f16_bits(scale / 256.0 * (0.5 + u[:supers]))
        dmin = _f16_bits(scale / 512.0 * (0.5 + synth.uniform(seed, tag + "/m", supers)))
        rest = synth.integers(seed, tag + "/q", supers * 140, 0, 255).astype(np.uint8).reshape(supers, 140)
        blk = np.zeros((supers, 144), np.uint8)
        blk[:, 0:2] = d.astype("<u2").view(np.uint8).reshape(supers, 2)
        blk[:, 2:4] = dmin.astype("<u2").view(np.uint8).reshape(supers, 2)
        blk[:, 4:] = rest
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
            w = (1.0 + 0.1 * synth.normal(s, name, h)).astype(np.float32)
            if self.norm_type == T_F16:
                return (name, [h], T_F16, w.astype("<f2").tobytes())
            return (name, [h], T_F32, w.astype("<f4").tobytes())

        def mat(name, rows, cols, ttype):
            return (name, [cols, rows], ttype, payload(ttype, rows, cols, s, name, 1.0 / np.sqrt(cols)))

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
