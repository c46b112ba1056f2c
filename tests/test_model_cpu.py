"""Model-level exports on the CPU: the synthetic GGUF files are accepted by the
reference's own C ABI (oracle/_ref, core/src/c_api.cpp), and malformed files
are rejected by this library with the reference's messages.  Every rejection
here happens while the file is parsed, before this library touches the GPU
(tvara_model_open: gguf.hpp:43-209, gguf_model.hpp:46-108, model.hpp:140-155).
"""

import struct

import numpy as np
import pytest

from tvara_amd import gguf_writer as gf
from tvara_amd import native

@pytest.fixture(scope="module")
def ref_capi():
    from pathlib import Path

    p = Path(__file__).resolve().parents[1] / "oracle" / "_ref" / "libtvara_ref_capi.so"
    if not p.exists():
        pytest.skip("reference C ABI not built (make -C oracle ref)")
    return str(p)


def opened_error(path, library=None, **kw):
    try:
        m = native.NativeModel(path, library=library, **kw)
    except RuntimeError as e:
        return str(e)
    m.close()
    return None


@pytest.mark.parametrize("mtype", [gf.T_F32, gf.T_F16, gf.T_Q8_0, gf.T_Q4_0])
def test_reference_accepts_fixtures(tmp_path, ref_capi, mtype):
    spec = gf.LlamaSpec(matrix_type=mtype, embed_type=gf.T_F16 if mtype == gf.T_F16 else gf.T_F32)
    m = native.NativeModel(spec.write(tmp_path / "m.gguf"), library=ref_capi)
    assert (m.vocab_size, m.context_size) == (spec.vocab, spec.context)
    s = m.new_sequence()
    out = m.decode_batch(s, [1, 2, 3])
    assert out.shape == (3, spec.vocab) and np.isfinite(out).all()
    md = m.metadata
    assert md["llama.block_count"] == spec.layers and md["tokenizer.ggml.tokens"][5] == "t5"
    m.close()


def test_reference_accepts_q4_k(tmp_path, ref_capi):
    spec = gf.LlamaSpec(matrix_type=gf.T_Q4_K, hidden=256, intermediate=512)
    m = native.NativeModel(spec.write(tmp_path / "k.gguf"), library=ref_capi)
    assert np.isfinite(m.logits(m.new_sequence(), 3)).all()


def _meta_file(tmp_path, name, replace=None, drop=(), extra=()):
    spec = gf.LlamaSpec()
    meta = [(k, t, v) for k, t, v in spec.metadata() if k not in drop]
    if replace:
        meta = [(k, *replace[k]) if k in replace else (k, t, v) for k, t, v in meta]
    meta += list(extra)
    path = tmp_path / name
    gf.write_gguf(path, meta, spec.tensors())
    return path


def _raw(tmp_path, name, data):
    path = tmp_path / name
    path.write_bytes(data)
    return path


def _tensor_file(tmp_path, name, edit, alignment=32):
    spec = gf.LlamaSpec()
    tensors = edit(spec.tensors())
    path = tmp_path / name
    gf.write_gguf(path, spec.metadata(), tensors, alignment=alignment)
    return path


def malformed(tmp_path):
    """(label, path) of files that tvara_model_open must reject."""
    good = gf.LlamaSpec()
    cases = []
    hdr = b"GGUF" + struct.pack("<IQQ", 3, 0, 0)
    cases += [
        ("bad magic", _raw(tmp_path, "a", b"GGUX" + b"\0" * 60)),
        ("version 1", _raw(tmp_path, "b", b"GGUF" + struct.pack("<IQQ", 1, 0, 0) + b"\0" * 40)),
        ("truncated header", _raw(tmp_path, "c", b"GGUF" + struct.pack("<I", 3))),
        ("count limit", _raw(tmp_path, "d", b"GGUF" + struct.pack("<IQQ", 3, 2000000, 0) + b"\0" * 64)),
        ("counts exceed bytes", _raw(tmp_path, "e", b"GGUF" + struct.pack("<IQQ", 3, 10, 0) + b"\0" * 64)),
        ("no metadata", _raw(tmp_path, "f", hdr + b"\0" * 64)),
    ]

    def kv(key, vtype, payload):
        return gf._str(key) + struct.pack("<I", vtype) + payload

    def doc(*kvs):
        return b"GGUF" + struct.pack("<IQQ", 3, 0, len(kvs)) + b"".join(kvs) + b"\0" * 64

    cases += [
        ("invalid bool", _raw(tmp_path, "g", doc(kv("x", gf.BOOL, b"\x02")))),
        ("unsupported scalar", _raw(tmp_path, "h", doc(kv("x", 13, b"\0" * 8)))),
        ("empty key", _raw(tmp_path, "i", doc(kv("", gf.U32, b"\1\0\0\0")))),
        ("duplicate key", _raw(tmp_path, "j", doc(kv("x", gf.U32, b"\1\0\0\0"), kv("x", gf.U32, b"\1\0\0\0")))),
        ("array of arrays", _raw(tmp_path, "k", doc(kv("x", gf.ARR, struct.pack("<IQ", gf.ARR, 1))))),
        ("oversized string", _raw(tmp_path, "l", doc(kv("x", gf.STR, struct.pack("<Q", 1 << 30))))),
        ("string past end", _raw(tmp_path, "m", doc(kv("x", gf.STR, struct.pack("<Q", 500))))),
    ]
    cases += [
        ("architecture", _meta_file(tmp_path, "n", replace={"general.architecture": (gf.STR, "gpt2")})),
        ("architecture type", _meta_file(tmp_path, "o", replace={"general.architecture": (gf.U32, 1)})),
        ("no architecture", _meta_file(tmp_path, "p", drop=("general.architecture",))),
        ("no vocabulary", _meta_file(tmp_path, "q", drop=("tokenizer.ggml.tokens",))),
        ("empty vocabulary", _meta_file(tmp_path, "r", replace={"tokenizer.ggml.tokens": (gf.ARR, (gf.STR, []))})),
        ("signed dimension", _meta_file(tmp_path, "s", replace={"llama.block_count": (gf.I32, 2)})),
        ("zero dimension", _meta_file(tmp_path, "t", replace={"llama.context_length": (gf.U32, 0)})),
        ("huge dimension", _meta_file(tmp_path, "u", replace={"llama.context_length": (gf.U64, 2000000)})),
        ("no context", _meta_file(tmp_path, "v", drop=("llama.context_length",))),
        ("negative epsilon", _meta_file(tmp_path, "w",
                                        replace={"llama.attention.layer_norm_rms_epsilon": (gf.F32, -1.0)})),
        ("integer theta", _meta_file(tmp_path, "x", replace={"llama.rope.freq_base": (gf.U32, 10000)})),
        ("epsilon underflows float", _meta_file(tmp_path, "y",
                                                replace={"llama.attention.layer_norm_rms_epsilon": (gf.F64, 1e-60)})),
        ("head layout", _meta_file(tmp_path, "z", replace={"llama.attention.head_count_kv": (gf.U32, 3)})),
        ("scaled rope", _meta_file(tmp_path, "aa", extra=[("llama.rope.scaling.type", gf.STR, "linear")])),
        ("rope layout", _meta_file(tmp_path, "ab", extra=[("tvara.rope.layout", gf.STR, "sideways")])),
        ("rope layout type", _meta_file(tmp_path, "ac", extra=[("tvara.rope.layout", gf.U32, 1)])),
        ("alignment not a power of two", _meta_file(tmp_path, "ad", extra=[("general.alignment", gf.U32, 24)])),
        ("alignment type", _meta_file(tmp_path, "ae", extra=[("general.alignment", gf.I32, 32)])),
    ]

    def drop_tensor(name):
        return lambda ts: [t for t in ts if t[0] != name]

    def reshape(name, dims):
        return lambda ts: [(n, dims if n == name else d, ty, p) for n, d, ty, p in ts]

    def retype(name, ttype):
        return lambda ts: [(n, d, ttype if n == name else ty, p) for n, d, ty, p in ts]

    def dup(ts):
        return ts + [ts[0]]

    def grow_last(ts):  # the last tensor claims 64 times its payload
        return [(n, [d[0] * 64] + d[1:] if n == ts[-1][0] else d, ty, p) for n, d, ty, p in ts]

    cases += [
        ("missing tensor", _tensor_file(tmp_path, "af", drop_tensor("blk.1.ffn_down.weight"))),
        ("malformed tensor", _tensor_file(tmp_path, "ag", reshape("blk.0.attn_k.weight", [64, 64]))),
        ("duplicate tensor", _tensor_file(tmp_path, "ah", dup)),
        ("unsupported storage", _tensor_file(tmp_path, "ai", retype("blk.0.attn_q.weight", 3))),
        ("quantized row width", _tensor_file(tmp_path, "aj", retype("blk.0.attn_q.weight", gf.T_Q4_K))),
        ("payload past end", _tensor_file(tmp_path, "ak", grow_last)),
    ]
    # unaligned offset and overlapping payloads: patch the offset of the first tensor
    path = tmp_path / "al"
    gf.write_gguf(path, good.metadata(), good.tensors())
    data = bytearray(path.read_bytes())
    name = gf._str("token_embd.weight")
    at = data.index(name) + len(name) + 4 + 8 * 2 + 4
    struct.pack_into("<Q", data, at, 8)
    cases.append(("unaligned offset", _raw(tmp_path, "al2", bytes(data))))
    second = gf._str("output_norm.weight")
    at2 = data.index(second) + len(second) + 4 + 8 + 4
    struct.pack_into("<Q", data, at, 0)
    struct.pack_into("<Q", data, at2, 0)
    cases.append(("overlapping payloads", _raw(tmp_path, "al3", bytes(data))))
    cases.append(("missing file", tmp_path / "does-not-exist.gguf"))
    return cases


def test_rejections_match_reference(tmp_path, ref_capi):
    cases = malformed(tmp_path)
    mismatches = []
    for label, path in cases:
        mine = opened_error(path)
        ref = opened_error(path, ref_capi)
        assert ref is not None, f"{label}: the reference accepted it"
        if mine != ref:
            mismatches.append((label, mine, ref))
    assert not mismatches, mismatches


def test_empty_path_and_null_handles():
    lib = native._capi.lib()
    assert not lib.tvara_model_open(b"", 8, 16)
    assert lib.tvara_last_error() == b"empty model path"
    assert lib.tvara_model_vocab_size(None) == 0 and lib.tvara_last_error() == b"closed model"
    assert lib.tvara_model_context_size(None) == 0
    assert lib.tvara_model_metadata(None) is None and lib.tvara_last_error() == b"closed model"
    assert lib.tvara_sequence_create(None) == 0 and lib.tvara_last_error() == b"closed model"
    assert lib.tvara_sequence_drop(None, 1) == -1
    assert lib.tvara_sequence_truncate(None, 1, 0) == -1
    assert lib.tvara_sequence_decode(None, 1, 0, None, 0) == -1
    assert lib.tvara_last_error() == b"invalid logit output buffer"
    assert lib.tvara_sequence_decode_batch(None, 1, None, 0, None, 0) == -1
    assert lib.tvara_last_error() == b"invalid batch buffers"
    lib.tvara_model_close(None)
