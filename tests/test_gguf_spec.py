"""GGUF v3 container against a file hand-assembled from the published spec
(tests/golden/make_gguf_fixture.py, struct.pack only), read by both the
oracle's reader and the product's (gguf::File through the C ABI), plus
malformed variants of it that both must refuse without reading out of
bounds.  The expected values below are literals from the spec layout, not
recomputed by either reader."""
from __future__ import annotations

import ctypes as C
import struct
import sys
from pathlib import Path

import numpy as np
import pytest

import oracle

GOLD = Path(__file__).resolve().parent / "golden"
FIX = GOLD / "gguf_v3_spec.gguf"
SIZE, DATA0 = 1728, 960
# (name, ggml type, dims, offset in the data section, nbytes)
TENSORS = [("token_embd.weight", 0, [32, 4], 0, 512),
           ("blk.0.attn_norm.weight", 1, [32], 512, 64),
           ("output.weight", 8, [32, 4], 576, 136)]


@pytest.fixture(scope="module")
def raw() -> bytes:
    return FIX.read_bytes()


@pytest.fixture(scope="module")
def lib():
    from brolm_amd import _native
    return _native.lib()


def test_fixture_is_the_script_output(raw):
    sys.path.insert(0, str(GOLD))
    import make_gguf_fixture
    assert make_gguf_fixture.assemble() == raw


def test_layout_literals(raw):
    assert len(raw) == SIZE
    assert raw[:4] == b"GGUF" and struct.unpack_from("<IQQ", raw, 4) == (3, 3, 17)
    # first key: u64 length 20, "general.architecture", type 8 (string), "qwen3"
    assert struct.unpack_from("<Q", raw, 24)[0] == 20 and raw[32:52] == b"general.architecture"
    assert struct.unpack_from("<IQ", raw, 52) == (8, 5) and raw[64:69] == b"qwen3"
    # the data section starts on the 64-byte alignment, zero padded before it
    assert raw[DATA0:DATA0 + 4] == struct.pack("<f", -16.0)
    assert raw[DATA0 - 8:DATA0] == bytes(8)


def test_oracle_reader(raw):
    g = oracle.Gguf(str(FIX))
    assert g.tensor_names() == [t[0] for t in TENSORS]
    for name, gt, dims, off, nb in TENSORS:
        t, d, data = g.tensor(name)
        assert (t, d, data.size) == (gt, dims, nb)
        assert data.tobytes() == raw[DATA0 + off:DATA0 + off + nb]
    ints = {"general.alignment": 64, "qwen3.block_count": 1, "qwen3.embedding_length": 32,
            "qwen3.feed_forward_length": 64, "qwen3.attention.head_count": 2, "qwen3.attention.head_count_kv": 1,
            "qwen3.attention.key_length": 16, "qwen3.context_length": 512, "test.i8": -5, "test.flag": 1}
    for k, v in ints.items():
        assert g.meta_int(k) == v, k
    assert g.meta_f64("qwen3.attention.layer_norm_rms_epsilon") == pytest.approx(1e-6, rel=1e-7)
    assert g.meta_f64("qwen3.rope.freq_base") == 1e6
    assert g.meta_str("general.architecture") == "qwen3"
    # read only if the nested array before it was stepped over exactly
    assert g.meta_str("test.after_arrays") == "end"
    n = C.c_int64()
    for key, count in (("tokenizer.ggml.tokens", 4), ("test.u32s", 3), ("test.nested", 2)):
        assert oracle.lib().or_gguf_meta_array_len(C.c_void_p(g._h), key.encode(), C.byref(n)) == 0
        assert n.value == count


def test_product_reader(raw, lib):
    p = str(FIX).encode()
    n = C.c_int64()
    assert lib.brolm_gguf_tensor_count(p, C.byref(n)) == 0 and n.value == 3
    for name, gt, dims, off, nb in TENSORS:
        t, nd, nbytes = C.c_int(), C.c_int(), C.c_int64()
        d4 = (C.c_int64 * 4)()
        assert lib.brolm_gguf_tensor_info(p, name.encode(), C.byref(t), d4, C.byref(nd), C.byref(nbytes)) == 0
        assert (t.value, list(d4)[:nd.value], nbytes.value) == (gt, dims, nb)
        buf = (C.c_uint8 * nb)()
        assert lib.brolm_gguf_tensor_data(p, name.encode(), buf, nb) == nb
        assert bytes(buf) == raw[DATA0 + off:DATA0 + off + nb]
    v = C.c_int64()
    for k, want in (("qwen3.embedding_length", 32), ("qwen3.feed_forward_length", 64),
                    ("qwen3.attention.head_count", 2), ("qwen3.attention.head_count_kv", 1),
                    ("qwen3.attention.key_length", 16), ("qwen3.context_length", 512), ("test.i8", -5),
                    ("test.flag", 1), ("general.alignment", 64)):
        assert lib.brolm_gguf_meta_int(p, k.encode(), C.byref(v)) == 0 and v.value == want, k
    f = C.c_double()
    assert lib.brolm_gguf_meta_f64(p, b"qwen3.rope.freq_base", C.byref(f)) == 0 and f.value == 1e6
    s = C.create_string_buffer(16)
    assert lib.brolm_gguf_meta_str(p, b"test.after_arrays", s, 16) == 3 and s.raw[:3] == b"end"
    et, cnt = C.c_int(), C.c_int64()
    for key, t, count in (("tokenizer.ggml.tokens", 8, 4), ("test.u32s", 4, 3), ("test.nested", 9, 2)):
        assert lib.brolm_gguf_meta_array(p, key.encode(), C.byref(et), C.byref(cnt)) == 0
        assert (et.value, cnt.value) == (t, count)


def test_qwen3_config_and_dequant_from_spec_file():
    import brolm_amd as ba
    c = ba.Qwen3Config.from_gguf(str(FIX))
    assert (c.hidden_size, c.intermediate_size, c.num_hidden_layers, c.num_attention_heads,
            c.num_key_value_heads, c.head_dim, c.max_position_embeddings, c.vocab_size) == (32, 64, 1, 2, 1, 16, 512, 4)
    assert c.rms_norm_eps == pytest.approx(1e-6) and c.rope_theta == 1e6
    assert c.tie_word_embeddings is False   # no tie key, output.weight present
    g = oracle.Gguf(str(FIX))
    t, _, data = g.tensor("output.weight")
    w = oracle.dequant(t, data, 128)
    # row 2 (scale 1.5), element 5: q = (7*2 + 3*5) % 255 - 127 = -98; row 0, element 0: q = -127
    assert w[2 * 32 + 5] == -147.0 and w[0] == -63.5
    t, _, data = g.tensor("blk.0.attn_norm.weight")
    assert oracle.dequant(t, data, 32)[31] == 1.96875


def test_alignment_24_read_by_both():
    """general.alignment 24: a multiple of 8 (all the spec asks) and no power
    of two.  The same tensors, assembled at offsets 0, 528, 600 of a data
    section starting at 912 (the 911-byte header rounded up to 24), read back
    by both readers."""
    sys.path.insert(0, str(GOLD))
    import make_gguf_fixture
    b = make_gguf_fixture.assemble(align=24)
    data0 = 912
    offsets = [0, 528, 600]
    assert b[data0:data0 + 4] == struct.pack("<f", -16.0)
    from brolm_amd import _native
    lib = _native.lib()
    assert _product_ok(lib, b) and _oracle_ok(b)
    buf = C.create_string_buffer(b, len(b))
    h = oracle.lib().or_gguf_open_memory(C.cast(buf, C.c_void_p), len(b))
    assert h
    try:
        for (name, gt, dims, _, nb), off in zip(TENSORS, offsets):
            i = oracle.lib().or_gguf_find_tensor(C.c_void_p(h), name.encode())
            assert i >= 0 and oracle.lib().or_gguf_tensor_nbytes(C.c_void_p(h), i) == nb
            p = oracle.lib().or_gguf_tensor_data(C.c_void_p(h), i)
            assert C.string_at(p, nb) == b[data0 + off:data0 + off + nb], name
    finally:
        oracle.lib().or_gguf_close(C.c_void_p(h))
    import tempfile
    with tempfile.NamedTemporaryFile(suffix=".gguf") as f:
        f.write(b)
        f.flush()
        for (name, gt, dims, _, nb), off in zip(TENSORS, offsets):
            out = (C.c_uint8 * nb)()
            assert lib.brolm_gguf_tensor_data(f.name.encode(), name.encode(), out, nb) == nb
            assert bytes(out) == b[data0 + off:data0 + off + nb], name


# ----------------------------------------------------------------- malformed variants

def _product_ok(lib, b: bytes) -> bool:
    n = C.c_int64()
    arr = (C.c_uint8 * max(len(b), 1)).from_buffer_copy(b if b else b"\0")
    return lib.brolm_gguf_parse_memory(arr, len(b), C.byref(n)) == 0


def _oracle_ok(b: bytes) -> bool:
    buf = C.create_string_buffer(b, max(len(b), 1))
    h = oracle.lib().or_gguf_open_memory(C.cast(buf, C.c_void_p), len(b))
    if h:
        oracle.lib().or_gguf_close(C.c_void_p(h))
    return bool(h)


def _field(raw: bytes, name: str) -> int:
    """Byte position just after the gguf_string `name` in the tensor infos."""
    key = struct.pack("<Q", len(name)) + name.encode()
    pos = raw.index(key, 400)   # past the metadata
    return pos + len(key)


def test_truncations_are_refused(raw, lib):
    assert _product_ok(lib, raw) and _oracle_ok(raw)
    # the last tensor ends at DATA0 + 576 + 136: the tail padding is optional
    end = DATA0 + 576 + 136
    assert _product_ok(lib, raw[:end]) and _oracle_ok(raw[:end])
    for n in list(range(0, DATA0, 5)) + [DATA0, DATA0 + 100, end - 1]:
        assert not _product_ok(lib, raw[:n]), n
        assert not _oracle_ok(raw[:n]), n


def _patched(raw: bytes, pos: int, fmt: str, value) -> bytes:
    b = bytearray(raw)
    struct.pack_into(fmt, b, pos, value)
    return bytes(b)


@pytest.mark.parametrize("case", ["misaligned_offset", "offset_past_end", "offset_wraps", "dim_overflow",
                                  "zero_dim", "array_count_huge", "alignment_zero", "alignment_not_mult8",
                                  "alignment_huge",
                                  "version_2", "bad_magic", "unknown_value_type", "too_many_dims"])
def test_malformed_headers_are_refused(raw, lib, case):
    out_pos = _field(raw, "output.weight")          # u32 n_dims, u64 dims[2], u32 type, u64 offset
    emb_pos = _field(raw, "token_embd.weight")
    align_pos = raw.index(b"general.alignment") + len(b"general.alignment") + 4
    arr_pos = raw.index(b"test.u32s") + len(b"test.u32s") + 8   # past type + element type
    key_pos = raw.index(b"test.i8") + len(b"test.i8")
    b = {
        "misaligned_offset": lambda: _patched(raw, out_pos + 4 + 16 + 4, "<Q", 577),
        "offset_past_end": lambda: _patched(raw, out_pos + 4 + 16 + 4, "<Q", 1 << 20),
        "offset_wraps": lambda: _patched(raw, out_pos + 4 + 16 + 4, "<Q", (1 << 64) - 64),
        "dim_overflow": lambda: _patched(_patched(raw, emb_pos + 4, "<Q", 1 << 62), emb_pos + 12, "<Q", 1 << 62),
        "zero_dim": lambda: _patched(raw, emb_pos + 12, "<Q", 0),
        "array_count_huge": lambda: _patched(raw, arr_pos, "<Q", 1 << 60),
        "alignment_zero": lambda: _patched(raw, align_pos, "<I", 0),
        "alignment_not_mult8": lambda: _patched(raw, align_pos, "<I", 4),   # divides every offset
        "alignment_huge": lambda: _patched(raw, align_pos, "<I", 1 << 21),
        "version_2": lambda: _patched(raw, 4, "<I", 2),
        "bad_magic": lambda: b"GGUG" + raw[4:],
        "unknown_value_type": lambda: _patched(raw, key_pos, "<I", 13),
        "too_many_dims": lambda: _patched(raw, emb_pos, "<I", 5),
    }[case]()
    assert b != raw
    assert not _product_ok(lib, b)
    assert not _oracle_ok(b)
