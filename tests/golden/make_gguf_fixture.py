"""Hand-assembles tests/golden/gguf_v3_spec.gguf byte by byte from the
published GGUF v3 layout (ggml's docs/gguf.md), with struct.pack only: no
code of the product's writer or of either reader is involved, so a mistake
those share (a value-type width, string or array framing, alignment of the
data section, tensor offsets) shows up as a mismatch against the literals in
tests/test_gguf_spec.py.

Layout (all little-endian):
  header   "GGUF", u32 version = 3, u64 tensor_count, u64 metadata_kv_count
  kv       gguf_string key, u32 value_type, value
           gguf_string = u64 byte length + UTF-8 bytes (no terminator)
           array value = u32 element type + u64 count + elements
  tensors  gguf_string name, u32 n_dims, u64 dims[n_dims] (innermost
           first), u32 ggml_type, u64 offset (from the start of the data
           section; a multiple of the alignment)
  padding  zero bytes up to a multiple of general.alignment (default 32)
  data     tensor bytes at their offsets, each padded to the alignment

The file is a valid one-layer-less Qwen3 header (the keys
Qwen3Config::from_gguf reads, src/qwen.cpp:88-149) with three tensors: F32,
F16 and Q8_0.  Run from the repository root:
    python tests/golden/make_gguf_fixture.py
"""
from __future__ import annotations

import struct
import sys
from pathlib import Path

OUT = Path(__file__).resolve().parent / "gguf_v3_spec.gguf"

# GGUF metadata value types (docs/gguf.md, gguf_metadata_value_type)
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
# ggml tensor types used here
GGML_F32, GGML_F16, GGML_Q8_0 = 0, 1, 8
ALIGN = 64

SCALAR_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?",
              U64: "<Q", I64: "<q", F64: "<d"}


def gstr(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def value(t: int, v) -> bytes:
    if t == STRING:
        return gstr(v)
    if t == ARRAY:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(value(et, x) for x in items)
    return struct.pack(SCALAR_FMT[t], v)


# (key, type, value): every value type of the spec appears at least once
KV = [
    ("general.architecture", STRING, "qwen3"),
    ("general.alignment", U32, ALIGN),
    ("qwen3.block_count", U32, 1),
    ("qwen3.embedding_length", U64, 32),
    ("qwen3.feed_forward_length", I32, 64),
    ("qwen3.attention.head_count", U16, 2),
    ("qwen3.attention.head_count_kv", U8, 1),
    ("qwen3.attention.key_length", I64, 16),
    ("qwen3.attention.layer_norm_rms_epsilon", F32, 1e-6),
    ("qwen3.rope.freq_base", F64, 1000000.0),
    ("qwen3.context_length", I16, 512),
    ("test.i8", I8, -5),
    ("test.flag", BOOL, True),
    ("tokenizer.ggml.tokens", ARRAY, (STRING, ["a", "bc", "", "dé"])),
    ("test.u32s", ARRAY, (U32, [1, 2, 3000000000])),
    ("test.nested", ARRAY, (ARRAY, [(I16, [-1, 2]), (I16, [])])),
    ("test.after_arrays", STRING, "end"),
]


def f16_bits(x: float) -> int:
    return struct.unpack("<H", struct.pack("<e", x))[0]


def q8_0_block(scale: float, qs: list[int]) -> bytes:
    """One Q8_0 block: FP16 scale d, then 32 int8 quants (value = d * q)."""
    assert len(qs) == 32
    return struct.pack("<H", f16_bits(scale)) + struct.pack("<32b", *qs)


def tensors():
    """(name, ggml_type, dims innermost first, data bytes)."""
    emb = struct.pack("<128f", *[0.25 * (i - 64) for i in range(128)])                 # F32 (32, 4)
    norm = struct.pack("<32H", *[f16_bits(1.0 + i / 32.0) for i in range(32)])           # F16 (32)
    blocks = b"".join(q8_0_block(0.5 * (r + 1), [((7 * r + 3 * j) % 255) - 127 for j in range(32)])
                      for r in range(4))                                                 # Q8_0 (32, 4)
    return [("token_embd.weight", GGML_F32, [32, 4], emb),
            ("blk.0.attn_norm.weight", GGML_F16, [32], norm),
            ("output.weight", GGML_Q8_0, [32, 4], blocks)]


def assemble(align: int = ALIGN) -> bytes:
    """The fixture; with another `align` (written as general.alignment) the
    same tensors at offsets and a data section rounded to that multiple."""
    def pad(n: int) -> int:
        return (n + align - 1) // align * align

    ts = tensors()
    out = bytearray(b"GGUF" + struct.pack("<IQQ", 3, len(ts), len(KV)))
    for k, t, v in KV:
        out += gstr(k) + struct.pack("<I", t) + value(t, align if k == "general.alignment" else v)
    offsets, off = [], 0
    for _, _, _, data in ts:
        offsets.append(off)
        off = pad(off + len(data))
    for (name, gt, dims, _), o in zip(ts, offsets):
        out += gstr(name) + struct.pack("<I", len(dims)) + struct.pack(f"<{len(dims)}Q", *dims)
        out += struct.pack("<IQ", gt, o)
    out += b"\0" * (pad(len(out)) - len(out))
    data0 = len(out)
    for (_, _, _, data), o in zip(ts, offsets):
        out += b"\0" * (data0 + o - len(out)) + data
    out += b"\0" * (pad(len(out)) - len(out))
    return bytes(out)


def main() -> int:
    OUT.write_bytes(assemble())
    print(f"{OUT}: {OUT.stat().st_size} bytes")
    return 0


if __name__ == "__main__":
    sys.exit(main())
