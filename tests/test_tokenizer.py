"""Qwen3 tokenizer (brolm_amd/csrc/host/tokenizer.cpp, through the C ABI of
libbrolm.so) against the tokenizer oracle (oracle/tokenizer.py), and the
oracle against the reference's own known answers, its compiled BPE core
(oracle/_ref, where the reference sources exist) and HF `tokenizers`.
Host code only: no GPU."""
from __future__ import annotations

import ctypes as C
import json
import random
from pathlib import Path

import pytest

from conftest import ROOT, SMALL, write_synth
from gguf_meta import read_metadata
from oracle import tokenizer as otok

KAT = json.loads((Path(__file__).parent / "golden" / "tokenizer_kat.json").read_text(encoding="utf-8"))
REF_SO = ROOT / "oracle" / "_ref" / "libref_bpe.so"


def _ba():
    from conftest import _ensure_built
    _ensure_built()
    import brolm_amd as ba
    return ba


def _write_files(tmp: Path, vocab_pairs, merges_lines, stem="t"):
    vj = tmp / f"{stem}_vocab.json"
    mt = tmp / f"{stem}_merges.txt"
    vj.write_text("{" + ",".join(json.dumps(t, ensure_ascii=False) + ":" + str(i) for t, i in vocab_pairs) + "}",
                  encoding="utf-8")
    mt.write_text("\n".join(merges_lines) + "\n", encoding="utf-8")
    return vj, mt


@pytest.fixture(scope="module")
def kat_files(tmp_path_factory):
    return _write_files(tmp_path_factory.mktemp("kat"), KAT["vocab"], KAT["merges_txt"])


@pytest.fixture(scope="module")
def synth_vocab(tmp_path_factory):
    """The byte-level BPE vocabulary of a synthetic checkpoint (GGUF metadata)."""
    path = write_synth(tmp_path_factory.mktemp("tok"), SMALL, "small_tok")
    meta = read_metadata(str(path))
    return path, meta["tokenizer.ggml.tokens"], meta["tokenizer.ggml.merges"], meta["tokenizer.ggml.token_type"]


# ------------------------------------------------------------------ oracle pins

@pytest.mark.parametrize("impl", ["oracle", "product"])
def test_reference_known_answers(impl, kat_files):
    """Every known answer of the reference's tokenizer test, for the oracle and
    the product."""
    vj, mt = kat_files
    if impl == "oracle":
        t = otok.Tokenizer.from_files(str(vj), str(mt))
        enc, dec = t.encode, lambda ids: t.decode_bytes(ids).decode()
        counts = (len(t.vocab), len(t.ranks))
        ids = (t.endoftext_id, t.im_start_id, t.im_end_id, t.im_end_id)
    else:
        t = _ba().Tokenizer.load(str(vj), str(mt))
        enc, dec = t.encode, t.decode
        counts = (t.vocab_count(), t.merge_count())
        ids = (t.endoftext_id(), t.im_start_id(), t.im_end_id(), t.eos_id())
    assert counts == (KAT["counts"]["vocab"], KAT["counts"]["merges"])
    assert ids == tuple(KAT["ids"][k] for k in ("endoftext", "im_start", "im_end", "eos"))
    for text, add_special, want in KAT["encode"]:
        assert enc(text, add_special) == want, text
    for text in KAT["round_trip"]:
        assert dec(enc(text)) == text
    if impl == "product":
        chat = KAT["chat"]
        prompt = t.apply_chat_template([tuple(m) for m in chat["messages"]], True)
        assert prompt == chat["prompt"]
        assert enc(prompt)[0] == chat["first_id"] and dec(enc(prompt)) == prompt


def _ref_lib():
    if not REF_SO.exists():
        pytest.skip("oracle/_ref/libref_bpe.so not built (reference sources absent)")
    lib = C.CDLL(str(REF_SO))
    lib.ref_bpe_encode_piece.restype = C.c_int
    lib.ref_bpe_encode_piece.argtypes = [C.c_char_p, C.c_char_p, C.c_char_p, C.c_long, C.POINTER(C.c_int), C.c_int]
    lib.ref_bpe_special_match.restype = C.c_int
    lib.ref_bpe_special_match.argtypes = [C.c_char_p, C.c_char_p, C.c_long, C.c_long, C.POINTER(C.c_long),
                                          C.POINTER(C.c_int)]
    return lib


def _random_texts(rng: random.Random, n: int, words: list[str], specials=()) -> list[bytes]:
    pool_ascii = [chr(c) for c in range(32, 127)] + ["\n", "\t", "\r", "\x0b", "\x0c"]
    out = []
    for _ in range(n):
        parts = []
        for _ in range(rng.randint(0, 14)):
            r = rng.random()
            if r < 0.45:
                parts.append(rng.choice(words))
            elif r < 0.6:
                parts.append(" " * rng.randint(1, 3))
            elif r < 0.75:
                parts.append("".join(rng.choice(pool_ascii) for _ in range(rng.randint(1, 5))))
            elif r < 0.82:
                parts.append(rng.choice(["'s", "'t", "'re", "'ve", "'m", "'ll", "'d", "'", "''", "'x"]))
            elif r < 0.9:
                parts.append(rng.choice(["é", "ß", "日本", "😀", " ", "–"]))
            elif r < 0.95 and specials:
                parts.append(rng.choice(specials))
            else:
                parts.append(str(rng.randint(0, 99999)))
        s = "".join(parts).encode()
        if rng.random() < 0.1:   # raw bytes, not UTF-8
            s += bytes(rng.randint(128, 255) for _ in range(rng.randint(1, 4)))
        out.append(s)
    return out


def test_oracle_merge_loop_matches_reference_build(tmp_path, synth_vocab):
    """oracle piece encoding (byte alphabet, merge loop, vocab lookup) equals
    the reference's compiled encode_piece on every piece of random texts."""
    lib = _ref_lib()
    _, tokens, merges, types = synth_vocab
    vj, mt = _write_files(tmp_path, [(t, i) for i, t in enumerate(tokens)], merges)
    orc = otok.Tokenizer.from_lists(tokens, merges, types)
    words = [t.lstrip("Ġ") for t in tokens[256:600] if t.isascii() and t.strip("Ġ").isalpha()]
    buf = (C.c_int * 4096)()
    n_pieces = 0
    for text in _random_texts(random.Random(5), 400, words):
        for piece in otok.pre_tokenize(text):
            k = lib.ref_bpe_encode_piece(str(vj).encode(), str(mt).encode(), piece, len(piece), buf, 4096)
            assert k >= 0
            got = []
            orc._piece(piece, got)
            assert got == list(buf[:k]), piece
            n_pieces += 1
    assert n_pieces > 1000


def test_oracle_special_match_matches_reference_build():
    lib = _ref_lib()
    specials = ["<|a|>", "<|a|>b", "<|ab|>", "<", "xyz", "<|endoftext|>"]
    o = otok.Tokenizer()
    for i, s in enumerate(specials):
        o.add_special(s, i)
    rng = random.Random(3)
    ln, sid = C.c_long(), C.c_int()
    for _ in range(2000):
        text = "".join(rng.choice(["<|a|>", "b", "<|ab|>", "<", "|", "xyz", "x", "<|endoftext|>"])
                       for _ in range(rng.randint(1, 6))).encode()
        pos = rng.randrange(len(text))
        assert lib.ref_bpe_special_match("\n".join(specials).encode(), text, len(text), pos, C.byref(ln),
                                         C.byref(sid)) == 0
        assert o._match(text, pos) == (ln.value, sid.value if ln.value else -1)


def test_oracle_matches_hf_tokenizers_where_pre_tokenizers_agree(synth_vocab):
    """On texts of letter / digit / punctuation runs separated by single
    spaces (where GPT-2's pre-tokenizer regex and the reference's ASCII rules
    split alike), the oracle's ids equal HF tokenizers' byte-level BPE."""
    hf_mod = pytest.importorskip("tokenizers")
    _, tokens, merges, types = synth_vocab
    vocab = {}
    for i, t in enumerate(tokens):
        vocab.setdefault(t, i)
    hf = hf_mod.Tokenizer(hf_mod.models.BPE(vocab=vocab, merges=[tuple(m.split(" ", 1)) for m in merges]))
    hf.pre_tokenizer = hf_mod.pre_tokenizers.ByteLevel(add_prefix_space=False, use_regex=True)
    orc = otok.Tokenizer.from_lists(tokens, merges, types)
    words = [t.lstrip("Ġ") for t in tokens[256:700] if t.isascii() and t.strip("Ġ").isalpha()]
    rng = random.Random(11)
    for _ in range(500):
        parts = []
        for _ in range(rng.randint(1, 12)):
            r = rng.random()
            if r < 0.6:
                parts.append(rng.choice(words) + rng.choice(["", "", rng.choice(words)]))
            elif r < 0.8:
                parts.append(str(rng.randint(0, 10 ** rng.randint(1, 6))))
            else:
                parts.append("".join(rng.choice(".,;:!?()-+=*/#%&") for _ in range(rng.randint(1, 3))))
        text = " ".join(parts)
        assert orc.encode(text) == hf.encode(text).ids, text


# ------------------------------------------------------------------ product vs oracle

def test_product_from_gguf_matches_oracle(synth_vocab):
    path, tokens, merges, types = synth_vocab
    ba = _ba()
    tok = ba.Tokenizer.from_gguf(str(path))
    orc = otok.Tokenizer.from_lists(tokens, merges, types)
    assert tok.vocab_count() == len(orc.vocab) and tok.merge_count() == len(orc.ranks)
    assert (tok.endoftext_id(), tok.im_start_id(), tok.im_end_id()) == (orc.endoftext_id, orc.im_start_id,
                                                                         orc.im_end_id)
    words = [t.lstrip("Ġ") for t in tokens[256:700] if t.isascii() and t.strip("Ġ").isalpha()]
    specials = ["<|endoftext|>", "<|im_start|>", "<|im_end|>"]
    for text in _random_texts(random.Random(1), 600, words, specials) + [b"", b" ", b"  ", b"'", b"''s"]:
        ids = tok.encode(text)
        assert ids == orc.encode(text), text
        assert tok.decode_bytes(ids) == text          # every byte has its own token
        assert ids + [orc.endoftext_id] == tok.encode(text, add_special=True)
        assert tok.decode_bytes(ids) == orc.decode_bytes(ids)


def test_loaders_agree(tmp_path, synth_vocab):
    """vocab.json + merges.txt, tokenizer.json (string and pair merges,
    added_tokens) and GGUF give the same tokenizer."""
    path, tokens, merges, types = synth_vocab
    ba = _ba()
    vj, mt = _write_files(tmp_path, [(t, i) for i, t in enumerate(tokens)], ["#version: 0.2"] + merges)
    specials = [i for i, ty in enumerate(types) if ty == 3]
    model_vocab = {t: i for i, t in enumerate(tokens) if i not in specials}
    added = [{"id": i, "content": tokens[i], "special": True} for i in specials]
    tj1 = tmp_path / "tok1.json"
    tj1.write_text(json.dumps({"model": {"type": "BPE", "vocab": model_vocab, "merges": merges},
                               "added_tokens": added}, ensure_ascii=False), encoding="utf-8")
    tj2 = tmp_path / "tok2.json"
    tj2.write_text(json.dumps({"model": {"type": "BPE", "vocab": model_vocab,
                                         "merges": [m.split(" ", 1) for m in merges]},
                               "added_tokens": added}, ensure_ascii=False), encoding="utf-8")
    toks = [ba.Tokenizer.from_gguf(str(path)), ba.Tokenizer.load(str(vj), str(mt)),
            ba.Tokenizer.from_tokenizer_json(str(tj1)), ba.Tokenizer.from_tokenizer_json(str(tj2))]
    words = [t.lstrip("Ġ") for t in tokens[256:700] if t.isascii() and t.strip("Ġ").isalpha()]
    for text in _random_texts(random.Random(2), 200, words, ["<|im_start|>", "<|im_end|>"]):
        first = toks[0].encode(text)
        for t in toks[1:]:
            assert t.encode(text) == first, text
    for t in toks:
        assert (t.vocab_count(), t.merge_count(), t.eos_id()) == (toks[0].vocab_count(), toks[0].merge_count(),
                                                                  toks[0].eos_id())


def test_specials_and_edges(kat_files):
    ba = _ba()
    vj, mt = kat_files
    t = ba.Tokenizer.load(str(vj), str(mt), extra_special_tokens=["hi"])
    assert t.encode("chi") == [ord("c"), 300]          # "hi" now atomic, matched inside a word
    t.register_special_token("<|x|>", 300)              # a second name for id 300
    assert t.decode([300]) == "<|x|>"
    assert t.encode("<|x|>hi") == [300, 300]
    t.register_special_token("<|im_end|>", 77)          # re-bind: eos follows
    assert t.eos_id() == 77 and t.encode("<|im_end|>") == [77]
    assert t.decode([12345, 99999]) == ""               # unknown ids are skipped
    assert t.encode("") == [] and t.decode([]) == ""
    o = otok.Tokenizer.from_files(str(vj), str(mt), extra=["hi"])
    assert o.encode("chi") == [ord("c"), 300]


def test_loader_errors(tmp_path):
    ba = _ba()
    from brolm_amd._native import NativeError
    bad = tmp_path / "bad_merges.txt"
    bad.write_text("#v\nab\n")
    vj, _ = _write_files(tmp_path, KAT["vocab"], KAT["merges_txt"])
    with pytest.raises(NativeError, match="malformed"):
        ba.Tokenizer.load(str(vj), str(bad))
    with pytest.raises(NativeError, match="cannot open"):
        ba.Tokenizer.load(str(tmp_path / "missing.json"), str(bad))
    nj = tmp_path / "notbpe.json"
    nj.write_text('{"model": {"vocab": [1, 2]}}')
    with pytest.raises(NativeError, match="not an object"):
        ba.Tokenizer.from_tokenizer_json(str(nj))
