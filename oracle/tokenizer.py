"""CPU oracle of the Qwen3 byte-level BPE tokenizer: a plain-Python
restatement of the reference's algorithm, TEST INFRASTRUCTURE ONLY (the
product tokenizer is brolm_amd/csrc/host/tokenizer.cpp; nothing in the product
imports this module).

Follows reference src/qwen_tokenizer.cpp (pre-tokenization :38-111, loaders
:122-390, encode / decode :392-459) and src/detail/byte_level_bpe.cpp (byte
alphabet :60-105, merges.txt :225-251, merge loop :255-304, encode_piece
:306-328, special-token longest match :451-468).

Pinned by: the reference's own known-answer fixture (tests/test_qwen_tokenizer.cpp,
committed as tests/golden/tokenizer_kat.json), HF `tokenizers` byte-level BPE on
texts where GPT-2's pre-tokenizer regex and the reference's ASCII rules split
alike, the reference's compiled merge loop (oracle/_ref, built from
src/detail/byte_level_bpe.cpp where /root/reference exists), and round trips.
"""
from __future__ import annotations

import json

SPECIAL_NAMES = ("<|endoftext|>", "<|im_start|>", "<|im_end|>")
_CONTRACTIONS = ("'re", "'ve", "'ll", "'s", "'t", "'m", "'d")


def byte_alphabet() -> list[str]:
    """GPT-2 byte -> unicode: printable bytes map to themselves, the others to
    U+0100.. in byte order (byte_level_bpe.cpp:60-89)."""
    out, nxt = [], 256
    for b in range(256):
        if 33 <= b <= 126 or 161 <= b <= 172 or 174 <= b <= 255:
            out.append(chr(b))
        else:
            out.append(chr(nxt))
            nxt += 1
    return out


def _letter(c: int) -> bool:
    return 65 <= c <= 90 or 97 <= c <= 122


def _digit(c: int) -> bool:
    return 48 <= c <= 57


def _space(c: int) -> bool:
    return c in (32, 9, 10, 13, 12, 11)


def _contraction(t: bytes, i: int) -> int:
    for c in _CONTRACTIONS:
        if t.startswith(c.encode(), i):
            return len(c)
    return 0


def pre_tokenize(t: bytes) -> list[bytes]:
    """qwen_tokenizer.cpp:38-111 on raw bytes."""
    out, i, n = [], 0, len(t)
    while i < n:
        c = t[i]
        if c == 0x27:
            k = _contraction(t, i)
            if k:
                out.append(t[i:i + k])
                i += k
                continue
        start = i
        if c == 32:
            if i + 1 < n and not _space(t[i + 1]):
                i += 1
                c = t[i]
            else:
                out.append(t[i:i + 1])
                i += 1
                continue
        elif _space(c):
            j = i
            while j < n and _space(t[j]) and t[j] != 32:
                j += 1
            out.append(t[i:j])
            i = j
            continue
        j = i
        if _letter(c):
            while j < n and _letter(t[j]):
                j += 1
        elif _digit(c):
            while j < n and _digit(t[j]):
                j += 1
        else:
            while j < n:
                u = t[j]
                if _space(u) or _letter(u) or _digit(u):
                    break
                if u == 0x27 and j != i and _contraction(t, j):
                    break
                j += 1
        out.append(t[start:j])
        i = j
    return out


def bpe_merge(units: list[str], ranks: dict[tuple[str, str], int]) -> list[str]:
    """Lowest-rank adjacent pair, all its non-overlapping occurrences per pass
    (byte_level_bpe.cpp:255-304)."""
    w = list(units)
    while len(w) > 1:
        best = None
        for a, b in zip(w, w[1:]):
            r = ranks.get((a, b))
            if r is not None and (best is None or r < best[0]):
                best = (r, a, b)
        if best is None:
            break
        _, a, b = best
        nw, k = [], 0
        while k < len(w):
            if k + 1 < len(w) and w[k] == a and w[k + 1] == b:
                nw.append(a + b)
                k += 2
            else:
                nw.append(w[k])
                k += 1
        w = nw
    return w


class Tokenizer:
    def __init__(self):
        self.vocab: dict[str, int] = {}
        self.id_to_token: dict[int, str] = {}
        self.ranks: dict[tuple[str, str], int] = {}
        self.special_by_str: dict[str, int] = {}
        self.special_by_id: dict[int, str] = {}
        self.alpha = byte_alphabet()
        self.inv = {c: b for b, c in enumerate(self.alpha)}
        self.endoftext_id = self.im_start_id = self.im_end_id = -1

    # ---- loaders
    def _merge(self, a: str, b: str, rank: int) -> None:
        self.ranks.setdefault((a, b), rank)

    def add_special(self, tok: str, id_: int) -> None:
        if not tok:
            return
        old = self.special_by_str.get(tok)
        if old is not None and self.special_by_id.get(old) == tok:
            del self.special_by_id[old]
        self.special_by_str[tok] = id_
        self.special_by_id[id_] = tok

    def _finish(self, extra=()) -> "Tokenizer":
        for s in list(SPECIAL_NAMES) + list(extra):
            if s in self.vocab:
                self.add_special(s, self.vocab[s])
        self.endoftext_id = self.vocab.get("<|endoftext|>", -1)
        self.im_start_id = self.vocab.get("<|im_start|>", -1)
        self.im_end_id = self.vocab.get("<|im_end|>", -1)
        return self

    @classmethod
    def from_lists(cls, tokens, merges, token_types=None, extra=()) -> "Tokenizer":
        """from_gguf (qwen_tokenizer.cpp:181-247) on the metadata arrays."""
        t = cls()
        for i, s in enumerate(tokens):
            t.vocab.setdefault(s, i)
            t.id_to_token[i] = s
        for i, m in enumerate(merges):
            sp = m.index(" ")
            t._merge(m[:sp], m[sp + 1:], i)
        if token_types is not None:
            for i, ty in enumerate(token_types[:len(tokens)]):
                if ty == 3:
                    t.add_special(tokens[i], i)
        return t._finish(extra)

    @classmethod
    def from_files(cls, vocab_json: str, merges_txt: str, extra=()) -> "Tokenizer":
        """load (qwen_tokenizer.cpp:122-160, byte_level_bpe.cpp:225-251)."""
        t = cls()
        with open(vocab_json, encoding="utf-8") as f:
            pairs = json.load(f, object_pairs_hook=lambda kv: kv)
        for s, i in pairs:
            t.vocab.setdefault(s, int(i))
        for s, i in t.vocab.items():
            t.id_to_token.setdefault(i, s)
        rank, first = 0, True
        with open(merges_txt, encoding="utf-8", newline="") as f:
            for line in f.read().split("\n"):
                if line.endswith("\r"):
                    line = line[:-1]
                if not line:
                    continue
                if first:
                    first = False
                    if line[0] == "#":
                        continue
                sp = line.index(" ")
                t._merge(line[:sp], line[sp + 1:], rank)
                rank += 1
        return t._finish(extra)

    # ---- encode / decode
    def _match(self, text: bytes, pos: int):
        best, bid = 0, -1
        for s, i in self.special_by_str.items():
            b = s.encode()
            if len(b) > best and text.startswith(b, pos):
                best, bid = len(b), i
        return best, bid

    def _piece(self, piece: bytes, out: list[int]) -> None:
        if not piece:
            return
        for u in bpe_merge([self.alpha[b] for b in piece], self.ranks):
            if u in self.vocab:
                out.append(self.vocab[u])

    def encode(self, text, add_special: bool = False) -> list[int]:
        t = text.encode() if isinstance(text, str) else bytes(text)
        out, i, span = [], 0, 0
        while i < len(t):
            k, sid = self._match(t, i)
            if k == 0:
                i += 1
                continue
            if i > span:
                for p in pre_tokenize(t[span:i]):
                    self._piece(p, out)
            out.append(sid)
            i += k
            span = i
        if span < len(t):
            for p in pre_tokenize(t[span:]):
                self._piece(p, out)
        if add_special and self.endoftext_id >= 0:
            out.append(self.endoftext_id)
        return out

    def decode_bytes(self, ids) -> bytes:
        out, pending = bytearray(), []

        def flush():
            for ch in "".join(pending):
                if ch in self.inv:
                    out.append(self.inv[ch])
            pending.clear()

        for i in ids:
            if i in self.special_by_id:
                flush()
                out += self.special_by_id[i].encode()
            elif i in self.id_to_token:
                pending.append(self.id_to_token[i])
        flush()
        return bytes(out)
