"""Llama 3 byte-level BPE tokenizer and chat template over a GGUF vocabulary.

The reference's Tokenizer (inferencer.cu:361-451) and chat_prompt
(inferencer.cu:1534-1551), restated for the host side of this package:

* tokenizer.ggml.tokens (exactly 128256 entries, as the reference demands)
  and tokenizer.ggml.merges ("left right", rank = position) from the GGUF.
* Byte symbols: bytes 33..126, 161..172 and 174..255 stand for themselves,
  the other 68 bytes take code points 256, 257, ... in byte order
  (inferencer.cu:375-379) -- the byte-level alphabet of the vocabulary.
* Pre-tokenization by Llama 3's split pattern (inferencer.cu:381-385),
  compiled by the reference with PCRE2 in UTF + UCP mode.  PCRE2's UCP
  ``\\s`` is the separator category Z plus tab, LF, VT, FF and CR; the
  ``regex`` module's ``\\s`` also takes U+0085, so the pattern here spells
  PCRE2's class out.  Text between matches is encoded
  as its own piece (inferencer.cu:423-429).
* Each piece: its bytes as symbols, then the adjacent pair of lowest merge
  rank is joined -- the leftmost when a pair occurs twice -- until no pair
  has a rank (inferencer.cu:395-416); every final symbol must be a token.
* decode(id): the token's symbols mapped back to bytes (inferencer.cu:432-445).

Only the reference's pcre2 dependency is replaced: the regex engine here is
the ``regex`` module (Unicode general categories of its own Unicode
version).  Errors raise ValueError with the reference's conditions.
"""
from __future__ import annotations

import regex

# Llama 3's pre-tokenizer (inferencer.cu:381-385) with \s written as PCRE2
# UCP's class: separators (\p{Z}) and \t \n \x0b \f \r.
_SP = r"\t\n\x0b\f\r\p{Z}"
LLAMA3_SPLIT = (
    r"(?:'[sS]|'[tT]|'[rR][eE]|'[vV][eE]|'[mM]|'[lL][lL]|'[dD])|"
    r"[^\r\n\p{L}\p{N}]?\p{L}+|\p{N}{1,3}|"
    r" ?[^" + _SP + r"\p{L}\p{N}]+[\r\n]*|[" + _SP + r"]*[\r\n]+|[" + _SP + r"]+(?![^" + _SP + r"])|[" + _SP + r"]+"
)

LLAMA3_VOCAB = 128256
STOP_TOKENS = ("<|eot_id|>", "<|end_of_text|>", "<|eom_id|>")


def byte_symbols() -> list[str]:
    """symbol[b] for every byte b (inferencer.cu:375-379)."""
    out, extra = [], 256
    for b in range(256):
        if 33 <= b <= 126 or 161 <= b <= 172 or b >= 174:
            out.append(chr(b))
        else:
            out.append(chr(extra))
            extra += 1
    return out


def _text(s) -> str:
    return s.decode("utf-8") if isinstance(s, (bytes, bytearray)) else str(s)


class Tokenizer:
    def __init__(self, tokens, merges):
        tokens = [_text(t) for t in tokens]
        if len(tokens) != LLAMA3_VOCAB:
            raise ValueError("Expected Llama 3 tokenizer")
        self.tokens = tokens
        # First occurrence wins, as with unordered_map::emplace.
        self.ids: dict[str, int] = {}
        for i, t in enumerate(tokens):
            self.ids.setdefault(t, i)
        self.rank: dict[str, int] = {}
        for i, m in enumerate(merges):
            self.rank.setdefault(_text(m), i)
        self.symbol = byte_symbols()
        self.byte_of = {s: b for b, s in enumerate(self.symbol)}
        self.split = regex.compile(LLAMA3_SPLIT)
        self._cache: dict[bytes, tuple[int, ...]] = {}

    @classmethod
    def from_gguf(cls, model) -> "Tokenizer":
        """From an open GGUF (the package's GGUF class): tokens and merges."""
        return cls(model.tokens(0), model.tokens(1))

    def _bpe(self, piece: bytes) -> tuple[int, ...]:
        hit = self._cache.get(piece)
        if hit is not None:
            return hit
        parts = [self.symbol[b] for b in piece]
        rank = self.rank
        while len(parts) > 1:
            best, at = None, -1
            for i in range(len(parts) - 1):
                r = rank.get(parts[i] + " " + parts[i + 1])
                if r is not None and (best is None or r < best):
                    best, at = r, i
            if best is None:
                break
            parts[at:at + 2] = [parts[at] + parts[at + 1]]
        out = []
        for s in parts:
            i = self.ids.get(s)
            if i is None:
                raise ValueError("Tokenizer produced an unknown token")
            out.append(i)
        hit = tuple(out)
        self._cache[piece] = hit
        return hit

    def encode(self, text: str) -> list[int]:
        out: list[int] = []
        pos = 0
        for m in self.split.finditer(text):
            if m.start() > pos:
                out.extend(self._bpe(text[pos:m.start()].encode("utf-8")))
            out.extend(self._bpe(m.group().encode("utf-8")))
            pos = m.end()
        if pos < len(text):
            out.extend(self._bpe(text[pos:].encode("utf-8")))
        return out

    def decode(self, token_id: int) -> bytes:
        if not 0 <= token_id < len(self.tokens):
            raise ValueError("Invalid token id")
        out = bytearray()
        for ch in self.tokens[token_id]:
            b = self.byte_of.get(ch)
            if b is None:
                raise ValueError("Cannot decode token")
            out.append(b)
        return bytes(out)

    def special(self, name: str) -> int:
        i = self.ids.get(name)
        if i is None:
            raise ValueError("Missing special token " + name)
        return i

    def stop_ids(self) -> set[int]:
        """The ids that end a response (inferencer.cu:1892-1894)."""
        return {self.special(n) for n in STOP_TOKENS}


def chat_prompt(tok: Tokenizer, prompt: str) -> list[int]:
    """Llama 3 chat framing of one user turn (inferencer.cu:1534-1551)."""
    ids = [tok.special("<|begin_of_text|>"), tok.special("<|start_header_id|>")]
    ids += tok.encode("user")
    ids.append(tok.special("<|end_header_id|>"))
    ids += tok.encode("\n\n" + prompt)
    ids += [tok.special("<|eot_id|>"), tok.special("<|start_header_id|>")]
    ids += tok.encode("assistant")
    ids.append(tok.special("<|end_header_id|>"))
    ids += tok.encode("\n\n")
    return ids
