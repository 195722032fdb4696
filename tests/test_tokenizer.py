"""Llama 3 tokenizer and chat template (inferencer.cu:342-451, 1534-1551).

Pinned against an independent implementation: HF `tokenizers` (installed)
running byte-level BPE with the same split pattern and merge list, on a
vocabulary trained by HF's BPE trainer from a seeded synthetic corpus and
padded to Llama 3's 128256 entries with its special tokens.  The split
pattern itself is pinned by hand-worked splits, and against the reference's
original spelling (with \\s) on text where PCRE2's and the regex module's
\\s agree.  No GGUF tokenizer file exists in this environment, so the real
Llama 3 merges are not exercised: parity on them is unpinned."""
import pytest
import regex

import llama3_vocab as V
from conftest import load_package

load_package()
import inferencer_jetson_amd.tokenizer as T  # noqa: E402

# The reference's pattern as written there (inferencer.cu:382-385).
REF_PATTERN = (r"(?:'[sS]|'[tT]|'[rR][eE]|'[vV][eE]|'[mM]|'[lL][lL]|'[dD])|"
               r"[^\r\n\p{L}\p{N}]?\p{L}+|\p{N}{1,3}|"
               r" ?[^\s\p{L}\p{N}]+[\r\n]*|\s*[\r\n]+|\s+(?!\S)|\s+")

@pytest.fixture(scope="module")
def vocab():
    """(our Tokenizer, HF tokenizer) over one trained vocabulary."""
    tk = pytest.importorskip("tokenizers")
    from tokenizers import decoders, models
    tokens, merges = V.trained_vocab(T.LLAMA3_SPLIT)
    ours = T.Tokenizer([t.encode() for t in tokens], [m.encode() for m in merges])
    hf = tk.Tokenizer(models.BPE(vocab={t: i for i, t in enumerate(tokens)},
                                 merges=[tuple(m.split(" ")) for m in merges]))
    hf.pre_tokenizer = V.split_pre_tokenizer(T.LLAMA3_SPLIT)
    hf.decoder = decoders.ByteLevel()
    return ours, hf


def test_byte_symbols_are_the_byte_level_alphabet():
    sym = T.byte_symbols()
    assert len(set(sym)) == 256
    assert sym[ord("A")] == "A" and sym[33] == "!" and sym[126] == "~" and sym[174] == "®"
    assert sym[0] == chr(256) and sym[32] == chr(256 + 32) and sym[127] == chr(256 + 33)
    assert sym[173] == chr(256 + 67)          # the last of the 68 remapped bytes
    from tokenizers import pre_tokenizers
    assert set(sym) == set(pre_tokenizers.ByteLevel.alphabet())


@pytest.mark.parametrize("text,pieces", [
    ("Hello world", ["Hello", " world"]),
    ("I'm here", ["I", "'m", " here"]),
    ("THEY'RE", ["THEY", "'RE"]),
    ("12345678", ["123", "456", "78"]),
    ("a  b", ["a", " ", " b"]),
    ("x\n\n  y", ["x", "\n\n", " ", " y"]),
    ("end.\n", ["end", ".\n"]),
    ("  ", ["  "]),
    ("(ok)", ["(ok", ")"]),
    ("a b", ["a", " b"]),
])
def test_split_pattern_known_answers(text, pieces):
    assert regex.findall(T.LLAMA3_SPLIT, text) == pieces


def test_split_matches_reference_spelling_where_whitespace_agrees():
    ref = regex.compile(REF_PATTERN)
    ours = regex.compile(T.LLAMA3_SPLIT)
    for s in V.corpus(5, 400):
        assert ours.findall(s) == ref.findall(s), s
    # Where they differ: U+0085 (a Cc control) is not PCRE2 UCP whitespace
    # but is the regex module's: as whitespace the pair splits, as "other" it
    # stays one piece.
    assert ref.findall("a\u0085\u0085b") == ["a", "\u0085", "\u0085b"]
    assert ours.findall("a\u0085\u0085b") == ["a", "\u0085\u0085", "b"]


def test_encode_matches_hf_bpe(vocab):
    ours, hf = vocab
    texts = V.corpus(23, 600) + ["", " ", "\n", "a", "ab", "😀😀😀", "é" * 17, "9" * 10, "'s's's", " \t\r\n \n",
                               "\u0085", "\u001c", "word  word", "x" * 200]
    for s in texts:
        assert ours.encode(s) == hf.encode(s, add_special_tokens=False).ids, repr(s)


def test_decode_round_trip(vocab):
    ours, hf = vocab
    for s in V.corpus(31, 200):
        ids = ours.encode(s)
        assert b"".join(ours.decode(i) for i in ids) == s.encode("utf-8")
        assert hf.decode(ids) == s


def test_special_tokens_and_chat_template(vocab):
    ours, _ = vocab
    assert ours.special("<|eot_id|>") == 128009
    assert ours.stop_ids() == {128009, 128001, 128008}
    ids = T.chat_prompt(ours, "Hi there")
    assert ids[:2] == [128000, 128006] and ids[-1:] != [128009]
    hdr = ours.encode("user")
    assert ids[2:2 + len(hdr)] == hdr and ids[2 + len(hdr)] == 128007
    body = ours.encode("\n\nHi there")
    k = 3 + len(hdr)
    assert ids[k:k + len(body)] == body
    assert ids[k + len(body):k + len(body) + 2] == [128009, 128006]
    tail = ours.encode("assistant") + [128007] + ours.encode("\n\n")
    assert ids[-len(tail):] == tail
    assert ours.decode(128009) == b"<|eot_id|>"


def test_reference_error_conditions(vocab):
    ours, _ = vocab
    with pytest.raises(ValueError, match="Expected Llama 3 tokenizer"):
        T.Tokenizer([b"a"] * 1000, [])
    with pytest.raises(ValueError, match="Invalid token id"):
        ours.decode(T.LLAMA3_VOCAB)
    with pytest.raises(ValueError, match="Missing special token"):
        ours.special("<|no_such|>")
    # A vocabulary without the byte symbols cannot encode: unknown token.
    bare = T.Tokenizer([f"t{i}" for i in range(T.LLAMA3_VOCAB)], [])
    with pytest.raises(ValueError, match="unknown token"):
        bare.encode("q")
    # A token holding a character that is no byte symbol cannot be decoded.
    odd = T.Tokenizer(["一"] + [f"t{i}" for i in range(T.LLAMA3_VOCAB - 1)], [])
    with pytest.raises(ValueError, match="Cannot decode token"):
        odd.decode(0)


def test_first_duplicate_token_and_merge_win():
    toks = ["a", "b", "ab", "ab"] + [f"t{i}" for i in range(T.LLAMA3_VOCAB - 4)]
    tok = T.Tokenizer(toks, ["a b", "a b"])
    assert tok.encode("ab") == [2]
