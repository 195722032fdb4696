"""A Llama 3 shaped vocabulary for the tokenizer and command-line tests:
HF tokenizers' BPE trainer on a seeded synthetic corpus with the Llama 3
split pattern, padded to 128256 tokens with the special tokens at Llama 3's
ids.  Test infrastructure only."""
from __future__ import annotations

import functools
import json
import random

SPECIALS = {128000: "<|begin_of_text|>", 128001: "<|end_of_text|>", 128006: "<|start_header_id|>",
            128007: "<|end_header_id|>", 128008: "<|eom_id|>", 128009: "<|eot_id|>"}

WORDS = ["the", "The", "quantized", "matrix", "vector", "GPU", "décodé", "naïve", "straße", "Ωmega", "日本語",
         "テキスト", "привет", "مرحبا", "emoji", "😀", "🚀🚀", "x", "I", "you", "don't", "WE'LL", "it's", "they're",
         "I'VE", "she'd", "I'm", "12345", "3.14159", "1,000,000", "٣٤٥", "Ⅻ", "½", "→", "...", "?!", "--", "(a)",
         "[b]", "{c}", "#tag", "@user", "a_b", "tab\there", "new\nline", "cr\r\nlf", "  spaced  ", "\n\n",
         " nbsp", "é", "zero​width", "ﬁ", "Q4_K", "Q6_K", "MI355X", "llama", "token", "cache", "user",
         "assistant", "hello", "world"]


def corpus(seed: int, n: int) -> list[str]:
    rnd = random.Random(seed)
    out = []
    for _ in range(n):
        k = rnd.randint(1, 12)
        seps = [" ", " ", " ", "", "\n", "  ", "\t", ". ", ", "]
        out.append("".join(rnd.choice(WORDS) + rnd.choice(seps) for _ in range(k)))
    return out


def split_pre_tokenizer(pattern: str):
    from tokenizers import Regex, pre_tokenizers
    return pre_tokenizers.Sequence([pre_tokenizers.Split(Regex(pattern), behavior="isolated"),
                                    pre_tokenizers.ByteLevel(add_prefix_space=False, use_regex=False)])


@functools.lru_cache(maxsize=None)
def trained_vocab(pattern: str) -> tuple[tuple[str, ...], tuple[str, ...]]:
    """(tokens, merges): 128256 token strings and the merge list."""
    import tokenizers as tk
    from tokenizers import models, pre_tokenizers, trainers
    t = tk.Tokenizer(models.BPE())
    t.pre_tokenizer = split_pre_tokenizer(pattern)
    trainer = trainers.BpeTrainer(vocab_size=1500, min_frequency=2, show_progress=False,
                                  initial_alphabet=pre_tokenizers.ByteLevel.alphabet())
    t.train_from_iterator(corpus(11, 3000), trainer=trainer)
    model = json.loads(t.to_str())["model"]
    merges = [m if isinstance(m, str) else " ".join(m) for m in model["merges"]]
    tokens = [tok for tok, _ in sorted(model["vocab"].items(), key=lambda kv: kv[1])]
    while len(tokens) < 128256:
        tokens.append(f"<|reserved_special_token_{len(tokens)}|>")
    for i, name in SPECIALS.items():
        tokens[i] = name
    return tuple(tokens), tuple(merges)
