"""The reference's byte-level BPE tokenizer restated (three_llm_amd.tokenizer)
against its own tests (engine.test.ts:434-486) and against the Hugging Face
`tokenizers` implementation of the same algorithm (byte-level BPE with the
GPT-2 and Qwen2 pre-tokenizer regexes) on a vocabulary trained offline."""
import json

import pytest

import three_llm_amd.tokenizer as T


def test_reference_cases():
    tok = T.GPT2Tokenizer({"a": 0, "#": 1, "##": 2, "a#": 3, "<|endoftext|>": 4}, ["#version: 0.2", "# #", "a #"])
    assert tok.bpe("##") == "##" and tok.bpe("a#") == "a#"
    assert tok.encode("##") == [2]
    tok = T.GPT2Tokenizer({"a": 0, "<|endoftext|>": 1}, [], addedTokens=[
        {"id": 10, "content": "<|im_start|>"}, {"id": 11, "content": "<think>"}, {"id": 12, "content": "</think>"}])
    assert tok.encode("<|im_start|><think></think>") == [10, 11, 12]
    assert tok.decode([10, 11, 12]) == "<|im_start|><think></think>"
    vocab = {"<|endoftext|>": 0, "1": 1, "2": 2, "3": 3, "12": 5, "123": 4}
    qwen = T.GPT2Tokenizer(vocab, [], tokenPattern=r"(?i:'s)|\p{N}")
    llama3 = T.GPT2Tokenizer(vocab, ["1 2", "12 3"], tokenPattern=r"\p{N}{1,3}")
    assert qwen.encode("123") == [1, 2, 3]
    assert llama3.encode("123") == [4]


def test_tokenizer_kind():
    assert T.tokenizer_kind({"model_type": "qwen2"}) == "qwen"
    assert T.tokenizer_kind({"model_type": "llama", "_name_or_path": "HuggingFaceTB/SmolLM2-135M"}) == "smollm"
    assert T.tokenizer_kind({"model_type": "llama", "_name_or_path": "kakaocorp/kanana-nano"}) == "llama3"
    assert T.tokenizer_kind({"model_type": "llama"}) == "gpt2"
    assert T.tokenizer_kind({"text_config": {"model_type": "qwen3"}}) == "qwen"


def test_whitespace_is_javascripts():
    # JavaScript's \s includes U+FEFF; the pre-tokenizer keeps it with the spaces
    assert T.GPT2_TOKEN_PATTERN.findall("a﻿﻿b") == ["a", "﻿", "﻿", "b"]
    assert T.GPT2_TOKEN_PATTERN.findall("x  y") == ["x", " ", " y"]


TEXTS = [
    "Hello world! It's a test, isn't it? I'LL SEE... 12345 and 3.14159",
    "Once upon a time, there was a little girl named Lily.\n\nShe liked to play\toutside   .",
    "日本語のテキストと中文文本，还有한국어 텍스트. Ünïcödé façade naïve café",
    "emoji 😀🚀 combined é and é; numbers 0123456789 ١٢٣",
    "code: def f(x):\n    return x**2  # comment\r\n}",
    "   leading spaces and trailing   ",
    "'s 's 'S 'RE 've 'd 'LL quotes",
]


@pytest.fixture(scope="module")
def trained(tmp_path_factory):
    tk = pytest.importorskip("tokenizers")
    from tokenizers import Tokenizer, decoders, models, pre_tokenizers, trainers
    corpus = [t * 3 for t in TEXTS] + ["the quick brown fox jumps over the lazy dog " * 5,
                                       "Lily went to the park with her mom and dad. " * 5]
    tok = Tokenizer(models.BPE())
    tok.pre_tokenizer = pre_tokenizers.ByteLevel(add_prefix_space=False, use_regex=True)
    tok.decoder = decoders.ByteLevel()
    trainer = trainers.BpeTrainer(vocab_size=600, special_tokens=["<|endoftext|>"],
                                  initial_alphabet=pre_tokenizers.ByteLevel.alphabet(), show_progress=False)
    tok.train_from_iterator(corpus, trainer)
    d = tmp_path_factory.mktemp("tok")
    tok.model.save(str(d))
    return tk, tok, d


def test_gpt2_pattern_matches_hf_byte_level_bpe(trained):
    tk, hf, d = trained
    ours = T.GPT2Tokenizer.from_files(str(d / "vocab.json"), str(d / "merges.txt"))
    for text in TEXTS:
        assert ours.encode(text) == hf.encode(text).ids, text
        assert ours.decode(ours.encode(text)) == text


def test_qwen_pattern_matches_hf_split_then_byte_level(trained):
    tk, hf, d = trained
    from tokenizers import Regex, Tokenizer, models, pre_tokenizers
    qwen_regex = (r"(?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\r\n\p{L}\p{N}]?\p{L}+|\p{N}| ?[^\s\p{L}\p{N}]+[\r\n]*"
                  r"|\s*[\r\n]+|\s+(?!\S)|\s+")  # Qwen2's tokenizer.json pre-tokenizer
    vocab = json.load(open(d / "vocab.json"))
    merges = [l for l in open(d / "merges.txt", encoding="utf-8").read().split("\n")]
    hq = Tokenizer(models.BPE.from_file(str(d / "vocab.json"), str(d / "merges.txt")))
    hq.pre_tokenizer = pre_tokenizers.Sequence([
        pre_tokenizers.Split(Regex(qwen_regex), behavior="isolated", invert=False),
        pre_tokenizers.ByteLevel(add_prefix_space=False, use_regex=False)])
    # the reference's Qwen pattern also admits combining marks (\p{M}) in letter runs
    ours = T.GPT2Tokenizer(vocab, merges, tokenPattern=T.QWEN_TOKEN_PATTERN)
    for text in TEXTS:
        if any(0x300 <= ord(c) <= 0x36F for c in text):
            continue  # combining marks: \p{L}\p{M} (reference) vs \p{L} (Qwen2's tokenizer.json)
        assert ours.encode(text) == hq.encode(text).ids, text
