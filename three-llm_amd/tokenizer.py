"""Byte-level BPE tokenizer of the reference (load/GPT2Tokenizer.ts:8-271) and
the tokenizer choice of a local Hugging Face directory (load/HFModelBundle.ts:
44-104, load/DecoderRecipe.ts:75-89).

The pre-tokenizer patterns are the reference's JavaScript regular expressions
written for Python's `regex` module; `\\s` / `\\S` are spelled out as
JavaScript's whitespace set (it includes U+FEFF, which Unicode's does not).
"""
from __future__ import annotations

import json
import os
import unicodedata
from typing import Dict, Iterable, List, Optional, Sequence

import regex

_WS = "\\t\\n\\x0b\\x0c\\r \\u00a0\\u1680\\u2000-\\u200a\\u2028\\u2029\\u202f\\u205f\\u3000\\ufeff"
_S = f"[{_WS}]"
_NS = f"[^{_WS}]"


def _js(pattern: str) -> "regex.Pattern":
    """A JS /u pattern with \\s and \\S replaced by JavaScript's whitespace class."""
    out, i = [], 0
    while i < len(pattern):
        c = pattern[i]
        if c == "\\" and i + 1 < len(pattern):
            nxt = pattern[i + 1]
            in_class = _inside_class(pattern, i)
            if nxt == "s":
                out.append(_WS if in_class else _S)
            elif nxt == "S":
                out.append(_NS)  # only used outside classes by these patterns
            else:
                out.append(pattern[i:i + 2])
            i += 2
            continue
        out.append(c)
        i += 1
    return regex.compile("".join(out), regex.V1)


def _inside_class(p: str, at: int) -> bool:
    depth, i = 0, 0
    while i < at:
        if p[i] == "\\":
            i += 2
            continue
        if p[i] == "[":
            depth += 1
        elif p[i] == "]" and depth:
            depth -= 1
        i += 1
    return depth > 0


# GPT2Tokenizer.ts:205-211
GPT2_TOKEN_PATTERN = _js(r"'s|'t|'re|'ve|'m|'ll|'d| ?\p{L}+| ?\p{N}+| ?[^\s\p{L}\p{N}]+|\s+(?!\S)|\s+")
QWEN_TOKEN_PATTERN = _js(r"(?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\r\n\p{L}\p{N}]?[\p{L}\p{M}]+|\p{N}"
                         r"| ?[^\s\p{L}\p{M}\p{N}]+[\r\n]*|\s*[\r\n]+|\s+(?!\S)|\s+")
SMOLLM_TOKEN_PATTERN = _js(r"'s|'t|'re|'ve|'m|'ll|'d| ?\p{L}+|\p{N}| ?[^\s\p{L}\p{N}]+|\s+(?!\S)|\s+")
LLAMA3_TOKEN_PATTERN = _js(r"(?i:'s|'t|'re|'ve|'m|'ll|'d)| ?\p{L}+|\p{N}{1,3}| ?[^\s\p{L}\p{N}]+[\r\n]*"
                           r"|\s*[\r\n]+|\s+(?!\S)|\s+")
PATTERNS = {"gpt2": GPT2_TOKEN_PATTERN, "qwen": QWEN_TOKEN_PATTERN, "smollm": SMOLLM_TOKEN_PATTERN,
            "llama3": LLAMA3_TOKEN_PATTERN}


def bytes_to_unicode() -> Dict[int, str]:
    """bytesToUnicode, GPT2Tokenizer.ts:213-239: printable bytes map to
    themselves, the rest to 256 + n in byte order."""
    bs = list(range(33, 127)) + list(range(161, 173)) + list(range(174, 256))
    cs = list(bs)
    n = 0
    for b in range(256):
        if b not in bs:
            bs.append(b)
            cs.append(256 + n)
            n += 1
    return {b: chr(c) for b, c in zip(bs, cs)}


class GPT2Tokenizer:
    """GPT2Tokenizer (GPT2Tokenizer.ts:8-203): encode, decode, bpe."""

    def __init__(self, vocab: Dict[str, int], merges: Sequence[str], unknownToken: Optional[str] = None,
                 endOfTextToken: Optional[str] = None, tokenPattern=None, normalizer: Optional[str] = None,
                 addedTokens: Iterable[dict] = (), stopTokenIds: Optional[List[int]] = None):
        self.encoder = dict(vocab)
        self.unknownToken = unknownToken or "<|endoftext|>"
        self.endOfTextToken = endOfTextToken or "<|endoftext|>"
        self.tokenPattern = tokenPattern if tokenPattern is not None else GPT2_TOKEN_PATTERN
        if isinstance(self.tokenPattern, str):
            self.tokenPattern = _js(self.tokenPattern)
        self.normalizer = normalizer
        self.addedTokenIds: Dict[str, int] = {}
        for added in addedTokens:
            if added is None or added.get("content") is None or added.get("id") is None:
                continue
            self.encoder[added["content"]] = added["id"]
            self.addedTokenIds[added["content"]] = added["id"]
        self.addedTokenPattern = None
        if self.addedTokenIds:
            escaped = "|".join(regex.escape(t) for t in sorted(self.addedTokenIds, key=len, reverse=True))
            self.addedTokenPattern = regex.compile(f"({escaped})")
        self.endOfTextTokenId = self.encoder.get(self.endOfTextToken)
        self.stopTokenIds = list(stopTokenIds) if stopTokenIds is not None else None
        self.decoder: Dict[int, str] = {i: t for t, i in self.encoder.items()}
        self.byteEncoder = bytes_to_unicode()
        self.byteDecoder = {c: b for b, c in self.byteEncoder.items()}
        self.bpeRanks: Dict[tuple, int] = {}
        for merge in merges:
            merge = merge.strip()
            if merge == "" or merge.startswith("#version"):
                continue
            pair = tuple(regex.split(r"\s+", merge))
            if pair not in self.bpeRanks:
                self.bpeRanks[pair] = len(self.bpeRanks)
        self.cache: Dict[str, str] = {}

    @classmethod
    def from_files(cls, vocab_path: str, merges_path: str, **options) -> "GPT2Tokenizer":
        """fromURLs for local vocab.json + merges.txt."""
        with open(vocab_path, encoding="utf-8") as f:
            vocab = json.load(f)
        with open(merges_path, encoding="utf-8") as f:
            merges = regex.split(r"\r?\n", f.read())
        return cls(vocab, merges, **options)

    @classmethod
    def from_tokenizer_json(cls, path: str, **options) -> "GPT2Tokenizer":
        """fromTokenizerJSONURL for a local tokenizer.json."""
        with open(path, encoding="utf-8") as f:
            tj = json.load(f)
        model = tj.get("model") or {}
        if model.get("vocab") is None or model.get("merges") is None:
            raise ValueError("GPT2Tokenizer: tokenizer.json does not contain a BPE vocab and merges.")
        merges = [" ".join(m) if isinstance(m, list) else m for m in model["merges"]]
        norm = tj.get("normalizer") or {}
        normalizers = norm.get("normalizers") or [] if "normalizers" in norm else [norm]
        has_nfc = any((n or {}).get("type") == "NFC" for n in normalizers)
        opts = dict(options)
        opts.setdefault("unknownToken", model.get("unk_token"))
        if opts.get("normalizer") is None:
            opts["normalizer"] = "nfc" if has_nfc else None
        opts["addedTokens"] = list(tj.get("added_tokens") or []) + list(options.get("addedTokens") or [])
        return cls(model["vocab"], merges, **opts)

    def encode(self, text: str) -> List[int]:
        tokens: List[int] = []
        source = unicodedata.normalize("NFC", str(text)) if self.normalizer == "nfc" else str(text)
        chunks = [source] if self.addedTokenPattern is None else self.addedTokenPattern.split(source)
        for chunk in chunks:
            if chunk == "":
                continue
            if chunk in self.addedTokenIds:
                tokens.append(self.addedTokenIds[chunk])
                continue
            for match in self.tokenPattern.findall(chunk):
                encoded = "".join(self.byteEncoder[b] for b in match.encode("utf-8"))
                for token in self.bpe(encoded).split(" "):
                    tid = self.encoder.get(token)
                    tokens.append(self.encoder.get(self.unknownToken) if tid is None else tid)
        return tokens

    def decode(self, token_ids: Iterable[int]) -> str:
        text = "".join(self.decoder.get(int(i), "") for i in token_ids)
        data = bytes(self.byteDecoder[c] for c in text if c in self.byteDecoder)
        return data.decode("utf-8", errors="replace")

    def bpe(self, token: str) -> str:
        if token in self.cache:
            return self.cache[token]
        word = list(token)
        pairs = _pairs(word)
        if not pairs:
            return token
        while True:
            best, best_rank = None, None
            for pair in pairs:
                rank = self.bpeRanks.get(pair)
                if rank is not None and (best_rank is None or rank < best_rank):
                    best, best_rank = pair, rank
            if best is None:
                break
            first, second = best
            nxt, i = [], 0
            while i < len(word):
                if word[i] == first and i < len(word) - 1 and word[i + 1] == second:
                    nxt.append(first + second)
                    i += 2
                else:
                    nxt.append(word[i])
                    i += 1
            word = nxt
            if len(word) == 1:
                break
            pairs = _pairs(word)
        value = " ".join(word)
        self.cache[token] = value
        return value


def _pairs(word: List[str]):
    return {(word[i], word[i + 1]) for i in range(len(word) - 1)}


def tokenizer_kind(config: dict) -> str:
    """denseTokenizer, DecoderRecipe.ts:75-89."""
    text = config.get("text_config") if isinstance(config.get("text_config"), dict) else config
    mtype = text.get("model_type")
    name = text.get("_name_or_path") or text.get("name_or_path") or text.get("model_id") or ""
    name = name.lower() if isinstance(name, str) else ""
    if mtype in ("qwen2", "qwen3") or "qwen" in name or "deepseek-r1-distill-qwen" in name:
        return "qwen"
    if mtype == "kanana2_tiny" or "kanana" in name:
        return "llama3"
    if "smollm2" in name:
        return "smollm"
    return "gpt2"


def load_tokenizer(root: str, config: dict, stop_token_ids: Optional[List[int]] = None) -> GPT2Tokenizer:
    """loadTokenizer (HFModelBundle.ts:44-104) for a local directory: added
    tokens from tokenizer_config.json, vocab.json + merges.txt, else
    tokenizer.json."""
    kind = tokenizer_kind(config)
    added: List[dict] = []
    try:
        with open(os.path.join(root, "tokenizer_config.json"), encoding="utf-8") as f:
            dec = json.load(f).get("added_tokens_decoder") or {}
        added = [{"id": int(k), "content": v["content"]} for k, v in dec.items()]
    except (OSError, ValueError, KeyError):
        added = []
    opts = dict(tokenPattern=PATTERNS.get(kind), addedTokens=added, stopTokenIds=stop_token_ids,
                endOfTextToken="<|end_of_text|>" if kind == "llama3" else "<|endoftext|>",
                normalizer="nfc" if kind == "qwen" else None)
    vocab, merges = os.path.join(root, "vocab.json"), os.path.join(root, "merges.txt")
    if os.path.isfile(vocab) and os.path.isfile(merges):
        return GPT2Tokenizer.from_files(vocab, merges, **opts)
    return GPT2Tokenizer.from_tokenizer_json(os.path.join(root, "tokenizer.json"), **opts)
