"""Text front-end: the three GGUF tokenizers and their chat framings, restated from the
reference's host modules (src/core/bpe.ts, tokenizer.ts, gpt2-tokenizer.ts,
qwen-tokenizer.ts) so ``PagedEngine.generate`` can take messages instead of token ids.

* ``Tokenizer``: SentencePiece BPE with merge scores and UTF-8 byte fallback (Gemma,
  tokenizer.ts:5-58).
* ``Gpt2Tokenizer``: byte-level BPE with ranked merges and a per-vocabulary pre-tokenizer
  (Llama 3, Mistral, SmolLM, Qwen2/3; gpt2-tokenizer.ts:1-132), with Llama 3 / ChatML /
  Mistral framing.
* ``QwenTokenizer``: NFC + the qwen35 pre-tokenizer + byte-level BPE, ChatML with explicit
  non-thinking framing (qwen-tokenizer.ts:1-63).

The JavaScript semantics the reference relies on are kept: ``\\s`` is ECMAScript white space
(written out below, since Python's differs), ``TextEncoder`` turns lone surrogates into
U+FFFD, and decoding is a streaming UTF-8 decode that withholds an unfinished trailing
sequence and replaces invalid bytes with U+FFFD.
"""
from __future__ import annotations

import codecs
import heapq
import unicodedata
from typing import Callable, Dict, List, Mapping, Optional, Sequence

import regex

# ------------------------------------------------------------------ shared BPE (bpe.ts)


def byte_alphabet() -> List[str]:
    """The GPT-2 byte -> printable code point table (bpe.ts:2-6): printable Latin-1 bytes map
    to themselves, the rest to 256, 257, ... in byte order."""
    kept = {b for b in range(256) if 33 <= b <= 126 or 161 <= b <= 172 or b >= 174}
    out, extra = [], 256
    for b in range(256):
        if b in kept:
            out.append(chr(b))
        else:
            out.append(chr(extra))
            extra += 1
    return out


def merge_symbols(symbols: List[str], score: Callable[[str, str], Optional[float]]) -> List[str]:
    """Adjacent-pair BPE (bpe.ts:9-40): repeatedly merge the best-scoring adjacent pair;
    higher scores win and ties go to the leftmost pair. A heap of candidate pairs with
    per-position versions drops pairs whose sides changed since they were queued."""
    n = len(symbols)
    if n < 2:
        return list(symbols)
    sym = list(symbols)
    nxt = [i + 1 if i + 1 < n else -1 for i in range(n)]
    prev = [i - 1 for i in range(n)]
    version = [0] * n
    heap: List[tuple] = []

    def enqueue(left: int) -> None:
        if left < 0 or nxt[left] < 0:
            return
        right = nxt[left]
        value = score(sym[left], sym[right])
        if value is None or not value > float("-inf"):
            return
        heapq.heappush(heap, (-value, left, right, version[left], version[right]))

    for i in range(n - 1):
        enqueue(i)
    while heap:
        _, left, right, lv, rv = heapq.heappop(heap)
        if nxt[left] != right or version[left] != lv or version[right] != rv:
            continue
        sym[left] += sym[right]
        version[left] += 1
        version[right] += 1
        nxt[left] = nxt[right]
        if nxt[right] >= 0:
            prev[nxt[right]] = left
        nxt[right] = -1
        enqueue(prev[left])
        enqueue(left)
    out, i = [], 0
    while i >= 0:
        out.append(sym[i])
        i = nxt[i]
    return out


def _utf8(text: str) -> bytes:
    """TextEncoder: UTF-8 with each lone surrogate as U+FFFD."""
    try:
        return text.encode("utf-8")
    except UnicodeEncodeError:
        return "".join("\ufffd" if 0xD800 <= ord(c) <= 0xDFFF else c for c in text).encode("utf-8")


def _decode_stream(data: bytes) -> str:
    """TextDecoder().decode(bytes, {stream: true}) on a fresh decoder: invalid sequences
    become U+FFFD, an unfinished trailing sequence is withheld."""
    return codecs.getincrementaldecoder("utf-8")(errors="replace").decode(data, final=False)


def _meta(m: Mapping, key: str, default=None):
    return m.get(key, default) if hasattr(m, "get") else default


# ------------------------------------------------------------------ SentencePiece (tokenizer.ts)


class Tokenizer:
    """SentencePiece BPE merge scores from GGUF, with UTF-8 byte fallback (Gemma)."""

    def __init__(self, m: Mapping) -> None:
        if _meta(m, "tokenizer.ggml.model") != "llama":
            raise ValueError("Only the Gemma SentencePiece tokenizer is supported.")
        self.tokens: List[str] = list(_meta(m, "tokenizer.ggml.tokens") or [])
        self.scores: List[float] = list(_meta(m, "tokenizer.ggml.scores") or [])
        types = _meta(m, "tokenizer.ggml.token_type")
        self.types: Optional[List[int]] = list(types) if types is not None else None
        if not self.tokens or len(self.tokens) != len(self.scores):
            raise ValueError("Invalid tokenizer metadata.")
        self.ids: Dict[str, int] = {}
        for i, s in enumerate(self.tokens):
            self.ids[s] = i
        self.bos = int(_meta(m, "tokenizer.ggml.bos_token_id", 2))
        self.eos = {int(_meta(m, "tokenizer.ggml.eos_token_id", 1)), self.special("<end_of_turn>")}
        # GGUF's SentencePiece default is true unless the model explicitly overrides it.
        self.prefix = _meta(m, "tokenizer.ggml.add_space_prefix") is not False

    def _type(self, i: int) -> int:
        return self.types[i] if self.types is not None and i < len(self.types) else 1

    def special(self, s: str) -> int:
        i = self.ids.get(s)
        if i is None:
            raise ValueError(f"Tokenizer lacks {s}.")
        return i

    def encode_text(self, text: str) -> List[int]:
        # identity normalization; U+2581 stands for a space
        chars = ["▁" if c == " " else c for c in ((" " if self.prefix else "") + text)]

        def score(a: str, b: str) -> Optional[float]:
            i = self.ids.get(a + b)
            return self.scores[i] if i is not None and self._type(i) == 1 else None

        out: List[int] = []
        for symbol in merge_symbols(chars, score):
            i = self.ids.get(symbol)
            if i is not None and self._type(i) == 1:
                out.append(i)
            else:
                out.extend(self.special(f"<0x{b:02X}>") for b in _utf8(symbol))
        return out

    def chat(self, messages: Sequence[Mapping]) -> List[int]:
        ids = [self.bos]
        for msg in messages:
            ids.append(self.special("<start_of_turn>"))
            role = "model" if msg["role"] == "assistant" else "user"
            ids.extend(self.encode_text(f"{role}\n{msg['content'].strip()}"))
            ids.append(self.special("<end_of_turn>"))
            ids.extend(self.encode_text("\n"))
        ids.append(self.special("<start_of_turn>"))
        ids.extend(self.encode_text("model\n"))
        return ids

    def decode(self, ids: Sequence[int]) -> str:
        data = bytearray()
        for i in ids:
            t = self.tokens[i] if 0 <= i < len(self.tokens) else ""
            if len(t) == 6 and t.startswith("<0x") and t.endswith(">") and all(c in "0123456789ABCDEF" for c in t[3:5]):
                data.append(int(t[3:5], 16))
            elif self._type(i) != 3:
                data += _utf8(t.replace("▁", " "))
        return _decode_stream(bytes(data))


# ------------------------------------------------------------------ byte-level BPE (gpt2-tokenizer.ts)

# ECMAScript \s (white space and line terminators), which the reference's patterns use.
_WS = "\\t\\n\\x0b\\x0c\\r \\xa0\\u1680\\u2000-\\u200a\\u2028\\u2029\\u202f\\u205f\\u3000\\ufeff"
_S = f"[{_WS}]"
_NS = f"[^{_WS}]"
_CONTRACTION = "'[sStT]|'[rR][eE]|'[vV][eE]|'[mM]|'[lL][lL]|'[dD]"
_LLAMA = (f"(?:{_CONTRACTION})|[^\\r\\n\\p{{L}}\\p{{N}}]?\\p{{L}}+|\\p{{N}}{{1,3}}| ?[^{_WS}\\p{{L}}\\p{{N}}]+[\\r\\n]*"
          f"|{_S}*[\\r\\n]+|{_S}+(?!{_NS})|{_S}+")
_PATTERNS = {
    "llama-bpe": _LLAMA, "llama3": _LLAMA, "smollm": _LLAMA, "deepseek-llm": _LLAMA,
    "qwen2": (f"(?:{_CONTRACTION})|[^\\r\\n\\p{{L}}\\p{{N}}]?\\p{{L}}+|\\p{{N}}| ?[^{_WS}\\p{{L}}\\p{{N}}]+[\\r\\n]*"
              f"|{_S}*[\\r\\n]+|{_S}+(?!{_NS})|{_S}+"),
    "qwen35": (f"(?:{_CONTRACTION})|[^\\r\\n\\p{{L}}\\p{{N}}]?[\\p{{L}}\\p{{M}}]+|\\p{{N}}| ?[^{_WS}\\p{{L}}\\p{{M}}\\p{{N}}]+[\\r\\n]*"
               f"|{_S}*[\\r\\n]+|{_S}+(?!{_NS})|{_S}+"),
    "gpt2": f"(?:{_CONTRACTION})| ?\\p{{L}}+| ?\\p{{N}}+| ?[^{_WS}\\p{{L}}\\p{{N}}]+|{_S}+(?!{_NS})|{_S}+",
    "default": f"(?:{_CONTRACTION})| ?\\p{{L}}+| ?\\p{{N}}+| ?[^{_WS}\\p{{L}}\\p{{N}}]+|{_S}+(?!{_NS})|{_S}+",
}
_COMPILED: Dict[str, "regex.Pattern"] = {}


def pre_tokenizer(name) -> "regex.Pattern":
    """The pre-tokenizer of a ``tokenizer.ggml.pre`` name (gpt2-tokenizer.ts:21-27);
    unknown names get the default pattern."""
    key = name if isinstance(name, str) and name in _PATTERNS else "default"
    if key not in _COMPILED:
        _COMPILED[key] = regex.compile(_PATTERNS[key])
    return _COMPILED[key]


def chat_style_for(m: Mapping, ids: Mapping[str, int]) -> str:
    """'llama3', 'chatml' or 'mistral' from the GGUF chat template, else from the control
    tokens the vocabulary holds (gpt2-tokenizer.ts:32-44)."""
    template = _meta(m, "tokenizer.chat_template")
    if isinstance(template, str):
        if "<|start_header_id|>" in template:
            return "llama3"
        if "<|im_start|>" in template:
            return "chatml"
        if "[INST]" in template:
            return "mistral"
    if "<|start_header_id|>" in ids:
        return "llama3"
    if "<|im_start|>" in ids:
        return "chatml"
    if "[INST]" in ids:
        return "mistral"
    raise ValueError("This model does not declare a chat template this runtime understands. "
                     "Use a chat or instruct GGUF (Llama 3, Qwen2/3, Mistral).")


_END_TOKENS = ("<|eot_id|>", "<|eom_id|>", "<|end_of_text|>", "<|im_end|>", "<|endoftext|>", "<|end|>", "</s>",
               "<end_of_turn>")


def _ranked_merge(piece: str, alphabet: List[str], ranks: Mapping[str, int]) -> List[str]:
    return merge_symbols([alphabet[b] for b in _utf8(piece)],
                         lambda a, b: (-ranks[a + " " + b]) if (a + " " + b) in ranks else None)


class Gpt2Tokenizer:
    """Byte-level BPE with the GPT-2 alphabet and ranked merges."""

    def __init__(self, m: Mapping) -> None:
        if _meta(m, "tokenizer.ggml.model") != "gpt2":
            raise ValueError("This model does not use a byte-level BPE tokenizer.")
        tokens = _meta(m, "tokenizer.ggml.tokens")
        merges = _meta(m, "tokenizer.ggml.merges")
        types = _meta(m, "tokenizer.ggml.token_type")
        if not isinstance(tokens, (list, tuple)) or not isinstance(merges, (list, tuple)) or \
                any(not isinstance(s, str) or " " not in s for s in merges):
            raise ValueError("Invalid byte-BPE tokenizer metadata.")
        self.tokens: List[str] = list(tokens)
        self.types: List[int] = list(types) if isinstance(types, (list, tuple)) else []
        self.ids: Dict[str, int] = {}
        for i, s in enumerate(self.tokens):
            self.ids[s] = i
        self.ranks: Dict[str, int] = {}
        for r, s in enumerate(merges):
            self.ranks[s] = r
        self.alphabet = byte_alphabet()
        self.bytes = {s: b for b, s in enumerate(self.alphabet)}
        self.pattern = pre_tokenizer(_meta(m, "tokenizer.ggml.pre"))
        self.eos = set()
        for key in ("tokenizer.ggml.eos_token_id", "tokenizer.ggml.eot_token_id"):
            v = _meta(m, key)
            if isinstance(v, int) and not isinstance(v, bool) and v >= 0:
                self.eos.add(v)
        many = _meta(m, "tokenizer.ggml.eos_token_ids")
        if isinstance(many, (list, tuple)):
            self.eos.update(int(v) for v in many if isinstance(v, int) and not isinstance(v, bool))
        for name in _END_TOKENS:
            if name in self.ids:
                self.eos.add(self.ids[name])
        self.style = chat_style_for(m, self.ids)

    def _control(self, name: str, ids: List[int]) -> None:
        if name in self.ids:
            ids.append(self.ids[name])
        else:
            ids.extend(self.encode_text(name))

    def encode_text(self, text: str) -> List[int]:
        out: List[int] = []
        for match in self.pattern.finditer(text):
            for symbol in _ranked_merge(match.group(0), self.alphabet, self.ranks):
                i = self.ids.get(symbol)
                if i is None:
                    raise ValueError("Invalid byte-BPE merge result.")
                out.append(i)
        return out

    def chat(self, messages: Sequence[Mapping]) -> List[int]:
        ids: List[int] = []
        text = lambda s: ids.extend(self.encode_text(s))  # noqa: E731
        if self.style == "llama3":
            if "<|begin_of_text|>" in self.ids:
                ids.append(self.ids["<|begin_of_text|>"])
            for msg in messages:
                self._control("<|start_header_id|>", ids)
                text("assistant" if msg["role"] == "assistant" else "user")
                self._control("<|end_header_id|>", ids)
                text("\n\n")
                text(msg["content"].strip())
                self._control("<|eot_id|>", ids)
            self._control("<|start_header_id|>", ids)
            text("assistant")
            self._control("<|end_header_id|>", ids)
            text("\n\n")
        elif self.style == "chatml":
            for msg in messages:
                self._control("<|im_start|>", ids)
                text(f"{msg['role']}\n")
                text(msg["content"].strip())
                self._control("<|im_end|>", ids)
                text("\n")
            self._control("<|im_start|>", ids)
            text("assistant\n")
        else:
            if "<s>" in self.ids:
                ids.append(self.ids["<s>"])
            for msg in messages:
                if msg["role"] == "user":
                    self._control("[INST]", ids)
                    text(f" {msg['content'].strip()} ")
                    self._control("[/INST]", ids)
                else:
                    text(msg["content"].strip())
                    if "</s>" in self.ids:
                        ids.append(self.ids["</s>"])
        return ids

    def decode(self, ids: Sequence[int]) -> str:
        data = bytearray()
        for i in ids:
            if (self.types[i] if 0 <= i < len(self.types) else 1) == 3:
                continue
            for ch in (self.tokens[i] if 0 <= i < len(self.tokens) else ""):
                b = self.bytes.get(ch)
                if b is not None:
                    data.append(b)
        return _decode_stream(bytes(data))


# ------------------------------------------------------------------ Qwen (qwen-tokenizer.ts)


class QwenTokenizer:
    """Qwen's Unicode pre-tokenizer (contractions case-insensitive, letter/mark classes
    not), GPT-2 byte encoding and ranked BPE, after NFC normalization."""

    def __init__(self, m: Mapping) -> None:
        if _meta(m, "tokenizer.ggml.model") != "gpt2" or _meta(m, "tokenizer.ggml.pre") != "qwen35":
            raise ValueError("Qwen3.8 requires the qwen35 byte-BPE tokenizer.")
        tokens = _meta(m, "tokenizer.ggml.tokens")
        merges = _meta(m, "tokenizer.ggml.merges")
        types = _meta(m, "tokenizer.ggml.token_type")
        if not isinstance(tokens, (list, tuple)) or not isinstance(merges, (list, tuple)) or \
                not isinstance(types, (list, tuple)) or len(types) != len(tokens) or \
                any(not isinstance(s, str) or " " not in s for s in merges):
            raise ValueError("Invalid Qwen tokenizer metadata.")
        self.tokens: List[str] = list(tokens)
        self.types: List[int] = list(types)
        self.ids = {s: i for i, s in enumerate(self.tokens)}  # a repeated string keeps its last id
        self.ranks = {s: r for r, s in enumerate(merges)}
        self.alphabet = byte_alphabet()
        self.bytes = {s: b for b, s in enumerate(self.alphabet)}
        self.pattern = pre_tokenizer("qwen35")
        self.eos = {self.special("<|im_end|>"), self.special("<|endoftext|>")}

    def special(self, s: str) -> int:
        i = self.ids.get(s)
        if i is None:
            raise ValueError(f"Qwen tokenizer lacks {s}.")
        return i

    def encode_text(self, text: str) -> List[int]:
        out: List[int] = []
        for match in self.pattern.finditer(unicodedata.normalize("NFC", text)):
            for symbol in _ranked_merge(match.group(0), self.alphabet, self.ranks):
                i = self.ids.get(symbol)
                if i is None or self.types[i] != 1:
                    raise ValueError("Invalid byte-BPE merge result.")
                out.append(i)
        return out

    def chat(self, messages: Sequence[Mapping]) -> List[int]:
        def empty_thinking() -> List[int]:
            return [self.special("<think>"), *self.encode_text("\n\n"), self.special("</think>"), *self.encode_text("\n\n")]
        ids: List[int] = []
        for msg in messages:
            ids.append(self.special("<|im_start|>"))
            ids.extend(self.encode_text(msg["role"] + "\n"))
            if msg["role"] == "assistant":
                ids.extend(empty_thinking())
            ids.extend(self.encode_text(msg["content"].strip()))
            ids.append(self.special("<|im_end|>"))
            ids.extend(self.encode_text("\n"))
        # explicit non-thinking mode
        ids.append(self.special("<|im_start|>"))
        ids.extend(self.encode_text("assistant\n"))
        ids.extend(empty_thinking())
        return ids

    def decode(self, ids: Sequence[int]) -> str:
        data = bytearray()
        for i in ids:
            if not (0 <= i < len(self.types)) or self.types[i] != 1:
                continue
            for ch in self.tokens[i]:
                b = self.bytes.get(ch)
                if b is None:
                    raise ValueError("Invalid byte-BPE output token.")
                data.append(b)
        return _decode_stream(bytes(data))


def tokenizer_for(metadata: Mapping, architecture: str, family: str):
    """The model's tokenizer as engine.ts:67-69 picks it: qwen35 architecture -> Qwen, the
    dense family (llama / qwen2 / qwen3 architectures) -> byte-level BPE, else
    SentencePiece. None when the GGUF carries no tokenizer."""
    if _meta(metadata, "tokenizer.ggml.model") is None:
        return None
    if architecture == "qwen35":
        return QwenTokenizer(metadata)
    if family == "llama":
        return Gpt2Tokenizer(metadata)
    return Tokenizer(metadata)
