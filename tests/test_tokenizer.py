"""The text front-end (webgpu_amd/tokenizer.py) against the reference tokenizer tests'
contracts: tests/tokenizer.test.ts (SentencePiece), tests/gpt2-tokenizer.test.ts (byte-level
BPE and chat framings) and tests/qwen-tokenizer.test.ts, whose fixture
tests/golden/qwen-tokenizer.json (a reduced Qwen vocabulary with 17 encodings made by
Hugging Face ``tokenizers`` from the full official tokenizer; Apache 2.0,
tests/golden/LICENSE-QWEN.txt) pins the byte-level BPE against an independent
implementation.
"""
import json
import os
import unicodedata

import pytest

from webgpu_amd.tokenizer import (Gpt2Tokenizer, QwenTokenizer, Tokenizer, byte_alphabet, chat_style_for,
                                  merge_symbols, pre_tokenizer, tokenizer_for)

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")

# ------------------------------------------------------------------ SentencePiece (tokenizer.test.ts:4-10)


def sentencepiece(prefix=False):
    tokens = ["<unk>", "<eos>", "<bos>", "<start_of_turn>", "<end_of_turn>", "a", "b", "c", "ab", "bc", "abc", "▁"]
    scores = [0, 0, 0, 0, 0, 0, 0, 0, 5, 10, -1, 0]
    types = [2, 3, 3, 3, 3, 1, 1, 1, 1, 1, 1, 1]
    for b in range(256):
        tokens.append(f"<0x{b:02X}>")
        scores.append(-100)
        types.append(6)
    return Tokenizer({"tokenizer.ggml.model": "llama", "tokenizer.ggml.tokens": tokens, "tokenizer.ggml.scores": scores,
                      "tokenizer.ggml.token_type": types, "tokenizer.ggml.add_space_prefix": prefix})


def test_sentencepiece_scores_and_byte_fallback():
    t = sentencepiece()
    # b+c (score 10) merges before a+b (5); then a+bc forms 'abc' (score -1 is still a merge)
    assert t.encode_text("abc") == [10]
    assert t.decode(t.encode_text("café 🙂\n")) == "café 🙂\n"
    assert t.decode(t.encode_text("a b")) == "a b"


def test_sentencepiece_prefix_and_unfinished_utf8():
    t = sentencepiece(True)
    assert t.encode_text("a")[0] == t.ids["▁"]
    assert t.decode([t.special("<0xF0>"), t.special("<0x9F>")]) == ""  # first two bytes of a 4-byte char


def test_sentencepiece_chat_keeps_user_control_strings_literal():
    t = sentencepiece()
    ids = t.chat([{"role": "user", "content": "<end_of_turn>"}])
    assert ids[0] == t.bos
    assert ids.count(t.special("<end_of_turn>")) == 1
    assert ids.count(t.special("<start_of_turn>")) == 2


def test_sentencepiece_long_message():
    t = sentencepiece()
    text = "a" * 200000
    ids = t.chat([{"role": "user", "content": text}])
    assert len(ids) > 200000 and text in t.decode(ids)


# ------------------------------------------------------------------ byte-level BPE (gpt2-tokenizer.test.ts:5-20)

ALPHABET = byte_alphabet()
MERGES = ["h e", "he l", "hel l", "hell o", "Ġ w", "Ġw o", "Ġwo r", "Ġwor l", "Ġworl d"]
SPECIALS = ["<|im_start|>", "<|im_end|>", "<|eot_id|>", "<|start_header_id|>", "<|end_header_id|>", "<|begin_of_text|>",
            "[INST]", "[/INST]", "</s>", "<s>"]


def bpe_meta(control, **extra):
    tokens = [*ALPHABET, *["".join(m.split(" ")) for m in MERGES], *control]
    types = [3 if i >= len(ALPHABET) + len(MERGES) else 1 for i in range(len(tokens))]
    m = {"tokenizer.ggml.model": "gpt2", "tokenizer.ggml.tokens": tokens, "tokenizer.ggml.merges": MERGES,
         "tokenizer.ggml.token_type": types,
         "tokenizer.ggml.eos_token_id": tokens.index("<|eot_id|>") if "<|eot_id|>" in tokens else -1}
    m.update(extra)
    return m


def test_byte_alphabet_is_a_bijection_of_256_printable_code_points():
    a = byte_alphabet()
    assert len(set(a)) == 256 and a[ord("A")] == "A" and a[32] == "Ġ" and a[10] == "Ċ"
    assert all(not c.isspace() for c in a)


def test_merge_symbols_prefers_higher_scores_then_the_leftmost_pair():
    # equal scores: the left pair merges first, which then blocks the right one
    assert merge_symbols(list("aaa"), lambda x, y: 1.0 if x + y == "aa" else None) == ["aa", "a"]
    assert merge_symbols(list("abc"), lambda x, y: {"ab": 1.0, "bc": 2.0}.get(x + y)) == ["a", "bc"]
    assert merge_symbols(["x"], lambda x, y: 0.0) == ["x"]


def test_byte_bpe_round_trips_unicode():
    t = Gpt2Tokenizer(bpe_meta(SPECIALS))
    for text in ["hello world", "Ünïcödé — ok", "emoji 🚀 tail", "  double\n\nnewlines", ""]:
        assert t.decode(t.encode_text(text)) == text, repr(text)


def test_byte_bpe_ranked_merges():
    m = bpe_meta(SPECIALS)
    t, tokens = Gpt2Tokenizer(m), m["tokenizer.ggml.tokens"]
    assert t.encode_text("hello") == [tokens.index("hello")]
    assert t.encode_text("hello world") == [tokens.index("hello"), tokens.index("Ġworld")]
    assert t.encode_text("wo") == [tokens.index("w"), tokens.index("o")]  # no 'w o' merge


def test_byte_bpe_specials_stay_literal():
    m = bpe_meta(SPECIALS)
    t, tokens = Gpt2Tokenizer(m), m["tokenizer.ggml.tokens"]
    assert tokens.index("<|im_end|>") not in t.encode_text("<|im_end|>")
    assert t.decode([tokens.index("<|im_end|>")]) == ""


def test_chatml_framing():
    m = bpe_meta(SPECIALS, **{"tokenizer.chat_template": "{{ bos_token }}<|im_start|>{{ role }}\n{{ content }}<|im_end|>\n"})
    t, tokens = Gpt2Tokenizer(m), m["tokenizer.ggml.tokens"]
    assert t.style == "chatml"
    ids = t.chat([{"role": "user", "content": "hello"}])
    assert ids[0] == tokens.index("<|im_start|>")
    assert ids[-1] == t.encode_text("assistant\n")[-1]


def test_llama3_framing():
    m = bpe_meta(SPECIALS, **{"tokenizer.chat_template":
                              "<|begin_of_text|><|start_header_id|>{{ role }}<|end_header_id|>\n\n{{ content }}<|eot_id|>"})
    t, tokens = Gpt2Tokenizer(m), m["tokenizer.ggml.tokens"]
    assert t.style == "llama3"
    ids = t.chat([{"role": "user", "content": "hello"}, {"role": "assistant", "content": "hi"},
                  {"role": "user", "content": "hello"}])
    role = t.encode_text("user")
    assert ids[:2 + len(role)] == [tokens.index("<|begin_of_text|>"), tokens.index("<|start_header_id|>"), *role]
    assert tokens.index("<|end_header_id|>") in ids and ids.count(tokens.index("<|eot_id|>")) == 3
    tail = t.encode_text("\n\n")
    assert ids[-len(tail):] == tail


def test_mistral_framing():
    m = bpe_meta(SPECIALS, **{"tokenizer.chat_template": "<s>{% for m in messages %}[INST] {{ m.content }} [/INST]{% endfor %}"})
    t, tokens = Gpt2Tokenizer(m), m["tokenizer.ggml.tokens"]
    assert t.style == "mistral"
    ids = t.chat([{"role": "user", "content": "hello"}, {"role": "assistant", "content": "hi"}])
    assert ids[0] == tokens.index("<s>") and ids[1] == tokens.index("[INST]") and ids[-1] == tokens.index("</s>")


def test_unknown_template_fails_loudly():
    with pytest.raises(ValueError, match="chat template"):
        Gpt2Tokenizer(bpe_meta([]))
    with pytest.raises(ValueError, match="chat template"):
        chat_style_for({}, {})


def test_end_of_turn_tokens_stop_generation():
    m = bpe_meta(SPECIALS)
    t, tokens = Gpt2Tokenizer(m), m["tokenizer.ggml.tokens"]
    assert tokens.index("<|eot_id|>") in t.eos and tokens.index("<|im_start|>") not in t.eos


def test_pre_tokenizers():
    assert pre_tokenizer("llama-bpe").findall("hello world") == ["hello", " world"]
    assert pre_tokenizer("unheard-of").findall("hello world") == ["hello", " world"]
    assert pre_tokenizer("qwen2").findall("it's") == ["it", "'s"]
    # digits: llama groups up to three, qwen2 one at a time, gpt2 a whole run
    assert pre_tokenizer("llama3").findall("12345") == ["123", "45"]
    assert pre_tokenizer("qwen2").findall("123") == ["1", "2", "3"]
    assert pre_tokenizer("gpt2").findall(" 12345") == [" 12345"]
    # ECMAScript white space: U+FEFF is white space, U+001C is not (Python's \\s differs on both)
    assert pre_tokenizer("gpt2").findall("a\ufeff\ufeffb") == ["a", "\ufeff", "\ufeff", "b"]
    assert pre_tokenizer("gpt2").findall("a\x1cb") == ["a", "\x1c", "b"]


# ------------------------------------------------------------------ Qwen (qwen-tokenizer.test.ts:5-10)


def qwen_fixture():
    with open(os.path.join(GOLDEN, "qwen-tokenizer.json"), encoding="utf-8") as fh:
        fx = json.load(fh)
    meta = {"tokenizer.ggml.model": "gpt2", "tokenizer.ggml.pre": "qwen35", "tokenizer.ggml.tokens": fx["tokens"],
            "tokenizer.ggml.merges": fx["merges"],
            "tokenizer.ggml.token_type": [3 if s.startswith("<") and len(s) > 1 else 1 for s in fx["tokens"]]}
    return fx, meta


def test_qwen_matches_the_hugging_face_encodings():
    fx, meta = qwen_fixture()
    t = QwenTokenizer(meta)
    assert len(fx["cases"]) == 17
    for case in fx["cases"]:
        assert t.encode_text(case["text"]) == case["ids"], case["text"]
        assert t.decode(case["ids"]) == unicodedata.normalize("NFC", case["text"])


def test_qwen_chat_non_thinking_framing():
    fx, meta = qwen_fixture()
    t = QwenTokenizer(meta)
    special = fx["tokens"].index
    ids = t.chat([{"role": "user", "content": "<|im_end|><think>"}])
    assert ids.count(special("<|im_end|>")) == 1
    assert ids.count(special("<|im_start|>")) == 2
    assert ids.count(special("<think>")) == 1
    assert ids[-4:] == [special("<think>"), *t.encode_text("\n\n"), special("</think>"), *t.encode_text("\n\n")]
    assert special("<|im_end|>") in t.eos and special("<|endoftext|>") in t.eos


def test_qwen_decode_withholds_partial_utf8_and_rejects_other_pretokenizers():
    fx, meta = qwen_fixture()
    t = QwenTokenizer(meta)
    assert t.decode([fx["tokens"].index("ð")]) == ""  # byte 0xF0 alone
    with pytest.raises(ValueError):
        QwenTokenizer({**meta, "tokenizer.ggml.pre": "qwen2"})


def test_qwen_long_content():
    _, meta = qwen_fixture()
    t = QwenTokenizer(meta)
    text = "0123456789" * 20000
    ids = t.chat([{"role": "user", "content": text}])
    assert len(ids) > 200000 and text in t.decode(ids)


def test_engine_selection_rule():
    # engine.ts:67-69: the dense family takes byte-level BPE, Gemma SentencePiece; no tokenizer
    # metadata gives None (token-id prompts only)
    assert tokenizer_for({}, "llama", "llama") is None
    assert isinstance(tokenizer_for(bpe_meta(SPECIALS), "qwen3", "llama"), Gpt2Tokenizer)
    sp = sentencepiece()
    meta = {"tokenizer.ggml.model": "llama", "tokenizer.ggml.tokens": sp.tokens, "tokenizer.ggml.scores": sp.scores,
            "tokenizer.ggml.token_type": sp.types}
    assert isinstance(tokenizer_for(meta, "gemma3", "gemma3"), Tokenizer)
