"""Host WordPiece tokenizer (C++, futon_amd/csrc/host/tokenizer.cpp) against
the reference's tokenizer tests (native/tokenizer_test.go): the committed
bert-base-uncased vocab hash, the HF-fast-tokenizer fixtures for three
models at their max_seq_len and at 16, special handling, and well-formed
output for arbitrary bytes."""
import hashlib
import json
import os
import random

import pytest

from futon_amd import native

HERE = os.path.dirname(os.path.abspath(__file__))
VOCAB = os.path.join(HERE, "golden", "vocab_bert_uncased.txt")
FIXTURES = os.path.join(HERE, "golden", "tokenizer_fixtures.json")
EXPECTED_VOCAB_SHA256 = "07eced375cec144d27c900241f3e339478dec958f92fddbc551f295c992038a3"  # tokenizer_test.go:19


def default_tok():
    return native.NewTokenizer(VOCAB, {"do_lower_case": True, "tokenize_chinese_chars": True})


def test_committed_vocab_hash():
    assert hashlib.sha256(open(VOCAB, "rb").read()).hexdigest() == EXPECTED_VOCAB_SHA256


def fixture_cases():
    fx = json.load(open(FIXTURES))
    for model, m in sorted(fx["models"].items()):
        for c in m["cases"]:
            yield pytest.param(model, m["max_seq_len"], c, id=f"{model}:{c['name']}")


@pytest.fixture(scope="module")
def tok():
    return default_tok()


def test_fixture_corpus_size():
    fx = json.load(open(FIXTURES))
    assert len(fx["models"]) == 3
    for m in fx["models"].values():
        assert len(m["cases"]) >= 24


@pytest.mark.parametrize("model,max_seq_len,case", list(fixture_cases()))
def test_tokenizer_conformance(tok, model, max_seq_len, case):
    assert tok.Encode(case["text"], max_seq_len) == case["ids"], case["name"]
    assert tok.Encode(case["text"], 16) == case["ids_max16"], case["name"]


def test_tokenizer_specials(tok):
    assert tok.VocabSize() == 30522
    for text in ["", "   \t\n "]:
        assert tok.Encode(text, 512) == [101, 102]
    # Literal special tokens split the raw text into independent segments.
    assert tok.Encode("[CLS]x[SEP]", 512) == [101, 101, tok.Encode("x", 512)[1], 102, 102]
    assert tok.Encode("hello", 2) == [101, 102]
    assert tok.Encode("hello", 0) == [101, 102]


def test_tokenizer_missing_vocab():
    with pytest.raises(native.PackError):
        native.NewTokenizer(os.path.join(HERE, "golden", "does-not-exist.txt"), {})


def test_tokenizer_special_not_in_vocab(tmp_path):
    p = tmp_path / "v.txt"
    p.write_text("[PAD]\n[UNK]\n[CLS]\n[SEP]\nhello\n")
    with pytest.raises(native.PackError, match="MASK"):
        native.NewTokenizer(str(p), {})


def test_tokenizer_vocab_lines(tmp_path):
    """bufio.ScanLines semantics: CRLF trimmed, no trailing empty token, a
    repeated token keeps its last id."""
    p = tmp_path / "v.txt"
    p.write_bytes(b"[PAD]\r\n[UNK]\n[CLS]\n[SEP]\n[MASK]\nhello\nworld\nhello")
    t = native.NewTokenizer(str(p), {"do_lower_case": True})
    assert t.VocabSize() == 7
    assert t.Encode("Hello world", 16) == [2, 7, 6, 3]


def test_tokenizer_fuzz_well_formed(tok):
    """FuzzTokenizerEncode (tokenizer_test.go): arbitrary bytes never crash
    and always give [CLS] … [SEP] within bounds and within the vocab."""
    rng = random.Random(1234)
    seeds = ["", " ", "hello world", "Élodie café ☃", "自然言語処理", "[CLS][SEP][UNK]", "a" * 300,
             "ﬁ ﬂ Ǆ ǅ İ ẞ", "́̀a̧", "한국어 텍스트", "\x00\x01\x7f​﻿"]
    cases = [s.encode() for s in seeds]
    for _ in range(300):
        n = rng.randrange(0, 64)
        cases.append(bytes(rng.randrange(256) for _ in range(n)))
    for raw in cases:
        for m in (2, 3, 16, 512):
            ids = tok.Encode(raw, m)
            assert 2 <= len(ids) <= max(m, 2)
            assert ids[0] == 101 and ids[-1] == 102
            assert all(0 <= i < 30522 for i in ids)
