"""Tokenizer (CPU): nnmetal/src/tokenizer_test.zig restated case by case,
the parser's error paths, and an independent check against the Hugging Face
``tokenizers`` library: a byte-level BPE trained here (no download) must
encode the same ids and decode the same bytes as this tokenizer on text
where the reference's simplified pre-tokenizer and the GPT-2 regex agree
(words, single spaces, punctuation; no digits, no runs of spaces).
"""
import json

import pytest

from nnzap_amd import tokenizer as T


def tok(vocab, merges=(), added=()):
    return T.Tokenizer.from_json(json.dumps(
        {"model": {"type": "BPE", "vocab": vocab, "merges": list(merges)},
         "added_tokens": list(added)}))


# -- tokenizer_test.zig ---------------------------------------------------------------

def test_byte_map_is_a_bijection():
    cps = T.BYTE_TO_CP
    assert len(set(cps)) == 256 and max(cps) < 324
    assert all(T.CP_TO_BYTE[cp] == b for b, cp in enumerate(cps))


def test_direct_mapped_bytes():
    for b in list(range(33, 127)) + list(range(161, 173)) + list(range(174, 256)):
        assert T.BYTE_TO_CP[b] == b
    assert T.BYTE_TO_CP[32] != 32 and T.BYTE_TO_CP[32] >= 256
    assert T.BYTE_TO_CP[32] == 0x120          # GPT-2's space, "Ġ"


@pytest.mark.parametrize("text,n", [
    (b"hello world", 5), (b" world", 6), (b"a", 1),                   # letter chunks
    (b"123456", 3), (b"42abc", 2), (b"7", 1),                         # digit chunks
    (b"'s great", 2), (b"'t do", 2), (b"'re done", 3), (b"'ll go", 3),  # contractions
    (b"!!!", 3), (b" !!!", 4),                                        # symbols
    (b"\n", 1), (b"\n\n", 2), (b"   abc", 3),                         # whitespace
])
def test_pretokenizer(text, n):
    assert T.next_pretoken_chunk(text) == n


def test_utf8_codepoint():
    assert T.decode_utf8_codepoint(b"a") == ord("a")
    assert T.decode_utf8_codepoint(bytes([0xC4, 0xA0])) == 0x120
    assert T.decode_utf8_codepoint(bytes([0xE2, 0x82, 0xAC])) == 0x20AC


def test_bpe_merge_known_sequence():
    t = tok({"a": 0, "b": 1, "c": 2, "ab": 3, "abc": 4}, ["a b", "ab c"])
    assert t.vocab_size == 5 and t.id_to_vocab[0] == "a" and t.id_to_vocab[4] == "abc"
    assert t.bpe_merge([0, 1, 2]) == [4]


def test_encode_decode_round_trip_ascii():
    t = tok({"a": 0, "b": 1, "c": 2, "d": 3, "ab": 4, "cd": 5, "abcd": 6},
            ["a b", "c d", "ab cd"])
    assert t.encode("abcd") == [6]
    assert t.decode([6]) == b"abcd"


def test_encode_preserves_partial_merges():
    t = tok({"a": 0, "b": 1, "x": 2, "c": 3, "d": 4, "ab": 5, "cd": 6}, ["a b", "c d"])
    assert t.encode("abxcd") == [5, 2, 6]


def test_special_tokens_not_split():
    t = tok({"a": 0, "b": 1, "ab": 2, "<s>": 10}, ["a b"],
            [{"id": 10, "content": "<s>", "special": True}])
    assert t.special_token_count == 1
    assert t.encode("ab<s>ab") == [2, 10, 2]


def test_decode_special_tokens():
    t = tok({"a": 0, "b": 1, "ab": 2, "<s>": 10}, ["a b"],
            [{"id": 10, "content": "<s>", "special": True}])
    assert t.decode([2, 10, 2]) == b"ab<s>ab"


def test_empty_input():
    assert tok({"a": 0}).encode("") == []


def test_single_bytes_without_merges():
    assert tok({"a": 0, "b": 1, "c": 2}).encode("abc") == [0, 1, 2]


def test_special_ids_resolved():
    t = tok({"a": 0}, added=[{"id": 100, "content": "<|endoftext|>", "special": True},
                             {"id": 101, "content": "<|im_start|>", "special": True},
                             {"id": 102, "content": "<|im_end|>", "special": True}])
    assert (t.eos_token_id, t.im_start_token_id, t.im_end_token_id) == (100, 101, 102)


def test_chat_template_structure():
    vocab = {c: i for i, c in enumerate("Hiuseratn")}
    vocab.update({"Ċ": 20, "<|im_start|>": 100, "<|im_end|>": 101})   # "\n" is byte 0x0A
    t = tok(vocab, added=[{"id": 100, "content": "<|im_start|>", "special": True},
                          {"id": 101, "content": "<|im_end|>", "special": True}])
    assert (t.im_start_token_id, t.im_end_token_id) == (100, 101)
    ids = t.apply_chat_template("Hi")
    enc = lambda s: [vocab[c] for c in s]
    assert ids == ([100] + enc("user") + [20] + enc("Hi") + [101, 20, 100] + enc("assistant")
                   + [20])


def test_decode_token_to_bytes():
    assert T.decode_token_to_bytes("hello") == b"hello"
    assert T.decode_token_to_bytes(bytes([0xC4, 0xA0])) == b" "
    assert T.decode_token_to_bytes("€") == "€".encode()   # outside the map: as is


def test_merge_priority_lowest_rank():
    t = tok({"a": 0, "b": 1, "c": 2, "ab": 3, "bc": 4}, ["b c", "a b"])
    assert t.encode("abc") == [0, 4]


# -- error paths and limits ------------------------------------------------------------

@pytest.mark.parametrize("doc,kind", [
    ("[1]", "InvalidJson"), ("{", "InvalidJson"), ("{}", "MissingField"),
    ('{"model": 3}', "InvalidJson"), ('{"model": {}}', "MissingField"),
    ('{"model": {"vocab": {"a": -1}}}', "InvalidVocabEntry"),
    ('{"model": {"vocab": {"a": "x"}}}', "InvalidVocabEntry"),
    ('{"model": {"vocab": {"a": 200000}}}', "VocabTooLarge"),
    ('{"model": {"vocab": {"a": 0}, "merges": [["a"]]}}', "InvalidMergeEntry"),
    ('{"model": {"vocab": {"a": 0}, "merges": [3]}}', "InvalidMergeEntry"),
])
def test_parse_errors(doc, kind):
    with pytest.raises(T.TokenizerError) as e:
        T.Tokenizer.from_json(doc)
    assert e.value.kind == kind


def test_encode_decode_errors():
    t = tok({"a": 0, "b": 1})
    with pytest.raises(T.TokenizerError) as e:
        t.encode("abz")
    assert e.value.kind == "UnknownByte"
    with pytest.raises(T.TokenizerError) as e:
        t.decode([0, 5])
    assert e.value.kind == "UnknownTokenId"
    with pytest.raises(T.TokenizerError) as e:
        t.encode("a" * (T.MAX_TOKEN_LENGTH + 1))
    assert e.value.kind == "ChunkTooLong"


def test_pair_merges_and_longest_special_match():
    t = tok({"a": 0, "b": 1, "ab": 2, "<x>": 5, "<x>>": 6}, [["a", "b"]],
            [{"id": 5, "content": "<x>", "special": True},
             {"id": 6, "content": "<x>>", "special": True}])
    assert t.encode("ab<x>>ab") == [2, 6, 2]


# -- independent check: Hugging Face tokenizers on a freshly trained BPE ---------------

CORPUS = [
    "The capital of France is Paris. The capital of Italy is Rome!",
    "Tokenizers split text into pieces, and pieces into merges; merges make words.",
    "A quick brown fox jumps over the lazy dog. Is it quick? Yes, it is quick.",
    "Café crème brûlée, naïve façade: déjà vu for the résumé.",
    "We'll see what they've done; it's fine, isn't it? You're right, I'm sure.",
] * 20

AGREE = [
    "The capital of France is Paris.",
    "Is it quick? Yes, it is quick!",
    "Café crème, naïve façade: déjà vu.",
    "We'll see what they've done; it's fine.",
    "merges make words, pieces make merges",
    "Unseen words like zyxwv still encode byte by byte.",
]


@pytest.fixture(scope="module")
def trained():
    tokenizers = pytest.importorskip("tokenizers")
    from tokenizers import decoders, models, pre_tokenizers, trainers
    hf = tokenizers.Tokenizer(models.BPE())
    hf.pre_tokenizer = pre_tokenizers.ByteLevel(add_prefix_space=False)
    hf.decoder = decoders.ByteLevel()
    trainer = trainers.BpeTrainer(vocab_size=700, show_progress=False,
                                  special_tokens=["<|endoftext|>", "<|im_start|>", "<|im_end|>"],
                                  initial_alphabet=pre_tokenizers.ByteLevel.alphabet())
    hf.train_from_iterator(CORPUS, trainer)
    return hf, T.Tokenizer.from_json(hf.to_str())


@pytest.mark.parametrize("text", AGREE)
def test_matches_hf_tokenizers(trained, text):
    hf, t = trained
    want = hf.encode(text, add_special_tokens=False).ids
    got = t.encode(text)
    assert got == want
    assert t.decode(got) == text.encode()
    assert hf.decode(got) == text


def test_chat_template_with_trained_vocab(trained):
    hf, t = trained
    ids = t.apply_chat_template("The capital of France is")
    assert ids[0] == t.im_start_token_id == hf.token_to_id("<|im_start|>")
    assert t.decode(ids) == (b"<|im_start|>user\nThe capital of France is<|im_end|>\n"
                             b"<|im_start|>assistant\n")
    assert t.stop_tokens() == [hf.token_to_id("<|endoftext|>"), hf.token_to_id("<|im_end|>")]
