"""Byte-level BPE tokenizer and the Qwen3 chat template.

Mirrors nnmetal/src/tokenizer.zig (host code; nothing here touches the GPU):

* parses a Hugging Face ``tokenizer.json``: ``model.vocab`` (string -> id),
  ``model.merges`` ("a b" strings or ["a", "b"] pairs, rank = position) and
  ``added_tokens`` (special ones split the input before BPE) (:372-621);
* the GPT-2 byte <-> unicode map: bytes 33-126, 161-172 and 174-255 map to
  themselves, the other 68 to 256.. in byte order (:56-110);
* encode: special-token segments (longest match), then the reference's
  simplified GPT-4-style pre-tokenizer (contractions, optional non-letter +
  letters, 1-3 digits, symbol runs with an optional leading space, newline
  runs, other whitespace runs; bytes >= 0x80 count as letters) (:936-1063),
  then greedy BPE inside each chunk: repeatedly merge the leftmost pair of
  lowest rank whose concatenation is in the vocabulary, stopping when a
  ranked pair's concatenation is missing (:761-933);
* decode: vocabulary strings mapped back through the byte map, codepoints
  outside it passed through as UTF-8 (:1066-1135);
* apply_chat_template: ``<|im_start|>`` "user\\n" prompt ``<|im_end|>`` "\\n"
  ``<|im_start|>`` "assistant\\n", each piece encoded on its own
  (:330-367).

Limits and error names follow the reference (``TokenizerError.kind``).
The pre-tokenizer is the reference's approximation, not the Qwen3 regex:
on digit runs and some whitespace patterns its chunks differ from the
Hugging Face ``tokenizers`` library's.
"""
from __future__ import annotations

import json
import os

MAX_VOCAB_SIZE = 200_000
MAX_TOKEN_LENGTH = 512
MAX_SPECIAL_TOKENS = 256
MAX_INPUT_LENGTH = 1024 * 1024
MAX_ENCODE_TOKENS = 65_536
MAX_JSON_FILE_BYTES = 32 * 1024 * 1024


class TokenizerError(ValueError):
    def __init__(self, kind: str, msg: str):
        super().__init__(f"{kind}: {msg}")
        self.kind = kind


def _direct(b: int) -> bool:
    return 33 <= b <= 126 or 161 <= b <= 172 or b >= 174


def _build_byte_map():
    fwd, rev, extra = [0] * 256, {}, 0
    for b in range(256):
        if _direct(b):
            cp = b
        else:
            cp = 256 + extra
            extra += 1
        fwd[b] = cp
        rev[cp] = b
    return fwd, rev


BYTE_TO_CP, CP_TO_BYTE = _build_byte_map()


# -- pre-tokenizer (byte classification on raw UTF-8 bytes) -----------------------

def _is_letter(b: int) -> bool:
    return 97 <= b <= 122 or 65 <= b <= 90 or b >= 0x80


def _is_digit(b: int) -> bool:
    return 48 <= b <= 57


def _is_ws(b: int) -> bool:
    return b in (0x20, 0x09, 0x0A, 0x0D, 0x0B, 0x0C)


def _is_newline(b: int) -> bool:
    return b in (0x0A, 0x0D)


def _is_symbol(b: int) -> bool:
    return not _is_letter(b) and not _is_digit(b) and not _is_ws(b)


def next_pretoken_chunk(text: bytes) -> int:
    """Byte length of the next pre-tokenization chunk (nextPretokenChunk)."""
    n = min(len(text), MAX_INPUT_LENGTH)
    c0 = text[0]
    if c0 == 0x27 and n >= 2:                      # contractions
        c1 = text[1] | 0x20
        if c1 in b"stmd":
            return 2
        if n >= 3:
            c2 = text[2] | 0x20
            if (c1, c2) in ((0x72, 0x65), (0x76, 0x65), (0x6C, 0x6C)):   # re ve ll
                return 3
    if _is_letter(c0):                             # letters
        e = 0
        while e < n and _is_letter(text[e]):
            e += 1
        return e
    if n > 1 and not (_is_letter(c0) or _is_digit(c0)) and not _is_newline(c0) \
            and _is_letter(text[1]):               # one non-letter + letters
        e = 1
        while e < n and _is_letter(text[e]):
            e += 1
        return e
    if _is_digit(c0):                              # 1-3 digits
        e = 1
        while e < n and e < 3 and _is_digit(text[e]):
            e += 1
        return e
    if _is_symbol(c0):                             # symbol run
        e = 1
        while e < n and _is_symbol(text[e]):
            e += 1
        return e
    if c0 == 0x20 and n > 1 and _is_symbol(text[1]):   # space + symbols
        e = 2
        while e < n and _is_symbol(text[e]):
            e += 1
        return e
    if _is_newline(c0):                            # newline run
        e = 1
        while e < n and _is_newline(text[e]):
            e += 1
        return e
    if _is_ws(c0):                                 # other whitespace run
        e = 1
        while e < n and _is_ws(text[e]) and not _is_newline(text[e]):
            e += 1
        return e
    return 1


def _utf8_len(first: int) -> int:
    if first < 0xC0:
        return 1
    if first < 0xE0:
        return 2
    if first < 0xF0:
        return 3
    return 4


def decode_utf8_codepoint(b: bytes) -> int:
    """decodeUtf8Codepoint: the payload bits of a 1-4 byte sequence."""
    if len(b) == 1:
        return b[0]
    if len(b) == 2:
        return (b[0] & 0x1F) << 6 | (b[1] & 0x3F)
    if len(b) == 3:
        return (b[0] & 0x0F) << 12 | (b[1] & 0x3F) << 6 | (b[2] & 0x3F)
    return (b[0] & 0x07) << 18 | (b[1] & 0x3F) << 12 | (b[2] & 0x3F) << 6 | (b[3] & 0x3F)


def decode_token_to_bytes(token: str | bytes) -> bytes:
    """decodeTokenToBytes: map each codepoint of a vocabulary string back to
    its byte; codepoints outside the byte map pass through as UTF-8."""
    s = token.encode("utf-8") if isinstance(token, str) else bytes(token)
    out, i = bytearray(), 0
    while i < len(s):
        L = _utf8_len(s[i])
        if i + L > len(s):
            out.append(s[i])
            i += 1
            continue
        cp = decode_utf8_codepoint(s[i:i + L])
        if cp in CP_TO_BYTE:
            out.append(CP_TO_BYTE[cp])
        else:
            out += s[i:i + L]
        i += L
    return bytes(out)


class Tokenizer:
    """Tokenizer.initFromJson / encode / decode / applyChatTemplate."""

    def __init__(self):
        self.vocab_to_id: dict[str, int] = {}
        self.id_to_vocab: dict[int, str] = {}
        self.vocab_size = 0
        self.merge_ranks: dict[str, int] = {}
        self.special_tokens: list[tuple[bytes, int]] = []
        self.byte_to_token_id = [None] * 256
        self.eos_token_id = 0
        self.im_start_token_id = 0
        self.im_end_token_id = 0

    # -- construction -----------------------------------------------------------------
    @classmethod
    def from_file(cls, path: str | os.PathLike) -> "Tokenizer":
        size = os.path.getsize(path)
        if size > MAX_JSON_FILE_BYTES:
            raise TokenizerError("FileTooBig", f"{path}: {size} bytes > {MAX_JSON_FILE_BYTES}")
        with open(path, "rb") as f:
            return cls.from_json(f.read())

    @classmethod
    def from_json(cls, data: str | bytes) -> "Tokenizer":
        self = cls()
        try:
            root = json.loads(data)
        except (json.JSONDecodeError, UnicodeDecodeError) as e:
            raise TokenizerError("InvalidJson", str(e)) from None
        if not isinstance(root, dict):
            raise TokenizerError("InvalidJson", "JSON root is not an object")
        self._parse_model(root)
        self._parse_added(root)
        self._resolve_special_ids()
        for b in range(256):
            self.byte_to_token_id[b] = self.vocab_to_id.get(chr(BYTE_TO_CP[b]))
        return self

    def _parse_model(self, root):
        if "model" not in root:
            raise TokenizerError("MissingField", "missing 'model'")
        model = root["model"]
        if not isinstance(model, dict):
            raise TokenizerError("InvalidJson", "'model' is not an object")
        if "vocab" not in model:
            raise TokenizerError("MissingField", "missing 'model.vocab'")
        vocab = model["vocab"]
        if not isinstance(vocab, dict):
            raise TokenizerError("InvalidJson", "'model.vocab' is not an object")
        for key, v in vocab.items():
            if not isinstance(v, int) or isinstance(v, bool) or not 0 <= v < 2 ** 32:
                raise TokenizerError("InvalidVocabEntry", f"vocab entry {key!r}: {v!r}")
            if v >= MAX_VOCAB_SIZE:
                raise TokenizerError("VocabTooLarge", f"vocab ID {v} >= {MAX_VOCAB_SIZE}")
            self.vocab_to_id[key] = v
            self.id_to_vocab[v] = key
            self.vocab_size = max(self.vocab_size, v + 1)
        merges = model.get("merges")
        if merges is None:
            return
        if not isinstance(merges, list):
            raise TokenizerError("InvalidJson", "'model.merges' is not an array")
        for rank, m in enumerate(merges):
            if isinstance(m, str):
                self.merge_ranks[m] = rank
            elif isinstance(m, list) and len(m) == 2 and all(isinstance(p, str) for p in m):
                self.merge_ranks[f"{m[0]} {m[1]}"] = rank
            else:
                raise TokenizerError("InvalidMergeEntry", f"merge {rank}: {m!r}")

    def _parse_added(self, root):
        added = root.get("added_tokens")
        if added is None:
            return
        if not isinstance(added, list):
            raise TokenizerError("InvalidJson", "'added_tokens' is not an array")
        for item in added:
            if not isinstance(item, dict):
                continue
            i = item.get("id")
            if not (isinstance(i, int) and not isinstance(i, bool) and 0 <= i < 2 ** 32):
                continue
            if "content" not in item:
                continue                    # the reference skips entries it cannot read
            content = item["content"]
            if not isinstance(content, str):
                continue
            if i < MAX_VOCAB_SIZE:
                self.id_to_vocab.setdefault(i, content)
                if not self.id_to_vocab[i]:
                    self.id_to_vocab[i] = content
                self.vocab_to_id[content] = i
                self.vocab_size = max(self.vocab_size, i + 1)
            if item.get("special") is True:
                if len(self.special_tokens) >= MAX_SPECIAL_TOKENS:
                    continue
                self.special_tokens.append((content.encode("utf-8"), i))

    def _resolve_special_ids(self):
        for content, i in self.special_tokens:
            if content == b"<|endoftext|>":
                self.eos_token_id = i
            elif content == b"<|im_start|>":
                self.im_start_token_id = i
            elif content == b"<|im_end|>":
                self.im_end_token_id = i

    @property
    def special_token_count(self) -> int:
        return len(self.special_tokens)

    # -- encode -----------------------------------------------------------------------
    def _special_at(self, text: bytes, pos: int):
        best = None
        for content, i in self.special_tokens:
            if (best is None or len(content) > len(best[0])) and text.startswith(content, pos):
                best = (content, i)
        return best

    def encode(self, text: str | bytes) -> list[int]:
        data = text.encode("utf-8") if isinstance(text, str) else bytes(text)
        if len(data) > MAX_INPUT_LENGTH:
            raise TokenizerError("InputTooLong", f"{len(data)} bytes > {MAX_INPUT_LENGTH}")
        out: list[int] = []
        pos = 0
        while pos < len(data):
            st = self._special_at(data, pos)
            if st is not None:
                out.append(st[1])
                pos += len(st[0])
            else:
                end = pos + 1
                while end < len(data) and self._special_at(data, end) is None:
                    end += 1
                seg = data[pos:end]
                p = 0
                while p < len(seg):
                    n = next_pretoken_chunk(seg[p:])
                    out += self._encode_chunk(seg[p:p + n])
                    p += n
                pos = end
            if len(out) > MAX_ENCODE_TOKENS:
                raise TokenizerError("OutputBufferTooSmall", f"more than {MAX_ENCODE_TOKENS} tokens")
        return out

    def _encode_chunk(self, chunk: bytes) -> list[int]:
        if len(chunk) > MAX_TOKEN_LENGTH:
            raise TokenizerError("ChunkTooLong", f"{len(chunk)} bytes > {MAX_TOKEN_LENGTH}")
        toks = []
        for b in chunk:
            t = self.byte_to_token_id[b]
            if t is None:
                raise TokenizerError("UnknownByte", f"no base token for byte 0x{b:02x}")
            toks.append(t)
        return self.bpe_merge(toks)

    def bpe_merge(self, tokens: list[int]) -> list[int]:
        """bpeMerge: merge the leftmost lowest-rank pair until none is ranked
        (or a ranked pair's concatenation is not in the vocabulary)."""
        toks = list(tokens)
        while len(toks) > 1:
            best_rank, best_i = None, 0
            for i in range(len(toks) - 1):
                a, b = self.id_to_vocab.get(toks[i], ""), self.id_to_vocab.get(toks[i + 1], "")
                r = self.merge_ranks.get(a + " " + b)
                if r is not None and (best_rank is None or r < best_rank):
                    best_rank, best_i = r, i
            if best_rank is None:
                break
            merged = self.vocab_to_id.get(self.id_to_vocab[toks[best_i]] +
                                          self.id_to_vocab[toks[best_i + 1]])
            if merged is None:
                break
            toks[best_i:best_i + 2] = [merged]
        return toks

    # -- decode -----------------------------------------------------------------------
    def decode(self, ids) -> bytes:
        ids = list(ids)
        if len(ids) > MAX_ENCODE_TOKENS:
            raise TokenizerError("OutputBufferTooSmall", f"more than {MAX_ENCODE_TOKENS} tokens")
        out = bytearray()
        for i in ids:
            s = self.id_to_vocab.get(int(i), "") if 0 <= int(i) < self.vocab_size else ""
            if not s:
                raise TokenizerError("UnknownTokenId", f"unknown token ID {int(i)}")
            out += decode_token_to_bytes(s)
        return bytes(out)

    # -- chat template ----------------------------------------------------------------
    def apply_chat_template(self, prompt: str | bytes) -> list[int]:
        return ([self.im_start_token_id] + self.encode("user\n") + self.encode(prompt)
                + [self.im_end_token_id] + self.encode("\n") + [self.im_start_token_id]
                + self.encode("assistant\n"))

    def stop_tokens(self) -> list[int]:
        """generate's stop tokens: <|endoftext|> and <|im_end|>
        (bonsai_golden.zig:142-146)."""
        return [self.eos_token_id, self.im_end_token_id]
