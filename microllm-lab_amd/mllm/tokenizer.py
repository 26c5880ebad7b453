"""Byte-level BPE tokenizer and chat templates (engine/tokenizer.js:1-272).

The caller side of the decode path: text -> prompt ids -> (engine) -> ids ->
text.  `load_tokenizer(spec)` takes a parsed tokenizer.json (the files shipped
beside each model) and returns an object with the reference's API:
encode(text), decode(ids, skip_special=False), unk_id, special, vocab_size.

The algorithm (tokenizer.js:1-183):
- split the text into pieces with the GPT-2 pattern (contractions, letters,
  numbers, other symbols, whitespace), JavaScript's Unicode semantics for \\s;
- map each piece's UTF-8 bytes to the printable characters of the byte-level
  alphabet (bytes 33-126, 161-172, 174-255 as themselves, the rest to 256+);
- merge adjacent symbols, the lowest merge rank first (leftmost on ties),
  until no pair has a rank; look each symbol up in the vocabulary (unknown ->
  the unk id: vocab[String(unk_token)], else 1);
- special tokens (added_tokens with "special") are matched first, longest
  first, and the text between them is encoded as above; text longer than
  32768 characters keeps its last 32768;
- decode maps ids back to symbols, symbols to bytes, and decodes UTF-8 with
  replacement of invalid sequences.

encode_messages (tokenizer.js:199-272) lays out a conversation for the
"completion", "chatml" and "petitgpt" templates.
"""
from __future__ import annotations

import json
from typing import Dict, Iterable, List, Optional

import regex

# JavaScript's \s (ECMA-262 WhiteSpace + LineTerminator), which the reference's
# /u regex uses: it differs from Python's (no \x1c-\x1f, \x85; has ﻿)
_WS = "\\t\\n\\x0b\\x0c\\r \\u00a0\\u1680\\u2000-\\u200a\\u2028\\u2029\\u202f\\u205f\\u3000\\ufeff"
PATTERN = regex.compile(
    "'s|'t|'re|'ve|'m|'ll|'d| ?\\p{L}+| ?\\p{N}+| ?[^" + _WS + "\\p{L}\\p{N}]+|[" + _WS + "]+(?![^" + _WS + "])|[" +
    _WS + "]+")

MAX_CHARS = 32768  # tokenizer.js:92-94, 201-203


def _byte_alphabet():
    printable = list(range(33, 127)) + list(range(161, 173)) + list(range(174, 256))
    to_char, to_byte = {}, {}
    extra = 0
    for b in range(256):
        if b in printable:
            cp = b
        else:
            cp = 256 + extra
            extra += 1
        to_char[b] = chr(cp)
        to_byte[chr(cp)] = b
    return to_char, to_byte


BYTE_TO_CHAR, CHAR_TO_BYTE = _byte_alphabet()


def _js_text(text: str, limit: int = MAX_CHARS) -> str:
    """The text as the reference sees it: JavaScript strings count UTF-16
    units, so the cut to the last `limit` characters can split a surrogate
    pair, and TextEncoder writes a lone surrogate as U+FFFD."""
    if all(ord(c) < 0xD800 for c in text):  # no astral characters or surrogates
        return text[-limit:] if len(text) > limit else text
    units = text.encode("utf-16-le", "surrogatepass")
    if len(units) > 2 * limit:
        units = units[-2 * limit:]
    return units.decode("utf-16-le", "surrogatepass").encode("utf-16", "surrogatepass").decode("utf-16", "replace")

# tokenizer.js:185-193: the petitgpt template's fixed ids
SPECIAL = {"PAD": 0, "UNK": 1, "BOS": 2, "EOS": 3, "SYSTEM": 4, "USER": 5, "ASSISTANT": 6}


def js_key(obj: dict, name: str) -> str:
    """The property name JavaScript forms from obj[name] when it is used as a
    key (String(value)): "undefined" when absent, "null", "true" / "false",
    integral numbers without a fraction, strings as they are."""
    if name not in obj:
        return "undefined"
    v = obj[name]
    if v is None:
        return "null"
    if isinstance(v, bool):
        return "true" if v else "false"
    if isinstance(v, float) and v.is_integer():
        return str(int(v))
    return str(v)


class Tokenizer:
    def __init__(self, spec: dict):
        model = spec["model"]
        self.vocab: Dict[str, int] = model["vocab"]
        # tokenizer.js:60 looks the unk token up as a property name,
        # vocab[String(unk_token)] ?? 1: a null unk_token finds the entry
        # "null" (18220 in the SmolLM2 vocabularies, 8423 in GPT-2's)
        self.unk_id = self.vocab.get(js_key(model, "unk_token"), 1)
        self.ranks: Dict[tuple, int] = {}
        for i, m in enumerate(model.get("merges") or []):
            if isinstance(m, (list, tuple)):
                a, b = m[0], m[1]
            else:
                a, _, b = m.partition(" ")
            self.ranks[(a, b)] = i  # a repeated pair keeps its last rank, as Map.set does
        self.special: Dict[str, int] = {t["content"]: t["id"] for t in spec.get("added_tokens") or [] if t.get("special")}
        self._special_order = sorted(self.special, key=len, reverse=True)
        self._special_ids = set(self.special.values())
        self.id_to_tok: Dict[int, str] = {v: k for k, v in self.vocab.items()}
        self.vocab_size = len(self.vocab)
        self._cache: Dict[str, List[str]] = {}

    # ------------------------------------------------------------ encode
    def _bpe(self, word: str) -> List[str]:
        hit = self._cache.get(word)
        if hit is not None:
            return hit
        syms = list(word)
        while len(syms) > 1:
            best, at = None, -1
            for i in range(len(syms) - 1):
                r = self.ranks.get((syms[i], syms[i + 1]))
                if r is not None and (best is None or r < best):
                    best, at = r, i
            if at < 0:
                break
            syms[at:at + 2] = [syms[at] + syms[at + 1]]
        if len(self._cache) < 100000:
            self._cache[word] = syms
        return syms

    def _encode_plain(self, text: str) -> List[int]:
        ids = []
        for piece in PATTERN.findall(text):
            mapped = "".join(BYTE_TO_CHAR[b] for b in piece.encode("utf-8"))
            for sym in self._bpe(mapped):
                ids.append(self.vocab.get(sym, self.unk_id))
        return ids

    def encode(self, text) -> List[int]:
        if not text:
            return []
        if not isinstance(text, str):
            text = str(text)
        text = _js_text(text)
        if not self._special_order:
            return self._encode_plain(text)
        ids: List[int] = []
        i, n = 0, len(text)
        while i < n:
            hit = next((s for s in self._special_order if text.startswith(s, i)), None)
            if hit is not None:
                ids.append(self.special[hit])
                i += len(hit)
                continue
            j = i + 1
            while j < n and not any(text.startswith(s, j) for s in self._special_order):
                j += 1
            ids.extend(self._encode_plain(text[i:j]))
            i = j
        return ids

    # ------------------------------------------------------------ decode
    def decode(self, ids: Iterable[int], skip_special: bool = False) -> str:
        out = bytearray()
        for i in ids:
            i = int(i)
            if skip_special and i in self._special_ids:
                continue
            sym = self.id_to_tok.get(i)
            if not sym:
                continue
            for ch in sym:
                b = CHAR_TO_BYTE.get(ch)
                if b is not None:
                    out.append(b)
        return out.decode("utf-8", "replace")


def load_tokenizer(spec) -> Tokenizer:
    """loadTokenizerFromJson (tokenizer.js:57-183): spec is the parsed
    tokenizer.json, its text, or a path to it."""
    if isinstance(spec, (str, bytes)) and not str(spec).lstrip().startswith("{"):
        with open(spec, "rb") as f:
            spec = json.load(f)
    elif isinstance(spec, (str, bytes)):
        spec = json.loads(spec)
    return Tokenizer(spec)


def encode_chat(tok: Tokenizer, messages, default_system: Optional[str] = None) -> List[int]:
    """encodeChat (tokenizer.js:195-197): the petitgpt template."""
    return encode_messages(tok, messages, {"template": "petitgpt", "defaultSystem": default_system})


def encode_messages(tok: Tokenizer, messages, card: Optional[dict] = None) -> List[int]:
    """encodeMessages (tokenizer.js:199-272): the conversation as prompt ids
    for the card's template ("completion", "chatml", or "petitgpt")."""
    card = card or {}
    msgs = []
    for m in messages:
        content = "" if m.get("content") is None else str(m.get("content"))
        content = _js_text(content)
        msgs.append({"role": str(m.get("role")).strip().lower(), "content": content})
    tpl = card.get("template") or "petitgpt"
    specials = card.get("specials") or {}
    if tpl == "completion":
        return tok.encode(msgs[-1]["content"] if msgs else "")
    if tpl == "chatml":
        sys_msg = card.get("defaultSystem")
        if sys_msg and (not msgs or msgs[0]["role"] != "system"):
            msgs.insert(0, {"role": "system", "content": sys_msg})

        def first(*vals):
            return next(v for v in vals if v is not None)

        im_start = first(tok.special.get("<|im_start|>"), specials.get("<|im_start|>"), card.get("bosId"), 1)
        im_end = first(tok.special.get("<|im_end|>"), specials.get("<|im_end|>"), card.get("eosId"), 2)
        ids: List[int] = []
        for m in msgs:
            ids.append(im_start)
            ids += tok.encode(m["role"]) + tok.encode("\n") + tok.encode(m["content"])
            ids.append(im_end)
            ids += tok.encode("\n")
        ids.append(im_start)
        ids += tok.encode("assistant") + tok.encode("\n")
        return ids
    default_system = card.get("defaultSystem")
    if default_system and (not msgs or msgs[0]["role"] != "system"):
        msgs.insert(0, {"role": "system", "content": default_system})
    bos = card.get("bosId") if card.get("bosId") is not None else SPECIAL["BOS"]
    eos = card.get("eosId") if card.get("eosId") is not None else SPECIAL["EOS"]
    def marker(name, default):  # `??`: a null entry falls back too
        v = specials.get(name)
        return default if v is None else v

    role_id = {
        "system": marker("<|system|>", SPECIAL["SYSTEM"]),
        "user": marker("<|user|>", SPECIAL["USER"]),
        "assistant": marker("<|assistant|>", SPECIAL["ASSISTANT"]),
    }
    ids = [bos]
    for m in msgs:
        if role_id.get(m["role"]) is None:
            raise ValueError(f"invalid role {m['role']}")
        content_ids = tok.encode(m["content"])
        if not content_ids:
            raise ValueError("empty message encoding")
        ids.append(role_id[m["role"]])
        ids += content_ids
        if m["role"] == "assistant":
            ids.append(eos)
    if not msgs or msgs[-1]["role"] != "user":
        raise ValueError("prompt must end with a user turn")
    ids.append(role_id["assistant"])
    return ids
