"""The byte-level BPE tokenizer and chat templates (mllm/tokenizer.py,
restating engine/tokenizer.js).

Pins:
- encode: the HuggingFace `tokenizers` library (installed; a byte-level BPE
  the reference says it matches, tokenizer.js:1) loading the same
  tokenizer.json, on the models the reference ships (read from the reference
  checkout when present; skipped otherwise), over fixed texts and seeded
  random Unicode strings; where JavaScript and Rust regex semantics differ
  (which characters \\s matches) the JavaScript split is checked by hand;
- decode: decode(encode(text)) == text for valid text; skip_special;
- the byte alphabet: a bijection of 256 bytes fixing 33-126, 161-172, 174-255;
- the merge loop: the lowest rank first, leftmost on ties, on hand-made specs;
- the templates: their token layout on hand-made tokenizers.
"""
import json
import os
import random

import pytest

from mllm import tokenizer as T

REF_MODELS = "/root/reference/models"
MODELS = ["gpt2", "l20-edu-135m", "minimind2", "smollm2-135m-instruct", "petitgpt"]

TEXTS = [
    "Hello! How can I help you today?",
    "The capital of France is Paris.",
    "  leading spaces and   runs\n\n\tof whitespace  ",
    "def add(a, b):\n    return a + b  # 42\n",
    "Numbers 12345 and 3.14159, 1e-5, 2024-12-01",
    "ünïcödé café naïve — “quotes” ‘single’ … ½ ² ℃",
    "日本語のテキストと中文混合 한국어",
    "emoji 😀🎉👍🏽 family 👨‍👩‍👧 flags 🇫🇷",
    "<|im_start|>user\nhi<|im_end|>\n<|im_start|>assistant\n",
    "<|endoftext|>after<|endoftext|><|endoftext|>",
    "don't won't I'm you're they've we'll he'd 'S 'LL",
    "tabs\tand\rcarriage\x0breturns\x0cff",
    "  nbsp  emspace 　ideo  ls",
    "a" * 50 + " " + "b" * 70,
    "x",
    "",
]


def hf_or_skip(name):
    path = os.path.join(REF_MODELS, name, "tokenizer.json")
    if not os.path.exists(path):
        pytest.skip("the reference's tokenizer files are not present")
    tokenizers = pytest.importorskip("tokenizers")
    return T.load_tokenizer(path), tokenizers.Tokenizer.from_file(path)


def random_texts(seed, n=60, astral=True):
    rng = random.Random(seed)
    pools = [range(0x20, 0x7F), range(0xA0, 0x250), range(0x370, 0x3FF), range(0x400, 0x4FF), range(0x4E00, 0x4F00),
             range(0x3040, 0x30FF), [0x20, 0x20, 0x0A, 0x09]] + ([range(0x1F600, 0x1F650)] if astral else [])
    out = []
    for _ in range(n):
        k = rng.randint(1, 80)
        out.append("".join(chr(rng.choice(rng.choice(pools))) for _ in range(k)))
    return out


@pytest.mark.parametrize("name", MODELS)
def test_encode_matches_hf_tokenizers(name):
    tok, hf = hf_or_skip(name)
    for text in TEXTS + random_texts(hash(name) & 0xFFFF):
        assert tok.encode(text) == hf.encode(text, add_special_tokens=False).ids, repr(text[:60])


@pytest.mark.parametrize("name", MODELS)
def test_decode_round_trip_and_skip_special(name):
    tok, hf = hf_or_skip(name)
    for text in TEXTS + random_texts(7):
        assert tok.decode(tok.encode(text)) == text
    if tok.special:
        s, sid = next(iter(tok.special.items()))
        ids = tok.encode("a" + s + "b")
        assert sid in ids
        assert tok.decode(ids) == "a" + s + "b"
        assert tok.decode(ids, skip_special=True) == "ab"
    # ids outside the vocabulary are dropped; a cut UTF-8 sequence is replaced
    assert tok.decode([10 ** 9]) == ""
    euro = tok.encode("€")
    if len(euro) > 1:
        assert tok.decode(euro[:1]).endswith("�")


def test_long_text_keeps_the_last_32768_characters():
    tok, hf = hf_or_skip("gpt2")
    text = "".join(random_texts(3, 2000, astral=False))
    text = (text * (40000 // len(text) + 1))[:40000]
    assert tok.encode(text) == hf.encode(text[-32768:], add_special_tokens=False).ids
    # JavaScript counts UTF-16 units: an astral character is two of them, and
    # a cut through a pair leaves a lone surrogate that TextEncoder writes as
    # U+FFFD
    emo = "\U0001F600"
    assert T._js_text(emo * 20000) == emo * 16384
    assert T._js_text("a" + emo * 16384) == emo * 16384
    assert T._js_text(emo * 16385 + "c") == "\ufffd" + emo * 16383 + "c"
    assert T._js_text("\ud800x") == "\ufffdx"


def test_javascript_whitespace_class():
    """\\s of the reference's /u regex is ECMA-262's: U+0085 and U+001C..1F are
    not whitespace there (Python and Rust count them), U+FEFF is."""
    split = T.PATTERN.findall
    assert split("a\x85b") == ["a", "\x85", "b"]
    assert split("a\x1cb") == ["a", "\x1c", "b"]
    # as whitespace, each U+FEFF is its own piece (only U+0020 joins a word);
    # as a symbol (Python's \s) the two would be one piece
    assert split("a\ufeff\ufeffb") == ["a", "\ufeff", "\ufeff", "b"]
    assert split("a  b") == ["a", " ", " b"]      # \s+(?!\S) leaves the last space to the word
    assert split("a  \n") == ["a", "  \n"]
    assert split("x's 'll") == ["x", "'s", " '", "ll"]


def test_byte_alphabet_is_the_gpt2_bijection():
    assert len(set(T.BYTE_TO_CHAR.values())) == 256
    for b in list(range(33, 127)) + list(range(161, 173)) + list(range(174, 256)):
        assert T.BYTE_TO_CHAR[b] == chr(b)
    others = [b for b in range(256) if T.BYTE_TO_CHAR[b] != chr(b)]
    assert [ord(T.BYTE_TO_CHAR[b]) for b in others] == list(range(256, 256 + len(others)))
    assert all(T.CHAR_TO_BYTE[T.BYTE_TO_CHAR[b]] == b for b in range(256))


def toy(merges, extra_vocab=(), added=()):
    vocab = {}
    for sym in [T.BYTE_TO_CHAR[b] for b in range(256)] + list(extra_vocab):
        vocab.setdefault(sym, len(vocab))
    return T.load_tokenizer({"model": {"type": "BPE", "vocab": vocab, "merges": merges},
                             "added_tokens": [dict(content=c, id=i, special=s) for c, i, s in added]})


def test_merge_order_lowest_rank_leftmost():
    tok = toy(["a a", "b c", "a b"], ["aa", "bc", "ab", "aaa"])
    assert tok._bpe("aaa") == ["aa", "a"]          # the leftmost of equal ranks first
    assert tok._bpe("abc") == ["a", "bc"]          # rank 1 (b c) before rank 2 (a b)
    assert tok._bpe("aab") == ["aa", "b"]
    # list-form merges are the same ranks
    tok2 = T.load_tokenizer({"model": {"vocab": tok.vocab, "merges": [["a", "a"], ["b", "c"], ["a", "b"]]}})
    assert tok2._bpe("abc") == ["a", "bc"]
    # a symbol missing from the vocabulary encodes as the unk id (1 without unk_token)
    assert tok.encode("aaaa") == [tok.vocab["aa"], tok.vocab["aa"]]
    assert toy(["a a"]).encode("aa") == [1]


def test_specials_longest_first_and_between_text():
    tok = toy([], added=[("<s>", 900, True), ("<s><s>", 901, True), ("<x>", 902, False)])
    a = tok.vocab["a"]
    assert tok.encode("<s><s>a<s>") == [901, a, 900]
    # non-special added tokens are plain text
    assert 902 not in tok.encode("<x>")


def test_templates():
    tok = toy([], added=[("<|im_start|>", 500, True), ("<|im_end|>", 501, True)])
    nl = tok.encode("\n")
    msgs = [{"role": "User", "content": "hi"}]
    ids = T.encode_messages(tok, msgs, {"template": "chatml", "defaultSystem": "sys"})
    assert ids == ([500] + tok.encode("system") + nl + tok.encode("sys") + [501] + nl + [500] + tok.encode("user") +
                   nl + tok.encode("hi") + [501] + nl + [500] + tok.encode("assistant") + nl)
    assert T.encode_messages(tok, [{"role": "user", "content": "q"}], {"template": "completion"}) == tok.encode("q")
    # petitgpt: BOS, role ids, content, EOS after assistant turns, assistant role last
    conv = [{"role": "user", "content": "a"}, {"role": "assistant", "content": "b"}, {"role": "user", "content": "c"}]
    assert T.encode_chat(tok, conv) == [2, 5] + tok.encode("a") + [6] + tok.encode("b") + [3, 5] + tok.encode("c") + [6]
    with pytest.raises(ValueError, match="end with a user turn"):
        T.encode_chat(tok, conv[:2])
    with pytest.raises(ValueError, match="invalid role"):
        T.encode_chat(tok, [{"role": "tool", "content": "x"}])
    with pytest.raises(ValueError, match="empty"):
        T.encode_chat(tok, [{"role": "user", "content": ""}])


def test_templates_with_the_reference_cards():
    """The cards shipped beside the models (card.json): petitgpt's template with
    its own role ids, chatml with SmolLM2's <|im_start|> / <|im_end|>."""
    import json

    tok, _ = hf_or_skip("petitgpt")
    card = json.load(open(os.path.join(REF_MODELS, "petitgpt", "card.json")))
    conv = [{"role": "system", "content": "Be brief."}, {"role": "user", "content": "What is 2 + 2?"}]
    ids = T.encode_messages(tok, conv, card)
    sp = card["specials"]
    assert ids == ([card["bosId"], sp["<|system|>"]] + tok.encode("Be brief.") + [sp["<|user|>"]] +
                   tok.encode("What is 2 + 2?") + [sp["<|assistant|>"]])
    tok2, _ = hf_or_skip("smollm2-135m-instruct")
    card2 = dict(json.load(open(os.path.join(REF_MODELS, "smollm2-135m-instruct", "card.json"))), template="chatml")
    ids2 = T.encode_messages(tok2, conv[1:], card2)
    assert ids2[0] == tok2.special["<|im_start|>"] == 1 and ids2.count(tok2.special["<|im_end|>"]) == 1
    assert tok2.decode(ids2) == "<|im_start|>user\nWhat is 2 + 2?<|im_end|>\n<|im_start|>assistant\n"


@pytest.mark.parametrize("name,want", [("smollm2-135m-instruct", 18220), ("smollm2-360m-instruct", 18220),
                                       ("l20-edu-135m", 18220), ("gpt2", 8423), ("petitgpt", 1), ("minimind2", 1)])
def test_unk_id_follows_the_reference_lookup(name, want):
    """tokenizer.js:60 takes vocab[spec.model.unk_token] ?? 1, a property
    lookup by String(unk_token): the shipped SmolLM2 and GPT-2 files have
    unk_token null, so the entry "null" is the unk id; petitgpt's "[UNK]"
    and minimind2's null miss and give 1.  A symbol missing from the
    vocabulary then encodes as that id."""
    path = os.path.join(REF_MODELS, name, "tokenizer.json")
    if not os.path.exists(path):
        pytest.skip("the reference's tokenizer files are not present")
    spec = json.load(open(path, encoding="utf-8"))
    tok = T.load_tokenizer(spec)
    assert tok.unk_id == want
    assert T.js_key(spec["model"], "unk_token") == ("null" if spec["model"].get("unk_token") is None
                                                     else spec["model"]["unk_token"])


def test_js_key_rules():
    assert T.js_key({}, "u") == "undefined"
    assert T.js_key({"u": None}, "u") == "null"
    assert T.js_key({"u": True}, "u") == "true"
    assert T.js_key({"u": 3.0}, "u") == "3"
    assert T.js_key({"u": "<unk>"}, "u") == "<unk>"
    vocab = {T.BYTE_TO_CHAR[b]: b + 10 for b in range(256)}
    vocab["null"] = 5
    tok = T.load_tokenizer({"model": {"vocab": vocab, "merges": [], "unk_token": None}})
    assert tok.unk_id == 5
    tok = T.load_tokenizer({"model": {"vocab": vocab, "merges": []}})
    assert tok.unk_id == 1  # vocab["undefined"] is absent
