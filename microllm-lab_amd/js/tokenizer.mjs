/**
 * Byte-level BPE tokenizer and chat templates for the Node host
 * (engine/tokenizer.js:1-272): text -> prompt ids -> (HipPetitGPT) -> ids ->
 * text.  The JavaScript twin of mllm/tokenizer.py, with the same API:
 *
 *   const tok = loadTokenizer("models/x/tokenizer.json");  // path, JSON text or object
 *   const ids = tok.encode("Hello");
 *   const text = tok.decode(ids, { skipSpecial: true });
 *   const prompt = encodeMessages(tok, [{ role: "user", content: "hi" }], card);
 *
 * The algorithm (tokenizer.js:1-183):
 * - text longer than 32768 UTF-16 units keeps its last 32768 (a cut through a
 *   surrogate pair leaves a lone surrogate, which TextEncoder writes as U+FFFD);
 * - special tokens (added_tokens marked special) match first, longest first;
 *   the text between them is split into pieces by the GPT-2 pattern
 *   (contractions, letters, numbers, other symbols, whitespace; \s is
 *   JavaScript's own class under the /u flag);
 * - each piece's UTF-8 bytes map to the printable byte-level alphabet
 *   (bytes 33-126, 161-172, 174-255 as themselves, the rest to U+0100 on);
 * - adjacent symbols merge, the lowest merge rank first (leftmost on ties),
 *   until no pair has a rank; each symbol is looked up in the vocabulary
 *   (missing: vocab[String(unk_token)], else 1);
 * - decode maps ids to symbols, symbols to bytes and decodes UTF-8 with
 *   U+FFFD for invalid sequences (ids outside the vocabulary are dropped).
 * encodeMessages (tokenizer.js:199-272) lays out a conversation for the
 * "completion", "chatml" and "petitgpt" templates.
 */
import { readFileSync } from "fs";

export const MAX_CHARS = 32768;
// tokenizer.js:185-193: the petitgpt template's fixed ids
export const SPECIAL = { PAD: 0, UNK: 1, BOS: 2, EOS: 3, SYSTEM: 4, USER: 5, ASSISTANT: 6 };

export const PATTERN = /'s|'t|'re|'ve|'m|'ll|'d| ?\p{L}+| ?\p{N}+| ?[^\s\p{L}\p{N}]+|\s+(?!\S)|\s+/gu;

function byteAlphabet() {
  const toChar = new Array(256);
  const toByte = new Map();
  let extra = 0;
  for (let b = 0; b < 256; b++) {
    const printable = (b >= 33 && b <= 126) || (b >= 161 && b <= 172) || (b >= 174 && b <= 255);
    const ch = String.fromCharCode(printable ? b : 256 + extra++);
    toChar[b] = ch;
    toByte.set(ch, b);
  }
  return [toChar, toByte];
}
export const [BYTE_TO_CHAR, CHAR_TO_BYTE] = byteAlphabet();

const utf8 = new TextEncoder();

/** The text the reference tokenizes: its last MAX_CHARS UTF-16 units. */
export function jsText(text) {
  return text.length > MAX_CHARS ? text.slice(text.length - MAX_CHARS) : text;
}

export class Tokenizer {
  constructor(spec) {
    const model = spec.model;
    this.vocab = new Map(Object.entries(model.vocab));
    // tokenizer.js:60, vocab[spec.model.unk_token] ?? 1: the property name is
    // String(unk_token), so a null unk_token finds the entry "null"
    const unkKey = String(model.unk_token);
    this.unkId = this.vocab.has(unkKey) && this.vocab.get(unkKey) != null ? this.vocab.get(unkKey) : 1;
    this.ranks = new Map();
    (model.merges || []).forEach((m, i) => {
      const [a, b] = Array.isArray(m) ? m : [m.slice(0, m.indexOf(" ")), m.slice(m.indexOf(" ") + 1)];
      this.ranks.set(a + "\u0000" + b, i);  // a repeated pair keeps its last rank
    });
    this.special = new Map();
    for (const t of spec.added_tokens || []) if (t.special) this.special.set(t.content, t.id);
    this.specialOrder = [...this.special.keys()].sort((x, y) => y.length - x.length);
    this.specialIds = new Set(this.special.values());
    this.idToTok = new Map();
    for (const [k, v] of this.vocab) this.idToTok.set(v, k);
    this.vocabSize = this.vocab.size;
    this.cache = new Map();
  }

  bpe(word) {
    const hit = this.cache.get(word);
    if (hit) return hit;
    const syms = Array.from(word);
    while (syms.length > 1) {
      let best = -1, at = -1;
      for (let i = 0; i + 1 < syms.length; i++) {
        const r = this.ranks.get(syms[i] + "\u0000" + syms[i + 1]);
        if (r !== undefined && (best < 0 || r < best)) {
          best = r;
          at = i;
        }
      }
      if (at < 0) break;
      syms.splice(at, 2, syms[at] + syms[at + 1]);
    }
    if (this.cache.size < 100000) this.cache.set(word, syms);
    return syms;
  }

  encodePlain(text, ids) {
    for (const piece of text.match(PATTERN) || []) {
      let mapped = "";
      for (const b of utf8.encode(piece)) mapped += BYTE_TO_CHAR[b];
      for (const sym of this.bpe(mapped)) ids.push(this.vocab.has(sym) ? this.vocab.get(sym) : this.unkId);
    }
    return ids;
  }

  specialAt(text, i) {
    for (const s of this.specialOrder) if (text.startsWith(s, i)) return s;
    return null;
  }

  encode(text) {
    if (text == null || text === "") return [];
    text = jsText(String(text));
    const ids = [];
    if (this.specialOrder.length === 0) return this.encodePlain(text, ids);
    let i = 0;
    while (i < text.length) {
      const hit = this.specialAt(text, i);
      if (hit !== null) {
        ids.push(this.special.get(hit));
        i += hit.length;
        continue;
      }
      let j = i + 1;
      while (j < text.length && this.specialAt(text, j) === null) j++;
      this.encodePlain(text.slice(i, j), ids);
      i = j;
    }
    return ids;
  }

  decode(ids, { skipSpecial = false } = {}) {
    const out = [];
    for (const v of ids) {
      const id = Number(v);
      if (skipSpecial && this.specialIds.has(id)) continue;
      const sym = this.idToTok.get(id);
      if (!sym) continue;
      for (const ch of sym) {
        const b = CHAR_TO_BYTE.get(ch);
        if (b !== undefined) out.push(b);
      }
    }
    return new TextDecoder("utf-8").decode(Uint8Array.from(out));
  }
}

/** loadTokenizerFromJson (tokenizer.js:57-183): a parsed tokenizer.json, its text, or a path. */
export function loadTokenizer(spec) {
  if (typeof spec === "string") spec = JSON.parse(spec.trimStart().startsWith("{") ? spec : readFileSync(spec, "utf8"));
  return new Tokenizer(spec);
}

/** encodeChat (tokenizer.js:195-197): the petitgpt template. */
export function encodeChat(tok, messages, defaultSystem = null) {
  return encodeMessages(tok, messages, { template: "petitgpt", defaultSystem });
}

// The first of its arguments that is neither undefined nor null (the
// reference's `??` chains; Node 12 has no `??`).
const pick = (...vals) => vals.find((v) => v !== undefined && v !== null);

// A conversation's turns as every layout reads them: the role trimmed and
// lower-cased, the content a string cut to its last MAX_CHARS units.
function turnsOf(messages) {
  return messages.map((m) => ({
    role: String(m.role).trim().toLowerCase(),
    content: jsText(m.content == null ? "" : String(m.content)),
  }));
}

// The card's default system turn in front, unless the conversation opens with one.
function withSystem(turns, text) {
  return text && !(turns.length && turns[0].role === "system") ? [{ role: "system", content: text }].concat(turns) : turns;
}

// One id layout per template name (tokenizer.js:208-271).  The ids and the
// error messages are the interface: a prompt must come out as the same ids,
// and a bad conversation must fail with the same message.
const LAYOUTS = {
  // the last turn's text alone
  completion(tok, turns) {
    return tok.encode(turns.length ? turns[turns.length - 1].content : "");
  },
  // <|im_start|>role\n content <|im_end|>\n per turn, then the assistant's header;
  // the markers from the tokenizer's specials, then the card's, then its bos / eos
  chatml(tok, turns, card, specials) {
    const open = pick(tok.special.get("<|im_start|>"), specials["<|im_start|>"], card.bosId, 1);
    const close = pick(tok.special.get("<|im_end|>"), specials["<|im_end|>"], card.eosId, 2);
    const nl = tok.encode("\n");
    const header = (role) => [open].concat(tok.encode(role), nl);
    const out = [];
    for (const turn of withSystem(turns, card.defaultSystem)) out.push(...header(turn.role), ...tok.encode(turn.content), close, ...nl);
    return out.concat(header("assistant"));
  },
  // bos, then per turn its role marker and text (an assistant turn closed by
  // eos); the conversation must end with the user, and the assistant's marker
  // follows.  Turns are checked in order, as they are laid out.
  petitgpt(tok, turns, card, specials) {
    const marker = {
      system: pick(specials["<|system|>"], SPECIAL.SYSTEM),
      user: pick(specials["<|user|>"], SPECIAL.USER),
      assistant: pick(specials["<|assistant|>"], SPECIAL.ASSISTANT),
    };
    const all = withSystem(turns, card.defaultSystem || null);
    const out = [pick(card.bosId, SPECIAL.BOS)];
    for (const turn of all) {
      const id = marker[turn.role];
      if (id === undefined || id === null) throw new Error(`invalid role ${turn.role}`);
      const text = tok.encode(turn.content);
      if (text.length === 0) throw new Error("empty message encoding");
      out.push(id, ...text);
      if (turn.role === "assistant") out.push(pick(card.eosId, SPECIAL.EOS));
    }
    if (!all.length || all[all.length - 1].role !== "user") throw new Error("prompt must end with a user turn");
    out.push(marker.assistant);
    return out;
  },
};

/** encodeMessages (tokenizer.js:199-272): a conversation as prompt ids for the card's template. */
export function encodeMessages(tok, messages, card = {}) {
  card = card || {};
  const layout = card.template || "petitgpt";
  // any other template name takes the petitgpt layout, as in the reference
  const build = layout === "completion" || layout === "chatml" ? LAYOUTS[layout] : LAYOUTS.petitgpt;
  return build(tok, turnsOf(messages), card, card.specials || {});
}
