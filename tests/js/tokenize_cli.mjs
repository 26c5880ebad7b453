/**
 * Batch front end of tokenizer.mjs for scripts and tests:
 *   node tokenize_cli.mjs cases.json
 * cases.json: { tokenizer: <path | tokenizer.json object>,
 *               encode: [text...], decode: [[id...]...], decodeSkip: [[id...]...],
 *               messages: [{ messages, card }...] }
 * prints { unkId, encode: [[id...]...], decode: [text...], decodeSkip: [text...],
 *          messages: [[id...] | { error }...] } as one JSON line.
 */
import { readFileSync } from "fs";
import { loadTokenizer, encodeMessages } from "../../microllm-lab_amd/js/tokenizer.mjs";

const cases = JSON.parse(readFileSync(process.argv[2], "utf8"));
const tok = loadTokenizer(cases.tokenizer);
const out = {
  unkId: tok.unkId,
  encode: (cases.encode || []).map((t) => tok.encode(t)),
  decode: (cases.decode || []).map((ids) => tok.decode(ids)),
  decodeSkip: (cases.decodeSkip || []).map((ids) => tok.decode(ids, { skipSpecial: true })),
  messages: (cases.messages || []).map((c) => {
    try {
      return encodeMessages(tok, c.messages, c.card);
    } catch (e) {
      return { error: String(e.message) };
    }
  }),
};
process.stdout.write(JSON.stringify(out) + "\n");
