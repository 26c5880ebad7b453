/**
 * Host-logic self-test (no GPU): parsePgw on a file written by the Python
 * writer, lookupDraft / argmax / argmaxGpt2 against cases given as JSON.
 *   node selftest.mjs <model.pgw> <cases.json>   -> prints one JSON line
 */
import fs from "fs";
import { parsePgw, tensorTable } from "../../microllm-lab_amd/js/weights.mjs";
import { argmax, argmaxGpt2, lookupDraft } from "../../microllm-lab_amd/js/sampling.mjs";

const [, , pgwPath, casesPath] = process.argv;
const buf = fs.readFileSync(pgwPath);
const bundle = parsePgw(buf);
const cases = JSON.parse(fs.readFileSync(casesPath, "utf8"));
const out = {
  kind: bundle.kind,
  cfg: bundle.cfg,
  payloadOff: bundle.payloadOff,
  table: tensorTable(bundle),
  drafts: cases.drafts.map((c) => lookupDraft(c.seq, c.k, c.n)),
  argmax: cases.argmax.map((l) => argmax(Float32Array.from(l))),
  argmaxGpt2: cases.gpt2.map((c) => argmaxGpt2(Float32Array.from(c.logits), c.hist)),
};
let bad = null;
try {
  parsePgw(new Uint8Array([1, 2, 3, 4, 0, 0, 0, 0]));
} catch (e) {
  bad = String(e.message);
}
out.badMagic = bad;
console.log(JSON.stringify(out));
