/**
 * Drive HipPetitGPT on a .pgw file (the flow of engine/worker.js:34-181:
 * load -> new engine -> generate with streaming onToken).
 *   node run_generate.mjs <model.pgw> <spec.json>   -> prints one JSON line
 * spec: { prompt: [...], maxNewTokens, eosId, mode, specK, kvFp16, execMode, prefillMin,
 *         decodeLogits: [ids...], debug: {maxLayers, noAttn, noMlp, mlpTo} }
 *         (decodeLogits: teacher-forced tokens whose logits are returned for
 *         comparison; debug: GpuPetitGPT's debug knobs, set as properties the
 *         way app.js:1317-1325 sets them)
 */
import fs from "fs";
import { parsePgw } from "../../microllm-lab_amd/js/weights.mjs";
import { HipPetitGPT } from "../../microllm-lab_amd/js/engine.mjs";

async function main() {
  const [, , pgwPath, specPath] = process.argv;
  const spec = JSON.parse(fs.readFileSync(specPath, "utf8"));
  const bundle = parsePgw(fs.readFileSync(pgwPath));
  const model = new HipPetitGPT(bundle, { kvFp16: !!spec.kvFp16, execMode: spec.execMode, prefillMin: spec.prefillMin });
  if (spec.debug) {
    if (spec.debug.maxLayers !== undefined) model.debugMaxLayers = spec.debug.maxLayers;
    if (spec.debug.noAttn !== undefined) model.debugNoAttn = spec.debug.noAttn;
    if (spec.debug.noMlp !== undefined) model.debugNoMlp = spec.debug.noMlp;
    if (spec.debug.mlpTo !== undefined) model.debugMlpTo = spec.debug.mlpTo;
  }
  const streamed = [];
  const res = await model.generate(spec.prompt, {
    maxNewTokens: spec.maxNewTokens,
    eosId: spec.eosId !== undefined ? spec.eosId : -1,
    mode: spec.mode || "greedy",
    specK: spec.specK || 4,
    onToken: async (t) => {
      streamed.push(t);
    },
  });
  const rows = [];
  if (spec.decodeLogits) {
    model.resetCache();
    rows.push(Array.from(model.forwardPrompt(spec.prompt)));
    for (const t of spec.decodeLogits) rows.push(Array.from(model.forwardDecode(t)));
  }
  const out = {
    generatedIds: res.generatedIds,
    streamed,
    stopReason: res.stopReason,
    specHits: res.specHits,
    specTries: res.specTries,
    mode: res.mode,
    bytesAllocated: model.bytesAllocated,
    rows,
  };
  model.destroy();
  let destroyedError = null;
  try {
    model.forwardDecode(1);
  } catch (e) {
    destroyedError = String(e.message);
  }
  out.destroyedError = destroyedError;
  console.log(JSON.stringify(out));
}

main().catch((e) => {
  console.error(e && e.stack ? e.stack : String(e));
  process.exit(1);
});
