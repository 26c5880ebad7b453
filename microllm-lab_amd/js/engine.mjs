/**
 * HipPetitGPT: the PetitGPT model API of engine/infer.js:289-647 on the MI355X
 * decode step (libmllm through the N-API shim mllm_napi.node).
 *
 *   const model = new HipPetitGPT(parsePgw(arrayBuffer));
 *   const logits = model.forwardPrompt(ids);     // Float32Array (shared buffer)
 *   const next = model.forwardDecode(id);        // Float32Array (shared buffer)
 *   const r = await model.generate(ids, { maxNewTokens, eosId, onToken, mode });
 *   model.destroy();
 *
 * As in infer.js the logits array returned by forwardPrompt / forwardDecode is
 * the model's own buffer and is overwritten by the next call.  generate()
 * returns { generatedIds, stopReason, ttftMs, totalMs, mode, specHits,
 * specTries, timing } like GpuPetitGPT.generate (webgpu.js:1164-1282).
 * There is no CPU or WebGPU fallback: a missing addon or device throws.
 */
import { createRequire } from "module";
import { tensorTable } from "./weights.mjs";
import { argmax, argmaxGpt2, lookupDraft } from "./sampling.mjs";

const require = createRequire(import.meta.url);
const native = require("./mllm_napi.node");

function now() {
  const t = process.hrtime();
  return t[0] * 1e3 + t[1] / 1e6;
}

export class HipPetitGPT {
  /**
   * bundle: a parsePgw() result, or a CPU PetitGPT (its .bundle is used), so
   * the GpuPetitGPT construction of webgpu.js:867 (new X(cpu, info); await
   * x.init()) works unchanged.  The payload is copied to the device here; the
   * class keeps no reference to the host buffer afterwards.
   */
  constructor(source, opts) {
    const o = opts || {};
    const bundle = source && source.bundle && source.bundle.cfg ? source.bundle : source;
    if (!bundle || !bundle.cfg) throw new Error("HipPetitGPT needs a parsePgw() bundle or a PetitGPT");
    this.cfg = bundle.cfg;
    this.kind = bundle.kind;
    this.isGpt2 = bundle.cfg.arch === "gpt2";
    const c = bundle.cfg;
    const payload = new Uint8Array(bundle.buffer, bundle.payloadOff, bundle.buffer.byteLength - bundle.payloadOff);
    this._h = native.createModel(
      {
        arch: this.isGpt2 ? 1 : 0,
        vocabSize: c.vocabSize,
        nLayers: c.nLayers,
        dModel: c.dModel,
        nHeads: c.nHeads,
        nKvHeads: c.nKvHeads,
        dFf: c.dFf,
        maxSeqLen: c.maxSeqLen,
        ropeTheta: c.ropeTheta,
        ropePct: c.ropePct,
        normEps: o.normEps !== undefined ? o.normEps : 1e-6,
        kvFp16: o.kvFp16 ? 1 : 0,
      },
      payload,
      tensorTable(bundle),
    );
    this._logits = new Float32Array(c.vocabSize);
    this.maxPass = native.maxPassTokens(this._h);
    if (o.execMode !== undefined) native.setExecMode(this._h, o.execMode);
    // prompts of at least prefillMin ids run batched (mllm_set_prefill; 0 = 16-token passes)
    if (o.prefillMin !== undefined) native.setPrefill(this._h, o.prefillMin, o.prefillChunk || 0);
    this.mode = `hip-${bundle.kind}`;
    this.lastArgmax = 0;
    this.lastTiming = null;
  }

  /** GpuPetitGPT.init() counterpart: the device copy is made by the constructor. */
  async init() {
    return this;
  }

  get cacheLen() {
    return native.cacheLen(this._h);
  }

  set cacheLen(v) {
    native.setCacheLen(this._h, v);
  }

  get bytesAllocated() {
    return native.deviceBytes(this._h);
  }

  resetCache() {
    native.resetCache(this._h);
  }

  /** infer.js:553-577 */
  forwardPrompt(ids) {
    this.lastArgmax = native.forwardPrompt(this._h, Int32Array.from(ids), this._logits);
    return this._logits;
  }

  /** infer.js:579-601 */
  forwardDecode(tokenId) {
    this.lastArgmax = native.forwardDecode(this._h, tokenId, this._logits);
    return this._logits;
  }

  /** The k+1-row verify pass: one argmax per row. */
  forwardVerify(ids, wantLogits) {
    const am = new Int32Array(ids.length);
    const lg = wantLogits ? new Float32Array(ids.length * this.cfg.vocabSize) : null;
    native.forwardVerify(this._h, Int32Array.from(ids), am, lg);
    return { argmax: Array.from(am), logits: lg };
  }

  /** Device-chained greedy decode (CHAIN_TOK, webgpu-metal.js:609-610). */
  decodeChain(first, nSteps, eosId, hist) {
    const out = new Int32Array(nSteps);
    const n = native.decodeChain(this._h, first, nSteps, eosId, hist ? Int32Array.from(hist) : null, out);
    this.lastTiming = native.lastTiming(this._h);
    return Array.from(out.subarray(0, n));
  }

  /** model.gemv(name, x, y) -- the operator plug point of infer.js:338-346. */
  gemv(name, x, y) {
    native.gemv(this._h, name, x, y);
  }

  setExecMode(mode) {
    native.setExecMode(this._h, mode);
  }

  // GpuPetitGPT's debug knobs (webgpu-metal.js:1263-1279, set by app.js:1317-1325
  // from the page's query string): null / false restore the full network.
  _applyDebug() {
    const d = this._dbg;
    native.setDebug(this._h, d.maxLayers == null ? -1 : d.maxLayers, d.noAttn ? 1 : 0, d.noMlp ? 1 : 0,
                    d.mlpTo == null ? -1 : d.mlpTo);
  }

  get debugMaxLayers() {
    return this._dbg ? this._dbg.maxLayers : null;
  }

  set debugMaxLayers(v) {
    this._dbg = Object.assign({}, this._dbg || {}, { maxLayers: v });
    this._applyDebug();
  }

  get debugNoAttn() {
    return this._dbg ? !!this._dbg.noAttn : false;
  }

  set debugNoAttn(v) {
    this._dbg = Object.assign({}, this._dbg || {}, { noAttn: !!v });
    this._applyDebug();
  }

  get debugNoMlp() {
    return this._dbg ? !!this._dbg.noMlp : false;
  }

  set debugNoMlp(v) {
    this._dbg = Object.assign({}, this._dbg || {}, { noMlp: !!v });
    this._applyDebug();
  }

  get debugMlpTo() {
    return this._dbg ? this._dbg.mlpTo : null;
  }

  set debugMlpTo(v) {
    this._dbg = Object.assign({}, this._dbg || {}, { mlpTo: v });
    this._applyDebug();
  }

  timing() {
    return native.lastTiming(this._h);
  }

  /**
   * Greedy generation.  mode: "greedy" (host loop, infer.js:603-646),
   * "chain" (device-chained, webgpu.js:1202-1226) or "spec" (prompt-lookup
   * speculation, webgpu.js:1239-1270; llama models).
   */
  async generate(inIds, opts) {
    const o = opts || {};
    const maxNewTokens = o.maxNewTokens !== undefined ? o.maxNewTokens : 64;
    const eosId = o.eosId !== undefined ? o.eosId : -1;
    const onToken = o.onToken || null;
    const mode = o.mode || "greedy";
    const specK = o.specK !== undefined ? o.specK : 4;
    const ngram = o.ngram !== undefined ? o.ngram : 3;
    const chainChunk = o.chainChunk || 64;
    const maxSeq = this.cfg.maxSeqLen || 2048;
    let ids = Array.from(inIds);
    const maxPrompt = Math.max(1, maxSeq - maxNewTokens - 1);
    if (ids.length > maxPrompt) ids = ids.slice(ids.length - maxPrompt);
    if (mode === "spec" && this.isGpt2) throw new Error("speculative decode needs a llama-style model");
    this.resetCache();
    const t0 = now();
    const logits = this.forwardPrompt(ids);
    const ttft = now() - t0;
    const out = [];
    let next = this.isGpt2 ? argmaxGpt2(logits, []) : this.lastArgmax;
    out.push(next);
    let specHits = 0;
    let specTries = 0;
    let stopReason = "max_new_tokens";
    if (onToken) await onToken(next, { phase: "prefill", ms: ttft });
    if (next === eosId) {
      stopReason = "eos";
    } else if (mode === "greedy") {
      for (let i = 1; i < maxNewTokens; i++) {
        if (ids.length + out.length >= this.cfg.maxSeqLen) break;
        const step = this.forwardDecode(next);
        next = this.isGpt2 ? argmaxGpt2(step, out) : this.lastArgmax;
        out.push(next);
        if (onToken) await onToken(next, { phase: "decode" });
        if (next === eosId) {
          stopReason = "eos";
          break;
        }
      }
    } else if (mode === "chain") {
      while (out.length < maxNewTokens) {
        if (this.cacheLen >= maxSeq - 1) {
          stopReason = "context_limit";
          break;
        }
        const n = Math.min(chainChunk, maxNewTokens - out.length, maxSeq - 1 - this.cacheLen);
        const got = this.decodeChain(out[out.length - 1], n, eosId, this.isGpt2 ? out : null);
        for (const tok of got) {
          out.push(tok);
          if (onToken) await onToken(tok, { phase: "chain" });
        }
        if (got.length && got[got.length - 1] === eosId) {
          stopReason = "eos";
          break;
        }
      }
    } else if (mode === "spec") {
      const seq = ids.concat(out);
      while (out.length < maxNewTokens) {
        if (this.cacheLen >= maxSeq - 1) break;
        const x = out[out.length - 1];
        const pos = this.cacheLen;
        const room = Math.min(specK, this.maxPass - 1, maxSeq - 1 - pos);
        const draft = room > 0 ? lookupDraft(seq, room, ngram) : [];
        specTries++;
        const r = this.forwardVerify([x].concat(draft), false).argmax;
        out.push(r[0]);
        seq.push(r[0]);
        let newLen = pos + 1;
        if (onToken) await onToken(r[0], { phase: "decode" });
        if (r[0] !== eosId) {
          for (let k = 0; k < draft.length; k++) {
            if (r[k] !== draft[k] || out.length >= maxNewTokens) break;
            const nxt = r[k + 1];
            specHits++;
            out.push(nxt);
            seq.push(nxt);
            newLen = pos + 2 + k;
            if (onToken) await onToken(nxt, { phase: "spec" });
            if (nxt === eosId) break;
          }
        }
        this.cacheLen = newLen;
        if (out[out.length - 1] === eosId) {
          stopReason = "eos";
          break;
        }
      }
    } else {
      throw new Error(`unknown mode ${mode}`);
    }
    return {
      generatedIds: out,
      stopReason,
      ttftMs: ttft,
      totalMs: now() - t0,
      mode: `${this.mode}-${mode}`,
      specHits,
      specTries,
      timing: this.lastTiming,
    };
  }

  /** Frees the device memory; later calls throw "model was destroyed". */
  destroy() {
    native.destroy(this._h);
  }
}

export { argmax, argmaxGpt2, lookupDraft };
