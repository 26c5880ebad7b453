/**
 * PGW1 container reader (the format of engine/weights.js:5-39).
 *
 * parsePgw(buffer) -> { kind, cfg, tensors, buffer, payloadOff }, with the
 * header fields, the JSON tensor table keyed by name, and the arch fix-up of
 * weights.js:36-38 (a "gpt2" header over llama tensor names reads as llama).
 */
export const DTYPE_CODE = { 0: "f32", 1: "f16", 2: "bf16", 3: "q8", 4: "q4" };
export const STORAGE_CODE = { f32: 0, f16: 1, bf16: 2, q8: 3, q4: 4, q8g32: 5 };

function readUtf8(bytes) {
  if (typeof TextDecoder !== "undefined") return new TextDecoder().decode(bytes);
  return Buffer.from(bytes.buffer, bytes.byteOffset, bytes.byteLength).toString("utf8");
}

export function parsePgw(buffer) {
  const ab = buffer instanceof ArrayBuffer ? buffer : buffer.buffer.slice(buffer.byteOffset, buffer.byteOffset + buffer.byteLength);
  const view = new DataView(ab);
  const magic = String.fromCharCode(view.getUint8(0), view.getUint8(1), view.getUint8(2), view.getUint8(3));
  if (magic !== "PGW1") throw new Error(`bad magic ${magic}`);
  const kind = DTYPE_CODE[view.getUint8(4)] || "f32";
  const arch = view.getUint8(5) === 1 ? "gpt2" : "llama";
  const cfg = {
    arch,
    vocabSize: view.getUint32(8, true),
    nLayers: view.getUint32(12, true),
    dModel: view.getUint32(16, true),
    nHeads: view.getUint32(20, true),
    nKvHeads: view.getUint32(24, true),
    dFf: view.getUint32(28, true),
    maxSeqLen: view.getUint32(32, true),
    qGroup: view.getUint32(36, true) || 32,
    ropeTheta: view.getFloat64(56, true) || 10000,
    ropePct: view.getFloat64(64, true) || 1,
  };
  const tableOff = view.getUint32(40, true);
  const tableLen = view.getUint32(44, true);
  const payloadOff = view.getUint32(48, true);
  const table = JSON.parse(readUtf8(new Uint8Array(ab, tableOff, tableLen)));
  const tensors = Object.create(null);
  for (const e of table) tensors[e.name] = e;
  if (cfg.arch === "gpt2" && !tensors["blocks.0.ln1"] && tensors["blocks.0.norm1"]) cfg.arch = "llama";
  return { kind, cfg, tensors, buffer: ab, payloadOff };
}

export function f32View(bundle, name) {
  const t = bundle.tensors[name];
  if (!t) throw new Error(`missing tensor ${name}`);
  if (t.storage !== "f32") throw new Error(`${name} is ${t.storage}, not f32`);
  return new Float32Array(bundle.buffer, bundle.payloadOff + t.offset, t.nbytes / 4);
}

/** The tensor table in the shape the native layer takes. */
export function tensorTable(bundle) {
  const out = [];
  for (const name of Object.keys(bundle.tensors)) {
    const t = bundle.tensors[name];
    const shape = t.shape;
    out.push({
      name,
      storage: STORAGE_CODE[t.storage],
      rows: shape.length === 2 ? shape[0] : 1,
      cols: shape.length === 2 ? shape[1] : shape[0],
      group: t.group || 32,
      offset: t.offset,
      nbytes: t.nbytes,
      scaleOffset: t.scaleOffset || 0,
      scaleNbytes: t.scaleNbytes || 0,
    });
  }
  return out;
}
