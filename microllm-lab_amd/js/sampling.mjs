/**
 * Host-side token selection and prompt-lookup drafting.
 *   argmax      first index of the maximum (engine/infer.js:240-250)
 *   argmaxGpt2  3-gram block + 1.15 repetition penalty (engine/infer.js:252-287)
 *   lookupDraft prompt-lookup draft (engine/webgpu.js:846-865)
 */
export function argmax(logits) {
  let bi = 0;
  let bv = logits[0];
  for (let i = 1; i < logits.length; i++) {
    if (logits[i] > bv) {
      bv = logits[i];
      bi = i;
    }
  }
  return bi;
}

export function argmaxGpt2(logits, history, opts) {
  const noRepeatNgram = opts && opts.noRepeatNgram !== undefined ? opts.noRepeatNgram : 3;
  const penalty = opts && opts.penalty !== undefined ? opts.penalty : 1.15;
  const hist = history || [];
  const n = hist.length;
  const banned = new Set();
  if (noRepeatNgram === 3 && n >= 2) {
    const t1 = hist[n - 2];
    const t2 = hist[n - 1];
    for (let h = 0; h < n - 2; h++) if (hist[h] === t1 && hist[h + 1] === t2) banned.add(hist[h + 2]);
  }
  const recent = new Set(hist.slice(Math.max(0, n - 32)));
  let bestIdx = 0;
  let bestVal = -Infinity;
  for (let i = 0; i < logits.length; i++) {
    let v = logits[i];
    if (banned.has(i)) v = -1e9;
    if (penalty > 1.0 && v > -1e8 && recent.has(i)) v = v > 0 ? v / penalty : v * penalty;
    if (v > bestVal) {
      bestVal = v;
      bestIdx = i;
    }
  }
  return bestIdx;
}

export function lookupDraft(seq, k, n) {
  const len = seq.length;
  if (len < n + 1) return [];
  for (let i = len - n - 1; i >= 0; i--) {
    let ok = true;
    for (let j = 0; j < n; j++) {
      if (seq[i + j] !== seq[len - n + j]) {
        ok = false;
        break;
      }
    }
    if (ok) {
      const d = [];
      for (let t = 0; t < k && i + n + t < len; t++) d.push(seq[i + n + t]);
      return d;
    }
  }
  return [];
}
