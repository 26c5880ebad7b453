"""Stage probe of the chained decode kernel k_flow3.

    python microllm-lab_amd/build.py probe            # libmllm_probe.so (-DMLLM_STAGE_PROBE)
    python microllm-lab_amd/stage_probe.py [135m|360m] [prompt] [steps]

Runs a greedy chain on libmllm_probe.so (the same sources with thread-0
s_memrealtime stamps at fixed points of every item, 100 MHz) and prints where
a layer's time goes: each stage's handoff and the segments inside its items,
as medians over the last 16 recorded positions and layers 1 .. L-1, in us.
The stamps cost a few percent of the step, so the layer period here is a
little longer than in the default build.  The stamp points are listed at the
stage-probe block of csrc/mllm_engine.hip.
"""
from __future__ import annotations

import ctypes as C
import json
import os
import sys

import numpy as np

PKG = os.path.dirname(os.path.abspath(__file__))
PROBE_LIB = os.path.join(PKG, "libmllm_probe.so")
NPOS, PSLOTS, PNI, PK, PROBE_TOP, PROBE_LM = 16, 34, 256, 8, 32, 33
TICK_US = 0.01  # s_memrealtime runs at 100 MHz


def run(name: str, plen: int, steps: int, warm: int = 32):
    os.environ["MLLM_LIBRARY"] = PROBE_LIB
    sys.path.insert(0, PKG)
    import mllm
    from mllm import pgw

    cfg = pgw.CONFIGS[{"135m": "smollm2-135m", "360m": "smollm2-360m"}[name]]
    bundle = pgw.parse_pgw(pgw.make_llama(cfg, seed=0))
    prompt = [int(v) for v in np.random.default_rng(1).integers(0, cfg.vocab_size, plen)]
    g = mllm.PetitGPT(bundle, exec_mode=3, kv_fp16=name == "360m")
    assert g.decodeKernel == "k_flow3", g.decodeKernel
    lib = mllm.abi.lib()
    lib.mllm_probe_read.argtypes = [C.c_void_p]
    g.forwardPrompt(prompt)
    g.decodeChain(g.last_argmax, warm)
    g.forwardPrompt(prompt)
    assert lib.mllm_probe_clear() == 0
    g.decodeChain(g.last_argmax, steps)
    ms, n = g.last_timing()
    buf = np.zeros(NPOS * PSLOTS * PNI * PK, np.uint64)
    assert lib.mllm_probe_read(buf.ctypes.data) == 0
    g.destroy()
    geo = {"L": cfg.n_layers, "NH": cfg.n_heads, "NKV": cfg.n_kv_heads, "nm": cfg.d_ff // 64,
           "nsplit": (cfg.max_seq_len + 255) // 256, "first": plen, "steps": steps,
           "us_per_token": ms * 1e3 / max(n, 1)}
    return buf.reshape(NPOS, PSLOTS, PNI, PK).astype(np.int64), geo


def analyse(b, geo):
    L, NH, NKV = geo["L"], geo["NH"], geo["NKV"]
    ia = 2 * (NH + 2 * NKV)
    im = ia + NH * geo["nsplit"]
    ni = im + geo["nm"]
    last = geo["first"] + geo["steps"] - 1
    rows = {}

    def add(k, v):
        rows.setdefault(k, []).append(float(v) * TICK_US)

    for pos in range(last - NPOS + 1, last + 1):
        s = pos & 15
        for li in range(1, L):
            Q, A, M, Mp = b[s, li, :ia], b[s, li, ia:im], b[s, li, im:ni], b[s, li - 1, im:ni]
            A = A[A[:, 1] > 0]  # items past the reached splits return at once
            t0 = Mp[:, 7].max()
            add("QKV: inputs gathered after the previous MLP stage (first item)", Q[:, 1].min() - t0)
            add("QKV: inputs gathered after the previous MLP stage (last item)", Q[:, 1].max() - t0)
            add("QKV: residual + norm scale (wave 0)", np.median(Q[:, 5] - Q[:, 1]))
            add("QKV: records staged (wave 0)", np.median(Q[:, 6] - Q[:, 5]))
            add("QKV: barrier after the records", np.median(Q[:, 2] - Q[:, 6]))
            add("QKV: chunk dots", np.median(Q[:, 3] - Q[:, 2]))
            add("QKV: row sums", np.median(Q[:, 4] - Q[:, 3]))
            add("QKV: RoPE + q/k/v and cache stores", np.median(Q[:, 7] - Q[:, 4]))
            add("QKV stage (previous MLP stage done -> last QKV item done)", Q[:, 7].max() - t0)
            tq = Q[:, 7].max()
            add("ATT: q/k/v rows in after the QKV stage (first item)", A[:, 1].min() - tq)
            add("ATT: q/k/v rows in after the QKV stage (last item)", A[:, 1].max() - tq)
            add("ATT: K/V of the split assembled", np.median(A[:, 4] - A[:, 1]))
            add("ATT: scores, softmax statistics, P.V (wave 0)", np.median(A[:, 5] - A[:, 4]))
            add("ATT: store wait + barrier", np.median(A[:, 2] - A[:, 5]))
            add("ATT: split merges + head-output records", np.median(A[:, 3] - A[:, 2]))
            add("ATT: W_o slice", np.median(A[:, 7] - A[:, 3]))
            add("ATT stage (QKV stage done -> last attention item done)", A[:, 7].max() - tq)
            ta = A[:, 7].max()
            add("MLP: inputs gathered after the attention stage (first item)", M[:, 1].min() - ta)
            add("MLP: inputs gathered after the attention stage (last item)", M[:, 1].max() - ta)
            add("MLP: residual + norm scale (wave 0)", np.median(M[:, 5] - M[:, 1]))
            add("MLP: records staged (wave 0)", np.median(M[:, 6] - M[:, 5]))
            add("MLP: barrier after the records", np.median(M[:, 2] - M[:, 6]))
            add("MLP: gate/up chunk dots", np.median(M[:, 3] - M[:, 2]))
            add("MLP: row sums + activation records", np.median(M[:, 4] - M[:, 3]))
            add("MLP: down slice", np.median(M[:, 7] - M[:, 4]))
            add("MLP stage (attention stage done -> last MLP item done)", M[:, 7].max() - ta)
            add("layer period", M[:, 7].max() - t0)
        tl = b[s, L - 1, im:ni, 7].max()
        lm = b[s, PROBE_LM]
        lm = lm[lm[:, 3] > 0]
        add("LM: last layer's flags seen after its last MLP item (last workgroup)", lm[:, 1].max() - tl)
        add("LM: final-norm records in after the last MLP item (median)", np.median(lm[:, 2] - tl))
        add("LM: last tile done after the last MLP item", lm[:, 3].max() - tl)
        if pos < last:
            n = (pos + 1) & 15
            top = b[n, PROBE_TOP, 0]
            add("next step: token resolved (workgroup 0) after the last tile", top[1] - lm[:, 3].max())
            add("next step: first layer-0 QKV records after the resolve", b[n, 0, :ia, 2].min() - top[1])
            add("token period (last MLP item of the last layer to the next one's)",
                b[n, L - 1, im:ni, 7].max() - tl)
    return {k: (float(np.median(v)), float(np.percentile(v, 90))) for k, v in rows.items()}


def main():
    name = sys.argv[1] if len(sys.argv) > 1 else "135m"
    plen = int(sys.argv[2]) if len(sys.argv) > 2 else (32 if name == "135m" else 1536)
    steps = int(sys.argv[3]) if len(sys.argv) > 3 else 127
    b, geo = run(name, plen, steps)
    res = analyse(b, geo)
    print(f"k_flow3 stage probe, {name}, positions {plen + steps - 16}..{plen + steps - 1} "
          f"(chain of {steps} after a {plen}-token prompt), {geo['us_per_token']:.1f} us per token with the stamps")
    print("| segment | median us | p90 us |\n|---|---|---|")
    for k, (med, p90) in res.items():
        print(f"| {k} | {med:.2f} | {p90:.2f} |")
    out = os.environ.get("MLLM_PROBE_JSON")
    if out:
        with open(out, "w") as f:
            json.dump({"geo": geo, "stages": res}, f, indent=1)


if __name__ == "__main__":
    main()
