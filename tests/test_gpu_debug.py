"""The GPU engine's layer-truncation knobs (GpuPetitGPT.debugMaxLayers /
debugNoAttn / debugNoMlp / debugMlpTo, webgpu-metal.js:1263-1279, set by
app.js:1317-1325) against the oracle with the same knobs.

A dropped block adds nothing to the residual, so the engine's logits must be
the truncated network's: within LOGIT_TOL (max-abs 1e-2) of the oracle's,
argmax equal wherever the oracle's top-2 margin exceeds MARGIN, in the
kernel-per-phase mode and the persistent kernel, and verify rows bit for bit
the decode step's.  Clearing the knobs restores the full network.
"""
import numpy as np
import pytest

import mllm
from mllm import pgw

gpu = pytest.mark.gpu
LOGIT_TOL = 1e-2
MARGIN = 1e-2
KNOBS = [{"max_layers": 0}, {"max_layers": 1}, {"no_attn": True}, {"no_mlp": True}, {"mlp_to": 1},
         {"max_layers": 1, "no_mlp": True}]


def margin(logits):
    top2 = np.partition(logits, -2)[-2:]
    return float(top2[1] - top2[0])


def set_knobs(g, kw):
    g.debugMaxLayers = kw.get("max_layers")
    g.debugNoAttn = kw.get("no_attn", False)
    g.debugNoMlp = kw.get("no_mlp", False)
    g.debugMlpTo = kw.get("mlp_to")


def run(g, ref, prompt, follow):
    """The prompt's logits and teacher-forced decode steps, both models: the
    worst max-abs difference and whether the argmax agrees wherever the
    oracle's margin allows."""
    pairs = [(g.forwardPrompt(prompt).copy(), ref.forward_prompt(prompt))]
    for tok in follow:
        pairs.append((g.forwardDecode(tok).copy(), ref.forward_decode(tok)))
    worst = max(float(np.abs(a - b).max()) for a, b in pairs)
    agree = all(int(np.argmax(a)) == int(np.argmax(b)) or margin(b) <= MARGIN for a, b in pairs)
    return worst, agree


@gpu
@pytest.mark.parametrize("arch", ["llama", "gpt2"])
@pytest.mark.parametrize("mode", [1, 3])
def test_debug_knobs_equal_oracle(oracle_lib, arch, mode):
    bundle = pgw.parse_pgw(pgw.make_model(pgw.small_config(arch, n_layers=3, max_seq_len=128), seed=40,
                                          **({"bias_std": 0.02} if arch == "gpt2" else {})))
    g = mllm.PetitGPT(bundle, exec_mode=mode)
    ref = oracle_lib.OracleModel(bundle)
    rng = np.random.default_rng(41)
    prompt = [int(v) for v in rng.integers(0, bundle.cfg.vocab_size, 12)]
    follow = [int(v) for v in rng.integers(0, bundle.cfg.vocab_size, 6)]
    full = g.forwardPrompt(prompt).copy()
    for kw in KNOBS:
        print(f"debug knobs {arch} mode={mode}: {kw}", flush=True)
        set_knobs(g, kw)
        ref.set_debug(**kw)
        ref.reset_cache()
        worst, agree = run(g, ref, prompt, follow)
        assert worst < LOGIT_TOL and agree, (kw, worst)
        assert not np.array_equal(g.forwardPrompt(prompt), full), kw
    set_knobs(g, {})
    ref.set_debug()
    ref.reset_cache()
    worst, agree = run(g, ref, prompt, follow)
    assert worst < LOGIT_TOL and agree, worst
    g.destroy()
    ref.close()


@gpu
@pytest.mark.parametrize("kw", [{"max_layers": 1}, {"no_attn": True}, {"mlp_to": 1}])
def test_debug_knobs_verify_rows_bit_identical_to_decode(kw):
    """Under the knobs a verify pass (the persistent verify kernel) still
    gives every row bit for bit as single-token decode, and a chained decode
    the host loop's ids."""
    bundle = pgw.parse_pgw(pgw.make_llama(pgw.small_config("llama", n_layers=3, max_seq_len=128), seed=42))
    g = mllm.PetitGPT(bundle)
    set_knobs(g, kw)
    prompt = [3, 1, 4, 1, 5, 9, 2, 6]
    extra = [5, 3, 5, 8, 9]
    g.forwardPrompt(prompt)
    am, lg = g.forwardVerify(extra, want_logits=True)
    g.forwardPrompt(prompt)
    for i, t in enumerate(extra):
        row = g.forwardDecode(t).copy()
        assert np.array_equal(row.view(np.uint32), lg[i].view(np.uint32)), (kw, i)
        assert am[i] == g.last_argmax
    greedy = g.generate(prompt, maxNewTokens=16, mode="greedy")["generatedIds"]
    chain = g.generate(prompt, maxNewTokens=16, mode="chain")["generatedIds"]
    assert chain == greedy, kw
    g.destroy()
