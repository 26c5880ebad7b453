"""Prompt-lookup speculative decode (webgpu.js:846-865, 1239-1270) on the GPU:
the accepted-token sequence must equal plain greedy decode exactly (the verify
pass rows are bit-identical to single-token decode)."""
import numpy as np
import pytest

import mllm
from mllm import pgw

gpu = pytest.mark.gpu


def spans_prompt(rng, vocab, length, copy_frac=0.4):
    """BASELINE config 3 prompt: spans of 8..32 tokens, ~40% verbatim copies."""
    out = []
    while len(out) < length:
        n = int(rng.integers(8, 33))
        if out and rng.random() < copy_frac and len(out) > n:
            s = int(rng.integers(0, len(out) - n))
            out += out[s:s + n]
        else:
            out += [int(v) for v in rng.integers(0, vocab, n)]
    return out[:length]


@gpu
@pytest.mark.parametrize("k,mode", [(2, 1), (4, 1), (8, 1), (4, 2), (8, 2)])
def test_spec_equals_greedy_small(k, mode):
    bundle = pgw.parse_pgw(pgw.make_llama(pgw.small_config("llama", max_seq_len=256), seed=21))
    g = mllm.PetitGPT(bundle, exec_mode=mode)
    prompt = spans_prompt(np.random.default_rng(3), bundle.cfg.vocab_size, 96)
    greedy = g.generate(prompt, maxNewTokens=48, mode="greedy")
    spec = g.generate(prompt, maxNewTokens=48, mode="spec", specK=k)
    g.destroy()
    assert spec["generatedIds"] == greedy["generatedIds"]
    assert spec["specTries"] > 0
    assert spec["specHits"] + spec["specTries"] >= len(spec["generatedIds"]) - 1


@gpu
def test_spec_equals_greedy_135m_k8():
    cfg = pgw.CONFIGS["smollm2-135m"]
    bundle = pgw.parse_pgw(pgw.make_llama(cfg, seed=0))
    g = mllm.PetitGPT(bundle)
    prompt = spans_prompt(np.random.default_rng(3), cfg.vocab_size, 512)
    greedy = g.generate(prompt, maxNewTokens=40, mode="chain")
    spec = g.generate(prompt, maxNewTokens=40, mode="spec", specK=8)
    g.destroy()
    assert spec["generatedIds"] == greedy["generatedIds"]
