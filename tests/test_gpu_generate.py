"""Token sequences of the HIP engine against the oracle's generate
(engine/infer.js:603-646, restated as orc_generate).

north_star: accepted-token sequences must be bit-exact.  Every driver of the
decode step -- the host greedy loop, the device-chained decode (with and
without EOS), prompt-lookup speculation at k = 4 and 8 -- must give the
oracle's ids, stop reason and prompt truncation.  The models are chosen so
that the oracle's top-2 logit margin exceeds MARGIN at every step of its own
greedy path (checked here before the comparison): where it does, a logits
difference within the 1e-2 parity bar cannot change the argmax.
"""
import numpy as np
import pytest

import mllm
from mllm import pgw

gpu = pytest.mark.gpu
MARGIN = 1e-2


def adjusted(logits, hist):
    """The logits argmaxGpt2 ranks (infer.js:252-287): 3-gram block, 1.15
    penalty over the last 32 generated ids."""
    v = logits.astype(np.float64).copy()
    n = len(hist)
    if n >= 2:
        for h in range(n - 2):
            if hist[h] == hist[-2] and hist[h + 1] == hist[-1]:
                v[hist[h + 2]] = -1e9
    for t in set(hist[max(0, n - 32):]):
        if v[t] > -1e8:
            v[t] = v[t] / 1.15 if v[t] > 0 else v[t] * 1.15
    return v


def min_margin(ref, prompt, n_new, gpt2):
    """The smallest top-2 margin along the oracle's own greedy path, and the path."""
    lg = ref.forward_prompt(prompt)
    hist, worst = [], np.inf
    for i in range(n_new):
        v = adjusted(lg, hist) if gpt2 else lg.astype(np.float64)
        top2 = np.partition(v, -2)[-2:]
        worst = min(worst, float(top2[1] - top2[0]))
        tok = int(np.argmax(v))
        hist.append(tok)
        if i + 1 < n_new:
            lg = ref.forward_decode(tok)
    return worst, hist


def pick_model(oracle_lib, arch, prompts, n_new, seeds, **over):
    """The first seed whose oracle greedy path keeps every margin above MARGIN
    for each prompt that prompts(seed, vocab, ref) returns (weights N(0, 0.1):
    wider logits than the N(0, 0.02) bench models).  Returns the bundle, the
    oracle model, the prompts and their greedy paths."""
    for seed in seeds:
        cfg = pgw.small_config(arch, **over)
        bundle = pgw.parse_pgw(pgw.make_model(cfg, seed=seed, std=0.1))
        ref = oracle_lib.OracleModel(bundle)
        ps, paths, ok = prompts(seed, cfg.vocab_size, ref), [], True
        for p in ps:
            m, path = min_margin(ref, p, n_new, arch == "gpt2")
            ok &= m > MARGIN
            paths.append(path)
        if ok:
            return bundle, ref, ps, paths
        ref.close()
    pytest.fail(f"no seed in {seeds} keeps the oracle's margins above {MARGIN}")


def random_prompt(n):
    return lambda seed, vocab, ref: [[int(v) for v in np.random.default_rng(seed).integers(0, vocab, n)]]


@gpu
@pytest.mark.parametrize("arch", ["llama", "gpt2"])
@pytest.mark.parametrize("mode", [1, 3])
def test_greedy_and_chain_ids_equal_oracle_generate(oracle_lib, arch, mode):
    n_new = 40
    bundle, ref, (prompt,), (path,) = pick_model(oracle_lib, arch, random_prompt(12), n_new, range(40, 60))
    ids, stop = ref.generate(prompt, max_new_tokens=n_new, eos_id=-1)
    assert ids == path and stop == "max_new_tokens"
    print(f"generate {arch} mode={mode}", flush=True)
    g = mllm.PetitGPT(bundle, exec_mode=mode)
    for drv, kw in (("greedy", {}), ("chain", {"chainChunk": 9})):
        r = g.generate(prompt, maxNewTokens=n_new, eosId=-1, mode=drv, **kw)
        assert r["generatedIds"] == ids, drv
        assert r["stopReason"] == "max_new_tokens", drv
    g.destroy()
    ref.close()


@gpu
@pytest.mark.parametrize("mode", [1, 3])
def test_eos_stop_equals_oracle_generate(oracle_lib, mode):
    """EOS = the oracle's 7th token: every driver stops on its first
    occurrence with stopReason "eos"."""
    bundle, ref, (prompt,), (path,) = pick_model(oracle_lib, "llama", random_prompt(10), 24, range(60, 80))
    eos = path[6]
    ids, stop = ref.generate(prompt, max_new_tokens=24, eos_id=eos)
    assert stop == "eos" and ids == path[:path.index(eos) + 1]
    print(f"eos mode={mode}", flush=True)
    g = mllm.PetitGPT(bundle, exec_mode=mode)
    for drv in ("greedy", "chain", "spec"):
        r = g.generate(prompt, maxNewTokens=24, eosId=eos, mode=drv)
        assert r["generatedIds"] == ids and r["stopReason"] == "eos", drv
    g.destroy()
    ref.close()


@gpu
@pytest.mark.parametrize("k", [4, 8])
def test_spec_ids_equal_oracle_generate(oracle_lib, k):
    """Prompt-lookup speculation (webgpu.js:1239-1270) accepts exactly the
    oracle's greedy ids.  The second prompt is the first, the oracle's
    greedy continuation of it, and the first again: the model then tends to
    continue with that continuation, which lookupDraft finds after the first
    copy, so drafts of full length k are proposed and accepted."""
    n_new = 32

    def prompts(seed, vocab, ref):
        p = [int(v) for v in np.random.default_rng(seed).integers(0, vocab, 16)]
        cont = ref.generate(p, max_new_tokens=n_new, eos_id=-1)[0]
        return [p, p + cont + p]

    bundle, ref, ps, paths = pick_model(oracle_lib, "llama", prompts, n_new, range(80, 100), max_seq_len=256)
    g = mllm.PetitGPT(bundle)
    for p, path in zip(ps, paths):
        ids, _ = ref.generate(p, max_new_tokens=n_new, eos_id=-1)
        assert ids == path
        r = g.generate(p, maxNewTokens=n_new, eosId=-1, mode="spec", specK=k)
        print(f"spec k={k} prompt {len(p)}: hits {r['specHits']} tries {r['specTries']}", flush=True)
        assert r["generatedIds"] == ids
    g.destroy()
    ref.close()


@gpu
def test_prompt_truncation_equals_oracle_generate(oracle_lib):
    """A prompt longer than maxSeq - maxNew - 1 keeps its last tokens
    (infer.js:604-608): 70 tokens with max_seq 64 and 10 new tokens are cut
    to the last 53."""
    max_new = 10

    def prompts(seed, vocab, ref):
        p = [int(v) for v in np.random.default_rng(seed).integers(0, vocab, 70)]
        return [p[-(64 - max_new - 1):]]

    bundle, ref, (cut,), (path,) = pick_model(oracle_lib, "llama", prompts, max_new, range(100, 120))
    long_prompt = [int(v) for v in np.random.default_rng(7).integers(0, bundle.cfg.vocab_size, 17)] + cut
    ids, stop = ref.generate(long_prompt, max_new_tokens=max_new, eos_id=-1)
    assert ids == path and stop == "max_new_tokens"
    g = mllm.PetitGPT(bundle)
    for drv in ("greedy", "chain"):
        r = g.generate(long_prompt, maxNewTokens=max_new, eosId=-1, mode=drv)
        assert r["generatedIds"] == ids and r["stopReason"] == stop, drv
    g.destroy()
    ref.close()
