"""The persistent verify step (k_flowm, speculation's k + 1 rows,
webgpu.js:568-685) at the shapes it runs on in the benchmarks.

Every row of a verify pass must equal, bit for bit, single-token decode of
the same engine at that position (forwardDecode, the decode kernel k_flow3),
so that accepted-token sequences equal plain greedy ones exactly.  The
small-model tests in test_gpu_decode.py cover the rule; here it is checked
where the launch geometry differs:

- the full 135M model (config 1 / 3: d_model 576, 9 query / 3 KV heads,
  rep 3, 30 layers, vocabulary 49152) at M = 3, 5, 9 (the fused three-stage
  form) and M = 12 (the five-stage form with norm items and token groups);
- config 5's per-layer shape (d_model 960, 15 / 5 heads, d_ff 2560, f16 KV,
  2 layers, vocabulary 512) with the pass straddling the 1792-position
  attention split boundary, so that merging and non-merging split items and
  a token whose merge gathers 7 splits all occur in one pass.

Mode 4 launches the same kernel without the cooperative launch API (the
profilers' path).  Its workgroups are all resident only while the device
runs nothing else: these tests run in one process on a dedicated GPU, where
that holds, and a wait that could not complete would end in the kernel's
bounded-poll error, not a hang.
"""
import numpy as np
import pytest

import mllm
from mllm import pgw

gpu = pytest.mark.gpu


@pytest.fixture(scope="module")
def m135():
    cfg = pgw.CONFIGS["smollm2-135m"]
    return pgw.parse_pgw(pgw.make_llama(cfg, seed=0))


@pytest.fixture(scope="module")
def c5shape():
    cfg = pgw.Config("llama", 512, 2, 960, 15, 5, 2560, 2048, 32, 100000.0, 1.0)
    return pgw.parse_pgw(pgw.make_llama(cfg, seed=5))


def verify_vs_decode(g, prompt, extra):
    """One verify pass over `extra` after `prompt`, then the same tokens by
    single-token decode after the same prompt: every row's logits and argmax
    must be the same bits."""
    g.forwardPrompt(prompt)
    am, lg = g.forwardVerify(extra, want_logits=True)
    assert g.cacheLen == len(prompt) + len(extra)
    g.forwardPrompt(prompt)
    for i, t in enumerate(extra):
        row = g.forwardDecode(t).copy()
        assert np.array_equal(row.view(np.uint32), lg[i].view(np.uint32)), f"row {i}"
        assert am[i] == g.last_argmax, f"row {i}"


@gpu
@pytest.mark.parametrize("mode", [3, 4])
@pytest.mark.parametrize("m", [3, 5, 9, 12])
def test_verify_rows_full_135m(m135, m, mode):
    g = mllm.PetitGPT(m135, exec_mode=mode)
    assert g.flowVerifyTokens >= m
    rng = np.random.default_rng(30 + m)
    prompt = [int(v) for v in rng.integers(0, m135.cfg.vocab_size, 40)]
    extra = [int(v) for v in rng.integers(0, m135.cfg.vocab_size, m)]
    print(f"verify 135m m={m} mode={mode}", flush=True)
    verify_vs_decode(g, prompt, extra)
    g.destroy()


@gpu
@pytest.mark.parametrize("m,plen", [(5, 1789), (9, 1786), (10, 1785)])
def test_verify_rows_config5_shape_across_split(c5shape, m, plen):
    """Positions plen .. plen + m - 1 straddle 1792 = 7 x 256: tokens before
    it merge 7 splits, tokens after it 8."""
    g = mllm.PetitGPT(c5shape, kv_fp16=True)
    assert g.flowVerifyTokens >= m
    rng = np.random.default_rng(40 + m)
    prompt = [int(v) for v in rng.integers(0, c5shape.cfg.vocab_size, plen)]
    extra = [int(v) for v in rng.integers(0, c5shape.cfg.vocab_size, m)]
    assert plen < 1792 <= plen + m - 1
    print(f"verify config5 shape m={m} from {plen}", flush=True)
    verify_vs_decode(g, prompt, extra)
    g.destroy()


@pytest.fixture(scope="module")
def cycle135(oracle_lib):
    """The 135M shape with a 12-token greedy cycle (pgw.make_cycle_llama) and
    a prompt holding the cycle once: prompt-lookup drafts are then full
    length and accepted.  Returns the bundle, the prompt and the oracle's
    generate ids (infer.js:603-646) with their smallest top-2 margin."""
    cfg = pgw.CONFIGS["smollm2-135m"]
    rng = np.random.default_rng(7)
    cycle = [int(v) for v in rng.choice(cfg.vocab_size, 12, replace=False)]
    bundle = pgw.parse_pgw(pgw.make_cycle_llama(cfg, cycle, seed=0))
    prompt = [int(v) for v in rng.integers(0, cfg.vocab_size, 20)] + cycle + cycle[:2]
    ref = oracle_lib.OracleModel(bundle)
    print("oracle: 135m cycle model, 48 tokens", flush=True)
    ids, stop = ref.generate(prompt, max_new_tokens=48, eos_id=-1)
    ref.reset_cache()
    lg, worst = ref.forward_prompt(prompt), np.inf
    for tok in ids[:-1]:
        top2 = np.partition(lg, -2)[-2:]
        worst = min(worst, float(top2[1] - top2[0]))
        lg = ref.forward_decode(tok)
    ref.close()
    return bundle, prompt, cycle, ids, stop, worst


@gpu
@pytest.mark.parametrize("k", [4, 8])
def test_spec_ids_full_drafts_135m_equal_oracle_generate(cycle135, k):
    """Speculation at the 135M shape with full-length drafts (k + 1 = 5 and
    9 verify rows per pass): the ids equal the oracle's generate, and more
    than two drafted tokens are accepted per verify pass on average."""
    bundle, prompt, cycle, ids, stop, worst = cycle135
    assert worst > 1.0 and stop == "max_new_tokens"
    assert ids[:24] == [cycle[(2 + i) % 12] for i in range(24)]  # the model follows its cycle
    g = mllm.PetitGPT(bundle)
    r = g.generate(prompt, maxNewTokens=48, eosId=-1, mode="spec", specK=k)
    print(f"spec 135m cycle k={k}: hits {r['specHits']} tries {r['specTries']}", flush=True)
    assert r["generatedIds"] == ids
    assert r["specHits"] > 2 * r["specTries"]
    g.destroy()


@gpu
def test_refused_cooperative_launch_falls_back_to_phase_kernels(monkeypatch):
    """When the runtime refuses the cooperative launch (simulated by the
    MLLM_REFUSE_COOPERATIVE test hook) and mode 3 was only the default, the
    model switches to the phase kernels for good -- also when the first
    persistent launch is a verify step, as in spec decode -- and the ids
    are those of a model that ran mode 1 from the start."""
    bundle = pgw.parse_pgw(pgw.make_llama(pgw.small_config("llama", max_seq_len=256), seed=21))
    rng = np.random.default_rng(3)
    prompt = [int(v) for v in rng.integers(0, bundle.cfg.vocab_size, 40)]
    prompt = prompt + prompt[:20]
    ref = mllm.PetitGPT(bundle, exec_mode=1)
    want = ref.generate(prompt, maxNewTokens=24, mode="greedy")["generatedIds"]
    ref.destroy()
    monkeypatch.setenv("MLLM_REFUSE_COOPERATIVE", "1")
    for drv in ("spec", "chain"):
        g = mllm.PetitGPT(bundle)
        assert g.execMode == 3
        r = g.generate(prompt, maxNewTokens=24, mode=drv, specK=4)
        print(f"refused cooperative launch, {drv}: exec mode {g.execMode}", flush=True)
        assert g.execMode == 1 and g.flowVerifyTokens == 0
        assert r["generatedIds"] == want, drv
        g.destroy()
    # an explicit mode 3 reports the refusal instead
    g = mllm.PetitGPT(bundle, exec_mode=3)
    g.forwardPrompt(prompt[:8])
    with pytest.raises(mllm.abi.MllmError):
        g.forwardDecode(1)
    g.destroy()


@gpu
def test_epochs_restart_before_tags_wrap(monkeypatch):
    """Handoff tags are epoch * 128 + layer in 32 bits.  Started 20 epochs
    before 2^25 (MLLM_FLOW_EPOCH0 test hook), single steps, a verify step and
    a chain cross the point where the library clears the tagged buffers and
    restarts the epochs; logits and ids equal those of a model whose epochs
    start at 0."""
    bundle = pgw.parse_pgw(pgw.make_llama(pgw.small_config("llama", max_seq_len=256), seed=22))
    rng = np.random.default_rng(5)
    prompt = [int(v) for v in rng.integers(0, bundle.cfg.vocab_size, 12)]
    follow = [int(v) for v in rng.integers(0, bundle.cfg.vocab_size, 30)]
    outs = []
    for epoch0 in (None, str((1 << 25) - 20)):
        if epoch0:
            monkeypatch.setenv("MLLM_FLOW_EPOCH0", epoch0)
        g = mllm.PetitGPT(bundle)
        assert g.execMode == 3
        g.forwardPrompt(prompt)
        rows = [g.forwardDecode(t).copy() for t in follow]
        _, lv = g.forwardVerify(follow[:5], want_logits=True)
        ids = g.decodeChain(follow[5], 40)
        outs.append((np.stack(rows), lv, ids))
        g.destroy()
    assert np.array_equal(outs[0][0].view(np.uint32), outs[1][0].view(np.uint32))
    assert np.array_equal(outs[0][1].view(np.uint32), outs[1][1].view(np.uint32))
    assert outs[0][2] == outs[1][2]
