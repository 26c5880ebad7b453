"""The kind-generic decode step (mllm_generic.hip) against the oracle:
models whose matrices are not all Q4 group-32.  infer.js:313-346 binds every
matrix by its own storage -- f32, f16, bf16, per-row Q8, Q4 of any group --
and the reference's GPU engine runs Q8 / f16 / bf16 models
(webgpu.js:902-973; WRITEUP.md:31-35 times each); Q8 group-32 is this
library's format.  The oracle's arithmetic on each storage is pinned
against HF transformers in float64 (test_oracle_model.py).

Bars: logits within LOGIT_TOL of the oracle's, relative to
max(1, max |logit|) (f32 activations throughout; the oracle accumulates
in float64); generated ids equal orc_generate along paths whose top-2
margin exceeds MARGIN; verify rows bit-identical to decode (the same
kernels per token); the chained decode equal to the host loop.
"""
import dataclasses

import numpy as np
import pytest

import mllm
from mllm import abi, pgw

gpu = pytest.mark.gpu
KINDS = ["q8", "q8g32", "f16", "bf16", "f32"]
LOGIT_TOL = 1e-4
MARGIN = 1e-2


def make(arch, kind, seed, std=0.1, group=32, storages=None, bias_std=None, **over):
    cfg = pgw.small_config(arch, **over)
    kw = {"bias_std": bias_std} if bias_std is not None else {}
    return pgw.parse_pgw(pgw.make_model(cfg, seed=seed, std=std, kind=kind, group=group, storages=storages, **kw))


def compare(g, ref, prompt, follow):
    """Worst relative logits difference over the prompt and the
    teacher-forced decode steps, and whether every argmax agrees where the
    oracle's margin allows."""
    pairs = [(g.forwardPrompt(prompt).copy(), ref.forward_prompt(prompt))]
    for t in follow:
        pairs.append((g.forwardDecode(t).copy(), ref.forward_decode(t)))
    worst, agree = 0.0, True
    for a, b in pairs:
        scale = max(1.0, float(np.abs(b).max()))
        worst = max(worst, float(np.abs(a - b).max()) / scale)
        top2 = np.partition(b, -2)[-2:]
        agree &= int(np.argmax(a)) == int(np.argmax(b)) or float(top2[1] - top2[0]) <= MARGIN
    return worst, agree


@gpu
@pytest.mark.parametrize("arch", ["llama", "gpt2"])
@pytest.mark.parametrize("kind", KINDS)
def test_kind_logits_equal_oracle(oracle_lib, arch, kind):
    bundle = make(arch, kind, seed=21, n_layers=3, **({"bias_std": 0.02} if arch == "gpt2" else {}))
    print(f"kind {kind} {arch}: prompt + 6 decode steps", flush=True)
    g = mllm.PetitGPT(bundle)
    assert g.decodeKernel == "generic kernels"
    ref = oracle_lib.OracleModel(bundle)
    rng = np.random.default_rng(22)
    prompt = [int(v) for v in rng.integers(0, bundle.cfg.vocab_size, 12)]
    follow = [int(v) for v in rng.integers(0, bundle.cfg.vocab_size, 6)]
    worst, agree = compare(g, ref, prompt, follow)
    assert worst < LOGIT_TOL and agree, (kind, arch, worst)
    g.destroy()
    ref.close()


def greedy_path(ref, prompt, n_new, gpt2):
    """The oracle's own greedy path and its smallest top-2 margin (gpt2:
    on the argmaxGpt2-adjusted logits)."""
    lg = ref.forward_prompt(prompt)
    hist, worst = [], np.inf
    for i in range(n_new):
        v = lg.astype(np.float64).copy()
        if gpt2:
            n = len(hist)
            if n >= 2:
                for h in range(n - 2):
                    if hist[h] == hist[-2] and hist[h + 1] == hist[-1]:
                        v[hist[h + 2]] = -1e9
            for t in set(hist[max(0, n - 32):]):
                if v[t] > -1e8:
                    v[t] = v[t] / 1.15 if v[t] > 0 else v[t] * 1.15
        top2 = np.partition(v, -2)[-2:]
        worst = min(worst, float(top2[1] - top2[0]))
        tok = int(np.argmax(v))
        hist.append(tok)
        if i + 1 < n_new:
            lg = ref.forward_decode(tok)
    return hist, worst


@gpu
@pytest.mark.parametrize("arch,kind", [("llama", "q8"), ("gpt2", "f16"), ("llama", "bf16"), ("gpt2", "q8")])
def test_kind_generate_equals_oracle(oracle_lib, arch, kind):
    """Greedy, chained (and for llama speculative) generate give
    orc_generate's ids; a chain stops at an EOS with stopReason "eos"."""
    n_new = 24
    for seed in range(30, 50):
        bundle = make(arch, kind, seed=seed)
        ref = oracle_lib.OracleModel(bundle)
        prompt = [int(v) for v in np.random.default_rng(seed).integers(0, bundle.cfg.vocab_size, 10)]
        path, m = greedy_path(ref, prompt, n_new, arch == "gpt2")
        if m > MARGIN:
            break
        ref.close()
    else:
        pytest.fail("no seed keeps the oracle's margins above MARGIN")
    ids, stop = ref.generate(prompt, max_new_tokens=n_new, eos_id=-1)
    assert ids == path and stop == "max_new_tokens"
    print(f"generate {kind} {arch} seed {seed}", flush=True)
    g = mllm.PetitGPT(bundle)
    drivers = [("greedy", {}), ("chain", {"chainChunk": 7})] + ([("spec", {"specK": 4})] if arch == "llama" else [])
    for drv, kw in drivers:
        r = g.generate(prompt, maxNewTokens=n_new, eosId=-1, mode=drv, **kw)
        assert r["generatedIds"] == ids and r["stopReason"] == "max_new_tokens", drv
    eos = path[5]
    want, stop = ref.generate(prompt, max_new_tokens=n_new, eos_id=eos)
    assert stop == "eos"
    for drv in ("greedy", "chain"):
        r = g.generate(prompt, maxNewTokens=n_new, eosId=eos, mode=drv)
        assert r["generatedIds"] == want and r["stopReason"] == "eos", drv
    g.destroy()
    ref.close()


@gpu
@pytest.mark.parametrize("kind", ["q8", "f16"])
def test_kind_verify_rows_bit_identical_to_decode(kind):
    bundle = make("llama", kind, seed=23)
    g = mllm.PetitGPT(bundle)
    prompt = [3, 1, 4, 1, 5, 9, 2, 6]
    extra = [5, 3, 5, 8, 9, 7, 9, 3, 2]
    g.forwardPrompt(prompt)
    am, lg = g.forwardVerify(extra, want_logits=True)
    g.forwardPrompt(prompt)
    for i, t in enumerate(extra):
        row = g.forwardDecode(t).copy()
        assert np.array_equal(row.view(np.uint32), lg[i].view(np.uint32)), i
        assert am[i] == g.last_argmax
    g.destroy()


@gpu
def test_mixed_storages_and_q4_groups(oracle_lib):
    """A Q4 model with one per-row Q8 matrix (the gate of layer 0), a Q4
    model at group 64, and one mixing f16 attention with bf16 MLP matrices:
    each takes the kind-generic step and matches the oracle."""
    cases = [
        ("q4 + q8 gate", make("llama", "q4", seed=24, storages={"blocks.0.mlp.w1": "q8"})),
        ("q4 group 64", make("llama", "q4", seed=25, group=64)),
        ("f16 attn, bf16 mlp", make("llama", "f16", seed=26, storages={
            f"blocks.{i}.mlp.{m}": "bf16" for i in range(2) for m in ("w1", "w2", "w3")})),
        ("gpt2 q4 group 64", make("gpt2", "q4", seed=27, group=64, bias_std=0.02)),
    ]
    rng = np.random.default_rng(28)
    for name, bundle in cases:
        print(f"mixed: {name}", flush=True)
        g = mllm.PetitGPT(bundle)
        assert g.decodeKernel == "generic kernels", name
        ref = oracle_lib.OracleModel(bundle)
        prompt = [int(v) for v in rng.integers(0, bundle.cfg.vocab_size, 9)]
        follow = [int(v) for v in rng.integers(0, bundle.cfg.vocab_size, 4)]
        worst, agree = compare(g, ref, prompt, follow)
        assert worst < LOGIT_TOL and agree, (name, worst)
        g.destroy()
        ref.close()


@gpu
def test_q4_group32_models_keep_the_fused_step():
    g = mllm.PetitGPT(make("llama", "q4", seed=29))
    assert g.decodeKernel != "generic kernels"
    g.destroy()


@gpu
def test_unsupported_storage_refused():
    """A Q4 matrix whose group does not divide into 8-column chunks is
    refused at creation with MLLM_ERR_UNSUPPORTED naming the tensor."""
    bundle = make("llama", "q4", seed=30)
    name = "blocks.1.attn.proj"
    tensors = dict(bundle.tensors)
    tensors[name] = {**tensors[name], "group": 12}
    bad = dataclasses.replace(bundle, tensors=tensors)
    print("unsupported storage refused", flush=True)
    with pytest.raises(abi.MllmError, match=f"{name}.*unsupported") as e:
        mllm.PetitGPT(bad)
    assert "UNSUPPORTED" in str(e.value)


@gpu
def test_kind_modes_debug_knobs_and_gemv(oracle_lib):
    """Exec modes 1 and 2 run the same kernels (bit-identical logits); the
    persistent kernel (modes 3 / 4) and batched prompts are refused; the
    debug knobs truncate the network as the oracle's do; model.gemv reads
    every storage."""
    bundle = make("llama", "f16", seed=31, n_layers=3, storages={"blocks.1.mlp.w2": "q8", "blocks.2.attn.qkv": "bf16"})
    g = mllm.PetitGPT(bundle)
    ref = oracle_lib.OracleModel(bundle)
    prompt = [7, 77, 177, 277, 377, 477]
    a = g.forwardPrompt(prompt).copy()
    g.set_exec_mode(2)
    assert np.array_equal(a.view(np.uint32), g.forwardPrompt(prompt).view(np.uint32))
    for mode in (3, 4):
        with pytest.raises(abi.MllmError, match="UNSUPPORTED"):
            g.set_exec_mode(mode)
    with pytest.raises(abi.MllmError, match="UNSUPPORTED"):
        g.set_prefill(2)
    g.set_prefill(0)
    for kw in ({"max_layers": 1}, {"no_attn": True}, {"no_mlp": True}, {"mlp_to": 2}):
        print(f"generic debug knobs {kw}", flush=True)
        g.debugMaxLayers = kw.get("max_layers")
        g.debugNoAttn = kw.get("no_attn", False)
        g.debugNoMlp = kw.get("no_mlp", False)
        g.debugMlpTo = kw.get("mlp_to")
        ref.set_debug(**kw)
        ref.reset_cache()
        worst, agree = compare(g, ref, prompt, [9, 99])
        assert worst < LOGIT_TOL and agree, (kw, worst)
    g.debugMaxLayers = None
    g.debugNoAttn = g.debugNoMlp = False
    g.debugMlpTo = None
    ref.set_debug()
    ref.reset_cache()
    worst, agree = compare(g, ref, prompt, [9])
    assert worst < LOGIT_TOL and agree
    x = np.random.default_rng(32).standard_normal(bundle.cfg.d_ff).astype(np.float32)
    xd = x[:bundle.cfg.d_model].copy()
    for name, xv in (("blocks.0.attn.proj", xd), ("blocks.1.mlp.w2", x), ("blocks.2.attn.qkv", xd),
                     ("lm_head", xd)):
        y, want = g.gemv(name, xv), ref.gemv(name, xv)
        assert np.abs(y - want).max() <= 1e-5 * max(1.0, float(np.abs(want).max())), name
    g.destroy()
    ref.close()


@gpu
def test_kind_fp16_kv_cache(oracle_lib):
    """An f16 KV cache (config 5's choice) on a Q8 model: the cache rounds
    k and v to f16, so the bar is the fp16-KV one of the Q4 engine (1e-2)."""
    bundle = make("llama", "q8", seed=33)
    g = mllm.PetitGPT(bundle, kv_fp16=True)
    ref = oracle_lib.OracleModel(bundle)
    prompt = [int(v) for v in np.random.default_rng(34).integers(0, bundle.cfg.vocab_size, 20)]
    worst, agree = compare(g, ref, prompt, [1, 2, 3])
    assert worst < 1e-2 and agree, worst
    g.destroy()
    ref.close()


@gpu
@pytest.mark.parametrize("kind", ["q8", "bf16"])
def test_kind_smollm2_135m_shape_vs_oracle(oracle_lib, kind):
    """The full SmolLM2-135M shape (30 layers, d576, 9/3 heads, vocab 49152)
    stored per-row Q8 and bf16: a 16-token prompt and three decode steps
    against the oracle."""
    bundle = pgw.parse_pgw(pgw.make_model(pgw.CONFIGS["smollm2-135m"], seed=35, kind=kind))
    print(f"135M {kind}", flush=True)
    g = mllm.PetitGPT(bundle)
    ref = oracle_lib.OracleModel(bundle)
    prompt = [int(v) for v in np.random.default_rng(36).integers(0, bundle.cfg.vocab_size, 16)]
    worst, agree = compare(g, ref, prompt, [11, 22, 33])
    assert worst < LOGIT_TOL and agree, worst
    g.destroy()
    ref.close()
