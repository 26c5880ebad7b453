"""Config 5 (SmolLM2-360M shape, fp16 KV, 1536-token prompt decoded toward
the 2048 context) against the oracle (engine/infer.js:422-504, 553-601).

The per-layer shape is the 360M one -- d_model 960, 15 query / 5 KV heads,
d_ff 2560, max_seq 2048, f16 KV cache -- so the decode runs the d_model-960
instances of the fused attention item and of the persistent kernel, with 7
and then 8 attention splits of 256 positions merged per head.  Two layers
and a 512-token vocabulary keep the oracle's work to seconds; a second test
runs the full 32-layer 360M model on a short prompt.

Bars: logits within LOGIT_TOL (max-abs 1e-2) of the fp64-accumulating
oracle, greedy argmax identical wherever the oracle's top-2 margin exceeds
MARGIN.  The oracle keeps an f32 cache; the f16 cache rounds K and V, which
the 1e-2 bar absorbs (north_star's tolerance for config 5).
"""
import numpy as np
import pytest

import mllm
from mllm import pgw

gpu = pytest.mark.gpu
LOGIT_TOL = 1e-2
MARGIN = 1e-2


def margin(logits):
    top2 = np.partition(logits, -2)[-2:]
    return float(top2[1] - top2[0])


def agree(lg, lr):
    return int(np.argmax(lg)) == int(np.argmax(lr)) or margin(lr) <= MARGIN


@pytest.fixture(scope="module")
def c5(oracle_lib):
    """The oracle's logits for a 1536-token prompt, then every position of a
    teacher-forced continuation to 2048 (forward_multi continues from the
    cache, as infer.js's attention does with pastLen)."""
    cfg = pgw.Config("llama", 512, 2, 960, 15, 5, 2560, 2048, 32, 100000.0, 1.0)
    bundle = pgw.parse_pgw(pgw.make_llama(cfg, seed=5))
    rng = np.random.default_rng(5)
    prompt = [int(v) for v in rng.integers(0, cfg.vocab_size, 1536)]
    follow = [int(v) for v in rng.integers(0, cfg.vocab_size, 2048 - 1536)]
    ref = oracle_lib.OracleModel(bundle)
    print("oracle: 1536-token prompt", flush=True)
    first = ref.forward_prompt(prompt)
    print("oracle: positions 1536..2047", flush=True)
    rest = ref.forward_multi(follow)
    ref.close()
    return bundle, prompt, follow, first, rest


@gpu
@pytest.mark.parametrize("mode", [1, 3])
def test_config5_shape_to_2048_vs_oracle(c5, mode):
    """The batched prompt (1536 tokens in one chunk, f16 cache), then 512
    single-token decode steps to position 2047; every step's logits against
    the oracle's row for that position."""
    bundle, prompt, follow, first, rest = c5
    print(f"config5 shape mode={mode}", flush=True)
    g = mllm.PetitGPT(bundle, kv_fp16=True, exec_mode=mode)
    lg = g.forwardPrompt(prompt).copy()
    worst = float(np.abs(lg - first).max())
    ok = [agree(lg, first)]
    for i, tok in enumerate(follow):
        lg = g.forwardDecode(tok)
        worst = max(worst, float(np.abs(lg - rest[i]).max()))
        ok.append(agree(lg, rest[i]))
    assert g.cacheLen == 2048
    g.destroy()
    assert worst < LOGIT_TOL and all(ok), worst


@gpu
def test_config5_shape_chained_decode_equals_host_steps(c5):
    """From position 1792 (7 splits) the persistent chained decode and the
    phase kernels' host loop give the same ids across the 8th split."""
    bundle, prompt, follow, _, _ = c5
    outs = []
    for mode in (1, 3):
        g = mllm.PetitGPT(bundle, kv_fp16=True, exec_mode=mode)
        g.forwardPrompt(prompt + follow[:255])
        outs.append(g.decodeChain(follow[255], 200))
        g.destroy()
    assert outs[0] == outs[1]


@gpu
@pytest.mark.parametrize("mode", [1, 3])
def test_smollm2_360m_full_depth_vs_oracle(oracle_lib, mode):
    """The full 32-layer 360M model (vocabulary 49152, fp16 KV): a 32-token
    prompt and 4 greedy steps against the oracle."""
    cfg = pgw.CONFIGS["smollm2-360m"]
    bundle = pgw.parse_pgw(pgw.make_llama(cfg, seed=0))
    rng = np.random.default_rng(11)
    prompt = [int(v) for v in rng.integers(0, cfg.vocab_size, 32)]
    print(f"360m full depth mode={mode}", flush=True)
    g = mllm.PetitGPT(bundle, kv_fp16=True, exec_mode=mode)
    ref = oracle_lib.OracleModel(bundle)
    lg = g.forwardPrompt(prompt).copy()
    lr = ref.forward_prompt(prompt)
    worst, ok = float(np.abs(lg - lr).max()), [agree(lg, lr)]
    for _ in range(4):
        tok = int(np.argmax(lr))
        lg = g.forwardDecode(tok).copy()
        lr = ref.forward_decode(tok)
        worst = max(worst, float(np.abs(lg - lr).max()))
        ok.append(agree(lg, lr))
    g.destroy()
    ref.close()
    assert worst < LOGIT_TOL and all(ok), worst
