"""A HuggingFace-format checkpoint converted by the C++ converter
(pgw.convert_checkpoint, include/pgw_convert.h) runs on the GPU engine: the
prompt (batched path) and decode steps within LOGIT_TOL (max-abs 1e-2) of the
oracle on the same file."""
import json
import os

import numpy as np
import pytest

import mllm
from mllm import pgw

gpu = pytest.mark.gpu
LOGIT_TOL = 1e-2


@gpu
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_converted_llama_checkpoint_runs_on_the_engine(oracle_lib, tmp_path, dtype):
    import torch
    from safetensors.torch import save_file

    rng = np.random.default_rng(31)
    L, D, NH, NKV, FF, V = 2, 128, 2, 1, 256, 512

    def w(*shape):
        return torch.from_numpy(rng.standard_normal(shape, dtype=np.float32) * np.float32(0.05))

    s = {"model.embed_tokens.weight": w(V, D), "model.norm.weight": 1 + 0.1 * w(D)}
    for i in range(L):
        p = f"model.layers.{i}."
        s.update({p + "input_layernorm.weight": 1 + 0.1 * w(D), p + "post_attention_layernorm.weight": 1 + 0.1 * w(D),
                  p + "self_attn.q_proj.weight": w(D, D), p + "self_attn.k_proj.weight": w(NKV * 64, D),
                  p + "self_attn.v_proj.weight": w(NKV * 64, D), p + "self_attn.o_proj.weight": w(D, D),
                  p + "mlp.gate_proj.weight": w(FF, D), p + "mlp.up_proj.weight": w(FF, D),
                  p + "mlp.down_proj.weight": w(D, FF)})
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    d = str(tmp_path / "hf")
    os.makedirs(d)
    save_file({k: v.contiguous().to(tdt) for k, v in s.items()}, os.path.join(d, "model.safetensors"))
    with open(os.path.join(d, "config.json"), "w") as f:
        json.dump({"num_hidden_layers": L, "hidden_size": D, "num_attention_heads": NH, "num_key_value_heads": NKV,
                   "intermediate_size": FF, "vocab_size": V, "rope_theta": 10000.0, "tie_word_embeddings": True}, f)
    out = str(tmp_path / "model.q4.bin")
    pgw.convert_checkpoint(d, out, "llama", 512)
    bundle = pgw.parse_pgw(open(out, "rb").read())
    print(f"converted {dtype} checkpoint", flush=True)
    g = mllm.PetitGPT(bundle)
    ref = oracle_lib.OracleModel(bundle)
    prompt = [int(v) for v in rng.integers(0, V, 80)]
    worst = float(np.abs(g.forwardPrompt(prompt) - ref.forward_prompt(prompt)).max())
    for t in (3, 77, 200):
        worst = max(worst, float(np.abs(g.forwardDecode(t) - ref.forward_decode(t)).max()))
    g.destroy()
    assert worst < LOGIT_TOL, worst
