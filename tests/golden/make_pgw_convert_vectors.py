"""Write tests/golden/pgw_convert_vectors.npz from the reference converters' own
packaging functions.

The converters' tensor packaging -- add_tensor (tools/convert_hf_to_pgw.py:37-72),
add_q4 / add_f32 (tools/convert_gpt2_to_pgw.py:36-69): the payload bytes, the
JSON entries and their key order -- has no closed form that pins it byte for
byte, so its output is recorded once from the reference code, for two tiny
seeded models (`llama_state`, `gpt2_state` below; the test regenerates the same
arrays from the seeds).  Their convert() functions themselves cannot run here
(they download the model), so the tensors go through the packaging functions
in the order convert() uses (convert_hf_to_pgw.py:104-122,
convert_gpt2_to_pgw.py:133-164), with the transforms convert() applies first
(q ‖ k ‖ v rows; GPT-2: Conv1D transposes, lm_head times the channel scales,
ln_f divided by them) -- the order and transforms are read from the source and
stated here.

Run in the build container only (the reference is not present on the GPU box):
    python tests/golden/make_pgw_convert_vectors.py [/root/reference]
Nothing of the reference is copied here; only the recorded outputs are stored.
"""
from __future__ import annotations

import importlib.util
import json
import os
import sys
from io import BytesIO

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))

# tiny shapes: cols multiples of 32
LLAMA = dict(vocab=96, layers=2, d=64, heads=2, kv_heads=1, ff=128, rope_theta=50000.0)
GPT2 = dict(vocab=80, layers=2, d=64, heads=2, n_positions=48)


def _w(rng, shape, std=0.05):
    return (rng.standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float32)


def llama_state(seed: int = 11) -> dict:
    """HF LlamaForCausalLM state dict (names as in model.safetensors), f32."""
    c = LLAMA
    rng = np.random.default_rng(seed)
    d, ff, hd = c["d"], c["ff"], c["d"] // c["heads"]
    kv = c["kv_heads"] * hd
    s = {"model.embed_tokens.weight": _w(rng, (c["vocab"], d)), "lm_head.weight": _w(rng, (c["vocab"], d))}
    for i in range(c["layers"]):
        p = f"model.layers.{i}."
        s[p + "input_layernorm.weight"] = (1 + _w(rng, (d,), 0.1)).astype(np.float32)
        s[p + "self_attn.q_proj.weight"] = _w(rng, (d, d))
        s[p + "self_attn.k_proj.weight"] = _w(rng, (kv, d))
        s[p + "self_attn.v_proj.weight"] = _w(rng, (kv, d))
        s[p + "self_attn.o_proj.weight"] = _w(rng, (d, d))
        s[p + "post_attention_layernorm.weight"] = (1 + _w(rng, (d,), 0.1)).astype(np.float32)
        s[p + "mlp.gate_proj.weight"] = _w(rng, (ff, d))
        s[p + "mlp.up_proj.weight"] = _w(rng, (ff, d))
        s[p + "mlp.down_proj.weight"] = _w(rng, (d, ff))
    s["model.norm.weight"] = (1 + _w(rng, (d,), 0.1)).astype(np.float32)
    return s


def gpt2_state(seed: int = 12) -> dict:
    """HF GPT2LMHeadModel state dict (trunk names without the "transformer."
    prefix, as in the hub's model.safetensors; Conv1D weights [in, out]), f32;
    plus the calibrated channel scales under "scale_factors"."""
    c = GPT2
    rng = np.random.default_rng(seed)
    d = c["d"]
    s = {"wte.weight": _w(rng, (c["vocab"], d)), "wpe.weight": _w(rng, (c["n_positions"], d))}
    for i in range(c["layers"]):
        p = f"h.{i}."
        s[p + "ln_1.weight"] = (1 + _w(rng, (d,), 0.1)).astype(np.float32)
        s[p + "ln_1.bias"] = _w(rng, (d,), 0.1)
        s[p + "attn.c_attn.weight"] = _w(rng, (d, 3 * d))
        s[p + "attn.c_attn.bias"] = _w(rng, (3 * d,), 0.1)
        s[p + "attn.c_proj.weight"] = _w(rng, (d, d))
        s[p + "attn.c_proj.bias"] = _w(rng, (d,), 0.1)
        s[p + "ln_2.weight"] = (1 + _w(rng, (d,), 0.1)).astype(np.float32)
        s[p + "ln_2.bias"] = _w(rng, (d,), 0.1)
        s[p + "mlp.c_fc.weight"] = _w(rng, (d, 4 * d))
        s[p + "mlp.c_fc.bias"] = _w(rng, (4 * d,), 0.1)
        s[p + "mlp.c_proj.weight"] = _w(rng, (4 * d, d))
        s[p + "mlp.c_proj.bias"] = _w(rng, (d,), 0.1)
    s["ln_f.weight"] = (1 + _w(rng, (d,), 0.1)).astype(np.float32)
    s["ln_f.bias"] = _w(rng, (d,), 0.1)
    s["scale_factors"] = np.exp(rng.standard_normal(d).astype(np.float32) * np.float32(0.3)).astype(np.float32)
    return s


def _load(ref_root: str, name: str):
    path = os.path.join(ref_root, "tools", name)
    spec = importlib.util.spec_from_file_location("_ref_" + name[:-3], path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def record_llama(ref) -> tuple:
    c, s = LLAMA, llama_state()
    entries, blobs = [], BytesIO()
    ref.add_tensor(entries, blobs, "lm_head", s["lm_head.weight"], "q4")
    for i in range(c["layers"]):
        p = f"model.layers.{i}."
        ref.add_tensor(entries, blobs, f"blocks.{i}.norm1", s[p + "input_layernorm.weight"], "f32")
        qkv = np.concatenate([s[p + "self_attn.q_proj.weight"], s[p + "self_attn.k_proj.weight"],
                              s[p + "self_attn.v_proj.weight"]], axis=0)
        ref.add_tensor(entries, blobs, f"blocks.{i}.attn.qkv", qkv, "q4")
        ref.add_tensor(entries, blobs, f"blocks.{i}.attn.proj", s[p + "self_attn.o_proj.weight"], "q4")
        ref.add_tensor(entries, blobs, f"blocks.{i}.norm2", s[p + "post_attention_layernorm.weight"], "f32")
        ref.add_tensor(entries, blobs, f"blocks.{i}.mlp.w1", s[p + "mlp.gate_proj.weight"], "q4")
        ref.add_tensor(entries, blobs, f"blocks.{i}.mlp.w3", s[p + "mlp.up_proj.weight"], "q4")
        ref.add_tensor(entries, blobs, f"blocks.{i}.mlp.w2", s[p + "mlp.down_proj.weight"], "q4")
    ref.add_tensor(entries, blobs, "norm_f", s["model.norm.weight"], "f32")
    return entries, blobs.getvalue()


def record_gpt2(ref, max_seq: int) -> tuple:
    c, s = GPT2, gpt2_state()
    scale = s["scale_factors"]
    n_ctx = min(c["n_positions"], max_seq)
    entries, blobs = [], BytesIO()
    ref.add_f32(entries, blobs, "scale_factors", scale)
    ref.add_q4(entries, blobs, "lm_head", s["wte.weight"] * scale[None, :])
    ref.add_f32(entries, blobs, "wpe", s["wpe.weight"][:n_ctx])
    ref.add_f32(entries, blobs, "ln_f", np.concatenate([s["ln_f.weight"] / scale, s["ln_f.bias"] / scale]))
    for i in range(c["layers"]):
        p = f"h.{i}."
        ref.add_f32(entries, blobs, f"blocks.{i}.ln1", np.concatenate([s[p + "ln_1.weight"], s[p + "ln_1.bias"]]))
        ref.add_q4(entries, blobs, f"blocks.{i}.attn.qkv", s[p + "attn.c_attn.weight"].T)
        ref.add_f32(entries, blobs, f"blocks.{i}.attn.qkv_bias", s[p + "attn.c_attn.bias"])
        ref.add_q4(entries, blobs, f"blocks.{i}.attn.proj", s[p + "attn.c_proj.weight"].T)
        ref.add_f32(entries, blobs, f"blocks.{i}.attn.proj_bias", s[p + "attn.c_proj.bias"])
        ref.add_f32(entries, blobs, f"blocks.{i}.ln2", np.concatenate([s[p + "ln_2.weight"], s[p + "ln_2.bias"]]))
        ref.add_q4(entries, blobs, f"blocks.{i}.mlp.fc", s[p + "mlp.c_fc.weight"].T)
        ref.add_f32(entries, blobs, f"blocks.{i}.mlp.fc_bias", s[p + "mlp.c_fc.bias"])
        ref.add_q4(entries, blobs, f"blocks.{i}.mlp.proj", s[p + "mlp.c_proj.weight"].T)
        ref.add_f32(entries, blobs, f"blocks.{i}.mlp.proj_bias", s[p + "mlp.c_proj.bias"])
    return entries, blobs.getvalue()


GPT2_MAX_SEQ = 32  # below n_positions: wpe is cut


def main():
    ref_root = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    le, lp = record_llama(_load(ref_root, "convert_hf_to_pgw.py"))
    ge, gp = record_gpt2(_load(ref_root, "convert_gpt2_to_pgw.py"), GPT2_MAX_SEQ)
    path = os.path.join(HERE, "pgw_convert_vectors.npz")
    np.savez_compressed(path, llama_entries=np.frombuffer(json.dumps(le).encode(), np.uint8),
                        llama_payload=np.frombuffer(lp, np.uint8),
                        gpt2_entries=np.frombuffer(json.dumps(ge).encode(), np.uint8),
                        gpt2_payload=np.frombuffer(gp, np.uint8))
    print(f"wrote {path}: llama {len(le)} tensors / {len(lp)} B, gpt2 {len(ge)} tensors / {len(gp)} B")


if __name__ == "__main__":
    main()
