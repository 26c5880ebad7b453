"""Oracle pinning: the model forward (infer.js PetitGPT restatement) against
HF transformers' LlamaForCausalLM / GPT2LMHeadModel in float64, built from the
same dequantised weights.  The reference converters read exactly these HF
modules (tools/convert_hf_to_pgw.py:104-122, tools/convert_gpt2_to_pgw.py:135-164),
so agreement pins the tensor layout, RoPE convention, GQA grouping, SwiGLU /
GELU, LayerNorm and the tied embedding.  Also: the prefill/decode invariant
and the multi-token pass against sequential decode.
"""
import numpy as np
import pytest
import torch

from mllm import pgw

transformers = pytest.importorskip("transformers")


def _deq(bundle, name):
    """A matrix in float64 from its storage (weights.js:69-123 restated in
    numpy, independently of the oracle's C dequantisers)."""
    t = bundle.tensors[name]
    st, a = t["storage"], bundle.array(name)
    if st == "q4":
        return pgw.dequant_q4(a, bundle.scales(name), int(t.get("group", 32))).astype(np.float64)
    if st == "q8":
        return a.astype(np.float64) * bundle.scales(name).astype(np.float64).reshape(-1, 1)
    if st == "q8g32":
        return a.astype(np.float64) * np.repeat(bundle.scales(name).astype(np.float64), 32, axis=1)
    if st == "f16":
        return a.view(np.float16).astype(np.float64)
    if st == "bf16":
        return (a.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    return a.astype(np.float64)


def hf_llama(bundle):
    from transformers import LlamaConfig, LlamaForCausalLM

    c = bundle.cfg
    hc = LlamaConfig(vocab_size=c.vocab_size, hidden_size=c.d_model, intermediate_size=c.d_ff,
                     num_hidden_layers=c.n_layers, num_attention_heads=c.n_heads, num_key_value_heads=c.n_kv_heads,
                     rms_norm_eps=1e-6, rope_theta=c.rope_theta, max_position_embeddings=c.max_seq_len,
                     tie_word_embeddings=True, hidden_act="silu", attention_bias=False, mlp_bias=False,
                     bos_token_id=0, eos_token_id=0, pad_token_id=0)
    hc._attn_implementation = "eager"
    m = LlamaForCausalLM(hc).double().eval()
    hd = c.d_model // c.n_heads
    kv = c.n_kv_heads * hd
    T = lambda a: torch.tensor(a, dtype=torch.float64)  # noqa: E731
    with torch.no_grad():
        m.model.embed_tokens.weight.copy_(T(_deq(bundle, "lm_head")))
        m.lm_head.weight = m.model.embed_tokens.weight
        for i, layer in enumerate(m.model.layers):
            qkv = _deq(bundle, f"blocks.{i}.attn.qkv")
            layer.self_attn.q_proj.weight.copy_(T(qkv[:c.d_model]))
            layer.self_attn.k_proj.weight.copy_(T(qkv[c.d_model:c.d_model + kv]))
            layer.self_attn.v_proj.weight.copy_(T(qkv[c.d_model + kv:]))
            layer.self_attn.o_proj.weight.copy_(T(_deq(bundle, f"blocks.{i}.attn.proj")))
            layer.mlp.gate_proj.weight.copy_(T(_deq(bundle, f"blocks.{i}.mlp.w1")))
            layer.mlp.up_proj.weight.copy_(T(_deq(bundle, f"blocks.{i}.mlp.w3")))
            layer.mlp.down_proj.weight.copy_(T(_deq(bundle, f"blocks.{i}.mlp.w2")))
            layer.input_layernorm.weight.copy_(T(bundle.array(f"blocks.{i}.norm1")))
            layer.post_attention_layernorm.weight.copy_(T(bundle.array(f"blocks.{i}.norm2")))
        m.model.norm.weight.copy_(T(bundle.array("norm_f")))
    return m


def hf_gpt2(bundle):
    from transformers import GPT2Config, GPT2LMHeadModel

    c = bundle.cfg
    hc = GPT2Config(vocab_size=c.vocab_size, n_positions=c.max_seq_len, n_embd=c.d_model, n_layer=c.n_layers,
                    n_head=c.n_heads, n_inner=c.d_ff, activation_function="gelu_new", layer_norm_epsilon=1e-5,
                    resid_pdrop=0.0, embd_pdrop=0.0, attn_pdrop=0.0, bos_token_id=0, eos_token_id=0)
    hc._attn_implementation = "eager"
    m = GPT2LMHeadModel(hc).double().eval()
    D = c.d_model
    T = lambda a: torch.tensor(np.asarray(a, np.float64), dtype=torch.float64)  # noqa: E731
    with torch.no_grad():
        tr = m.transformer
        tr.wte.weight.copy_(T(_deq(bundle, "lm_head")))
        m.lm_head.weight = tr.wte.weight
        tr.wpe.weight.copy_(T(bundle.array("wpe")))
        lnf = bundle.array("ln_f")
        tr.ln_f.weight.copy_(T(lnf[:D]))
        tr.ln_f.bias.copy_(T(lnf[D:]))
        for i, blk in enumerate(tr.h):
            ln1, ln2 = bundle.array(f"blocks.{i}.ln1"), bundle.array(f"blocks.{i}.ln2")
            blk.ln_1.weight.copy_(T(ln1[:D]))
            blk.ln_1.bias.copy_(T(ln1[D:]))
            blk.ln_2.weight.copy_(T(ln2[:D]))
            blk.ln_2.bias.copy_(T(ln2[D:]))
            blk.attn.c_attn.weight.copy_(T(_deq(bundle, f"blocks.{i}.attn.qkv").T))  # Conv1D is [in, out]
            blk.attn.c_attn.bias.copy_(T(bundle.array(f"blocks.{i}.attn.qkv_bias")))
            blk.attn.c_proj.weight.copy_(T(_deq(bundle, f"blocks.{i}.attn.proj").T))
            blk.attn.c_proj.bias.copy_(T(bundle.array(f"blocks.{i}.attn.proj_bias")))
            blk.mlp.c_fc.weight.copy_(T(_deq(bundle, f"blocks.{i}.mlp.fc").T))
            blk.mlp.c_fc.bias.copy_(T(bundle.array(f"blocks.{i}.mlp.fc_bias")))
            blk.mlp.c_proj.weight.copy_(T(_deq(bundle, f"blocks.{i}.mlp.proj").T))
            blk.mlp.c_proj.bias.copy_(T(bundle.array(f"blocks.{i}.mlp.proj_bias")))
    return m


def hf_logits(m, ids):
    with torch.no_grad():
        return m(torch.tensor([ids])).logits[0].numpy()


@pytest.mark.parametrize("norm_gain", [1.0, 1.7])
def test_llama_forward_vs_hf(oracle_lib, norm_gain):
    cfg = pgw.small_config("llama", n_layers=2, n_heads=4, n_kv_heads=2, d_model=256, d_ff=512)
    bundle = pgw.parse_pgw(pgw.make_llama(cfg, seed=3, std=0.05, norm_gain=norm_gain))
    ref = oracle_lib.OracleModel(bundle)
    ids = [5, 77, 300, 12, 9, 500, 41]
    want = hf_logits(hf_llama(bundle), ids)
    got = ref.forward_prompt(ids)
    assert np.abs(got - want[-1]).max() < 2e-4 * max(1.0, np.abs(want[-1]).max())
    # decode continues consistently with the HF sequence
    got2 = ref.forward_decode(123)
    want2 = hf_logits(hf_llama(bundle), ids + [123])[-1]
    assert np.abs(got2 - want2).max() < 2e-4 * max(1.0, np.abs(want2).max())


KINDS = [("q8", 32), ("q8g32", 32), ("f16", 32), ("bf16", 32), ("f32", 32), ("q4", 64)]


@pytest.mark.parametrize("kind,group", KINDS)
def test_llama_kinds_vs_hf(oracle_lib, kind, group):
    """The oracle on every matrix storage infer.js:313-346 binds (and Q8
    group-32, Q4 at group 64): its GEMVs and embedding rows against HF in
    float64 on the same dequantised weights."""
    cfg = pgw.small_config("llama", n_layers=2, n_heads=4, n_kv_heads=2, d_model=256, d_ff=512)
    bundle = pgw.parse_pgw(pgw.make_llama(cfg, seed=3, std=0.05, kind=kind, group=group))
    assert bundle.tensors["blocks.0.mlp.w1"]["storage"] == kind and bundle.tensors["lm_head"]["storage"] == kind
    ref = oracle_lib.OracleModel(bundle)
    ids = [5, 77, 300, 12, 9, 500, 41]
    want = hf_logits(hf_llama(bundle), ids + [123])
    got = ref.forward_prompt(ids)
    assert np.abs(got - want[-2]).max() < 2e-4 * max(1.0, np.abs(want[-2]).max())
    got2 = ref.forward_decode(123)
    assert np.abs(got2 - want[-1]).max() < 2e-4 * max(1.0, np.abs(want[-1]).max())


@pytest.mark.parametrize("kind,group", KINDS)
def test_gpt2_kinds_vs_hf(oracle_lib, kind, group):
    cfg = pgw.small_config("gpt2", n_layers=2, n_heads=4, n_kv_heads=4, d_model=256, d_ff=1024, max_seq_len=32)
    bundle = pgw.parse_pgw(pgw.make_gpt2(cfg, seed=4, std=0.05, bias_std=0.05, kind=kind, group=group))
    ref = oracle_lib.OracleModel(bundle)
    ids = [3, 141, 59, 26, 5]
    want = hf_logits(hf_gpt2(bundle), ids)
    got = ref.forward_prompt(ids)
    assert np.abs(got - want[-1]).max() < 2e-4 * max(1.0, np.abs(want[-1]).max())


def test_gpt2_forward_vs_hf(oracle_lib):
    cfg = pgw.small_config("gpt2", n_layers=2, n_heads=4, n_kv_heads=4, d_model=256, d_ff=1024, max_seq_len=32)
    bundle = pgw.parse_pgw(pgw.make_gpt2(cfg, seed=4, std=0.05, bias_std=0.05))
    ref = oracle_lib.OracleModel(bundle)
    ids = [3, 141, 59, 26, 5]
    want = hf_logits(hf_gpt2(bundle), ids)
    got = ref.forward_prompt(ids)
    assert np.abs(got - want[-1]).max() < 2e-4 * max(1.0, np.abs(want[-1]).max())


def test_gpt2_scale_factors_vs_hf(oracle_lib):
    """SmoothQuant layout (convert_gpt2_to_pgw.py:124-145): lm_head holds W*s,
    ln_f holds gamma/s and beta/s, and embed divides the dequantised row by s
    (infer.js:416-419).  HF with an untied embedding wte = deq(W*s)/s computes
    the same function."""
    from transformers import GPT2Config, GPT2LMHeadModel

    cfg = pgw.small_config("gpt2", n_layers=1, d_model=128, n_heads=2, n_kv_heads=2, d_ff=256, max_seq_len=16)
    s = np.random.default_rng(0).uniform(0.5, 2.0, cfg.d_model).astype(np.float32)
    bundle = pgw.parse_pgw(pgw.make_gpt2(cfg, seed=9, std=0.05, scale_factors=s))
    m = hf_gpt2(bundle)
    D = cfg.d_model
    with torch.no_grad():
        lm = torch.tensor(_deq(bundle, "lm_head"))
        hc = m.config
        hc.tie_word_embeddings = False
        m2 = GPT2LMHeadModel(hc).double().eval()
        m2.load_state_dict({k: v for k, v in m.state_dict().items()}, strict=False)
        emb = (lm.numpy().astype(np.float32) / s[None, :]).astype(np.float64)
        m2.transformer.wte.weight.copy_(torch.tensor(emb))
        m2.lm_head.weight = torch.nn.Parameter(lm.clone())
        lnf = bundle.array("ln_f")
        m2.transformer.ln_f.weight.copy_(torch.tensor(lnf[:D].astype(np.float64)))
        m2.transformer.ln_f.bias.copy_(torch.tensor(lnf[D:].astype(np.float64)))
    ids = [1, 2, 3, 40]
    want = hf_logits(m2, ids)[-1]
    got = oracle_lib.OracleModel(bundle).forward_prompt(ids)
    assert np.abs(got - want).max() < 2e-4 * max(1.0, np.abs(want).max())


@pytest.mark.parametrize("arch", ["llama", "gpt2"])
def test_prefill_decode_and_multi_invariants(oracle_lib, arch):
    cfg = pgw.small_config(arch)
    bundle = pgw.parse_pgw(pgw.make_model(cfg, seed=11))
    m = oracle_lib.OracleModel(bundle)
    ids = [7, 8, 9, 10, 11, 12]
    l6 = m.forward_prompt(ids)
    m.reset_cache()
    m.forward_prompt(ids[:5])
    l5_1 = m.forward_decode(ids[5])
    assert np.array_equal(l6, l5_1)
    # a 3-token multi pass equals three sequential decodes, row by row
    m.reset_cache()
    m.forward_prompt(ids[:3])
    multi = m.forward_multi(ids[3:])
    m.reset_cache()
    m.forward_prompt(ids[:3])
    seq = np.stack([m.forward_decode(t) for t in ids[3:]])
    assert np.array_equal(multi, seq)
    assert m.cache_len == 6


def test_generate_truncation_and_eos(oracle_lib):
    cfg = pgw.small_config("llama", max_seq_len=16)
    m = oracle_lib.OracleModel(pgw.parse_pgw(pgw.make_llama(cfg, seed=2)))
    ids = list(range(20))
    out, stop = m.generate(ids, max_new_tokens=4)
    assert len(out) == 4 and stop == "max_new_tokens"
    # first emitted token as eos stops immediately
    out2, stop2 = m.generate(ids, max_new_tokens=4, eos_id=out[0])
    assert out2 == [out[0]] and stop2 == "eos"


def test_cycle_model_follows_its_cycle(oracle_lib):
    """pgw.make_cycle_llama (the speculation benchmark's model): from any
    token of the cycle, the oracle's greedy decode walks the cycle, with a
    wide top-2 margin; the prompt-lookup drafts along it are full length."""
    from mllm.engine import lookup_draft

    cfg = pgw.small_config("llama", max_seq_len=128)
    rng = np.random.default_rng(3)
    cycle = [int(v) for v in rng.choice(cfg.vocab_size, 9, replace=False)]
    ref = oracle_lib.OracleModel(pgw.parse_pgw(pgw.make_cycle_llama(cfg, cycle, seed=1)))
    prompt = [int(v) for v in rng.integers(0, cfg.vocab_size, 10)] + cycle + cycle[:4]
    lg = ref.forward_prompt(prompt)
    seq, worst = list(prompt), np.inf
    for i in range(20):
        top2 = np.partition(lg, -2)[-2:]
        worst = min(worst, float(top2[1] - top2[0]))
        tok = int(np.argmax(lg))
        assert tok == cycle[(4 + i) % 9], i
        assert lookup_draft(seq, 4, 3) == [cycle[(4 + i + j) % 9] for j in range(4)]
        seq.append(tok)
        lg = ref.forward_decode(tok)
    ref.close()
    assert worst > 1.0, worst


def test_oracle_debug_knobs(oracle_lib):
    """The GPU engine's layer-truncation knobs restated in the oracle
    (webgpu-metal.js:1263-1279).  With no layer run, the logits are the
    closed form lm_head . (rmsnorm(embedding) * norm_f) (infer.js:134-143,
    360-420, 597-600) for every token; dropping both blocks everywhere is no
    layer at all; max_layers = L and mlp_to = L are the full network; and the
    knobs restore it."""
    cfg = pgw.small_config("llama", max_seq_len=64)
    bundle = pgw.parse_pgw(pgw.make_llama(cfg, seed=31))
    ref = oracle_lib.OracleModel(bundle)
    t = bundle.tensors
    def arr(name, dtype, key="offset", nb="nbytes"):
        return np.frombuffer(bundle.buffer, dtype, t[name][nb] // np.dtype(dtype).itemsize,
                             bundle.payload_off + t[name][key])
    lm = oracle_lib.dequant_q4(arr("lm_head", np.uint8).reshape(cfg.vocab_size, -1),
                               arr("lm_head", np.float32, "scaleOffset", "scaleNbytes").reshape(cfg.vocab_size, -1))
    gf = arr("norm_f", np.float32).astype(np.float64)
    ids = [5, 17, 3, 99]
    full = ref.forward_prompt(ids)
    ref.set_debug(max_layers=0)
    for i, tok in enumerate(ids):
        ref.reset_cache()
        got = ref.forward_prompt(ids[:i + 1])
        e = lm[tok].astype(np.float64)
        xn = (e / np.sqrt(np.mean(e * e) + 1e-6) * gf).astype(np.float32).astype(np.float64)
        want = lm.astype(np.float64) @ xn
        assert np.abs(got - want).max() < 1e-4 * np.abs(want).max()
    ref.reset_cache()
    none = ref.forward_prompt(ids)
    ref.set_debug(no_attn=True, no_mlp=True)
    ref.reset_cache()
    assert np.array_equal(ref.forward_prompt(ids), none)
    for kw in ({"max_layers": cfg.n_layers}, {"mlp_to": cfg.n_layers}, {}):
        ref.set_debug(**kw)
        ref.reset_cache()
        assert np.array_equal(ref.forward_prompt(ids), full)
    ref.set_debug(no_mlp=True)
    ref.reset_cache()
    assert not np.array_equal(ref.forward_prompt(ids), full)
    ref.close()
