"""Oracle pinning: GEMV, norms, activations, RoPE, softmax, argmax, draft (CPU).

Each oracle function is checked against an independent computation (numpy
float64 matmul, torch float64 ops, a complex-rotation form of RoPE, brute
force), chosen so a dropped term, wrong sign or swapped index fails.
"""
import numpy as np
import pytest
import torch

from mllm import engine as host
from mllm import pgw


def q4(rng, m, n, std=0.02):
    w = (rng.standard_normal((m, n)) * std).astype(np.float32)
    return pgw.quant_q4(w)


@pytest.mark.parametrize("m,n", [(7, 32), (33, 96), (64, 576), (16, 1536)])
def test_gemv_q4_js_vs_float64_matmul(oracle_lib, rng, m, n):
    p, s = q4(rng, m, n)
    x = rng.standard_normal(n).astype(np.float32)
    W = oracle_lib.dequant_q4(p, s).astype(np.float64)
    ref = W @ x.astype(np.float64)
    y = oracle_lib.gemv_q4(p, s, x, mode="js")
    # fp64 accumulation then one f32 rounding
    assert np.allclose(y, ref.astype(np.float32), rtol=0, atol=np.abs(ref).max() * 1e-6 + 1e-12)
    yw = oracle_lib.gemv_q4(p, s, x, mode="wasm")
    assert np.abs(yw - ref).max() <= 1e-5 * (np.abs(W) @ np.abs(x)).max() + 1e-9


def test_gemv_q8_and_f32_vs_float64(oracle_lib, rng):
    m, n = 24, 160
    w = (rng.standard_normal((m, n)) * 0.02).astype(np.float32)
    x = rng.standard_normal(n).astype(np.float32)
    q, s = pgw.quant_q8row(w)
    ref = (q.astype(np.float64) @ x.astype(np.float64)) * s.astype(np.float64)
    assert np.allclose(oracle_lib.gemv_q8(q, s, x), ref, atol=1e-6)
    assert np.allclose(oracle_lib.gemv_q8(q, s, x, mode="wasm"), ref, atol=1e-4)
    qg, sg = pgw.quant_q8g32(w)
    refg = oracle_lib.dequant_q8g32(qg, sg).astype(np.float64) @ x.astype(np.float64)
    assert np.allclose(oracle_lib.gemv_q8g32(qg, sg, x), refg, atol=1e-6)
    reff = w.astype(np.float64) @ x.astype(np.float64)
    assert np.allclose(oracle_lib.gemv_f32(w, x), reff, atol=1e-6)
    assert np.allclose(oracle_lib.gemv_f32(w, x, mode="wasm"), reff, atol=1e-5)


def test_rms_norm_vs_torch(oracle_lib, rng):
    x = rng.standard_normal((3, 96)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 96).astype(np.float32)
    ref = torch.nn.functional.rms_norm(torch.tensor(x, dtype=torch.float64), (96,),
                                       torch.tensor(w, dtype=torch.float64), eps=1e-6).numpy()
    assert np.allclose(oracle_lib.rms_norm(x, w, 1e-6, "js"), ref, atol=1e-6)
    assert np.allclose(oracle_lib.rms_norm(x, w, 1e-6, "wasm"), ref, atol=1e-5)
    # eps matters: a wrong eps at tiny inputs is visible
    tiny = (x * 1e-4).astype(np.float32)
    ref2 = torch.nn.functional.rms_norm(torch.tensor(tiny, dtype=torch.float64), (96,),
                                        torch.tensor(w, dtype=torch.float64), eps=1e-6).numpy()
    assert np.allclose(oracle_lib.rms_norm(tiny, w, 1e-6), ref2, atol=1e-6)
    assert not np.allclose(oracle_lib.rms_norm(tiny, w, 1e-5), ref2, atol=1e-3)


def test_layer_norm_vs_torch(oracle_lib, rng):
    x = rng.standard_normal((2, 64)).astype(np.float32) + 3.0
    g = rng.uniform(0.5, 1.5, 64).astype(np.float32)
    b = rng.standard_normal(64).astype(np.float32)
    ref = torch.nn.functional.layer_norm(torch.tensor(x, dtype=torch.float64), (64,),
                                         torch.tensor(g, dtype=torch.float64), torch.tensor(b, dtype=torch.float64),
                                         eps=1e-5).numpy()
    assert np.allclose(oracle_lib.layer_norm(x, np.concatenate([g, b])), ref, atol=1e-5)


def test_silu_gelu_softmax_vs_torch(oracle_lib, rng):
    a = (rng.standard_normal(200) * 4).astype(np.float32)
    b = rng.standard_normal(200).astype(np.float32)
    ta, tb = torch.tensor(a, dtype=torch.float64), torch.tensor(b, dtype=torch.float64)
    ref = (torch.nn.functional.silu(ta) * tb).numpy()
    assert np.allclose(oracle_lib.silu_mul(a, b), ref, atol=1e-6)
    assert np.allclose(oracle_lib.silu_mul(a, b, "wasm"), ref, atol=1e-5)
    refg = torch.nn.functional.gelu(ta, approximate="tanh").numpy()
    assert np.allclose(oracle_lib.gelu_new(a), refg, atol=1e-6)
    refs = torch.softmax(ta, 0).numpy()
    assert np.allclose(oracle_lib.softmax(a), refs, atol=1e-7)


def test_rope_vs_complex_rotation(oracle_lib, rng):
    """rotate_half with cat(freqs, freqs) == multiplying (x_d + i x_{d+half}) by e^{i p w_d}."""
    hd, maxs, theta = 64, 40, 1e5
    cos, sin, rd = oracle_lib.build_rope(maxs, hd, theta)
    assert rd == 64
    nh, t, off = 3, 4, 17
    q = rng.standard_normal((nh, t, hd)).astype(np.float32)
    out = oracle_lib.apply_rope(q, nh, t, hd, cos, sin, rd, off).reshape(nh, t, hd)
    half = hd // 2
    inv = (1.0 / theta ** (2 * np.arange(half) / hd)).astype(np.float32).astype(np.float64)
    for ti in range(t):
        ang = (off + ti) * inv
        z = (q[:, ti, :half] + 1j * q[:, ti, half:]).astype(np.complex128) * np.exp(1j * ang)
        assert np.allclose(out[:, ti, :half], z.real, atol=1e-5)
        assert np.allclose(out[:, ti, half:], z.imag, atol=1e-5)
    # partial rotary (ropePct 0.5): dims >= rd pass through
    c2, s2, rd2 = oracle_lib.build_rope(maxs, hd, theta, 0.5)
    assert rd2 == 32
    out2 = oracle_lib.apply_rope(q, nh, t, hd, c2, s2, rd2, off).reshape(nh, t, hd)
    assert np.array_equal(out2[..., 32:], q[..., 32:])


def test_argmax_first_maximum(oracle_lib):
    v = np.array([0.1, 0.7, 0.7, -1, 0.7], np.float32)
    assert oracle_lib.argmax(v) == 1
    assert host.argmax(v) == 1


def brute_argmax_gpt2(logits, hist):
    """Literal statement of the rule, candidate by candidate."""
    n = len(hist)
    best, bi = -np.inf, 0
    for i in range(len(logits)):
        v = float(logits[i])
        if n >= 2 and any(hist[h] == hist[n - 2] and hist[h + 1] == hist[n - 1] and hist[h + 2] == i
                          for h in range(n - 2)):
            v = -1e9
        if v > -1e8 and i in hist[max(0, n - 32):]:
            v = v / 1.15 if v > 0 else v * 1.15
        if v > best:
            best, bi = v, i
    return bi


def test_argmax_gpt2_brute_force(oracle_lib, rng):
    for trial in range(40):
        V = 12
        logits = (rng.standard_normal(V) * 0.5).astype(np.float32)
        hist = [int(v) for v in rng.integers(0, V, rng.integers(0, 40))]
        want = brute_argmax_gpt2(logits, hist)
        assert oracle_lib.argmax_gpt2(logits, hist) == want
        assert host.argmax_gpt2(logits, hist) == want
    # the 3-gram block removes an otherwise winning token
    logits = np.zeros(6, np.float32)
    logits[5] = 1.0
    hist = [1, 2, 5, 3, 1, 2]
    assert oracle_lib.argmax_gpt2(logits, hist) != 5
    # the penalty on a recent token flips a close race
    logits = np.array([0, 1.0, 0.95, 0, 0, 0], np.float32)
    assert oracle_lib.argmax_gpt2(logits, [1]) == 2


@pytest.mark.parametrize("seq,k,n,want", [
    ([1, 2, 3], 4, 3, []),                                  # too short
    ([1, 2, 3, 9, 9, 1, 2, 3], 4, 3, [9, 9, 1, 2]),          # match at the start
    ([5, 1, 2, 3, 7, 1, 2, 3, 8, 1, 2, 3], 2, 3, [8, 1]),    # most recent earlier match wins
    ([1, 1, 1, 1], 4, 3, [1]),                              # overlapping suffix, truncated at the end
    ([4, 5, 6, 7, 8], 3, 3, []),                            # no match
    ([2, 3, 4, 2, 3, 4, 2, 3, 4], 8, 3, [2, 3, 4]),          # draft truncated by the sequence end
])
def test_lookup_draft_cases(oracle_lib, seq, k, n, want):
    assert oracle_lib.lookup_draft(seq, k, n) == want
    assert host.lookup_draft(seq, k, n) == want


def test_lookup_draft_random_agrees(oracle_lib, rng):
    for _ in range(200):
        seq = [int(v) for v in rng.integers(0, 4, rng.integers(0, 30))]
        k = int(rng.integers(1, 9))
        assert oracle_lib.lookup_draft(seq, k, 3) == host.lookup_draft(seq, k, 3)
