"""Oracle pinning: quantiser and dequantiser (CPU).

quant_q4 is pinned against golden vectors written by the reference's own
quant_q4 (tools/convert_hf_to_pgw.py:18-34) via tests/golden/make_quant_q4_vectors.py;
the dequantiser is pinned by the error bound and exact requantisation, which a
swapped nibble order or a wrong offset would break.
"""
import os

import numpy as np
import pytest

from mllm import pgw

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "quant_q4_vectors.npz")


def golden_cases():
    z = np.load(GOLDEN)
    names = sorted({k.split("__")[0] for k in z.files})
    return [(n, z[n + "__x"], z[n + "__packed"], z[n + "__scales"]) for n in names]


@pytest.mark.parametrize("case", golden_cases(), ids=lambda c: c[0])
def test_quant_q4_matches_reference_golden(oracle_lib, case):
    name, x, packed, scales = case
    p, s = oracle_lib.quant_q4(x)
    assert np.array_equal(p, packed), name
    assert np.array_equal(s.view(np.uint32), scales.view(np.uint32)), name
    p2, s2 = pgw.quant_q4(x)  # the vectorised writer used for synthetic models
    assert np.array_equal(p2, packed), name
    assert np.array_equal(s2.view(np.uint32), scales.view(np.uint32)), name


def test_near_tie_case_discriminates_division_precision():
    """The golden near-tie row is one where a float64 division would pick a
    different nibble than the reference's float32 division."""
    z = np.load(GOLDEN)
    x, packed, sc = z["near_ties__x"], z["near_ties__packed"], z["near_ties__scales"]
    q = np.empty(x.shape, np.uint8)
    q[:, 0::2] = packed & 15
    q[:, 1::2] = packed >> 4
    q64 = np.clip(np.rint(x.astype(np.float64) / np.repeat(sc.astype(np.float64), 32, axis=1)) + 8, 0, 15)
    assert (q64.astype(np.uint8) != q).any()


def test_quant_q4_special_cases(oracle_lib):
    x = np.zeros((1, 32), np.float32)
    p, s = oracle_lib.quant_q4(x)
    assert s[0, 0] == 1.0 and (p == 0x88).all()  # amax 0 -> sc 1, every q = 8
    x[0, 0], x[0, 1] = 3.0, -3.0
    p, s = oracle_lib.quant_q4(x)
    assert s[0, 0] == np.float32(3.0 / 8)
    assert p[0, 0] & 15 == 15  # +amax -> 16 clipped to 15
    assert p[0, 0] >> 4 == 0  # -amax -> 0
    # ties to even: amax 8 -> sc 1; 0.5 -> 0 (+8 = 8), 1.5 -> 2 (10), -0.5 -> -0 (8), 2.5 -> 2 (10)
    x = np.zeros((1, 32), np.float32)
    x[0, :5] = [8.0, 0.5, 1.5, -0.5, 2.5]
    p, _ = oracle_lib.quant_q4(x)
    q = [p[0, 0] & 15, p[0, 0] >> 4, p[0, 1] & 15, p[0, 1] >> 4, p[0, 2] & 15]
    assert q == [15, 8, 10, 8, 10]


def test_quant_q4_brute_force_small(oracle_lib, rng):
    """Every element's nibble is the nearest representable level (brute force over 0..15)."""
    x = (rng.standard_normal((8, 64)) * 0.05).astype(np.float32)
    p, s = oracle_lib.quant_q4(x)
    deq = oracle_lib.dequant_q4(p, s)
    for r in range(8):
        for c in range(64):
            sc = s[r, c // 32]
            levels = (np.arange(16) - 8) * np.float64(sc)
            err = np.abs(levels - x[r, c])
            best = err.min()
            assert abs(deq[r, c] - x[r, c]) <= best + 1e-12 + sc * 1e-6


def test_dequant_error_bound_and_requant(oracle_lib, rng):
    x = (rng.standard_normal((16, 96)) * 0.02).astype(np.float32)
    p, s = oracle_lib.quant_q4(x)
    d = oracle_lib.dequant_q4(p, s)
    bound = np.repeat(s, 32, axis=1) * 0.5000001
    inside = x < np.repeat(s * 7.5, 32, axis=1)  # above 7.5*sc the +8 level clips to +7
    assert (np.abs(d - x)[inside] <= bound[inside]).all()
    # the dequantised matrix requantises to the same nibbles where its amax is unchanged
    p2, s2 = oracle_lib.quant_q4(d)
    same = np.repeat(s2 == s, 16, axis=1)
    assert np.array_equal(p2[same], p[same])
    # vectorised dequant agrees bit for bit
    assert np.array_equal(pgw.dequant_q4(p, s).view(np.uint32), d.view(np.uint32))


def test_dequant_exhaustive_bytes(oracle_lib):
    """All 256 byte values x scale edge cases (1, 0, the smallest subnormal, a
    large finite value): element 2k = low nibble, 2k+1 = high nibble, each
    (nib - 8) * sc rounded once to float32."""
    packed = np.tile(np.arange(256, dtype=np.uint8), (4, 1))
    scales = np.array([[1.0] * 16, [0.0] * 16, [1.4e-45] * 16, [3.0e38] * 16], np.float32)
    d = oracle_lib.dequant_q4(packed, scales)
    b = np.arange(256)
    lo = ((b & 15) - 8).astype(np.float64)
    hi = ((b >> 4) - 8).astype(np.float64)
    with np.errstate(over="ignore"):
        for r in range(4):
            s = np.float64(scales[r, 0])
            want = np.empty(512, np.float32)
            want[0::2] = (lo * s).astype(np.float32)
            want[1::2] = (hi * s).astype(np.float32)
            assert np.array_equal(d[r].view(np.uint32), want.view(np.uint32)), r
    # the closed form at the ends: byte 0x80 -> (-8, 0), byte 0x7F -> (7, -1)
    assert d[0, 2 * 0x80] == -8.0 and d[0, 2 * 0x80 + 1] == 0.0
    assert d[0, 2 * 0x7F] == 7.0 and d[0, 2 * 0x7F + 1] == -1.0
    assert np.isinf(d[3, 0]) and d[3, 0] < 0  # -8 * 3e38 overflows float32


def _q8_brute(x, sc):
    """The nearest of the 255 levels q * sc (q in [-127, 127]) to each x, ties
    to the even q; levels and distances in float64."""
    q = np.arange(-127, 128, dtype=np.float64)
    lv = q * np.float64(sc)
    out = np.empty(x.size, np.int64)
    for i, v in enumerate(x.astype(np.float64)):
        err = np.abs(lv - v)
        best = np.flatnonzero(err == err.min())
        if best.size > 1:  # an exact tie between two levels: the even one
            best = best[(q[best] % 2) == 0]
        out[i] = int(q[best[0]])
    return out


def test_quant_q8_rules(oracle_lib, rng):
    """Build-defined Q8 (the reference ships no Q8 quantiser): the scale is
    float32(amax / 127) exactly (amax = max |x| of the span; 1 when amax is 0),
    the element of largest magnitude maps to +-127, and every other element
    to the nearest level (brute force over all 255 levels).  A scale of
    amax / 126 or amax / 128, a truncating rounding or a clip at 128 fails
    one of these."""
    x = (rng.standard_normal((4, 64)) * 0.02).astype(np.float32)
    x[1, 5] = -np.abs(x[1]).max() * 1.5  # a negative maximum magnitude
    x[2, :32] = 0.0  # an all-zero group
    for quant, span in ((oracle_lib.quant_q8g32, 32), (oracle_lib.quant_q8row, 64)):
        q, s = quant(x)
        s = s.reshape(4, -1)
        for r in range(4):
            for g in range(64 // span):
                xs = x[r, g * span:(g + 1) * span]
                qs = q[r, g * span:(g + 1) * span].astype(np.int64)
                amax = np.abs(xs).max()
                if amax == 0:
                    assert s[r, g] == 1.0 and (qs == 0).all()
                    continue
                assert s[r, g] == np.float32(np.float64(amax) / 127.0)
                assert s[r, g] != np.float32(np.float64(amax) / 126.0)
                k = int(np.argmax(np.abs(xs)))
                assert qs[k] == (127 if xs[k] > 0 else -127)
                # the division x / sc is float32 as in rintf(x / sc); brute
                # force over levels agrees except where that float32 quotient
                # lands on the other side of a half level (none in this data)
                assert np.array_equal(qs, _q8_brute(xs, s[r, g]))
    q, s = oracle_lib.quant_q8g32(x)
    q2, s2 = pgw.quant_q8g32(x)
    assert np.array_equal(q, q2) and np.array_equal(s, s2)
    qr, sr = oracle_lib.quant_q8row(x)
    qr2, sr2 = pgw.quant_q8row(x)
    assert np.array_equal(qr, qr2) and np.array_equal(sr, sr2)
    d = oracle_lib.dequant_q8g32(q, s)
    assert (np.abs(d - x) <= np.repeat(s, 32, axis=1) * 0.5000001).all()
    dr = oracle_lib.dequant_q8row(qr, sr)
    assert (np.abs(dr - x) <= sr[:, None] * 0.5000001).all()


def test_quant_q8_ties_to_even(oracle_lib):
    """amax 127 gives sc = 1, so x = k + 0.5 is an exact tie: rint rounds to
    the even neighbour (0.5 -> 0, 1.5 -> 2, -2.5 -> -2), and 127 -> 127."""
    x = np.zeros((1, 32), np.float32)
    x[0, :6] = [127.0, 0.5, 1.5, -2.5, 3.5, -0.5]
    q, s = oracle_lib.quant_q8g32(x)
    assert s[0, 0] == 1.0
    assert list(q[0, :6]) == [127, 0, 2, -2, 4, 0]


def test_bf16_bits_round_to_nearest_even():
    """pgw.f32_to_bf16_bits against torch's float32 -> bfloat16 conversion
    (round to nearest even), including exact halfway cases and infinities."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(7)
    x = rng.standard_normal(4096).astype(np.float32) * np.float32(3.0)
    # exact halfway patterns: low 16 bits 0x8000 with even and odd bf16 lsb
    u = np.array([0x3F808000, 0x3F818000, 0xBF808000, 0xBF818000, 0x7F7F8000], np.uint32)
    x = np.concatenate([x, u.view(np.float32), np.array([np.inf, -np.inf, 0.0, -0.0], np.float32)])
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(pgw.f32_to_bf16_bits(x), want)


@pytest.mark.parametrize("storage", ["q4", "q8", "q8g32", "f16", "bf16", "f32"])
def test_add_matrix_round_trip(storage):
    """A matrix written by PgwWriter.add_matrix reads back (Bundle.array /
    scales, weights.js:42-67) as its quantiser's output, each blob 16-byte
    aligned; q4 at group 32 is add_q4's layout byte for byte."""
    rng = np.random.default_rng(11)
    m = rng.standard_normal((48, 128)).astype(np.float32)
    w = pgw.PgwWriter()
    w.add_f32("pad", np.ones(3, np.float32))  # misaligns the blob on purpose
    w.add_matrix("m", m, storage, group=64 if storage == "q4" else 32)
    cfg = pgw.small_config("llama")
    b = pgw.parse_pgw(w.finish(cfg, kind=storage if storage != "q8g32" else "q8"))
    t = b.tensors["m"]
    assert t["storage"] == storage and t["offset"] % 16 == 0
    a = b.array("m")
    if storage == "q4":
        p, s = pgw.quant_q4(m, 64)
        assert t["group"] == 64 and np.array_equal(a, p) and np.array_equal(b.scales("m"), s)
    elif storage == "q8":
        q, s = pgw.quant_q8row(m)
        assert np.array_equal(a, q) and np.array_equal(b.scales("m").ravel(), s)
    elif storage == "q8g32":
        q, s = pgw.quant_q8g32(m)
        assert np.array_equal(a, q) and np.array_equal(b.scales("m"), s)
    elif storage == "f16":
        assert np.array_equal(a.view(np.float16), m.astype(np.float16))
    elif storage == "bf16":
        assert np.array_equal(a, pgw.f32_to_bf16_bits(m))
    else:
        assert np.array_equal(a, m)
    # group-32 q4 through add_matrix is add_q4 byte for byte
    w1, w2 = pgw.PgwWriter(), pgw.PgwWriter()
    w1.add_matrix("m", m, "q4")
    w2.add_q4("m", m)
    assert w1.finish(cfg) == w2.finish(cfg)
