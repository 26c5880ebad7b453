"""GPU parity of the operator-level C ABI against the oracle.

Bars: dequant bit-exact; GEMV rows within a float32 accumulation bound of the
fp64 oracle (|err| <= 2e-6 * sum|w||x| + 1e-7, written per row); the t-token
GEMM and the batched GEMV bit-identical to the single GEMV.
"""
import ctypes as C

import numpy as np
import pytest

from mllm import abi, pgw

torch = pytest.importorskip("torch")
gpu = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def ptr(t):
    return C.c_void_p(t.data_ptr())


def row_bound(W, x):
    return 2e-6 * (np.abs(W.astype(np.float64)) @ np.abs(x.astype(np.float64))) + 1e-7


def within(y, ref, bound):
    """Every row within its bound; otherwise the failing rows' values."""
    bad = np.nonzero(~(np.abs(y - ref) <= bound))[0]
    return bad.size == 0, [(int(i), float(y[i]), float(ref[i]), float(bound[i])) for i in bad[:8]], int(bad.size)


SHAPES = [(7, 32), (33, 64), (576, 576), (960, 576), (3072, 576), (576, 1536), (960, 960), (320, 960),
          (2560, 960), (960, 2560), (2304, 768), (768, 3072), (49152, 960), (50257, 768), (64, 8192), (3, 16384)]


@gpu
@pytest.mark.parametrize("m,n", SHAPES)
def test_gemv_q4_vs_oracle(oracle_lib, m, n):
    rng = np.random.default_rng(m * 7 + n)
    w = (rng.standard_normal((m, n)) * 0.02).astype(np.float32)
    packed, sc = pgw.quant_q4(w)
    x = rng.standard_normal(n).astype(np.float32)
    dp, ds, dx = dev(packed), dev(sc), dev(x)
    dy = torch.empty(m, dtype=torch.float32, device="cuda")
    print(f"gemv_q4 m={m} n={n}", flush=True)
    abi.call("mllm_gemv_q4", m, n, ptr(dp), ptr(ds), 32, ptr(dx), ptr(dy), None)
    y = host(dy)
    ref = oracle_lib.gemv_q4(packed, sc, x, mode="js")
    W = oracle_lib.dequant_q4(packed, sc)
    ok, rows, nbad = within(y, ref, row_bound(W, x))
    assert ok, (nbad, rows)


@gpu
def test_gemm_q4_rows_bit_identical_to_gemv():
    rng = np.random.default_rng(5)
    m, n, t = 1000, 960, 9
    packed, sc = pgw.quant_q4((rng.standard_normal((m, n)) * 0.02).astype(np.float32))
    x = rng.standard_normal((t, n)).astype(np.float32)
    dp, ds, dx = dev(packed), dev(sc), dev(x)
    dy = torch.empty((t, m), dtype=torch.float32, device="cuda")
    abi.call("mllm_gemm_q4", t, m, n, ptr(dp), ptr(ds), 32, ptr(dx), ptr(dy), None)
    y = host(dy)
    for i in range(t):
        d1 = torch.empty(m, dtype=torch.float32, device="cuda")
        abi.call("mllm_gemv_q4", m, n, ptr(dp), ptr(ds), 32, ptr(dx[i]), ptr(d1), None)
        assert np.array_equal(host(d1).view(np.uint32), y[i].view(np.uint32))


@gpu
def test_gemv_q4_batched_matches_single():
    rng = np.random.default_rng(6)
    count, m, n = 5, 320, 960
    mats = [pgw.quant_q4((rng.standard_normal((m, n)) * 0.02).astype(np.float32)) for _ in range(count)]
    xs = [dev(rng.standard_normal(n).astype(np.float32)) for _ in range(count)]
    dps = [dev(p) for p, _ in mats]
    dss = [dev(s) for _, s in mats]
    ys = [torch.empty(m, dtype=torch.float32, device="cuda") for _ in range(count)]
    table = lambda ts: dev(np.array([t.data_ptr() for t in ts], np.uint64))  # noqa: E731
    tp, ts_, tx, ty = table(dps), table(dss), table(xs), table(ys)
    abi.call("mllm_gemv_q4_batched", count, m, n, ptr(tp), ptr(ts_), ptr(tx), ptr(ty), None)
    torch.cuda.synchronize()
    for i in range(count):
        d1 = torch.empty(m, dtype=torch.float32, device="cuda")
        abi.call("mllm_gemv_q4", m, n, ptr(dps[i]), ptr(dss[i]), 32, ptr(xs[i]), ptr(d1), None)
        assert np.array_equal(host(d1), host(ys[i]))


@gpu
@pytest.mark.parametrize("m,n", [(320, 960), (960, 2560)])
def test_gemv_q8_g32_batched_matches_single(m, n):
    """A stacked launch of Q8 group-32 GEMVs (config 2's Q8 variant): every
    matrix's rows carry the bits of a single mllm_gemv_q8_g32 call."""
    rng = np.random.default_rng(9)
    count = 6
    mats = [pgw.quant_q8g32((rng.standard_normal((m, n)) * 0.02).astype(np.float32)) for _ in range(count)]
    xs = [dev(rng.standard_normal(n).astype(np.float32)) for _ in range(count)]
    dqs = [dev(q) for q, _ in mats]
    dss = [dev(s) for _, s in mats]
    ys = [torch.empty(m, dtype=torch.float32, device="cuda") for _ in range(count)]
    table = lambda ts: dev(np.array([t.data_ptr() for t in ts], np.uint64))  # noqa: E731
    tq, ts_, tx, ty = table(dqs), table(dss), table(xs), table(ys)
    abi.call("mllm_gemv_q8_g32_batched", count, m, n, ptr(tq), ptr(ts_), ptr(tx), ptr(ty), None)
    torch.cuda.synchronize()
    for i in range(count):
        d1 = torch.empty(m, dtype=torch.float32, device="cuda")
        abi.call("mllm_gemv_q8_g32", m, n, ptr(dqs[i]), ptr(dss[i]), ptr(xs[i]), ptr(d1), None)
        assert np.array_equal(host(d1).view(np.uint32), host(ys[i]).view(np.uint32)), i


@gpu
@pytest.mark.parametrize("n", [2048, 2560, 4096, 8192])
def test_gemv_q4_rows_do_not_depend_on_the_workgroup_width(n):
    """960 x n alone (64 to 256 groups per row) and 32 of them stacked launch
    different tile plans (workgroup width, passes per tile).  Every row must
    carry the same bits: its summation order depends only on the row length."""
    rng = np.random.default_rng(8)
    count, m = 32, 960
    packed, sc = pgw.quant_q4((rng.standard_normal((m, n)) * 0.02).astype(np.float32))
    dp, ds = dev(packed), dev(sc)
    xs = [dev(rng.standard_normal(n).astype(np.float32)) for _ in range(count)]
    ys = [torch.empty(m, dtype=torch.float32, device="cuda") for _ in range(count)]
    table = lambda ts: dev(np.array([t.data_ptr() for t in ts], np.uint64))  # noqa: E731
    tp, ts_, tx, ty = table([dp] * count), table([ds] * count), table(xs), table(ys)
    abi.call("mllm_gemv_q4_batched", count, m, n, ptr(tp), ptr(ts_), ptr(tx), ptr(ty), None)
    torch.cuda.synchronize()
    for i in range(count):
        d1 = torch.empty(m, dtype=torch.float32, device="cuda")
        abi.call("mllm_gemv_q4", m, n, ptr(dp), ptr(ds), 32, ptr(xs[i]), ptr(d1), None)
        assert np.array_equal(host(d1).view(np.uint32), host(ys[i]).view(np.uint32)), i


@gpu
@pytest.mark.parametrize("m,n", [(96, 64), (960, 960), (320, 960), (2560, 960), (960, 2560), (49152, 960)])
def test_gemv_q8_row_and_g32_vs_oracle(oracle_lib, m, n):
    rng = np.random.default_rng(m + n)
    w = (rng.standard_normal((m, n)) * 0.02).astype(np.float32)
    x = rng.standard_normal(n).astype(np.float32)
    dx = dev(x)
    q, s = pgw.quant_q8row(w)
    dq, ds = dev(q), dev(s)  # keep the device buffers alive until the kernel has run
    dy = torch.empty(m, dtype=torch.float32, device="cuda")
    abi.call("mllm_gemv_q8", m, n, ptr(dq), ptr(ds), ptr(dx), ptr(dy), None)
    ref = oracle_lib.gemv_q8(q, s, x)
    W = oracle_lib.dequant_q8row(q, s)
    ok, rows, nbad = within(host(dy), ref, row_bound(W, x))
    assert ok, ("q8 per-row", nbad, rows)
    qg, sg = pgw.quant_q8g32(w)
    dqg, dsg = dev(qg), dev(sg)
    abi.call("mllm_gemv_q8_g32", m, n, ptr(dqg), ptr(dsg), ptr(dx), ptr(dy), None)
    refg = oracle_lib.gemv_q8g32(qg, sg, x)
    Wg = oracle_lib.dequant_q8g32(qg, sg)
    ok, rows, nbad = within(host(dy), refg, row_bound(Wg, x))
    assert ok, ("q8 g32", nbad, rows)


@gpu
@pytest.mark.parametrize("m,n", [(5, 7), (64, 576), (300, 1000)])
def test_gemv_f32_vs_oracle(oracle_lib, m, n):
    rng = np.random.default_rng(n)
    w = rng.standard_normal((m, n)).astype(np.float32)
    x = rng.standard_normal(n).astype(np.float32)
    dy = torch.empty(m, dtype=torch.float32, device="cuda")
    dw, dx = dev(w), dev(x)
    abi.call("mllm_gemv_f32", m, n, ptr(dw), ptr(dx), ptr(dy), None)
    assert (np.abs(host(dy) - oracle_lib.gemv_f32(w, x)) <= row_bound(w, x)).all()


@gpu
def test_rms_norm_and_silu_mul_vs_oracle(oracle_lib):
    rng = np.random.default_rng(8)
    x = rng.standard_normal((3, 576)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 576).astype(np.float32)
    out = torch.empty((3, 576), dtype=torch.float32, device="cuda")
    dx, dw = dev(x), dev(w)
    abi.call("mllm_rms_norm", 576, ptr(dx), ptr(dw), ptr(out), 3, C.c_float(1e-6), None)
    assert np.allclose(host(out), oracle_lib.rms_norm(x, w, 1e-6, "js"), rtol=2e-6, atol=2e-6)
    a = (rng.standard_normal(1536) * 3).astype(np.float32)
    b = rng.standard_normal(1536).astype(np.float32)
    da, db = dev(a), dev(b)
    abi.call("mllm_silu_mul", 1536, ptr(da), ptr(db), None)
    assert np.allclose(host(da), oracle_lib.silu_mul(a, b, "js"), rtol=4e-6, atol=1e-7)


@gpu
def test_dequant_q4_bit_exact(oracle_lib):
    rng = np.random.default_rng(9)
    m, n = 70, 576
    packed = rng.integers(0, 256, (m, n // 2), dtype=np.uint8)
    sc = (rng.standard_normal((m, n // 32)) * 0.01).astype(np.float32)
    sc[0, :] = [0.0, 1.4e-45, 3e38, -1.0] * 4 + [1e-38, 7.0]
    out = torch.empty((m, n), dtype=torch.float32, device="cuda")
    dp, ds = dev(packed), dev(sc)
    abi.call("mllm_dequant_q4", m, n, ptr(dp), ptr(ds), 32, ptr(out), None)
    assert np.array_equal(host(out).view(np.uint32), oracle_lib.dequant_q4(packed, sc).view(np.uint32))


@gpu
def test_gemv_q4_linearity_full_lm_head():
    """Size-independent property at the 360M lm_head shape: W(a+b) = Wa + Wb
    within float32 rounding."""
    rng = np.random.default_rng(10)
    m, n = 49152, 960
    packed, sc = pgw.quant_q4((rng.standard_normal((m, n)) * 0.02).astype(np.float32))
    dp, ds = dev(packed), dev(sc)
    a = rng.standard_normal(n).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    outs = []
    for v in (a, b, (a + b).astype(np.float32)):
        dy = torch.empty(m, dtype=torch.float32, device="cuda")
        dv = dev(v)
        abi.call("mllm_gemv_q4", m, n, ptr(dp), ptr(ds), 32, ptr(dv), ptr(dy), None)
        torch.cuda.synchronize()
        outs.append(host(dy))
    assert np.abs(outs[2] - (outs[0] + outs[1])).max() < 1e-4


@gpu
def test_gpu_abi_against_the_oracle_abi_on_the_same_arguments(oracle_lib):
    """Each operator of include/mllm.h and its host-pointer counterpart in the
    oracle (oracle/mllm_cpu.h, kernels.rs semantics) on one argument list:
    dequant bit-exact, the rest within the row bound."""
    lib = C.CDLL(oracle_lib.build())
    rng = np.random.default_rng(42)
    m, n, t = 300, 960, 3
    w = (rng.standard_normal((m, n)) * 0.02).astype(np.float32)
    packed, sc = pgw.quant_q4(w)
    W = oracle_lib.dequant_q4(packed, sc)
    x = rng.standard_normal((t, n)).astype(np.float32)
    hp = lambda a: C.c_void_p(a.ctypes.data)  # noqa: E731
    print("cpu abi: gemv_q4 / gemm_q4 / dequant_q4", flush=True)
    y_cpu = np.zeros((t, m), np.float32)
    assert lib.mllm_cpu_gemm_q4(t, m, n, hp(packed), hp(sc), 32, hp(x), hp(y_cpu), None) == 0
    # device copies held for the whole test: a temporary's memory may be
    # reused by the next allocation before the kernel runs
    dp, ds, dx = dev(packed), dev(sc), dev(x)
    dy = torch.empty((t, m), dtype=torch.float32, device="cuda")
    abi.call("mllm_gemm_q4", t, m, n, ptr(dp), ptr(ds), 32, ptr(dx), ptr(dy), None)
    for i in range(t):
        assert (np.abs(host(dy)[i] - y_cpu[i]) <= 2 * row_bound(W, x[i])).all()
    y1 = np.zeros(m, np.float32)
    assert lib.mllm_cpu_gemv_q4(m, n, hp(packed), hp(sc), 32, hp(x[0]), hp(y1), None) == 0
    assert np.array_equal(y1, y_cpu[0])
    d_cpu = np.zeros((m, n), np.float32)
    assert lib.mllm_cpu_dequant_q4(m, n, hp(packed), hp(sc), 32, hp(d_cpu), None) == 0
    dd = torch.empty((m, n), dtype=torch.float32, device="cuda")
    abi.call("mllm_dequant_q4", m, n, ptr(dp), ptr(ds), 32, ptr(dd), None)
    assert np.array_equal(host(dd).view(np.uint32), d_cpu.view(np.uint32))
    print("cpu abi: rms_norm / silu_mul / gemv_f32", flush=True)
    g = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    o_cpu = np.zeros((t, n), np.float32)
    assert lib.mllm_cpu_rms_norm(n, hp(x), hp(g), hp(o_cpu), t, C.c_float(1e-6), None) == 0
    dg = dev(g)
    do = torch.empty((t, n), dtype=torch.float32, device="cuda")
    abi.call("mllm_rms_norm", n, ptr(dx), ptr(dg), ptr(do), t, C.c_float(1e-6), None)
    assert np.abs(host(do) - o_cpu).max() <= 1e-5 * np.abs(o_cpu).max()
    a = rng.standard_normal(n).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    a_cpu = a.copy()
    assert lib.mllm_cpu_silu_mul(n, hp(a_cpu), hp(b), None) == 0
    da, db = dev(a), dev(b)
    abi.call("mllm_silu_mul", n, ptr(da), ptr(db), None)
    assert np.abs(host(da) - a_cpu).max() <= 1e-5 * np.abs(a_cpu).max() + 1e-6
    f_cpu = np.zeros(m, np.float32)
    assert lib.mllm_cpu_gemv_f32(m, n, hp(w), hp(x[0]), hp(f_cpu), None) == 0
    dw, dx0 = dev(w), dev(x[0])
    df = torch.empty(m, dtype=torch.float32, device="cuda")
    abi.call("mllm_gemv_f32", m, n, ptr(dw), ptr(dx0), ptr(df), None)
    assert (np.abs(host(df) - f_cpu) <= 2 * row_bound(w, x[0])).all()


def host_argmax(y):
    """infer.js:240-250: best = 0, bestV = y[0]; a later row wins only when
    strictly larger (so NaN rows never win and a NaN y[0] keeps 0)."""
    best, bv = 0, y[0]
    for i in range(1, y.size):
        if y[i] > bv:
            best, bv = i, y[i]
    return best


def argmax_case(rng, m, n, kind):
    w = (rng.standard_normal((m, n)) * 0.02).astype(np.float32)
    x = rng.standard_normal(n).astype(np.float32)
    if kind == "tie":  # three equal maximal rows: the first one wins
        w[[m // 3, m // 2, m - 1]] = w[m // 2] * 3
    packed, sc = pgw.quant_q4(w)
    if kind == "nan0":  # row 0 NaN keeps index 0
        sc[0, 0] = np.nan
    if kind == "nan_rows":  # NaN rows elsewhere never win
        sc[1:m:7, 0] = np.nan
    if kind == "all_nan":
        x[:] = np.nan
    if kind == "last":  # the maximum in the last row (the last tile)
        w[-1] = np.abs(w[-1]) * np.sign(x) * 4
        packed, sc = pgw.quant_q4(w)
    return packed, sc, x


@gpu
@pytest.mark.parametrize("m,n,kind", [(49152, 960, "rand"), (49152, 576, "tie"), (50257, 768, "last"),
                                      (2000, 960, "nan0"), (2000, 960, "nan_rows"), (300, 64, "all_nan"),
                                      (7, 32, "rand")])
def test_gemv_q4_argmax(m, n, kind):
    """y bit-identical to mllm_gemv_q4, and the index equal to the reference
    argmax rule over y (first maximum, NaN rules of infer.js:240-250)."""
    rng = np.random.default_rng(m + n)
    packed, sc, x = argmax_case(rng, m, n, kind)
    dp, ds, dx = dev(packed), dev(sc), dev(x)
    dy = torch.empty(m, dtype=torch.float32, device="cuda")
    dy1 = torch.empty(m, dtype=torch.float32, device="cuda")
    di = torch.full((1,), -5, dtype=torch.int32, device="cuda")
    print(f"gemv_q4_argmax m={m} n={n} {kind}", flush=True)
    abi.call("mllm_gemv_q4_argmax", m, n, ptr(dp), ptr(ds), 32, ptr(dx), ptr(dy), ptr(di), None)
    abi.call("mllm_gemv_q4", m, n, ptr(dp), ptr(ds), 32, ptr(dx), ptr(dy1), None)
    y = host(dy)
    assert np.array_equal(y.view(np.uint32), host(dy1).view(np.uint32))
    assert int(host(di)[0]) == host_argmax(y)
