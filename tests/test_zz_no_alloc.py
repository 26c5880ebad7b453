"""The no-allocation variant of the GEMV + argmax entry point
(mllm_gemv_q4_argmax_noalloc): its scratch is a fixed device array, not
memory the library allocates.  Through the C ABI its logits and index must
equal mllm_gemv_q4_argmax's -- bit for bit, the same kernel -- on two calls
in a row, the second with a smaller input (the array keeps the first call's
contents), and a shape beyond the array's capacity is refused before
anything runs."""
import ctypes as C

import numpy as np
import pytest

from mllm import abi, pgw

torch = pytest.importorskip("torch")
gpu = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def ptr(t):
    return C.c_void_p(t.data_ptr())


def run(fn, packed, sc, x, m, n):
    dp, ds, dx = dev(packed), dev(sc), dev(x)
    dy = torch.empty(m, dtype=torch.float32, device="cuda")
    di = torch.full((1,), -5, dtype=torch.int32, device="cuda")
    abi.call(fn, m, n, ptr(dp), ptr(ds), 32, ptr(dx), ptr(dy), ptr(di), None)
    torch.cuda.synchronize()
    return dy.cpu().numpy(), int(di.cpu().numpy()[0])


@gpu
def test_noalloc_equals_allocating_variant_twice_second_smaller():
    rng = np.random.default_rng(77)
    for m, n in ((49152, 960), (3000, 576)):
        w = (rng.standard_normal((m, n)) * 0.02).astype(np.float32)
        packed, sc = pgw.quant_q4(w)
        x = rng.standard_normal(n).astype(np.float32)
        print(f"noalloc m={m} n={n}", flush=True)
        y0, i0 = run("mllm_gemv_q4_argmax_noalloc", packed, sc, x, m, n)
        y1, i1 = run("mllm_gemv_q4_argmax", packed, sc, x, m, n)
        assert np.array_equal(y0.view(np.uint32), y1.view(np.uint32))
        assert i0 == i1 == int(np.argmax(y1))


def test_noalloc_refuses_shapes_beyond_its_scratch():
    """1,048,128 rows of 960 columns need 16377 tiles of 64 rows, one more
    than the fixed array holds: refused with MLLM_ERR_UNSUPPORTED before any
    device work (the pointers are never read)."""
    buf = (C.c_uint8 * 64)()
    a = C.addressof(buf) + (-C.addressof(buf) % 16)
    rc = abi.lib().mllm_gemv_q4_argmax_noalloc(1048128, 960, C.c_void_p(a), C.c_void_p(a), 32, C.c_void_p(a),
                                               C.c_void_p(a), C.c_void_p(a), None)
    assert rc == 4
    assert b"no-allocation scratch" in abi.lib().mllm_last_error()
