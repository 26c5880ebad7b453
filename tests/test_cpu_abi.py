"""The oracle's host-pointer operator entry points (oracle/mllm_cpu.h, test
infrastructure): the operator names of include/mllm.h with identical
signatures, and the same argument checks -- every bad argument list gets the
same return code from the GPU library (which checks before touching the GPU)
and from the oracle."""
import ctypes as C
import os
import re

import pytest

from mllm import abi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
OPS = ["gemv_f32", "gemv_q8", "gemv_q4", "gemv_q8_g32", "gemm_q4", "rms_norm", "silu_mul", "dequant_q4"]


def signatures(path, prefix):
    text = re.sub(r"/\*.*?\*/", "", open(path).read(), flags=re.S)
    out = {}
    for m in re.finditer(r"\bint\s+(" + prefix + r"[a-z0-9_]+)\s*\(([^)]*)\)", text):
        out[m.group(1)[len(prefix):]] = re.sub(r"\s+", " ", m.group(2)).strip()
    return out


def test_signatures_identical_to_the_gpu_abi():
    gpu = signatures(os.path.join(ROOT, "include", "mllm.h"), "mllm_")
    cpu = signatures(os.path.join(ROOT, "oracle", "mllm_cpu.h"), "mllm_cpu_")
    for op in OPS:
        assert cpu[op] == gpu[op], op


def test_oracle_library_exports_them(oracle_lib):
    lib = C.CDLL(oracle_lib.build())
    for op in OPS + ["kernel_version"]:
        assert hasattr(lib, "mllm_cpu_" + op), op
    lib.mllm_cpu_kernel_version.restype = C.c_int
    assert lib.mllm_cpu_kernel_version() == abi.lib().mllm_kernel_version()


BUF = (C.c_uint8 * 256)()
B = C.addressof(BUF)
BAD = [
    ("gemv_q4", (4, 64, B, B, 64, B, B, None)),       # group 64: unsupported
    ("gemv_q4", (4, 48, B, B, 32, B, B, None)),       # n not a multiple of 32
    ("gemv_q4", (0, 64, B, B, 32, B, B, None)),       # m = 0
    ("gemv_q4", (4, 1 << 15, B, B, 32, B, B, None)),  # too many columns
    ("gemv_q4", (4, 64, None, None, 32, None, None, None)),
    ("gemm_q4", (0, 4, 64, B, B, 32, B, B, None)),
    ("gemm_q4", (2, 4, 64, B, B, 16, B, B, None)),
    ("gemv_f32", (0, 16, B, B, B, None)),
    ("gemv_f32", (4, 16, None, B, B, None)),
    ("gemv_q8", (4, -1, B, B, B, B, None)),
    ("gemv_q8_g32", (4, 0, B, B, B, B, None)),
    ("rms_norm", (0, B, B, B, 1, C.c_float(1e-6), None)),
    ("rms_norm", (16, None, B, B, 1, C.c_float(1e-6), None)),
    ("silu_mul", (0, B, B, None)),
    ("silu_mul", (4, None, B, None)),
    ("dequant_q4", (4, 64, B, B, 16, B, None)),
    ("dequant_q4", (4, 40, B, B, 32, B, None)),
]


@pytest.mark.parametrize("op,args", BAD, ids=[f"{o}-{i}" for i, (o, _) in enumerate(BAD)])
def test_same_argument_errors_as_the_gpu_abi(oracle_lib, op, args):
    lib = C.CDLL(oracle_lib.build())
    lib.mllm_cpu_last_error.restype = C.c_char_p
    rc_gpu = getattr(abi.lib(), "mllm_" + op)(*args)
    rc_cpu = getattr(lib, "mllm_cpu_" + op)(*args)
    assert rc_gpu != 0 and rc_cpu == rc_gpu, (rc_gpu, rc_cpu)
    assert lib.mllm_cpu_last_error()
