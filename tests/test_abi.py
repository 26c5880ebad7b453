"""CPU checks of the C-ABI library: it loads, exports every entry point that
include/mllm.h declares, and rejects bad arguments before touching the GPU."""
import ctypes as C
import json
import os
import re

import pytest

from mllm import abi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "mllm.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mllm_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_what_the_binding_binds():
    assert set(declared_symbols()) == set(abi.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = abi.lib()
    for name in declared_symbols():
        assert hasattr(lib, name), name


def test_kernel_version_and_error_string():
    assert abi.lib().mllm_kernel_version() == 1
    assert isinstance(abi.lib().mllm_last_error(), bytes)


@pytest.mark.parametrize("m,n,group,code", [(4, 64, 64, 4), (4, 48, 32, 1), (0, 64, 32, 1), (4, 1 << 15, 32, 4)])
def test_gemv_q4_argument_errors(m, n, group, code):
    buf = (C.c_uint8 * 64)()
    rc = abi.lib().mllm_gemv_q4(m, n, C.addressof(buf), C.addressof(buf), group, C.addressof(buf),
                                C.addressof(buf), None)
    assert rc == code
    assert abi.lib().mllm_last_error()


def test_null_pointer_errors():
    assert abi.lib().mllm_gemv_q4(4, 64, None, None, 32, None, None, None) == 1
    assert abi.lib().mllm_rms_norm(0, None, None, None, 1, C.c_float(1e-6), None) == 1
    assert abi.lib().mllm_model_create(None, None, 0, None, 0, None) == 1
    assert abi.lib().mllm_model_destroy(None) == 0
    assert abi.lib().mllm_cache_len(None) == -1


def test_no_kernel_uses_scratch_memory():
    """The build records each kernel's resources (compiler remarks); a kernel
    whose register arrays went to scratch memory pays a memory round trip per
    access and extra HBM traffic."""
    path = os.path.join(ROOT, "microllm-lab_amd", "_build", "resource_usage.json")
    if not os.path.exists(path):
        pytest.skip("library not built in this tree")
    with open(path) as f:
        usage = json.load(f)
    assert usage, "no kernels recorded"
    assert {k: v["ScratchSize"] for k, v in usage.items() if v.get("ScratchSize", 0)} == {}
