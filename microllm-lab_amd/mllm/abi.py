"""ctypes binding of libmllm (include/mllm.h).

The library is built in-tree (microllm-lab_amd/build.py) as
microllm-lab_amd/libmllm.so.  Loading fails loudly when it is missing: there
is no CPU fallback for any entry point.
"""
from __future__ import annotations

import ctypes as C
import os

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
# MLLM_LIBRARY may name another build of the same library (e.g. one compiled
# with different tuning constants); it must export the same symbols.
LIB_PATH = os.environ.get("MLLM_LIBRARY") or os.path.join(PKG_DIR, "libmllm.so")

MLLM_OK = 0
ERR_NAMES = {1: "INVALID", 2: "HIP", 3: "OOM", 4: "UNSUPPORTED", 5: "DEVICE"}

# Every exported entry point with its argument and return types.
P = C.c_void_p
I = C.c_int
SIGNATURES = {
    "mllm_last_error": ([], C.c_char_p),
    "mllm_kernel_version": ([], I),
    "mllm_gemv_f32": ([I, I, P, P, P, P], I),
    "mllm_gemv_q8": ([I, I, P, P, P, P, P], I),
    "mllm_gemv_q4": ([I, I, P, P, I, P, P, P], I),
    "mllm_gemv_q8_g32": ([I, I, P, P, P, P, P], I),
    "mllm_gemm_q4": ([I, I, I, P, P, I, P, P, P], I),
    "mllm_gemv_q4_batched": ([I, I, I, P, P, P, P, P], I),
    "mllm_gemv_q8_g32_batched": ([I, I, I, P, P, P, P, P], I),
    "mllm_gemv_q4_argmax": ([I, I, P, P, I, P, P, P, P], I),
    "mllm_gemv_q4_argmax_noalloc": ([I, I, P, P, I, P, P, P, P], I),
    "mllm_rms_norm": ([I, P, P, P, I, C.c_float, P], I),
    "mllm_silu_mul": ([I, P, P, P], I),
    "mllm_dequant_q4": ([I, I, P, P, I, P, P], I),
    "mllm_model_create": ([P, P, C.c_uint64, P, I, P], I),
    "mllm_model_destroy": ([P], I),
    "mllm_reset_cache": ([P], I),
    "mllm_cache_len": ([P], I),
    "mllm_set_cache_len": ([P, I], I),
    "mllm_forward_prompt": ([P, P, I, P, P], I),
    "mllm_forward_decode": ([P, C.c_int32, P, P], I),
    "mllm_forward_verify": ([P, P, I, P, P], I),
    "mllm_max_pass_tokens": ([P], I),
    "mllm_decode_chain": ([P, C.c_int32, I, C.c_int32, P, I, P, P], I),
    "mllm_model_gemv": ([P, C.c_char_p, P, P], I),
    "mllm_set_exec_mode": ([P, I], I),
    "mllm_get_exec_mode": ([P], I),
    "mllm_decode_kernel_name": ([P], C.c_char_p),
    "mllm_flow_verify_tokens": ([P], I),
    "mllm_set_prefill": ([P, I, I], I),
    "mllm_set_debug": ([P, I, I, I, I], I),
    "mllm_model_device_bytes": ([P], C.c_uint64),
    "mllm_last_timing": ([P, P, P], I),
    "mllm_profile_decode": ([P, C.c_int32, I, P], I),
    "mllm_phase_name": ([I], C.c_char_p),
}


class MllmError(RuntimeError):
    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} -> {ERR_NAMES.get(code, code)}: {msg}")
        self.code = code


class MllmConfig(C.Structure):
    _fields_ = [("arch", C.c_int32), ("vocab_size", C.c_int32), ("n_layers", C.c_int32), ("d_model", C.c_int32),
                ("n_heads", C.c_int32), ("n_kv_heads", C.c_int32), ("d_ff", C.c_int32),
                ("max_seq_len", C.c_int32), ("rope_theta", C.c_double), ("rope_pct", C.c_double),
                ("norm_eps", C.c_float), ("kv_fp16", C.c_int32)]


class MllmTensor(C.Structure):
    _fields_ = [("name", C.c_char_p), ("storage", C.c_int32), ("rows", C.c_int32), ("cols", C.c_int32),
                ("group", C.c_int32), ("offset", C.c_uint64), ("nbytes", C.c_uint64),
                ("scale_offset", C.c_uint64), ("scale_nbytes", C.c_uint64)]


_lib = None


def lib() -> C.CDLL:
    """Load libmllm.so (raises if it was not built)."""
    global _lib
    if _lib is None:
        try:
            # torch ships its own HIP runtime under the same soname; loading it
            # first makes libmllm bind to that one, so the process holds a
            # single runtime and torch tensors and libmllm share the device.
            import torch  # noqa: F401
        except ImportError:
            pass
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"libmllm.so not built at {LIB_PATH}; run __graft_entry__.build()")
        L = C.CDLL(LIB_PATH)
        for name, (args, res) in SIGNATURES.items():
            f = getattr(L, name)
            f.argtypes = args
            f.restype = res
        _lib = L
    return _lib


def check(fn: str, rc: int):
    if rc != MLLM_OK:
        raise MllmError(fn, rc, lib().mllm_last_error().decode())


def call(fn: str, *args):
    rc = getattr(lib(), fn)(*args)
    check(fn, rc)
    return rc
