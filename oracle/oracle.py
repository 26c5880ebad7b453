"""ctypes binding of the CPU oracle (liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py.  The product path never imports this module.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from typing import List, Optional

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

STORAGE = {"f32": 0, "f16": 1, "bf16": 2, "q8": 3, "q4": 4, "q8g32": 5}


class OrcConfig(C.Structure):
    _fields_ = [("arch", C.c_int32), ("vocab_size", C.c_int32), ("n_layers", C.c_int32), ("d_model", C.c_int32),
                ("n_heads", C.c_int32), ("n_kv_heads", C.c_int32), ("d_ff", C.c_int32),
                ("max_seq_len", C.c_int32), ("rope_theta", C.c_double), ("rope_pct", C.c_double),
                ("norm_eps", C.c_double)]


class OrcTensor(C.Structure):
    _fields_ = [("name", C.c_char_p), ("storage", C.c_int32), ("rows", C.c_int32), ("cols", C.c_int32),
                ("group", C.c_int32), ("offset", C.c_uint64), ("nbytes", C.c_uint64),
                ("scale_offset", C.c_uint64), ("scale_nbytes", C.c_uint64)]


def build(force: bool = False) -> str:
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-s", "-B" if force else "liboracle.so"], cwd=HERE, check=True)
    return LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        P = C.c_void_p
        i = C.c_int
        for name, args in {
            "orc_quant_q4": [P, i, i, i, P, P],
            "orc_quant_q8g32": [P, i, i, P, P],
            "orc_quant_q8row": [P, i, i, P, P],
            "orc_dequant_q4": [P, P, i, i, i, P],
            "orc_dequant_q8row": [P, P, i, i, P],
            "orc_dequant_q8g32": [P, P, i, i, P],
            "orc_gemv_q4_js": [i, i, P, P, i, P, P],
            "orc_gemv_q8_js": [i, i, P, P, P, P],
            "orc_gemv_q8g32_js": [i, i, P, P, P, P],
            "orc_gemv_f32_js": [i, i, P, P, P],
            "orc_gemv_q4_wasm": [i, i, P, P, i, P, P],
            "orc_gemv_q8_wasm": [i, i, P, P, P, P],
            "orc_gemv_f32_wasm": [i, i, P, P, P],
            "orc_rms_norm_wasm": [i, P, P, P, i, C.c_float],
            "orc_silu_mul_wasm": [i, P, P],
            "orc_rms_norm_js": [P, P, P, i, i, C.c_double],
            "orc_layer_norm_js": [P, P, P, i, i, C.c_double],
            "orc_silu_mul_js": [P, P, i],
            "orc_gelu_new_js": [P, i],
            "orc_build_rope": [i, i, C.c_double, C.c_double, P, P, P],
            "orc_apply_rope_js": [P, i, i, i, P, P, i, i],
            "orc_softmax_js": [P, i],
            "orc_argmax": [P, i],
            "orc_argmax_gpt2": [P, i, P, i, i, C.c_double],
            "orc_lookup_draft": [P, i, i, i, P],
            "orc_model_create": [P, P, P, i],
            "orc_model_destroy": [P],
            "orc_reset_cache": [P],
            "orc_cache_len": [P],
            "orc_set_cache_len": [P, i],
            "orc_set_debug": [P, i, i, i, i],
            "orc_forward_prompt": [P, P, i],
            "orc_forward_decode": [P, C.c_int32],
            "orc_forward_multi": [P, P, i, P],
            "orc_model_gemv": [P, C.c_char_p, P, P],
            "orc_generate": [P, P, i, i, i, P, P],
        }.items():
            f = getattr(L, name)
            f.argtypes = args
        for name in ("orc_argmax", "orc_argmax_gpt2", "orc_lookup_draft", "orc_cache_len", "orc_model_gemv",
                     "orc_generate"):
            getattr(L, name).restype = C.c_int
        L.orc_model_create.restype = C.c_void_p
        L.orc_forward_prompt.restype = C.POINTER(C.c_float)
        L.orc_forward_decode.restype = C.POINTER(C.c_float)
        for name in ("orc_quant_q4", "orc_quant_q8g32", "orc_quant_q8row", "orc_dequant_q4", "orc_dequant_q8row",
                     "orc_dequant_q8g32", "orc_gemv_q4_js", "orc_gemv_q8_js", "orc_gemv_q8g32_js",
                     "orc_gemv_f32_js", "orc_gemv_q4_wasm", "orc_gemv_q8_wasm", "orc_gemv_f32_wasm",
                     "orc_rms_norm_wasm", "orc_silu_mul_wasm", "orc_rms_norm_js", "orc_layer_norm_js",
                     "orc_silu_mul_js", "orc_gelu_new_js", "orc_build_rope", "orc_apply_rope_js", "orc_softmax_js",
                     "orc_model_destroy", "orc_reset_cache", "orc_set_cache_len", "orc_forward_multi",
                     "orc_set_debug"):
            getattr(L, name).restype = None
        _lib = L
    return _lib


def ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


# ---------------------------------------------------------------- operators
def quant_q4(mat: np.ndarray, group: int = 32):
    mat = np.ascontiguousarray(mat, np.float32)
    r, c = mat.shape
    packed = np.empty((r, c // 2), np.uint8)
    sc = np.empty((r, c // group), np.float32)
    lib().orc_quant_q4(ptr(mat), r, c, group, ptr(packed), ptr(sc))
    return packed, sc


def quant_q8g32(mat):
    mat = np.ascontiguousarray(mat, np.float32)
    r, c = mat.shape
    q = np.empty((r, c), np.int8)
    sc = np.empty((r, c // 32), np.float32)
    lib().orc_quant_q8g32(ptr(mat), r, c, ptr(q), ptr(sc))
    return q, sc


def quant_q8row(mat):
    mat = np.ascontiguousarray(mat, np.float32)
    r, c = mat.shape
    q = np.empty((r, c), np.int8)
    sc = np.empty((r,), np.float32)
    lib().orc_quant_q8row(ptr(mat), r, c, ptr(q), ptr(sc))
    return q, sc


def dequant_q4(packed, scales, group: int = 32):
    packed = np.ascontiguousarray(packed, np.uint8)
    scales = np.ascontiguousarray(scales, np.float32)
    r = packed.shape[0]
    c = packed.shape[1] * 2
    out = np.empty((r, c), np.float32)
    lib().orc_dequant_q4(ptr(packed), ptr(scales), r, c, group, ptr(out))
    return out


def dequant_q8g32(q, scales):
    q = np.ascontiguousarray(q, np.int8)
    scales = np.ascontiguousarray(scales, np.float32)
    out = np.empty(q.shape, np.float32)
    lib().orc_dequant_q8g32(ptr(q), ptr(scales), q.shape[0], q.shape[1], ptr(out))
    return out


def dequant_q8row(q, scales):
    q = np.ascontiguousarray(q, np.int8)
    scales = np.ascontiguousarray(scales, np.float32)
    out = np.empty(q.shape, np.float32)
    lib().orc_dequant_q8row(ptr(q), ptr(scales), q.shape[0], q.shape[1], ptr(out))
    return out


def _gemv(fn, m, n, *arrays, group=None):
    x = np.ascontiguousarray(arrays[-1], np.float32)
    y = np.empty(m, np.float32)
    args = [m, n] + [ptr(np.ascontiguousarray(a)) for a in arrays[:-1]]
    if group is not None:
        args.append(group)
    fn(*args, ptr(x), ptr(y))
    return y


def gemv_q4(packed, scales, x, mode="js", group=32):
    m, n = packed.shape[0], packed.shape[1] * 2
    fn = lib().orc_gemv_q4_js if mode == "js" else lib().orc_gemv_q4_wasm
    return _gemv(fn, m, n, packed, scales, x, group=group)


def gemv_q8(q, scales, x, mode="js"):
    m, n = q.shape
    fn = lib().orc_gemv_q8_js if mode == "js" else lib().orc_gemv_q8_wasm
    return _gemv(fn, m, n, q, scales, x)


def gemv_q8g32(q, scales, x):
    m, n = q.shape
    return _gemv(lib().orc_gemv_q8g32_js, m, n, q, scales, x)


def gemv_f32(w, x, mode="js"):
    m, n = w.shape
    fn = lib().orc_gemv_f32_js if mode == "js" else lib().orc_gemv_f32_wasm
    return _gemv(fn, m, n, np.ascontiguousarray(w, np.float32), x)


def rms_norm(x, w, eps=1e-6, mode="js"):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    dim = w.shape[0]
    tokens = x.size // dim
    out = np.empty_like(x)
    if mode == "js":
        lib().orc_rms_norm_js(ptr(x), ptr(w), ptr(out), dim, tokens, eps)
    else:
        lib().orc_rms_norm_wasm(dim, ptr(x), ptr(w), ptr(out), tokens, eps)
    return out


def layer_norm(x, wb, eps=1e-5):
    x = np.ascontiguousarray(x, np.float32)
    wb = np.ascontiguousarray(wb, np.float32)
    dim = wb.shape[0] // 2
    out = np.empty_like(x)
    lib().orc_layer_norm_js(ptr(x), ptr(wb), ptr(out), dim, x.size // dim, eps)
    return out


def silu_mul(a, b, mode="js"):
    a = np.array(a, np.float32, copy=True)
    b = np.ascontiguousarray(b, np.float32)
    if mode == "js":
        lib().orc_silu_mul_js(ptr(a), ptr(b), a.size)
    else:
        lib().orc_silu_mul_wasm(a.size, ptr(a), ptr(b))
    return a


def gelu_new(a):
    a = np.array(a, np.float32, copy=True)
    lib().orc_gelu_new_js(ptr(a), a.size)
    return a


def build_rope(max_seq, head_dim, theta, pct=1.0):
    cos = np.zeros((max_seq, head_dim), np.float32)
    sin = np.zeros((max_seq, head_dim), np.float32)
    rd = C.c_int(0)
    lib().orc_build_rope(max_seq, head_dim, theta, pct, ptr(cos), ptr(sin), C.addressof(rd))
    return cos[:, :rd.value].copy(), sin[:, :rd.value].copy(), rd.value


def apply_rope(q, n_heads, t, head_dim, cos, sin, rope_dim, offset):
    q = np.array(q, np.float32, copy=True)
    cos = np.ascontiguousarray(cos, np.float32)
    sin = np.ascontiguousarray(sin, np.float32)
    lib().orc_apply_rope_js(ptr(q), n_heads, t, head_dim, ptr(cos), ptr(sin), rope_dim, offset)
    return q


def softmax(x):
    x = np.array(x, np.float32, copy=True)
    lib().orc_softmax_js(ptr(x), x.size)
    return x


def argmax(logits):
    logits = np.ascontiguousarray(logits, np.float32)
    return lib().orc_argmax(ptr(logits), logits.size)


def argmax_gpt2(logits, hist, no_repeat_ngram=3, penalty=1.15):
    logits = np.ascontiguousarray(logits, np.float32)
    h = np.ascontiguousarray(np.asarray(hist, np.int32).reshape(-1))
    hp = ptr(h) if h.size else 0
    return lib().orc_argmax_gpt2(ptr(logits), logits.size, hp, h.size, no_repeat_ngram, penalty)


def lookup_draft(seq, k, n=3) -> List[int]:
    s = np.ascontiguousarray(np.asarray(seq, np.int32).reshape(-1))
    out = np.zeros(max(k, 1), np.int32)
    cnt = lib().orc_lookup_draft(ptr(s) if s.size else 0, s.size, k, n, ptr(out))
    return [int(v) for v in out[:cnt]]


# ---------------------------------------------------------------- model
class OracleModel:
    """infer.js PetitGPT (CPU path) over a PGW bundle."""

    def __init__(self, bundle, norm_eps: float = 1e-6):
        c = bundle.cfg
        self.bundle = bundle
        self.cfg = c
        self._payload = np.frombuffer(bundle.buffer, dtype=np.uint8, offset=bundle.payload_off)
        names = list(bundle.tensors.keys())
        self._names = [n.encode() for n in names]
        arr = (OrcTensor * len(names))()
        for i, n in enumerate(names):
            t = bundle.tensors[n]
            shape = t["shape"]
            rows, cols = (shape[0], shape[1]) if len(shape) == 2 else (1, shape[0])
            arr[i] = OrcTensor(self._names[i], STORAGE[t["storage"]], rows, cols, int(t.get("group", 32) or 32),
                               t["offset"], t["nbytes"], t.get("scaleOffset", 0), t.get("scaleNbytes", 0))
        self._tensors = arr
        oc = OrcConfig(1 if c.arch == "gpt2" else 0, c.vocab_size, c.n_layers, c.d_model, c.n_heads,
                       c.n_kv_heads, c.d_ff, c.max_seq_len, c.rope_theta, c.rope_pct, norm_eps)
        self._cfg = oc
        h = lib().orc_model_create(C.byref(oc), ptr(self._payload), arr, len(names))
        if not h:
            raise ValueError("oracle: missing tensor in bundle")
        self.h = h

    def close(self):
        if getattr(self, "h", None):
            lib().orc_model_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    @property
    def cache_len(self) -> int:
        return lib().orc_cache_len(self.h)

    @cache_len.setter
    def cache_len(self, v: int):
        lib().orc_set_cache_len(self.h, v)

    def reset_cache(self):
        lib().orc_reset_cache(self.h)

    def set_debug(self, max_layers=None, no_attn=False, no_mlp=False, mlp_to=None):
        """The GPU engine's debug knobs (webgpu-metal.js:1263-1279)."""
        lib().orc_set_debug(self.h, -1 if max_layers is None else int(max_layers), int(bool(no_attn)),
                            int(bool(no_mlp)), -1 if mlp_to is None else int(mlp_to))

    def forward_prompt(self, ids) -> np.ndarray:
        a = np.ascontiguousarray(np.asarray(ids, np.int32))
        p = lib().orc_forward_prompt(self.h, ptr(a), a.size)
        return np.ctypeslib.as_array(p, shape=(self.cfg.vocab_size,)).copy()

    def forward_decode(self, tok: int) -> np.ndarray:
        p = lib().orc_forward_decode(self.h, int(tok))
        return np.ctypeslib.as_array(p, shape=(self.cfg.vocab_size,)).copy()

    def forward_multi(self, ids) -> np.ndarray:
        a = np.ascontiguousarray(np.asarray(ids, np.int32))
        out = np.empty((a.size, self.cfg.vocab_size), np.float32)
        lib().orc_forward_multi(self.h, ptr(a), a.size, ptr(out))
        return out

    def gemv(self, name: str, x) -> np.ndarray:
        t = self.bundle.tensors[name]
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty(t["shape"][0], np.float32)
        if lib().orc_model_gemv(self.h, name.encode(), ptr(x), ptr(y)) != 0:
            raise KeyError(name)
        return y

    def generate(self, ids, max_new_tokens=64, eos_id=-1):
        a = np.ascontiguousarray(np.asarray(ids, np.int32))
        out = np.zeros(max_new_tokens, np.int32)
        stop = C.c_int(0)
        n = lib().orc_generate(self.h, ptr(a), a.size, max_new_tokens, eos_id, ptr(out), C.addressof(stop))
        return [int(v) for v in out[:n]], ("eos" if stop.value == 1 else "max_new_tokens")
