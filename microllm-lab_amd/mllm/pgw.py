"""PGW1 weight container: reader, writer, quantisers and synthetic models.

Format (reader: engine/weights.js:5-39; writer: tools/convert_hf_to_pgw.py:125-144
and tools/convert_gpt2_to_pgw.py:166-184):

  bytes 0..3    "PGW1"
  byte  4       dtype code (weights.js:3): 0 f32, 1 f16, 2 bf16, 3 q8, 4 q4
  byte  5       arch: 0 llama, 1 gpt2
  u32 @ 8..36   vocab, nLayers, dModel, nHeads, nKvHeads, dFf, maxSeqLen, qGroup
  u32 @ 40/44/48 tableOff (=256), tableLen, payloadOff (16-aligned)
  f64 @ 56/64   ropeTheta, ropePct
  JSON table    [{name, shape, kind, storage, group, scaleOffset, scaleNbytes, offset, nbytes}]
  payload       per q4 tensor: f32 scales [rows][cols/32] then packed nibbles [rows][cols/2]

The tensor order and JSON key order follow the converters so a file written here
is laid out the way the reference writes one.
"""
from __future__ import annotations

import json
import struct
from dataclasses import dataclass, field
from io import BytesIO
from typing import Dict, List, Optional

import numpy as np

GROUP = 32
DTYPE_CODE = {0: "f32", 1: "f16", 2: "bf16", 3: "q8", 4: "q4"}
STORAGE_CODE = {"f32": 0, "f16": 1, "bf16": 2, "q8": 3, "q4": 4, "q8g32": 5}


# --------------------------------------------------------------------------
# quantisers
# --------------------------------------------------------------------------
def quant_q4(mat: np.ndarray, group: int = GROUP):
    """Vectorised restatement of convert_hf_to_pgw.py:18-34.

    Per group of 32: amax = max|x|; sc = amax/8 in f64 (1.0 if amax == 0),
    stored as f32; q = clip(rint(x / f32(sc)) + 8, 0, 15) computed in float32
    (NumPy divides a float32 array by a Python float in float32); the even
    element goes to the low nibble.
    """
    mat = np.ascontiguousarray(mat, dtype=np.float32)
    rows, cols = mat.shape
    if cols % group:
        raise ValueError(f"cols {cols} not divisible by group {group}")
    ng = cols // group
    ch = mat.reshape(rows, ng, group)
    amax = np.abs(ch).max(axis=-1)
    sc = np.where(amax > 0, amax.astype(np.float64) / 8.0, 1.0).astype(np.float32)
    q = np.clip(np.rint(ch / sc[..., None]) + np.float32(8.0), 0, 15).astype(np.uint8)
    packed = (q[..., 0::2] | (q[..., 1::2] << 4)).reshape(rows, cols // 2)
    return np.ascontiguousarray(packed), np.ascontiguousarray(sc)


def _quant_q8_spans(ch: np.ndarray):
    amax = np.abs(ch).max(axis=-1)
    sc = np.where(amax > 0, amax.astype(np.float64) / 127.0, 1.0).astype(np.float32)
    q = np.clip(np.rint(ch / sc[..., None]), -127, 127).astype(np.int8)
    return q, sc


def quant_q8g32(mat: np.ndarray):
    """Build-defined Q8 group-32 (the reference has no such format): i8 [m][n] + f32 [m][n/32]."""
    mat = np.ascontiguousarray(mat, dtype=np.float32)
    rows, cols = mat.shape
    q, sc = _quant_q8_spans(mat.reshape(rows, cols // 32, 32))
    return np.ascontiguousarray(q.reshape(rows, cols)), np.ascontiguousarray(sc)


def quant_q8row(mat: np.ndarray):
    """Per-row Q8 in the reference's storage layout (weights.js:96-104): i8 [m][n] + f32 [m]."""
    mat = np.ascontiguousarray(mat, dtype=np.float32)
    q, sc = _quant_q8_spans(mat)
    return np.ascontiguousarray(q), np.ascontiguousarray(sc)


def f32_to_bf16_bits(mat: np.ndarray) -> np.ndarray:
    """bf16 bit patterns of f32 values, rounded to nearest even (NaN kept quiet)."""
    u = np.ascontiguousarray(mat, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(np.asarray(mat, np.float32))
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)


def dequant_q4(packed: np.ndarray, scales: np.ndarray, group: int = GROUP) -> np.ndarray:
    """weights.js:106-123 (vectorised)."""
    rows = packed.shape[0]
    cols = packed.shape[1] * 2
    lo = (packed & 15).astype(np.int32) - 8
    hi = (packed >> 4).astype(np.int32) - 8
    q = np.empty((rows, cols), np.float64)
    q[:, 0::2] = lo
    q[:, 1::2] = hi
    sc = np.repeat(scales.astype(np.float64), group, axis=1)
    return (q * sc).astype(np.float32)


# --------------------------------------------------------------------------
# container
# --------------------------------------------------------------------------
@dataclass
class Config:
    arch: str = "llama"
    vocab_size: int = 49152
    n_layers: int = 30
    d_model: int = 576
    n_heads: int = 9
    n_kv_heads: int = 3
    d_ff: int = 1536
    max_seq_len: int = 2048
    q_group: int = GROUP
    rope_theta: float = 100000.0
    rope_pct: float = 1.0

    @property
    def head_dim(self) -> int:
        return self.d_model // self.n_heads


@dataclass
class Bundle:
    """What parsePgw returns (weights.js:39): kind, cfg, tensors, buffer, payloadOff."""

    kind: str
    cfg: Config
    tensors: Dict[str, dict]
    buffer: bytes
    payload_off: int
    order: List[str] = field(default_factory=list)

    @property
    def payload(self) -> memoryview:
        return memoryview(self.buffer)[self.payload_off:]

    def array(self, name: str) -> np.ndarray:
        """Typed view of a tensor's data (weights.js:42-62)."""
        t = self.tensors[name]
        st = t["storage"]
        dt = {"f32": np.float32, "f16": np.uint16, "bf16": np.uint16, "q8": np.int8, "q8g32": np.int8,
              "q4": np.uint8}[st]
        a = np.frombuffer(self.buffer, dtype=dt, count=t["nbytes"] // np.dtype(dt).itemsize,
                          offset=self.payload_off + t["offset"])
        shape = t["shape"]
        if st == "q4":
            return a.reshape(shape[0], shape[1] // 2)
        return a.reshape(shape)

    def scales(self, name: str) -> np.ndarray:
        """weights.js:64-67"""
        t = self.tensors[name]
        a = np.frombuffer(self.buffer, dtype=np.float32, count=t["scaleNbytes"] // 4,
                          offset=self.payload_off + t["scaleOffset"])
        rows = t["shape"][0]
        return a.reshape(rows, -1)


def parse_pgw(buf: bytes) -> Bundle:
    """Restatement of weights.js:5-39."""
    buf = bytes(buf)
    if buf[0:4] != b"PGW1":
        raise ValueError(f"bad magic {buf[0:4]!r}")
    kind = DTYPE_CODE.get(buf[4], "f32")
    arch = "gpt2" if buf[5] == 1 else "llama"
    vocab, nl, d, nh, nkv, dff, ms, qg = struct.unpack_from("<8I", buf, 8)
    table_off, table_len, payload_off = struct.unpack_from("<III", buf, 40)
    theta = struct.unpack_from("<d", buf, 56)[0] or 10000.0
    pct = struct.unpack_from("<d", buf, 64)[0] or 1.0
    cfg = Config(arch, vocab, nl, d, nh, nkv, dff, ms, qg or 32, theta, pct)
    table = json.loads(buf[table_off:table_off + table_len].decode("utf-8"))
    tensors = {e["name"]: e for e in table}
    if cfg.arch == "gpt2" and "blocks.0.ln1" not in tensors and "blocks.0.norm1" in tensors:
        cfg.arch = "llama"
    return Bundle(kind, cfg, tensors, buf, payload_off, [e["name"] for e in table])


class PgwWriter:
    """Accumulates tensors in the converters' blob order (convert_hf_to_pgw.py:37-72)."""

    def __init__(self):
        self.blobs = BytesIO()
        self.entries: List[dict] = []

    def add_q4(self, name: str, arr: np.ndarray):
        packed, scales = quant_q4(arr)
        self.add_q4_packed(name, packed, scales, arr.shape)

    def add_q4_packed(self, name, packed, scales, shape):
        scale_off = self.blobs.tell()
        self.blobs.write(np.ascontiguousarray(scales, np.float32).tobytes())
        data_off = self.blobs.tell()
        self.blobs.write(np.ascontiguousarray(packed, np.uint8).tobytes())
        self.entries.append({
            "name": name,
            "shape": [int(shape[0]), int(shape[1])],
            "kind": "q4",
            "storage": "q4",
            "group": GROUP,
            "scaleOffset": scale_off,
            "scaleNbytes": int(scales.size * 4),
            "offset": data_off,
            "nbytes": int(packed.size),
        })

    def add_f32(self, name: str, arr: np.ndarray):
        data = np.ascontiguousarray(arr, dtype=np.float32)
        off = self.blobs.tell()
        self.blobs.write(data.tobytes())
        self.entries.append({
            "name": name,
            "shape": list(data.shape),
            "kind": "q4",
            "storage": "f32",
            "offset": off,
            "nbytes": int(data.nbytes),
        })

    def add_matrix(self, name: str, arr: np.ndarray, storage: str = "q4", kind: Optional[str] = None,
                   group: int = GROUP):
        """A matrix in any storage weights.js reads (f32, f16, bf16, per-row
        q8, q4 of any group) or q8g32.  q4 at group 32 is add_q4 (the
        converters' layout, byte for byte); the other storages have no writer
        in the reference, so their blobs (scales first, then data) each start
        on a 16-byte boundary, which the GPU engine reads them with."""
        if storage == "q4" and group == GROUP and kind in (None, "q4"):
            self.add_q4(name, arr)
            return
        arr = np.ascontiguousarray(arr, dtype=np.float32)
        rows, cols = arr.shape
        scales = None
        if storage == "q4":
            data, scales = quant_q4(arr, group)
        elif storage == "q8":
            data, scales = quant_q8row(arr)
        elif storage == "q8g32":
            data, scales = quant_q8g32(arr)
        elif storage == "f16":
            data = arr.astype(np.float16).view(np.uint16)
        elif storage == "bf16":
            data = f32_to_bf16_bits(arr)
        elif storage == "f32":
            data = arr
        else:
            raise ValueError(storage)
        e = {"name": name, "shape": [int(rows), int(cols)], "kind": kind or storage, "storage": storage}
        if storage in ("q4", "q8g32"):
            e["group"] = int(group if storage == "q4" else 32)
        if scales is not None:
            self._pad16()
            e["scaleOffset"] = self.blobs.tell()
            e["scaleNbytes"] = int(scales.size * 4)
            self.blobs.write(np.ascontiguousarray(scales, np.float32).tobytes())
        self._pad16()
        e["offset"] = self.blobs.tell()
        e["nbytes"] = int(data.nbytes)
        self.blobs.write(np.ascontiguousarray(data).tobytes())
        self.entries.append(e)

    def _pad16(self):
        self.blobs.write(b"\x00" * (-self.blobs.tell() % 16))

    def finish(self, cfg: Config, header_group: Optional[int] = None, kind: str = "q4") -> bytes:
        payload = self.blobs.getvalue()
        table = json.dumps(self.entries, separators=(",", ":")).encode("utf-8")
        table_off = 256
        pad = (16 - ((table_off + len(table)) % 16)) % 16
        payload_off = table_off + len(table) + pad
        header = bytearray(256)
        header[0:4] = b"PGW1"
        header[4] = {v: k for k, v in DTYPE_CODE.items()}.get(kind, 4)
        header[5] = 1 if cfg.arch == "gpt2" else 0
        qg = GROUP if header_group is None else header_group
        struct.pack_into("<8I", header, 8, cfg.vocab_size, cfg.n_layers, cfg.d_model, cfg.n_heads,
                         cfg.n_kv_heads, cfg.d_ff, cfg.max_seq_len, qg)
        struct.pack_into("<III", header, 40, table_off, len(table), payload_off)
        struct.pack_into("<d", header, 56, cfg.rope_theta)
        struct.pack_into("<d", header, 64, cfg.rope_pct)
        return bytes(header) + table + b"\x00" * pad + payload


# --------------------------------------------------------------------------
# synthetic models (no checkpoints exist offline)
# --------------------------------------------------------------------------
CONFIGS = {
    # SmolLM2-135M shape (models/smollm2-135m-instruct/card.json)
    "smollm2-135m": Config("llama", 49152, 30, 576, 9, 3, 1536, 2048, 32, 100000.0, 1.0),
    # SmolLM2-360M shape (models/smollm2-360m-instruct/card.json)
    "smollm2-360m": Config("llama", 49152, 32, 960, 15, 5, 2560, 2048, 32, 100000.0, 1.0),
    # GPT-2 124M shape (models/gpt2/card.json)
    "gpt2-124m": Config("gpt2", 50257, 12, 768, 12, 12, 3072, 1024, 32, 10000.0, 1.0),
}


def _normal(rng: np.random.Generator, shape, std: float = 0.02) -> np.ndarray:
    return (rng.standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float32)


def _storages(kind: str, storages: Optional[Dict[str, str]]):
    """The matrix storage of each tensor name: `kind` (q4, q8, q8g32, f16,
    bf16, f32) unless `storages` names another (a mixed model)."""
    return lambda name: (storages or {}).get(name, kind)


def make_llama(cfg: Config, seed: int = 0, std: float = 0.02, norm_gain: float = 1.0, kind: str = "q4",
               storages: Optional[Dict[str, str]] = None, group: int = GROUP) -> bytes:
    """Llama-style PGW1 in convert_hf_to_pgw.py:104-122 order; weights N(0, std)
    stored as `kind` (q4: quant_q4, the converter's format); norm gains
    constant.  `storages` overrides the storage of named matrices; `group` is
    the Q4 group size."""
    rng = np.random.default_rng(seed)
    hd = cfg.d_model // cfg.n_heads
    kv = cfg.n_kv_heads * hd
    w = PgwWriter()
    st = _storages(kind, storages)

    def mat(name, shape):
        w.add_matrix(name, _normal(rng, shape, std), st(name), kind=kind, group=group)

    mat("lm_head", (cfg.vocab_size, cfg.d_model))
    ones = np.full(cfg.d_model, norm_gain, np.float32)
    for i in range(cfg.n_layers):
        w.add_f32(f"blocks.{i}.norm1", ones)
        mat(f"blocks.{i}.attn.qkv", (cfg.d_model + 2 * kv, cfg.d_model))
        mat(f"blocks.{i}.attn.proj", (cfg.d_model, cfg.d_model))
        w.add_f32(f"blocks.{i}.norm2", ones)
        mat(f"blocks.{i}.mlp.w1", (cfg.d_ff, cfg.d_model))
        mat(f"blocks.{i}.mlp.w3", (cfg.d_ff, cfg.d_model))
        mat(f"blocks.{i}.mlp.w2", (cfg.d_model, cfg.d_ff))
    w.add_f32("norm_f", ones)
    return w.finish(cfg, kind=kind if kind in DTYPE_CODE.values() else "q8")


def make_cycle_llama(cfg: Config, cycle, seed: int = 0, std: float = 0.02, layer_std: float = 0.002,
                     gain: float = 20.0) -> bytes:
    """A llama model whose greedy decode follows a token cycle: after token
    cycle[i] it emits cycle[(i + 1) % len(cycle)].  Synthetic N(0, std)
    weights cannot show prompt-lookup speculation at work -- their greedy
    output repeats one token or never repeats a 3-gram, so every draft is one
    token long or empty -- and no trained checkpoint is available offline.

    Layer 0's MLP carries the cycle.  Hidden unit i < len(cycle) has gate and
    up rows 0.5 * e_i (e_i the unit direction of cycle[i]'s embedding row),
    so it fires only for that token (silu(12) * 12 against ~0.1), and its
    down column adds gain * e_{i+1} / 144 to the residual, which then points
    at the next token's embedding.  The other units of the first 32 (one Q4
    group of the down rows) are zero, so the cycle's columns quantise on
    their own scale.  Every other weight is N(0, layer_std): the remaining
    layers do real work without turning the residual away from the next
    token.  The lm_head / embedding is N(0, std) as in make_llama."""
    cycle = [int(t) for t in cycle]
    c = len(cycle)
    assert 1 < c <= 32 <= cfg.d_ff and len(set(cycle)) == c
    rng = np.random.default_rng(seed)
    hd = cfg.d_model // cfg.n_heads
    kv = cfg.n_kv_heads * hd
    w = PgwWriter()
    emb = _normal(rng, (cfg.vocab_size, cfg.d_model), std)
    w.add_q4("lm_head", emb)
    unit = emb[cycle] / np.linalg.norm(emb[cycle], axis=1, keepdims=True)
    ones = np.ones(cfg.d_model, np.float32)
    for i in range(cfg.n_layers):
        w.add_f32(f"blocks.{i}.norm1", ones)
        w.add_q4(f"blocks.{i}.attn.qkv", _normal(rng, (cfg.d_model + 2 * kv, cfg.d_model), layer_std))
        w.add_q4(f"blocks.{i}.attn.proj", _normal(rng, (cfg.d_model, cfg.d_model), layer_std))
        w.add_f32(f"blocks.{i}.norm2", ones)
        w1 = _normal(rng, (cfg.d_ff, cfg.d_model), layer_std)
        w3 = _normal(rng, (cfg.d_ff, cfg.d_model), layer_std)
        w2 = _normal(rng, (cfg.d_model, cfg.d_ff), layer_std)
        if i == 0:
            w1[:32] = 0.0
            w3[:32] = 0.0
            w2[:, :32] = 0.0
            w1[:c] = 0.5 * unit
            w3[:c] = 0.5 * unit
            w2[:, :c] = (gain / 144.0) * np.roll(unit, -1, axis=0).T
        w.add_q4(f"blocks.{i}.mlp.w1", w1.astype(np.float32))
        w.add_q4(f"blocks.{i}.mlp.w3", w3.astype(np.float32))
        w.add_q4(f"blocks.{i}.mlp.w2", w2.astype(np.float32))
    w.add_f32("norm_f", ones)
    return w.finish(cfg)


def make_gpt2(cfg: Config, seed: int = 0, std: float = 0.02, scale_factors: Optional[np.ndarray] = None,
              bias_std: float = 0.0, kind: str = "q4", storages: Optional[Dict[str, str]] = None,
              group: int = GROUP) -> bytes:
    """GPT-2 PGW1 in convert_gpt2_to_pgw.py:135-164 order; header qGroup = 1 as the
    converter writes it (convert_gpt2_to_pgw.py:175).  LN gamma 1, beta 0,
    biases N(0, bias_std) (0 by default), scale_factors 1 unless given;
    matrices stored as `kind` (storages / group as in make_llama)."""
    rng = np.random.default_rng(seed)
    d, ff = cfg.d_model, cfg.d_ff
    w = PgwWriter()
    st = _storages(kind, storages)

    def mat(name, shape):
        w.add_matrix(name, _normal(rng, shape, std), st(name), kind=kind, group=group)

    sf = np.ones(d, np.float32) if scale_factors is None else np.asarray(scale_factors, np.float32)
    w.add_f32("scale_factors", sf)
    mat("lm_head", (cfg.vocab_size, d))
    w.add_f32("wpe", _normal(rng, (cfg.max_seq_len, d), std))
    w.add_f32("ln_f", np.concatenate([np.ones(d, np.float32) / sf, np.zeros(d, np.float32) / sf]))
    ln = np.concatenate([np.ones(d, np.float32), np.zeros(d, np.float32)])

    def bias(n):
        return _normal(rng, (n,), bias_std) if bias_std > 0 else np.zeros(n, np.float32)

    for i in range(cfg.n_layers):
        w.add_f32(f"blocks.{i}.ln1", ln)
        mat(f"blocks.{i}.attn.qkv", (3 * d, d))
        w.add_f32(f"blocks.{i}.attn.qkv_bias", bias(3 * d))
        mat(f"blocks.{i}.attn.proj", (d, d))
        w.add_f32(f"blocks.{i}.attn.proj_bias", bias(d))
        w.add_f32(f"blocks.{i}.ln2", ln)
        mat(f"blocks.{i}.mlp.fc", (ff, d))
        w.add_f32(f"blocks.{i}.mlp.fc_bias", bias(ff))
        mat(f"blocks.{i}.mlp.proj", (d, ff))
        w.add_f32(f"blocks.{i}.mlp.proj_bias", bias(d))
    return w.finish(cfg, header_group=1, kind=kind if kind in DTYPE_CODE.values() else "q8")


def make_model(cfg: Config, seed: int = 0, **kw) -> bytes:
    return make_gpt2(cfg, seed, **kw) if cfg.arch == "gpt2" else make_llama(cfg, seed, **kw)


def small_config(arch: str = "llama", **over) -> Config:
    """Tiny shapes for CPU-oracle parity tests."""
    if arch == "gpt2":
        c = Config("gpt2", 512, 2, 128, 2, 2, 512, 64, 32, 10000.0, 1.0)
    else:
        c = Config("llama", 512, 2, 128, 2, 1, 256, 64, 32, 10000.0, 1.0)
    for k, v in over.items():
        setattr(c, k, v)
    return c


# --------------------------------------------------------------------------
# checkpoint conversion (the C++ converter, libpgwconvert.so)
# --------------------------------------------------------------------------
def convert_checkpoint(hf_dir: str, out_path: str, arch: str = "llama", max_seq: Optional[int] = None,
                       scale_factors: Optional[np.ndarray] = None) -> None:
    """A HuggingFace checkpoint directory (config.json + safetensors) to a PGW1
    file, as tools/convert_hf_to_pgw.py (arch "llama") or
    tools/convert_gpt2_to_pgw.py after its calibration (arch "gpt2", with the
    calibrated channel scales) write it; see include/pgw_convert.h."""
    import ctypes as C
    import os

    lib_path = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "convert",
                            "libpgwconvert.so")
    lib = C.CDLL(lib_path)
    lib.pgwc_last_error.restype = C.c_char_p
    if arch == "llama":
        rc = lib.pgwc_convert_llama(hf_dir.encode(), out_path.encode(), C.c_int(max_seq or 2048))
    elif arch == "gpt2":
        sf = None if scale_factors is None else np.ascontiguousarray(scale_factors, np.float32)
        rc = lib.pgwc_convert_gpt2(hf_dir.encode(), out_path.encode(), C.c_int(max_seq or 1024),
                                   C.c_void_p(None if sf is None else sf.ctypes.data),
                                   C.c_int(0 if sf is None else sf.size))
    else:
        raise ValueError(f"arch {arch!r}")
    if rc:
        raise RuntimeError(f"pgw_convert: {lib.pgwc_last_error().decode()}")
