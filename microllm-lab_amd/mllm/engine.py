"""PetitGPT model API (engine/infer.js:289-647) over libmllm.

The class keeps the reference's method names so a caller of infer.js finds
the same surface: constructor(bundle), forwardPrompt, forwardDecode, generate,
resetCache, cacheLen, gemv, destroy.  All compute runs in libmllm's HIP
kernels; there is no CPU fallback.

generate() implements three drivers of the same decode step:
  mode="greedy"  host loop of forwardDecode + argmax (infer.js:603-646)
  mode="chain"   device-chained decode, argmax fed back on the GPU
                 (webgpu.js:1202-1226, CHAIN_TOK)
  mode="spec"    prompt-lookup speculation: draft k tokens with lookupDraft
                 (webgpu.js:846-865) and verify k+1 positions in one pass,
                 greedy acceptance (webgpu.js:1239-1270)
"""
from __future__ import annotations

import ctypes as C
import time
from typing import Callable, List, Optional

import numpy as np

from . import abi
from .pgw import STORAGE_CODE, Bundle


def lookup_draft(seq: List[int], k: int, n: int) -> List[int]:
    """webgpu.js:846-865: the k tokens that followed the most recent earlier
    occurrence of the last n tokens of seq (scanning i = len-n-1 .. 0)."""
    L = len(seq)
    if L < n + 1:
        return []
    suf = seq[L - n:]
    for i in range(L - n - 1, -1, -1):
        if seq[i:i + n] == suf:
            return [seq[i + n + t] for t in range(k) if i + n + t < L]
    return []


def argmax(logits: np.ndarray) -> int:
    """infer.js:240-250: the first index of the maximum."""
    return int(np.argmax(logits))


def argmax_gpt2(logits: np.ndarray, history: List[int], no_repeat_ngram: int = 3, penalty: float = 1.15) -> int:
    """infer.js:252-287: 3-gram block and repetition penalty over `history`."""
    v = logits.astype(np.float64).copy()
    n = len(history)
    if no_repeat_ngram == 3 and n >= 2:
        t1, t2 = history[-2], history[-1]
        banned = {history[h + 2] for h in range(n - 2) if history[h] == t1 and history[h + 1] == t2}
        for b in banned:
            v[b] = -1e9
    if penalty > 1.0:
        for tok in set(history[max(0, n - 32):]):
            if v[tok] > -1e8:
                v[tok] = v[tok] / penalty if v[tok] > 0 else v[tok] * penalty
    return int(np.argmax(v))


class PetitGPT:
    """infer.js PetitGPT on the MI355X decode step."""

    def __init__(self, bundle: Bundle, norm_eps: float = 1e-6, kv_fp16: bool = False,
                 exec_mode: Optional[int] = None):
        self.bundle = bundle
        self.cfg = bundle.cfg
        self.kind = bundle.kind
        c = bundle.cfg
        self.is_gpt2 = c.arch == "gpt2"
        names = list(bundle.tensors.keys())
        self._names = [n.encode() for n in names]
        arr = (abi.MllmTensor * len(names))()
        for i, n in enumerate(names):
            t = bundle.tensors[n]
            shape = t["shape"]
            rows, cols = (shape[0], shape[1]) if len(shape) == 2 else (1, shape[0])
            arr[i] = abi.MllmTensor(self._names[i], STORAGE_CODE[t["storage"]], rows, cols,
                                    int(t.get("group", 32) or 32), t["offset"], t["nbytes"],
                                    t.get("scaleOffset", 0), t.get("scaleNbytes", 0))
        cfg = abi.MllmConfig(1 if self.is_gpt2 else 0, c.vocab_size, c.n_layers, c.d_model, c.n_heads,
                             c.n_kv_heads, c.d_ff, c.max_seq_len, c.rope_theta, c.rope_pct, norm_eps,
                             1 if kv_fp16 else 0)
        payload = np.frombuffer(bundle.buffer, dtype=np.uint8, offset=bundle.payload_off)
        h = C.c_void_p()
        abi.call("mllm_model_create", C.byref(cfg), payload.ctypes.data, payload.size, arr, len(names),
                 C.byref(h))
        self._h = h
        self._logits = np.zeros(c.vocab_size, np.float32)
        self.max_pass = abi.lib().mllm_max_pass_tokens(h)
        self.exec_mode = None
        if exec_mode is not None:
            self.set_exec_mode(exec_mode)
        self.lastTiming = None

    # ---------------------------------------------------------------- state
    def destroy(self):
        if getattr(self, "_h", None):
            abi.lib().mllm_model_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass

    def set_exec_mode(self, mode: int):
        abi.call("mllm_set_exec_mode", self._h, int(mode))
        self.exec_mode = int(mode)

    @property
    def execMode(self) -> int:
        """The execution mode the next decode call uses (mllm_get_exec_mode)."""
        return int(abi.lib().mllm_get_exec_mode(self._h))

    @property
    def decodeKernel(self) -> str:
        """The kernel that runs the next decode step (mllm_decode_kernel_name)."""
        return abi.lib().mllm_decode_kernel_name(self._h).decode()

    @property
    def flowVerifyTokens(self) -> int:
        """Most tokens a verify pass runs in the persistent kernel (0: phase kernels)."""
        return int(abi.lib().mllm_flow_verify_tokens(self._h))

    # ---------------------------------------------------------------- debug knobs
    # GpuPetitGPT.debugMaxLayers / debugNoAttn / debugNoMlp / debugMlpTo
    # (webgpu-metal.js:1263-1279): None / False restore the full network.
    def _set_debug(self, **kw):
        d = dict(getattr(self, "_dbg", {"max_layers": None, "no_attn": False, "no_mlp": False, "mlp_to": None}))
        d.update(kw)
        abi.call("mllm_set_debug", self._h, -1 if d["max_layers"] is None else int(d["max_layers"]),
                 int(bool(d["no_attn"])), int(bool(d["no_mlp"])), -1 if d["mlp_to"] is None else int(d["mlp_to"]))
        self._dbg = d

    debugMaxLayers = property(lambda self: getattr(self, "_dbg", {}).get("max_layers"),
                              lambda self, v: self._set_debug(max_layers=v))
    debugNoAttn = property(lambda self: getattr(self, "_dbg", {}).get("no_attn", False),
                           lambda self, v: self._set_debug(no_attn=v))
    debugNoMlp = property(lambda self: getattr(self, "_dbg", {}).get("no_mlp", False),
                          lambda self, v: self._set_debug(no_mlp=v))
    debugMlpTo = property(lambda self: getattr(self, "_dbg", {}).get("mlp_to"),
                          lambda self, v: self._set_debug(mlp_to=v))

    def set_prefill(self, min_tokens: int, chunk_tokens: int = 0):
        """Prompts of at least min_tokens tokens take the batched path (0: never),
        in chunks of at most chunk_tokens (0: the largest)."""
        abi.call("mllm_set_prefill", self._h, int(min_tokens), int(chunk_tokens))

    def last_timing(self):
        """(gpu_ms, tokens) of the last call, from HIP events on the model stream."""
        ms = C.c_float(0)
        n = C.c_int(0)
        abi.call("mllm_last_timing", self._h, C.byref(ms), C.byref(n))
        return float(ms.value), int(n.value)

    N_PHASES = 6  # MLLM_PHASES

    @staticmethod
    def phase_names() -> list:
        return [abi.lib().mllm_phase_name(i).decode() for i in range(PetitGPT.N_PHASES)]

    def profile_decode(self, first: int, n_steps: int) -> dict:
        """Mean microseconds per launch of each decode phase: the kernels' own
        begin/end stamps (hipExtLaunchKernel events on the model stream)."""
        out = (C.c_float * self.N_PHASES)()
        abi.call("mllm_profile_decode", self._h, int(first), int(n_steps), out)
        return {name: float(out[i]) for i, name in enumerate(self.phase_names())}

    @property
    def bytesAllocated(self) -> int:
        return int(abi.lib().mllm_model_device_bytes(self._h))

    @property
    def cacheLen(self) -> int:
        return abi.lib().mllm_cache_len(self._h)

    @cacheLen.setter
    def cacheLen(self, v: int):
        abi.call("mllm_set_cache_len", self._h, int(v))

    def resetCache(self):
        abi.call("mllm_reset_cache", self._h)

    # ---------------------------------------------------------------- forward
    def forwardPrompt(self, ids) -> np.ndarray:
        """infer.js:553-577.  Like the reference, the returned array is the
        model's logits buffer and is overwritten by the next call."""
        a = np.ascontiguousarray(np.asarray(ids, np.int32))
        am = C.c_int32(0)
        abi.call("mllm_forward_prompt", self._h, a.ctypes.data, a.size, self._logits.ctypes.data, C.byref(am))
        self.last_argmax = am.value
        return self._logits

    def forwardDecode(self, token_id: int) -> np.ndarray:
        """infer.js:579-601 (returns the shared logits buffer)."""
        am = C.c_int32(0)
        abi.call("mllm_forward_decode", self._h, int(token_id), self._logits.ctypes.data, C.byref(am))
        self.last_argmax = am.value
        return self._logits

    def forwardVerify(self, ids, want_logits: bool = False):
        """The (k+1)-row pass: argmax per row (and optionally [n][V] logits)."""
        a = np.ascontiguousarray(np.asarray(ids, np.int32))
        am = np.zeros(a.size, np.int32)
        lg = np.zeros((a.size, self.cfg.vocab_size), np.float32) if want_logits else None
        abi.call("mllm_forward_verify", self._h, a.ctypes.data, a.size, am.ctypes.data,
                 lg.ctypes.data if lg is not None else None)
        return [int(v) for v in am], lg

    def decodeChain(self, first: int, n_steps: int, eos_id: int = -1, hist: Optional[List[int]] = None) -> List[int]:
        h = np.ascontiguousarray(np.asarray(hist if hist else [], np.int32))
        out = np.zeros(n_steps, np.int32)
        n = C.c_int(0)
        abi.call("mllm_decode_chain", self._h, int(first), int(n_steps), int(eos_id),
                 h.ctypes.data if h.size else None, h.size, out.ctypes.data, C.byref(n))
        return [int(v) for v in out[:n.value]]

    def gemv(self, name: str, x, y=None) -> np.ndarray:
        """model.gemv(name, x, y) (infer.js:338-346)."""
        t = self.bundle.tensors[name]
        xv = np.ascontiguousarray(x, np.float32)
        yv = y if y is not None else np.empty(t["shape"][0], np.float32)
        abi.call("mllm_model_gemv", self._h, name.encode(), xv.ctypes.data, yv.ctypes.data)
        return yv

    # ---------------------------------------------------------------- generate
    def _pick(self, logits: np.ndarray, out: List[int], device_argmax: int) -> int:
        if self.is_gpt2:
            return argmax_gpt2(logits, out)
        return device_argmax

    def generate(self, ids, maxNewTokens: int = 64, eosId: int = -1, onToken: Optional[Callable] = None,
                 mode: str = "greedy", specK: int = 4, ngram: int = 3, chainChunk: int = 64) -> dict:
        c = self.cfg
        max_seq = c.max_seq_len or 2048
        ids = list(ids)
        max_prompt = max(1, max_seq - maxNewTokens - 1)
        if len(ids) > max_prompt:
            ids = ids[len(ids) - max_prompt:]
        if mode == "spec" and self.is_gpt2:
            raise ValueError("speculative decode is a llama-path feature (webgpu.js:1239-1270)")
        self.resetCache()
        t0 = time.perf_counter()
        logits = self.forwardPrompt(ids)
        ttft = (time.perf_counter() - t0) * 1e3
        out: List[int] = []
        nxt = argmax_gpt2(logits, []) if self.is_gpt2 else self.last_argmax
        out.append(nxt)
        spec_hits = spec_tries = 0
        stop = "max_new_tokens"
        if onToken:
            onToken(nxt, {"phase": "prefill", "ms": ttft})
        if nxt == eosId:
            stop = "eos"
        elif mode == "greedy":
            for _ in range(1, maxNewTokens):
                if len(ids) + len(out) >= c.max_seq_len:
                    break
                lg = self.forwardDecode(nxt)
                nxt = self._pick(lg, out, self.last_argmax)
                out.append(nxt)
                if onToken:
                    onToken(nxt, {"phase": "decode"})
                if nxt == eosId:
                    stop = "eos"
                    break
        elif mode == "chain":
            while len(out) < maxNewTokens:
                if self.cacheLen >= max_seq - 1:
                    stop = "context_limit"
                    break
                n = min(chainChunk, maxNewTokens - len(out), max_seq - 1 - self.cacheLen)
                got = self.decodeChain(out[-1], n, eosId, out if self.is_gpt2 else None)
                for tok in got:
                    out.append(tok)
                    if onToken:
                        onToken(tok, {"phase": "chain"})
                if got and got[-1] == eosId:
                    stop = "eos"
                    break
        elif mode == "spec":
            seq = ids + out
            while len(out) < maxNewTokens:
                if self.cacheLen >= max_seq - 1:
                    break
                x = out[-1]
                pos = self.cacheLen
                room = min(specK, self.max_pass - 1, max_seq - 1 - pos)
                draft = lookup_draft(seq, room, ngram) if room > 0 else []
                spec_tries += 1
                r, _ = self.forwardVerify([x] + draft)
                out.append(r[0])
                seq.append(r[0])
                new_len = pos + 1
                if onToken:
                    onToken(r[0], {"phase": "decode"})
                if r[0] != eosId:
                    for k in range(len(draft)):
                        if r[k] != draft[k] or len(out) >= maxNewTokens:
                            break
                        nxt = r[k + 1]
                        spec_hits += 1
                        out.append(nxt)
                        seq.append(nxt)
                        new_len = pos + 2 + k
                        if onToken:
                            onToken(nxt, {"phase": "spec"})
                        if nxt == eosId:
                            break
                self.cacheLen = new_len
                if out[-1] == eosId:
                    stop = "eos"
                    break
        else:
            raise ValueError(f"unknown mode {mode}")
        return {
            "generatedIds": out,
            "stopReason": stop,
            "ttftMs": ttft,
            "totalMs": (time.perf_counter() - t0) * 1e3,
            "mode": f"hip-{self.kind}-{mode}",
            "specHits": spec_hits,
            "specTries": spec_tries,
        }
