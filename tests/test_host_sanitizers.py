"""Host code under AddressSanitizer and UndefinedBehaviorSanitizer (CPU only).

The CPU oracle (oracle/mllm_oracle.c, oracle/mllm_cpu.c) and the PGW1
converter (microllm-lab_amd/convert/pgw_convert.cc) are built here with
gcc / g++ -fsanitize=address,undefined -fno-sanitize-recover=all and run on
small workloads in child processes; the first report of either sanitizer
ends the child with a nonzero status.  The results must also equal those of
the regular builds bit for bit (the sanitizers add checks, not arithmetic):

- the oracle: quantisers and dequantisers, the js and wasm GEMVs, every
  storage kind of a small llama model and a small GPT-2 model through
  forward_prompt, forward_decode, forward_multi, the named GEMV and generate;
- the converter: the llama and GPT-2 command lines on synthetic HF
  checkpoints (safetensors, sharded and tied variants) and a checkpoint with a
  missing tensor (the error path).

The sanitizer runtimes come from the compiler (gcc -print-file-name); the
child Python process preloads them so that the ctypes-loaded oracle can use
them.  No GPU code is built with a sanitizer.
"""
import os
import shutil
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE = os.path.join(ROOT, "oracle")
CONV = os.path.join(ROOT, "microllm-lab_amd", "convert")
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", "-g"]


def _runtime(name):
    p = subprocess.run(["gcc", f"-print-file-name={name}"], capture_output=True, text=True).stdout.strip()
    return p if os.path.isabs(p) and os.path.exists(p) else None


def _san_env():
    asan, ubsan = _runtime("libasan.so"), _runtime("libubsan.so")
    if not (asan and ubsan):
        pytest.skip("the compiler's sanitizer runtimes are not installed")
    env = dict(os.environ)
    env["LD_PRELOAD"] = f"{asan}:{ubsan}"
    # the interpreter itself leaks by design; the checks that matter here are
    # the out-of-bounds, use-after-free and undefined-behaviour ones
    env["ASAN_OPTIONS"] = "detect_leaks=0:halt_on_error=1:abort_on_error=0"
    env["UBSAN_OPTIONS"] = "halt_on_error=1:print_stacktrace=1"
    return env


@pytest.fixture(scope="module")
def san_oracle(tmp_path_factory):
    if shutil.which("gcc") is None:
        pytest.skip("gcc not found")
    d = tmp_path_factory.mktemp("san_oracle")
    out = str(d / "liboracle_san.so")
    subprocess.run(["gcc", "-O1", "-std=c11", "-fPIC", "-ffp-contract=off", *SAN, "-shared", "-o", out,
                    os.path.join(ORACLE, "mllm_oracle.c"), os.path.join(ORACLE, "mllm_cpu.c"), "-lm"], check=True)
    return out


# The child's workload: every entry point of the oracle that the tests use,
# results saved to an npz.  LIB_PATH is set before the first call loads it.
ORACLE_WORK = r"""
import sys, numpy as np
sys.path[:0] = [{root!r}, {pkg!r}]
from oracle import oracle
oracle.LIB_PATH = {lib!r}
from mllm import pgw
rng = np.random.default_rng(7)
res = {{}}
w = rng.normal(0, 0.02, (48, 96)).astype(np.float32)
x = rng.normal(0, 1, 96).astype(np.float32)
pk, sc = oracle.quant_q4(w)
q8, s8 = oracle.quant_q8g32(w)
qr, sr = oracle.quant_q8row(w)
res["q4"] = pk; res["q4s"] = sc; res["q8"] = q8; res["q8s"] = s8; res["q8r"] = qr; res["q8rs"] = sr
res["dq4"] = oracle.dequant_q4(pk, sc); res["dq8"] = oracle.dequant_q8g32(q8, s8); res["dq8r"] = oracle.dequant_q8row(qr, sr)
for mode in ("js", "wasm"):
    res["g4" + mode] = oracle.gemv_q4(pk, sc, x, mode=mode)
    res["g8" + mode] = oracle.gemv_q8(qr, sr, x, mode=mode)
    res["gf" + mode] = oracle.gemv_f32(w, x, mode=mode)
res["g8g"] = oracle.gemv_q8g32(q8, s8, x)
res["draft"] = np.array(oracle.lookup_draft([1, 2, 3, 4, 1, 2, 3, 9, 9, 1, 2, 3], 4), np.int32)
for arch in ("llama", "gpt2"):
    for kind in (("q4", "q8", "f16", "bf16", "f32", "q8g32") if arch == "llama" else ("q4", "bf16")):
        bundle = pgw.parse_pgw(pgw.make_model(pgw.small_config(arch), seed=3, kind=kind))
        m = oracle.OracleModel(bundle)
        tag = arch + "_" + kind
        res[tag + "_p"] = m.forward_prompt([3, 9, 27, 81, 3, 9]).copy()
        res[tag + "_d"] = m.forward_decode(5).copy()
        res[tag + "_m"] = m.forward_multi([7, 11, 13]).copy()
        res[tag + "_gemv"] = m.gemv("blocks.0.attn.proj", np.ones(bundle.cfg.d_model, np.float32))
        m.reset_cache()
        ids, why = m.generate([3, 9, 27, 81, 3, 9, 27], max_new_tokens=12, eos_id=-1)
        res[tag + "_gen"] = np.array(ids, np.int32)
        m.close()
np.savez({out!r}, **res)
print("done")
"""


def _oracle_run(lib_path, out, env=None):
    code = ORACLE_WORK.format(root=ROOT, pkg=os.path.join(ROOT, "microllm-lab_amd"), lib=lib_path, out=out)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env, timeout=600)
    assert r.returncode == 0 and "done" in r.stdout, r.stderr[-4000:]
    return dict(np.load(out))


def test_oracle_under_asan_and_ubsan(san_oracle, oracle_lib, tmp_path):
    got = _oracle_run(san_oracle, str(tmp_path / "san.npz"), env=_san_env())
    ref = _oracle_run(oracle_lib.LIB_PATH, str(tmp_path / "ref.npz"))
    assert got.keys() == ref.keys()
    for k in ref:
        assert got[k].dtype == ref[k].dtype and np.array_equal(got[k].view(np.uint8), ref[k].view(np.uint8)), k


@pytest.fixture(scope="module")
def san_convert(tmp_path_factory):
    if shutil.which("g++") is None:
        pytest.skip("g++ not found")
    d = tmp_path_factory.mktemp("san_convert")
    out = str(d / "pgw_convert_san")
    subprocess.run(["g++", "-O1", "-std=c++17", *SAN, f"-I{os.path.join(ROOT, 'include')}", "-DPGW_CONVERT_MAIN",
                    os.path.join(CONV, "pgw_convert.cc"), "-o", out], check=True)
    return out


def test_converter_under_asan_and_ubsan(san_convert, tmp_path):
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    import test_pgw_convert as tc  # the checkpoint writers of the converter tests

    if not os.path.exists(tc.BIN):  # the regular converter, for the comparison
        sys.path.insert(0, os.path.join(ROOT, "microllm-lab_amd"))
        import build as mbuild

        mbuild.build_convert()
    env = _san_env()
    env.pop("LD_PRELOAD")  # a linked executable carries its runtimes
    cases = []
    for dtype, shards, tied in (("f32", 1, False), ("bf16", 3, False), ("f16", 2, True)):
        d = str(tmp_path / f"llama_{dtype}_{shards}")
        state = tc.gv.llama_state()
        if tied:
            state = {k: v for k, v in state.items() if k != "lm_head.weight"}
        cfg = tc.llama_config()
        cfg["tie_word_embeddings"] = tied
        tc.save_checkpoint(d, state, cfg, dtype=dtype, shards=shards)
        cases.append(("llama", d, ["--max-seq", "2048"]))
    d = str(tmp_path / "gpt2")
    tc.save_checkpoint(d, tc.gv.gpt2_state(), tc.gpt2_config())
    cases.append(("gpt2", d, ["--max-seq", str(tc.gv.GPT2_MAX_SEQ)]))
    for arch, d, extra in cases:
        a, b = str(tmp_path / "san.bin"), str(tmp_path / "ref.bin")
        r = subprocess.run([san_convert, arch, d, a, *extra], capture_output=True, text=True, env=env, timeout=300)
        assert r.returncode == 0, r.stderr[-4000:]
        subprocess.run([tc.BIN, arch, d, b, *extra], check=True, capture_output=True)
        assert open(a, "rb").read() == open(b, "rb").read(), (arch, d)
    # the error path: a checkpoint without one of its layers' tensors
    d = str(tmp_path / "broken")
    state = tc.gv.llama_state()
    state.pop(next(k for k in state if k.endswith("mlp.down_proj.weight")))
    tc.save_checkpoint(d, state, tc.llama_config())
    r = subprocess.run([san_convert, "llama", d, str(tmp_path / "x.bin")], capture_output=True, text=True, env=env,
                       timeout=300)
    assert r.returncode != 0 and "AddressSanitizer" not in r.stderr and "runtime error" not in r.stderr, r.stderr
