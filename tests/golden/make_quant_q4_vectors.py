"""Write tests/golden/quant_q4_vectors.npz from the reference's own quantiser.

quant_q4 (tools/convert_hf_to_pgw.py:18-34) is the one function on the path
whose exact behaviour (NumPy float32 division by a Python float, np.rint
ties-to-even, the +amax clip to 15) no closed form here pins bit for bit, so
its outputs are recorded once from the reference code itself.

Run in the build container only (the reference is not present on the GPU box):
    python tests/golden/make_quant_q4_vectors.py [/root/reference]
The reference module is loaded from its file; nothing of it is copied here --
only the input matrices and the packed/scale outputs are stored.
"""
from __future__ import annotations

import importlib.util
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def load_reference_quant(ref_root: str):
    path = os.path.join(ref_root, "tools", "convert_hf_to_pgw.py")
    spec = importlib.util.spec_from_file_location("_ref_convert_hf_to_pgw", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod.quant_q4


def cases():
    rng = np.random.default_rng(20261201)
    out = {}
    out["normal_002"] = (rng.standard_normal((6, 64), dtype=np.float32) * np.float32(0.02))
    out["normal_1"] = rng.standard_normal((5, 96), dtype=np.float32)
    out["uniform_wide"] = rng.uniform(-3e3, 3e3, size=(4, 64)).astype(np.float32)
    # exact half-way points: amax 8 -> sc 1 -> x/sc lands on k + 0.5 (ties to even)
    ties = np.zeros((2, 64), np.float32)
    ties[0, :32] = np.array([8.0] + [(k % 16) - 7.5 for k in range(31)], np.float32)
    ties[0, 32:] = np.array([-8.0] + [0.5 * (k - 15) for k in range(31)], np.float32)
    ties[1, :32] = np.array([4.0] + [(k % 8) * 0.25 - 1.75 for k in range(31)], np.float32)  # sc 0.5
    ties[1, 32:] = np.array([16.0] + [k - 15.0 for k in range(31)], np.float32)  # sc 2
    out["ties"] = ties
    # zero group -> sc 1, every nibble 8; +amax -> 16 clipped to 15; -amax -> 0
    edge = np.zeros((3, 64), np.float32)
    edge[1, :32] = np.linspace(-1, 1, 32, dtype=np.float32)
    edge[1, 32:] = -np.linspace(-0.3, 0.7, 32, dtype=np.float32)
    edge[2, :32] = np.float32(1e-40) * np.arange(32, dtype=np.float32)  # subnormal amax
    edge[2, 32:] = np.float32(1e30) * np.sin(np.arange(32, dtype=np.float32))
    out["edges"] = edge
    # values whose float32 quotient rounds onto .5 while the float64 one does not
    near = np.zeros((2, 32), np.float32)
    amax = np.float32(0.7)
    near[0, 0] = amax
    sc32 = np.float32(np.float64(amax) / 8.0)
    for k in range(1, 32):
        target = np.float32((k % 15) - 7 + 0.5) * sc32
        near[0, k] = np.nextafter(target, np.float32(np.inf) if k % 2 else np.float32(-np.inf))
    near[1] = rng.standard_normal(32).astype(np.float32)
    out["near_ties"] = near
    return out


def main():
    ref_root = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    quant = load_reference_quant(ref_root)
    arrays = {}
    for name, mat in cases().items():
        packed, scales = quant(mat)
        arrays[f"{name}__x"] = mat
        arrays[f"{name}__packed"] = packed
        arrays[f"{name}__scales"] = scales
    path = os.path.join(HERE, "quant_q4_vectors.npz")
    np.savez_compressed(path, **arrays)
    print(f"wrote {path} ({len(arrays) // 3} cases)")


if __name__ == "__main__":
    main()
