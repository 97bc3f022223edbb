"""Writes tests/golden/lut4_vectors.npz: input matrices and the reference's palettize_lut4 output
(packed indices + fp16 codebook) for them.

palettize_lut4 (aneforge/_blob.py:28-43: np.quantile edges, 20 Lloyd iterations, argmin ties,
low-nibble-first packing) has no closed form, known-answer test or stored vector in the
reference, so its output is recorded here from the reference function itself.  Run in the build
container only (the reference tree is not on the GPU box):

    python tests/golden/make_lut4_vectors.py /root/reference

The reference module is loaded by file path (it imports only numpy and struct); nothing of it
is copied into this repository, only the vectors it produced."""
import importlib.util
import os
import sys

import numpy as np


def cases():
    rng = np.random.default_rng(1234)
    yield "normal_8x64", rng.standard_normal((8, 64)).astype(np.float32)
    yield "normal_odd_6x33", rng.standard_normal((6, 33)).astype(np.float32)
    yield "uniform_16x48", rng.uniform(-2.0, 2.0, (16, 48)).astype(np.float32)
    # heavy ties: few distinct values, so argmin ties and empty clusters occur
    yield "ties_4x32", rng.integers(-3, 4, (4, 32)).astype(np.float32)
    yield "fp16_grid_32x16", rng.standard_normal((32, 16)).astype(np.float16).astype(np.float32)


def main(ref_root):
    path = os.path.join(ref_root, "aneforge", "_blob.py")
    spec = importlib.util.spec_from_file_location("reference_blob", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    out = {}
    for name, W in cases():
        packed, cb = mod.palettize_lut4(W)
        out[f"{name}__W"] = W
        out[f"{name}__packed"] = np.frombuffer(packed, np.uint8).reshape(W.shape[0], -1).copy()
        out[f"{name}__codebook"] = np.frombuffer(cb, np.float16).copy()
    dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lut4_vectors.npz")
    np.savez_compressed(dst, **out)
    print(f"wrote {dst}: {len(out) // 3} cases")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
