"""Writes tests/golden/pack_rows.npz: packer inputs and expected outputs.

Inputs are slices of the reference's own head weights (W^T rows of linear_8.w_0 of
PP-OCRv6_small_rec and linear_1.w_0 of PP-OCRv6_tiny_rec, read from the safetensors
files in the reference's models/ directory) plus hand-made special rows.  Expected q and
scales come from the independent numpy restatement (tests/packref.py) and are checked
against the C oracle before writing.  Run in a container where the reference is mounted:
    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np
from safetensors.numpy import load_file

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "tests"))
sys.path.insert(0, ROOT)
from packref import pack_numpy  # noqa: E402
from oracle import oracle as orc  # noqa: E402

MODELS = "/root/reference/models"


def rows_of(path, name, take):
    w = load_file(path)[name]
    w_t = np.ascontiguousarray(w.T)
    return np.ascontiguousarray(w_t[take])


def main():
    small = rows_of(os.path.join(MODELS, "PP-OCRv6_small_rec.safetensors"), "linear_8.w_0",
                    np.r_[0:256, 9000:9128, 18710 - 128:18710])
    tiny = rows_of(os.path.join(MODELS, "PP-OCRv6_tiny_rec.safetensors"), "linear_1.w_0",
                   np.r_[0:128, 6906 - 128:6906])
    special = np.zeros((8, 120), np.float32)
    special[1, :] = 5e-9
    special[2, 3] = 5.0
    special[3, 7] = -5.0
    special[3, 0] = 0.01
    special[4, :] = np.float32(1e-8)
    special[5, :9] = [127, 2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 126.5, -0.49999997]
    special[6, 0] = np.nan
    special[6, 1] = 0.5
    special[7, :] = np.linspace(-1, 1, 120, dtype=np.float32)
    out = {}
    for key, w in (("small_rec", small), ("tiny_rec", tiny), ("special", special)):
        q, s = pack_numpy(w)
        qo, so = orc.pack_int8(w)
        assert np.array_equal(q, qo) and np.array_equal(s.view(np.uint32), so.view(np.uint32)), key
        out[f"{key}_w_t"] = w
        out[f"{key}_q"] = q
        out[f"{key}_scales"] = s
    np.savez_compressed(os.path.join(HERE, "pack_rows.npz"), **out)
    print("wrote", os.path.join(HERE, "pack_rows.npz"))


if __name__ == "__main__":
    main()
