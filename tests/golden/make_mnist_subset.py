"""Writes mnist_034_subset.npz: the first 48 test images of each of the
digits 0, 3 and 4 from the data files the reference's MNIST test holds
(crates/thrml-models/tests/mnist_test_data/sep_images_test_{0,3,4}.npy,
bool [n, 784]), bit-packed.  Run in a container that has the reference
checkout; the GPU tests read only the .npz."""
import os
import sys

import numpy as np

REF = "/root/reference/crates/thrml-models/tests/mnist_test_data"
N = 48


def main():
    out = {}
    for d in (0, 3, 4):
        a = np.load(os.path.join(REF, f"sep_images_test_{d}.npy"), allow_pickle=False)
        assert a.dtype == np.bool_ and a.shape[1] == 784
        out[f"digit{d}"] = np.packbits(a[:N], axis=1)
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "mnist_034_subset.npz")
    np.savez_compressed(path, **out)
    print("wrote", path, {k: v.shape for k, v in out.items()})


if __name__ == "__main__":
    sys.exit(main())
