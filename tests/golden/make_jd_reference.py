"""Writes tests/golden/jd_reference.npz: the values of the reference's
``src/maloq/helm/Jd.pt`` (the list of J_l matrices, l = 0..11, that
eSEN_Backbone registers as buffers, esen_osh.py:267-270), as float64 arrays
``J0`` .. ``J11``.

The file is data (tensors), read with ``torch.load(..., weights_only=True)``,
which executes nothing from the file.  Run here, where the reference is
mounted:

    python tests/golden/make_jd_reference.py [/root/reference]
"""
import os
import sys

import numpy as np
import torch


def main(ref_root="/root/reference"):
    path = os.path.join(ref_root, "src", "maloq", "helm", "Jd.pt")
    jd = torch.load(path, map_location="cpu", weights_only=True)
    out = {f"J{l}": np.asarray(j.double().numpy()) for l, j in enumerate(jd)}
    dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), "jd_reference.npz")
    np.savez(dst, **out)
    print(f"wrote {dst}: {len(out)} matrices")


if __name__ == "__main__":
    main(*sys.argv[1:])
