"""Writes tests/golden/scale_shifts_nabladft.npz from the reference's
``src/maloq/fock_utils/element_scale_shifts_nablaDFT.pt`` (the
scale_shift_data dict training_workflow.py:193-197 loads): ``Z`` [k],
``means`` / ``stds`` [k, 50] (rows in the order of Z) and
``scalar_irrep_indices`` [50].  Read with torch.load(weights_only=True),
which executes nothing from the file.  Run here, where the reference is
mounted:

    python tests/golden/make_scale_shift_fixture.py [/root/reference]
"""
import os
import sys

import numpy as np
import torch


def main(ref_root="/root/reference"):
    path = os.path.join(ref_root, "src", "maloq", "fock_utils", "element_scale_shifts_nablaDFT.pt")
    d = torch.load(path, map_location="cpu", weights_only=True)
    Z = sorted(int(z) for z in d["element_scalar_means"])
    out = {"Z": np.asarray(Z, np.int64),
           "means": np.stack([np.asarray(d["element_scalar_means"][z], np.float64) for z in Z]),
           "stds": np.stack([np.asarray(d["element_scalar_stds"][z], np.float64) for z in Z]),
           "scalar_irrep_indices": np.asarray(d["scalar_irrep_indices"], np.int64)}
    dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), "scale_shifts_nabladft.npz")
    np.savez(dst, **out)
    print(f"wrote {dst}: {len(Z)} elements x {out['means'].shape[1]} scalar columns")


if __name__ == "__main__":
    main(*sys.argv[1:])
