"""Writes the scale-shift fixtures from the reference's element_scale_shifts
files (the scale_shift_data dicts training_workflow.py:193-197 loads):

* ``scale_shifts_nabladft.npz`` from ``element_scale_shifts_nablaDFT.pt``
  (def2-SVP, 50 scalar label columns);
* ``scale_shifts_omol.npz`` from ``element_scale_shifts_omol_csh_58k.pt``
  (def2-TZVPD over the whole dictionary, 4096-column labels, 114 scalar
  columns, f-f on-site pairs included).

Each holds ``Z`` [k], ``means`` / ``stds`` [k, n] (rows in the order of Z)
and ``scalar_irrep_indices`` [n].  Read with torch.load(weights_only=True),
which executes nothing from the file.  Run here, where the reference is
mounted:

    python tests/golden/make_scale_shift_fixture.py [/root/reference]
"""
import os
import sys

import numpy as np
import torch

FILES = {"scale_shifts_nabladft.npz": "element_scale_shifts_nablaDFT.pt",
         "scale_shifts_omol.npz": "element_scale_shifts_omol_csh_58k.pt"}


def main(ref_root="/root/reference"):
    for name, src in FILES.items():
        path = os.path.join(ref_root, "src", "maloq", "fock_utils", src)
        d = torch.load(path, map_location="cpu", weights_only=True)
        Z = sorted(int(z) for z in d["element_scalar_means"])
        out = {"Z": np.asarray(Z, np.int64),
               "means": np.stack([np.asarray(d["element_scalar_means"][z], np.float64) for z in Z]),
               "stds": np.stack([np.asarray(d["element_scalar_stds"][z], np.float64) for z in Z]),
               "scalar_irrep_indices": np.asarray(d["scalar_irrep_indices"], np.int64)}
        dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), name)
        np.savez_compressed(dst, **out)
        print(f"wrote {dst}: {len(Z)} elements x {out['means'].shape[1]} scalar columns")


if __name__ == "__main__":
    main(*sys.argv[1:])
