"""CPU restatement of the Fock matrix <-> label copy (test oracle only).

* ``single_matrix2label``        numpy_single_matrix2label, matrix2labels_kernels.py:1117-1170
* ``single_matrix2label_sparse`` block-list semantics of _single_matrix2label_fp32_sparse,
                                 matrix2labels_kernels.py:689-800 / 1038-1115
"""
from __future__ import annotations

import numpy as np

MAX_ELEMENTS = 100


def single_matrix2label(template, offsets, atomic_numbers, rows, cols, fock, target, forward):
    for r in range(len(rows)):
        i, j = int(rows[r]), int(cols[r])
        blk = (slice(offsets[i], offsets[i + 1]), slice(offsets[j], offsets[j + 1]))
        key = int(atomic_numbers[i]) * MAX_ELEMENTS + int(atomic_numbers[j])
        for rs, cs, os_ in template[key]:
            if forward:
                target[r, os_] = fock[blk][rs, cs].reshape(-1)
            else:
                fock[blk][rs, cs] = target[r, os_].reshape(rs.stop - rs.start, cs.stop - cs.start)


def block_data_offsets(offsets, rows, cols):
    sizes = [(offsets[i + 1] - offsets[i]) * (offsets[j + 1] - offsets[j]) for i, j in zip(rows, cols)]
    return np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64)


def single_matrix2label_sparse(template, offsets, atomic_numbers, rows, cols, data, bdo, target, forward):
    for b in range(len(rows)):
        i, j = int(rows[b]), int(cols[b])
        ni, nj = offsets[i + 1] - offsets[i], offsets[j + 1] - offsets[j]
        blk = data[bdo[b]: bdo[b] + ni * nj].reshape(ni, nj)
        key = int(atomic_numbers[i]) * MAX_ELEMENTS + int(atomic_numbers[j])
        for rs, cs, os_ in template[key]:
            if forward:
                target[b, os_] = blk[rs, cs].reshape(-1)
            else:
                blk[rs, cs] = target[b, os_].reshape(rs.stop - rs.start, cs.stop - cs.start)
