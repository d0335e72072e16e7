"""HIP Fock-matrix <-> label copy: drop-in for the CuPy wrappers.

``hip_single_matrix2label`` / ``hip_single_matrix2label_sparse`` keep the
arguments and in-place semantics of ``cupy_single_matrix2label`` /
``cupy_single_matrix2label_sparse`` (src/maloq/fock_utils/matrix2labels_kernels.py:
946-1115): ``forward=True`` fills ``target`` from the matrix, ``forward=False``
writes the covered entries of the matrix from ``target``.  Tensors are torch
tensors on the GPU instead of CuPy arrays; index arrays may be numpy or torch.
A pure copy: results are bit-exact.
"""
from __future__ import annotations

from typing import NamedTuple

import numpy as np
import torch

from . import _lib
from .basis_transform import _check_pairs_on_host
from .tensor_decomp import MAX_ELEMENTS


class SparseBlockMatrix(NamedTuple):
    """Block list of a sparse Fock matrix (matrix2labels_kernels.py:43-48)."""

    data: torch.Tensor                # (total_elements,) float32, block b row-major at block_data_offsets[b]
    block_data_offsets: torch.Tensor  # (num_blocks + 1,) int64
    fock_block_rows: torch.Tensor     # (num_blocks,) int32, atom index of the block's rows
    fock_block_cols: torch.Tensor     # (num_blocks,) int32
    fock_block_offsets: torch.Tensor  # (num_atoms + 1,) int32


_PACKED: dict = {}


def pack_orbital_template(orbital_template, device):
    """CSR of the template: ptr [100*100+1], entries [n, 5] = (r0, r1, c0, c1, out0)."""
    key = (id(orbital_template), str(device))
    hit = _PACKED.get(key)
    if hit is not None and hit[0] is orbital_template:
        return hit[1]
    ptr = np.zeros(MAX_ELEMENTS * MAX_ELEMENTS + 1, np.int32)
    ent = []
    for k, lst in enumerate(orbital_template):
        for rs, cs, os_ in lst:
            ent.append((rs.start, rs.stop, cs.start, cs.stop, os_.start))
        ptr[k + 1] = len(ent)
    ent = np.asarray(ent if ent else [(0, 0, 0, 0, 0)], np.int32).reshape(-1)
    packed = (torch.as_tensor(ptr, device=device), torch.as_tensor(ent, device=device))
    _PACKED[key] = (orbital_template, packed)
    return packed


def _dev_i32(a, device):
    if torch.is_tensor(a):
        return a.to(device=device, dtype=torch.int32).contiguous()
    return torch.as_tensor(np.ascontiguousarray(np.asarray(a, dtype=np.int32)), device=device)


def hip_single_matrix2label(orbital_templates, fock_block_offsets, idx_to_atomic_number,
                           fock_block_rows, fock_block_cols, fock_matrix, target,
                           orbital_template_ptrs=None, forward=True):
    """In-place gather (forward) or scatter (inverse) between a dense [n, n]
    matrix and label rows [R, T]; row r is atom pair (rows[r], cols[r])."""
    if target.dtype != fock_matrix.dtype:
        raise AssertionError("target and fock_matrix dtypes differ")
    if target.dtype != torch.float32:
        raise ValueError("Unsupported dtype for targets. Only float32 is supported.")
    _lib.require_cuda(fock_matrix, target)
    if fock_matrix.dim() != 2 or fock_matrix.stride(1) != 1 or target.stride(1) != 1:
        raise ValueError("fock_matrix and target must be 2-D with unit column stride")
    _check_pairs_on_host(fock_block_offsets, idx_to_atomic_number, fock_block_rows, fock_block_cols)
    dev = target.device
    tptr, tent = pack_orbital_template(orbital_templates, dev)
    rows = _dev_i32(fock_block_rows, dev)
    cols = _dev_i32(fock_block_cols, dev)
    off = _dev_i32(fock_block_offsets, dev)
    Z = _dev_i32(idx_to_atomic_number, dev)
    R = int(rows.shape[0])
    if R > target.shape[0]:
        raise ValueError("target has fewer rows than atom pairs")
    _lib.call("maloq_matrix2label", _lib.ptr(fock_matrix), fock_matrix.stride(0), None, _lib.ptr(off),
              _lib.ptr(Z), _lib.ptr(rows), _lib.ptr(cols), R, _lib.ptr(tptr), _lib.ptr(tent),
              _lib.ptr(target), target.stride(0), 1 if forward else 0, _lib.stream_of(dev))


def block_data_offsets_for(fock_block_offsets, rows, cols) -> torch.Tensor:
    off = fock_block_offsets.to(torch.int64)
    r = rows.to(torch.int64)
    c = cols.to(torch.int64)
    sizes = (off[r + 1] - off[r]) * (off[c + 1] - off[c])
    return torch.cat([torch.zeros(1, dtype=torch.int64, device=sizes.device), torch.cumsum(sizes, 0)])


def hip_single_matrix2label_sparse(orbital_templates, fock_block_offsets, idx_to_atomic_number,
                                  fock_block_rows, fock_block_cols, target, orbital_template_ptrs=None,
                                  forward=True, sparse_matrix=None, block_data_offsets=None):
    """Block-list twin (matrix2labels_kernels.py:1038-1115): label row b <-> block b."""
    if target.dtype != torch.float32:
        raise AssertionError("sparse kernel only implements fp32")
    _lib.require_cuda(target)
    _check_pairs_on_host(fock_block_offsets, idx_to_atomic_number, fock_block_rows, fock_block_cols)
    dev = target.device
    rows = _dev_i32(fock_block_rows, dev)
    cols = _dev_i32(fock_block_cols, dev)
    off = _dev_i32(fock_block_offsets, dev)
    Z = _dev_i32(idx_to_atomic_number, dev)
    if block_data_offsets is None:
        block_data_offsets = block_data_offsets_for(off, rows, cols)
    bdo = block_data_offsets.to(device=dev, dtype=torch.int64).contiguous()
    total = int(bdo[-1].item()) if bdo.numel() else 0
    if forward:
        assert sparse_matrix is not None, "sparse_matrix (with populated .data) is required when forward=True"
        data = sparse_matrix.data.contiguous()
        assert data.numel() == total, "sparse_matrix.data doesn't match the current block structure"
    else:
        data = torch.zeros(total, device=dev, dtype=torch.float32)
    tptr, tent = pack_orbital_template(orbital_templates, dev)
    R = int(rows.shape[0])
    _lib.call("maloq_matrix2label", _lib.ptr(data), 0, _lib.ptr(bdo), _lib.ptr(off), _lib.ptr(Z),
              _lib.ptr(rows), _lib.ptr(cols), R, _lib.ptr(tptr), _lib.ptr(tent), _lib.ptr(target),
              target.stride(0), 1 if forward else 0, _lib.stream_of(dev))
    return SparseBlockMatrix(data=data, block_data_offsets=bdo, fock_block_rows=rows,
                             fock_block_cols=cols, fock_block_offsets=off)
