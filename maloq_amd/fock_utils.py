"""The callers' hooks around the basis transform, on the GPU.

Mirrors the reference's label-side helpers (same names, arguments and
results) with HIP kernels of ``libmaloq_hip.so`` doing the per-element work:

* :class:`ScaleShift` -- ``Fock_Targets.scale_shift_node_blocks`` and
  ``undo_scale_shift`` (fock_utils/fock_targets_batched.py:1093-1115,
  :1157-1194): the l = 0 label columns of every node row shifted by the
  per-element means of ``scale_shift_data`` (``maloq_label_scalar_shift``);
* :func:`make_targets` -- the per-molecule body of ``Fock_Targets.make_targets``
  (fock_targets_batched.py:335-464): rows ``[edges..., on-site...]``, the fused
  Fock -> irreps transform, the node / edge split, the scale-shift;
* :func:`create_label_unpadding_mask` -- fock_targets_batched.py:1012-1080
  (``maloq_label_mask``);
* :func:`sort_by_m` -- fock_utils/utils_orca_out.py:402-465: ORCA / pyscf <->
  e3nn m-order of a Hamiltonian as one signed-permutation gather
  (``maloq_signed_permute``);
* :func:`sparse_block_matrix_to_scipy_csr` -- matrix2labels_kernels.py:16-42:
  the CSR arrays built on the GPU (``maloq_blocks_to_csr``), then handed to
  scipy.
"""
from __future__ import annotations

import numpy as np
import torch

from . import _lib

MAX_ELEMENTS = 100


def _i32(a, device):
    return torch.as_tensor(np.asarray(a, dtype=np.int32), device=device).contiguous()


# ------------------------------------------------------------ scale-shift
class ScaleShift:
    """Device tables of a ``scale_shift_data`` dict ({"element_scalar_means":
    {Z: [means]}, "element_scalar_stds": ..., "scalar_irrep_indices": [...]},
    as training_workflow.py:193-197 builds it; ``spin_string`` "_alpha" /
    "_beta" selects the open-shell means)."""

    def __init__(self, scale_shift_data, device, spin_string=""):
        means = scale_shift_data["element_scalar_means" + spin_string]
        idx = [int(i) for i in scale_shift_data["scalar_irrep_indices"]]
        if len(set(idx)) != len(idx):
            # one writer per label element: the kernel updates each (row, column) once
            raise ValueError("scalar_irrep_indices must not repeat a column")
        if min(idx, default=0) < 0:
            raise ValueError("scalar_irrep_indices must be non-negative")
        if isinstance(means, dict):
            max_z = max(int(z) for z in means)
            table = np.zeros((max_z + 1, len(idx)), np.float32)
            for z, v in means.items():
                v = np.asarray(v, dtype=np.float32).reshape(-1)
                if v.shape[0] != len(idx):
                    raise ValueError(f"element {z}: {v.shape[0]} means for {len(idx)} scalar columns")
                table[int(z)] = v
        else:
            table = np.asarray(torch.as_tensor(means).float().cpu().numpy(), np.float32)
            if table.ndim != 2 or table.shape[1] != len(idx):
                raise ValueError(f"means table must be [max Z + 1, {len(idx)}], got {tuple(table.shape)}")
        self.device = torch.device(device)
        self.means = torch.from_numpy(table).to(self.device)
        self.cols = _i32(idx, self.device)
        self.max_z = table.shape[0] - 1
        self.ncols = len(idx)
        self.max_col = max(idx) if idx else -1

    def _apply(self, labels, atomic_numbers, sign):
        _lib.require_cuda(labels)
        if labels.dtype != torch.float32 or labels.dim() != 2 or labels.stride(1) != 1:
            raise ValueError("node labels must be a float32 [N, T] tensor with unit column stride")
        Z = np.asarray(atomic_numbers.cpu() if torch.is_tensor(atomic_numbers) else atomic_numbers)
        if len(Z) != labels.shape[0]:
            raise ValueError("one atomic number per node row")
        if len(Z) and (Z.min() < 0 or Z.max() > self.max_z):
            raise IndexError(f"atomic numbers outside the scale-shift table (0..{self.max_z})")
        if self.max_col >= labels.shape[1]:
            raise IndexError("scalar irrep index outside the label rows")
        z = _i32(Z, labels.device)
        _lib.call("maloq_label_scalar_shift", _lib.ptr(labels), labels.stride(0), labels.shape[0], _lib.ptr(z),
                  _lib.ptr(self.means), _lib.ptr(self.cols), self.ncols, float(sign), _lib.stream_of(labels.device))
        return labels

    def scale_shift_node_blocks(self, node_blocks, node_atomic_numbers):
        """In place, as the reference (fock_targets_batched.py:1113)."""
        return self._apply(node_blocks, node_atomic_numbers, -1.0)

    def undo_scale_shift(self, node_blocks, atomic_numbers):
        """A new tensor, as unscale_shift_node_blocks (:1165 clones)."""
        return self._apply(node_blocks.clone(), atomic_numbers, 1.0)


# ------------------------------------------------------------ make_targets
def make_targets(decomp, fock_matrix, atomic_numbers, neighbour_list, orbitals_per_atom, orbital_template,
                 scale_shift=None, plan=None):
    """(node_labels [spins, N, T], edge_labels [spins, E, T]) of one molecule,
    as Fock_Targets.make_targets (fock_targets_batched.py:388-453): the rows are
    the edges then the on-site pairs, gathered by template and transformed to
    irreps in one launch per spin (``decomp``: a HipE3TensorDecomp), split, and
    the node rows' l = 0 columns shifted (``scale_shift``: a ScaleShift, or a
    pair for the alpha / beta spins of an open-shell fock_matrix [2, n, n])."""
    src, dst = (np.asarray(a) for a in neighbour_list)
    Z = np.asarray(atomic_numbers)
    num_atoms, num_edges = len(Z), len(src)
    rows = np.concatenate([src, np.arange(num_atoms)]).astype(np.int32)
    cols = np.concatenate([dst, np.arange(num_atoms)]).astype(np.int32)
    off = np.concatenate([[0], np.cumsum(orbitals_per_atom)]).astype(np.int32)
    open_shell = fock_matrix.dim() == 3
    spins = 2 if open_shell else 1
    T = decomp.total_h_dim
    node = torch.zeros(spins, num_atoms, T, device=fock_matrix.device)
    edge = torch.zeros(spins, num_edges, T, device=fock_matrix.device)
    for s in range(spins):
        H = fock_matrix[s] if open_shell else fock_matrix
        lab = decomp.fock_to_irreps(H, off, Z, rows, cols, orbital_template, plan=plan)
        node[s] = lab[num_edges:]
        edge[s] = lab[:num_edges]
        if scale_shift is not None:
            ss = scale_shift[s] if isinstance(scale_shift, (tuple, list)) else scale_shift
            ss.scale_shift_node_blocks(node[s], Z)
    return node, edge


# ------------------------------------------------------------ padding mask
_MASK_TABLES: dict = {}


def _template_kinds(orbital_template, target_len):
    key = (id(orbital_template), target_len)
    hit = _MASK_TABLES.get(key)
    if hit is not None and hit[0] is orbital_template:
        return hit[1], hit[2]
    pair_kind = np.full(MAX_ELEMENTS * MAX_ELEMENTS, -1, np.int32)
    covers = []
    for k, entries in enumerate(orbital_template):
        if not entries:
            continue
        cov = np.zeros(target_len, np.uint8)
        for _, _, out in entries:
            cov[out] = 1
        pair_kind[k] = len(covers)
        covers.append(cov)
    cover = np.stack(covers) if covers else np.zeros((1, target_len), np.uint8)
    _MASK_TABLES[key] = (orbital_template, pair_kind, cover)
    return pair_kind, cover


def create_label_unpadding_mask(orbital_template, atomic_numbers, src, dst, target_len, device):
    """(edge_mask [E, T], node_mask [N, T]) bool: True on the label columns the
    orbital template fills for each row's element pair (rows = edges, then
    on-site pairs; fock_targets_batched.py:1052-1080)."""
    Z = np.asarray(atomic_numbers)
    if len(Z) and (Z.min() < 0 or Z.max() >= MAX_ELEMENTS):
        raise IndexError("atomic numbers must lie in 0..99")
    num_atoms, num_edges = len(Z), len(src)
    if len(dst) != num_edges:
        raise ValueError("src and dst must have one entry per edge")
    if num_edges and (min(np.min(src), np.min(dst)) < 0 or max(np.max(src), np.max(dst)) >= num_atoms):
        raise IndexError("edge endpoints outside 0..num_atoms-1")
    rows = np.concatenate([np.asarray(src), np.arange(num_atoms)])
    cols = np.concatenate([np.asarray(dst), np.arange(num_atoms)])
    pair_kind, cover = _template_kinds(orbital_template, target_len)
    dev = torch.device(device)
    mask = torch.empty(num_edges + num_atoms, target_len, dtype=torch.uint8, device=dev)
    if mask.numel():
        # every device argument bound to a name until the launch is enqueued: a
        # temporary passed only through _lib.ptr() is freed before the call, and
        # the caching allocator hands its block to the next allocation
        r_d, c_d, z_d = _i32(rows, dev), _i32(cols, dev), _i32(Z, dev)
        pk_d, cov_d = _i32(pair_kind, dev), torch.from_numpy(cover).to(dev)
        _lib.call("maloq_label_mask", _lib.ptr(r_d), _lib.ptr(c_d), _lib.ptr(z_d), _lib.ptr(pk_d), _lib.ptr(cov_d),
                  target_len, num_edges + num_atoms, _lib.ptr(mask), _lib.stream_of(dev))
    mask = mask.bool()
    return mask[:num_edges], mask[num_edges:]


# ---------------------------------------------------------------- m order
_M_TO_M = {"orca": {0: [0], 1: [2, 0, 1], 2: [4, 2, 0, 1, 3], 3: [6, 4, 2, 0, 1, 3, 5],
                    4: [8, 6, 4, 2, 0, 1, 3, 5, 7]},
           "pyscf": {0: [0], 1: [2, 0, 1], 2: [0, 1, 2, 3, 4], 3: [0, 1, 2, 3, 4, 5, 6], 4: list(range(9))}}
_REFLECTION = {0: [1], 1: [1, 1, 1], 2: [1, 1, 1, 1, 1], 3: [-1, 1, 1, 1, 1, 1, -1],
               4: [-1, -1, 1, 1, 1, 1, 1, -1, -1]}


def m_order_permutation(orbital_basis, atomic_numbers, direction="orca_to_e3nn"):
    """(src [n] int32, sign [n] fp32) with sort_by_m(H)[i][j] = sign[i] sign[j]
    H[src[i]][src[j]]: per shell of angular momentum l, the signed permutation
    R P (orca_to_e3nn, e3nn_to_pyscf) or P^T R (e3nn_to_orca, pyscf_to_e3nn)
    of utils_orca_out.py:415-460."""
    if direction in ("orca_to_e3nn", "e3nn_to_orca"):
        table = _M_TO_M["orca"]
    elif direction in ("e3nn_to_pyscf", "pyscf_to_e3nn"):
        table = _M_TO_M["pyscf"]
    else:
        raise NotImplementedError(f"Direction {direction} not implemented")
    forward = direction in ("orca_to_e3nn", "e3nn_to_pyscf")
    src, sign = [], []
    b0 = 0
    for z in atomic_numbers:
        for l in orbital_basis[int(z)]:
            l = int(l) % 10
            perm, refl = table[l], _REFLECTION[l]
            n = 2 * l + 1
            for a in range(n):
                if forward:        # (R P)[a, perm[a]] = refl[a]
                    src.append(b0 + perm[a])
                    sign.append(refl[a])
                else:              # (P^T R)[a, b] = refl[b] where perm[b] = a
                    b = perm.index(a)
                    src.append(b0 + b)
                    sign.append(refl[b])
            b0 += n
    return np.asarray(src, np.int32), np.asarray(sign, np.float32)


_PERM_CACHE: dict = {}


def _signed_permutation_on(orbital_basis, atomic_numbers, direction, dev):
    """m_order_permutation as device arrays, kept per (basis, atomic numbers,
    direction, device): an eval loop over molecules of repeated composition
    builds and uploads each permutation once."""
    key = (tuple(sorted((int(z), tuple(int(l) for l in ls)) for z, ls in orbital_basis.items())),
           tuple(int(z) for z in atomic_numbers), direction, str(dev))
    hit = _PERM_CACHE.get(key)
    if hit is None:
        src, sign = m_order_permutation(orbital_basis, atomic_numbers, direction)
        if len(_PERM_CACHE) > 256:
            _PERM_CACHE.clear()
        hit = _PERM_CACHE[key] = (_i32(src, dev), torch.from_numpy(sign).to(dev))
    return hit


def sort_by_m(hamiltonian, orbital_basis, atomic_numbers, direction="orca_to_e3nn"):
    """The Hamiltonian [n, n] (fp32, on the GPU) with every shell's m-components
    reordered and reflected (utils_orca_out.py:402-465); a new tensor."""
    _lib.require_cuda(hamiltonian)
    if hamiltonian.dtype != torch.float32 or hamiltonian.dim() != 2 or hamiltonian.stride(1) != 1:
        raise ValueError("hamiltonian must be a float32 [n, n] tensor with unit column stride")
    dev = hamiltonian.device
    src_d, sign_d = _signed_permutation_on(orbital_basis, atomic_numbers, direction, dev)
    n = hamiltonian.shape[0]
    if src_d.shape[0] != n or hamiltonian.shape[1] != n:
        raise ValueError(f"the basis has {src_d.shape[0]} functions, the matrix is {tuple(hamiltonian.shape)}")
    out = torch.empty(n, n, device=dev, dtype=torch.float32)
    _lib.call("maloq_signed_permute", _lib.ptr(hamiltonian), n, hamiltonian.stride(0), _lib.ptr(src_d),
              _lib.ptr(sign_d), _lib.ptr(out), n, _lib.stream_of(dev))
    return out


# ------------------------------------------------------------- CSR export
def sparse_block_matrix_to_csr_arrays(sparse_matrix):
    """(indptr, indices, data) on the GPU of the CSR form of a SparseBlockMatrix
    (int64, int64, fp32); column indices ascending in every row."""
    data = sparse_matrix.data
    _lib.require_cuda(data)
    dev = data.device
    rows = sparse_matrix.fock_block_rows.to(device=dev, dtype=torch.int64)
    cols = sparse_matrix.fock_block_cols.to(device=dev, dtype=torch.int64)
    off = sparse_matrix.fock_block_offsets.to(device=dev, dtype=torch.int64)
    bdo = sparse_matrix.block_data_offsets.to(device=dev, dtype=torch.int64).contiguous()
    n = int(off[-1].item())
    nb = int(rows.shape[0])
    natoms = off.shape[0] - 1
    if cols.shape[0] != nb or bdo.shape[0] < nb:
        raise ValueError("one block row, column and data offset per block")
    if nb and (min(int(rows.min()), int(cols.min())) < 0 or max(int(rows.max()), int(cols.max())) >= natoms):
        raise IndexError("block atoms outside 0..num_atoms-1")
    ni, nj = off[rows + 1] - off[rows], off[cols + 1] - off[cols]
    if nb and (int(bdo[:nb].min()) < 0 or int((bdo[:nb] + ni * nj).max()) > data.numel()):
        raise IndexError("a block's data runs outside the data array")
    # columns of the blocks left of each block in its block row (blocks of one
    # row atom in column-atom order)
    keys = rows * (off.shape[0]) + cols
    order = torch.argsort(keys)
    if nb > 1 and bool((keys[order][1:] == keys[order][:-1]).any()):
        raise ValueError("blocks overlap: a (row atom, column atom) pair appears twice")
    ro, njo = rows[order], nj[order]
    run = torch.cumsum(njo, 0) - njo
    first = torch.zeros_like(run)
    starts = torch.ones(nb, dtype=torch.bool, device=dev)
    if nb > 1:
        starts[1:] = ro[1:] != ro[:-1]
    first[starts] = run[starts]
    first = torch.cummax(torch.where(starts, first, torch.zeros_like(first)), 0).values
    coloff = torch.empty(nb, dtype=torch.int64, device=dev)
    coloff[order] = run - first
    # row lengths: the columns of every block of the row's atom
    atom_len = torch.zeros(natoms, dtype=torch.int64, device=dev).index_add_(0, rows, nj)
    atom_of_row = torch.repeat_interleave(torch.arange(natoms, device=dev), off[1:] - off[:-1])
    indptr = torch.zeros(n + 1, dtype=torch.int64, device=dev)
    indptr[1:] = torch.cumsum(atom_len[atom_of_row], 0)
    nnz = int(indptr[-1].item())
    csr_data = torch.empty(nnz, dtype=torch.float32, device=dev)
    csr_idx = torch.empty(nnz, dtype=torch.int64, device=dev)
    data_d = data.float().contiguous()                 # alive across the launch
    rows_d, cols_d, off_d = rows.int().contiguous(), cols.int().contiguous(), off.int().contiguous()
    _lib.call("maloq_blocks_to_csr", _lib.ptr(data_d), _lib.ptr(bdo), _lib.ptr(rows_d), _lib.ptr(cols_d),
              _lib.ptr(off_d), _lib.ptr(coloff), _lib.ptr(indptr), nb, _lib.ptr(csr_data), _lib.ptr(csr_idx),
              _lib.stream_of(dev))
    return indptr, csr_idx, csr_data


def sparse_block_matrix_to_scipy_csr(sparse_matrix):
    """scipy.sparse.csr_matrix of a SparseBlockMatrix (matrix2labels_kernels.py:16-42),
    for writing to disk."""
    import scipy.sparse as sp
    indptr, idx, data = sparse_block_matrix_to_csr_arrays(sparse_matrix)
    n = indptr.shape[0] - 1
    return sp.csr_matrix((data.cpu().numpy(), idx.cpu().numpy(), indptr.cpu().numpy()), shape=(n, n))
