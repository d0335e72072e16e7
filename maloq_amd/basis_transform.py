"""HIP basis-transform backend: drop-in for BalancedTritonE3TensorDecompL2.

``HipE3TensorDecomp(base_decomp)`` keeps the backend protocol of the reference
(src/maloq/fock_utils/basis_transform_triton_backend.py:177-265, 1255-1438):

* ``get_H(net_out[R, T]) -> H[R, T]``, differentiable in ``net_out`` (the
  backward is the adjoint, ``grad @ W_global^T``, as TritonGetHFunctionL2,
  basis_transform_triton_backend.py:1064-1073);
* ``get_net_out(H[R, T]) -> net_out[R, T]`` (= ``H @ W_global_inv``);
* ``required_irreps_out`` forwarded from the base object.

On top of it, ``fock_to_irreps`` / ``irreps_to_fock`` fuse the shell-pair
gather of the Fock matrix (cupy_single_matrix2label, matrix2labels_kernels.py:
946-1115) with the CG contraction, for dense matrices and for the
``SparseBlockMatrix`` block list.  All index work is integer and exact; the
per-row arithmetic is the block-local dot product of the dense reference
restricted to its non-zero blocks.

``make_basis_transform(base, backend)`` is the 'hip' value of the
``basis_transform_backend`` switch (fock_targets_batched.py:152-165).
"""
from __future__ import annotations

import numpy as np
import torch

from . import _lib
from .tensor_decomp import MAX_ELEMENTS


def _i32(a, device):
    if torch.is_tensor(a):
        return a.to(device=device, dtype=torch.int32).contiguous()
    return torch.as_tensor(np.ascontiguousarray(np.asarray(a, dtype=np.int32)), device=device)


def _check_pairs_on_host(off, Z, rows, cols):
    """Range checks of the atom-pair structure where it is still on the host
    (numpy or CPU tensors, as the per-molecule callers hold it): the kernels
    index with these values unchecked.  Device tensors are the caller's
    responsibility (checking them would read them back, a sync per call)."""
    arrs = (off, Z, rows, cols)
    if any(torch.is_tensor(a) and a.is_cuda for a in arrs):
        return
    off, Z, rows, cols = (np.asarray(a.numpy() if torch.is_tensor(a) else a).reshape(-1) for a in arrs)
    natoms = off.shape[0] - 1
    if natoms < 0 or Z.shape[0] < natoms:
        raise ValueError("fock_block_offsets must have one entry per atom plus one, and atomic_numbers one per atom")
    if natoms > 0 and (np.any(np.diff(off) < 0) or off[0] < 0):
        raise ValueError("fock_block_offsets must be non-decreasing from >= 0")
    if rows.shape != cols.shape:
        raise ValueError("rows and cols must have the same length")
    if rows.size and (min(rows.min(), cols.min()) < 0 or max(rows.max(), cols.max()) >= natoms):
        raise IndexError("atom-pair index outside 0..num_atoms-1")
    if natoms and (Z[:natoms].min() < 0 or Z[:natoms].max() >= MAX_ELEMENTS):
        raise ValueError(f"atomic numbers must lie in 0..{MAX_ELEMENTS - 1}")


# (2 l1 + 1)(2 l2 + 1) for l1, l2 <= 3: the block sizes the kernel is built for
_SUPPORTED_N = frozenset((2 * a + 1) * (2 * b + 1) for a in range(4) for b in range(4))
_WAVES = 4  # block lists of the transform kernel's schedule


def _wave_schedule(costs):
    """Longest-processing-time split of the CG blocks into 4 lists, each in
    descending cost order (``costs[b]``: FMAs + LDS accesses per row of block
    b).  A 4-wave workgroup runs one list per wave, an 8-wave one every other
    block of a list per wave.  Layout: 5 offsets, then the block ids of list 0,
    list 1, ..."""
    load = [0] * _WAVES
    lists = [[] for _ in range(_WAVES)]
    for b in sorted(range(len(costs)), key=lambda i: (-costs[i], i)):
        w = min(range(_WAVES), key=lambda k: (load[k], k))
        lists[w].append(b)
        load[w] += costs[b]
    offs = np.cumsum([0] + [len(x) for x in lists])
    return np.concatenate([offs, np.concatenate([np.array(x, np.int64) for x in lists])]).astype(np.int32)


def cg_block_tables(decomp_obj):
    """Host tables of the transform kernels for an e3TensorDecomp (numpy):

    * ``blocks`` [nblocks, 3] = (n, first column, weight offset);
    * ``w_fwd`` / ``w_inv`` / ``w_adj``: the n x n block matrices, row-major
      [output column][input column], of get_net_out (W[t][h] = wms_H[b] as
      [n, n], utils_tensor_decomp.py:118), get_H (W[h][t] = wms[b] as [n, n],
      :117) and the transpose of get_H's block (its adjoint);
    * ``programs`` [3, nblocks]: per direction (fwd, inv, adj) the compiled CG
      program of libmaloq_hip.so whose matrix equals the block's exactly, or -1
      (the kernels then read the weights);
    * ``sched``: the per-wave block lists (_wave_schedule), costed by the
      nonzeros a compiled program computes or n^2 for a dense block.
    """
    ins, hs = decomp_obj.in_slices, decomp_obj.H_slices
    if list(map(int, ins)) != list(map(int, hs)):
        raise ValueError("label and irreps sides of the CG blocks must share their columns")
    blocks, w_fwd, w_inv, w_adj = [], [], [], []
    woff = 0
    for b in range(len(decomp_obj.out_js_list)):
        n = int(ins[b + 1]) - int(ins[b])
        if n not in _SUPPORTED_N:
            raise ValueError(f"CG block {b} of size {n} is not a shell pair with l <= 3")
        fwd = np.asarray(decomp_obj.wms_H[b].detach().cpu().double()).reshape(n, n)
        inv = np.asarray(decomp_obj.wms[b].detach().cpu().double()).reshape(n, n)
        blocks.append((n, int(ins[b]), woff))
        w_fwd.append(fwd.reshape(-1)); w_inv.append(inv.reshape(-1)); w_adj.append(inv.T.reshape(-1))
        woff += n * n
    w = [np.concatenate(w_fwd), np.concatenate(w_inv), np.concatenate(w_adj)]
    programs = _match_cg_programs(decomp_obj.out_js_list, blocks, w)
    costs = []
    for b, (n, _, woff) in enumerate(blocks):
        fma = int(np.count_nonzero(w[0][woff:woff + n * n])) if (programs[:, b] >= 0).all() else n * n
        costs.append(fma + 2 * n)
    return {"blocks": np.array(blocks, np.int32), "programs": programs, "sched": _wave_schedule(costs),
            "w_fwd": w[0], "w_inv": w[1], "w_adj": w[2]}


def _match_cg_programs(out_js_list, blocks, w):
    """[3, nblocks] int32: for direction d (0 fwd, 1 inv, 2 adj) and block b of
    shell pair (l1, l2), the program d * 16 + l1 * 4 + l2 if its compiled
    matrix (maloq_basis_cg_block) equals the block's fp32 matrix entry for
    entry, else -1."""
    lib = _lib.load()
    compiled = {}
    out = np.full((3, len(blocks)), -1, np.int32)
    for b, (n, _, woff) in enumerate(blocks):
        l1, l2 = (int(v) % 10 for v in out_js_list[b])
        for d in range(3):
            p = d * 16 + l1 * 4 + l2
            if p not in compiled:
                m = np.empty(n * n, np.float32)
                compiled[p] = m if lib.maloq_basis_cg_block(p, m.ctypes.data, n) == 0 else None
            ref = compiled[p]
            if ref is not None and ref.shape[0] == n * n and np.array_equal(ref, w[d][woff:woff + n * n].astype(np.float32)):
                out[d, b] = p
    return out


def template_slot_tables(orbital_template, h_slices):
    """Per element-pair tables of a template (numpy):

    * ``pair_kind`` [100*100]: element-pair key Z_i*100+Z_j -> kind, or -1;
    * ``raw_slot`` [kinds, maxe]: element q = a * n_j + b of an atom-pair block of
      that kind (row-major, n_i x n_j orbitals) goes to label column
      raw_slot[kind, q], -1 if no shell pair of the template covers it.  The
      columns are those of the template's row-major copies
      (numpy_single_matrix2label, matrix2labels_kernels.py:1117-1170);
      maxe = the largest n_i * n_j;
    * ``kind_blocks`` [kinds, 2] uint32: bit b set if the kind has CG block b
      (the block whose label columns start at h_slices[b]).
    """
    T = int(h_slices[-1])
    starts = {int(x): b for b, x in enumerate(h_slices[:-1])}
    pair_kind = np.full(MAX_ELEMENTS * MAX_ELEMENTS, -1, np.int32)
    kinds, masks = [], []
    for k, entries in enumerate(orbital_template):
        if not entries:
            continue
        ni = max(rs.stop for rs, _, _ in entries)
        nj = max(cs.stop for _, cs, _ in entries)
        if ni > 255 or nj > 255:
            raise ValueError("atom-pair blocks are limited to 255 x 255 orbitals")
        sl = np.full(ni * nj, -1, np.int64)
        mask = 0
        for rs, cs, os_ in entries:
            n1, n2 = rs.stop - rs.start, cs.stop - cs.start
            if os_.stop - os_.start != n1 * n2 or os_.stop > T or int(os_.start) not in starts:
                raise ValueError("orbital template entry does not match its CG block")
            a_, b_ = np.meshgrid(np.arange(rs.start, rs.stop), np.arange(cs.start, cs.stop), indexing="ij")
            sl[(a_ * nj + b_).reshape(-1)] = np.arange(os_.start, os_.stop)
            mask |= 1 << starts[int(os_.start)]
        pair_kind[k] = len(kinds)
        kinds.append(sl)
        masks.append(mask)
    maxe = max([len(x) for x in kinds] + [1])
    raw = np.full((max(len(kinds), 1), maxe), -1, np.int32)
    for k, sl in enumerate(kinds):
        raw[k, :len(sl)] = sl
    kb = np.zeros((max(len(kinds), 1), 2), np.uint32)
    for k, m in enumerate(masks):
        kb[k, 0] = m & 0xFFFFFFFF
        kb[k, 1] = (m >> 32) & 0xFFFFFFFF
    return pair_kind, raw, kb


class BasisPlan:
    """Row plan of the Fock-side transforms for one structure: per atom pair the
    block base, its original row index, element-pair kind and shape
    (maloq_basis_row_meta), in row order.  One small kernel builds it; build it
    once per (index lists, storage) to reuse it across fock_to_irreps /
    irreps_to_fock calls."""

    def __init__(self, meta, num_rows, ld, template_key):
        self.meta, self.num_rows, self.ld, self.template_key = meta, num_rows, ld, template_key


class _GetH(torch.autograd.Function):
    @staticmethod
    def forward(ctx, net_out, obj):
        ctx.obj = obj
        return obj._get_H_impl(net_out)

    @staticmethod
    def backward(ctx, grad):
        return ctx.obj._get_H_adjoint(grad.contiguous()), None


class HipE3TensorDecomp:
    def __init__(self, decomp_obj, device=None):
        self._decomp_obj = decomp_obj
        self.decomp_obj = decomp_obj
        self.device = torch.device(device) if device is not None else torch.device(decomp_obj.device)
        if self.device.type != "cuda":
            raise ValueError("HipE3TensorDecomp needs a ROCm GPU device")
        self.dtype = torch.float32
        self.num_blocks = len(decomp_obj.out_js_list)
        ins, hs = decomp_obj.in_slices, decomp_obj.H_slices
        self.total_in_dim, self.total_h_dim = int(ins[-1]), int(hs[-1])
        self.sort_perm = getattr(decomp_obj, "sort_perm", None)
        if decomp_obj.sort is not None and self.sort_perm is None:
            # a reference e3TensorDecomp: read the permutation off its sort module
            eye = torch.eye(int(decomp_obj.in_slices[-1]), dtype=torch.float64)
            self.sort_perm = torch.argmax(decomp_obj.sort(eye.to(decomp_obj.device)).cpu(), dim=0).numpy()
        if self.sort_perm is not None and not np.array_equal(np.sort(np.asarray(self.sort_perm)),
                                                             np.arange(self.total_in_dim)):
            # the kernels read and write every label column exactly once through it
            raise ValueError("sort_perm must be a permutation of the label columns")
        tabs = cg_block_tables(decomp_obj)
        dev = self.device
        # one blocks table per direction: (n, col0, woff, compiled program or -1)
        self._blocks_fwd, self._blocks_inv, self._blocks_adj = (
            _i32(np.concatenate([tabs["blocks"], tabs["programs"][d][:, None]], axis=1).reshape(-1), dev)
            for d in range(3))
        self.cg_programs = tabs["programs"]
        self._sched = _i32(tabs["sched"], dev)
        f32 = lambda a: torch.as_tensor(a.astype(np.float32), device=dev)
        self._w_fwd, self._w_inv, self._w_adj = f32(tabs["w_fwd"]), f32(tabs["w_inv"]), f32(tabs["w_adj"])
        # the weights the kernels read: none in a direction where every block
        # runs a compiled program (the kernel variant without the dense loops)
        self._wk_fwd, self._wk_inv, self._wk_adj = (
            None if (self.cg_programs[d] >= 0).all() else w for d, w in enumerate(
                (self._w_fwd, self._w_inv, self._w_adj)))
        self._perm = _i32(self.sort_perm, dev) if self.sort_perm is not None else None
        self.block_n2 = np.array([(2 * (l2 % 10) + 1) for _, l2 in decomp_obj.out_js_list], np.int32)
        self._templates = {}

    @property
    def required_irreps_out(self):
        return self._decomp_obj.required_irreps_out

    # ------------------------------------------------------------ labels
    def _check(self, x, width):
        _lib.require_cuda(x)
        if x.dtype != torch.float32:
            raise ValueError(f"HIP basis transform computes in fp32, got {x.dtype}")
        if x.dim() != 2 or x.shape[1] != width:
            raise ValueError(f"expected [R, {width}], got {tuple(x.shape)}")

    def _transform(self, x, blocks, w, perm_in=None, perm_out=None):
        x = x.contiguous()
        out = torch.empty_like(x)
        _lib.call("maloq_label_transform", _lib.ptr(x), _lib.ptr(perm_in), _lib.ptr(out), _lib.ptr(perm_out),
                  x.shape[0], x.shape[1], self.num_blocks, _lib.ptr(blocks), _lib.ptr(w),
                  _lib.ptr(self._sched), _lib.stream_of(x.device))
        return out

    def _get_H_impl(self, net_out):
        self._check(net_out, self.total_in_dim)
        return self._transform(net_out, self._blocks_inv, self._wk_inv, perm_in=self._perm)

    def _get_H_adjoint(self, grad):
        self._check(grad, self.total_h_dim)
        return self._transform(grad, self._blocks_adj, self._wk_adj, perm_out=self._perm)

    def get_H(self, net_out):
        return _GetH.apply(net_out, self)

    def get_net_out(self, H):
        self._check(H, self.total_h_dim)
        return self._transform(H, self._blocks_fwd, self._wk_fwd, perm_out=self._perm)

    # ------------------------------------------------ fused Fock <-> irreps
    def _template_tables(self, orbital_template):
        key = id(orbital_template)
        hit = self._templates.get(key)
        if hit is not None and hit[0] is orbital_template:
            return hit[1]
        pair_kind, raw, kb = template_slot_tables(orbital_template, self._decomp_obj.H_slices)
        dev = self.device
        tabs = {"pair_kind": _i32(pair_kind, dev), "raw": _i32(raw.reshape(-1), dev), "maxe": int(raw.shape[1]),
                "kind_blocks": (torch.as_tensor(kb.reshape(-1).view(np.int32), device=dev)
                                if self.num_blocks <= 64 else None)}
        self._templates[key] = (orbital_template, tabs)
        return tabs

    @staticmethod
    def _storage(fock, sparse_offsets):
        if sparse_offsets is None:
            if fock.dim() != 2 or fock.stride(1) != 1:
                raise ValueError("dense Fock matrix must be 2-D with unit column stride")
            return fock.stride(0), None
        # on the Fock matrix's device: the kernels read it there
        return 0, torch.as_tensor(sparse_offsets).to(device=fock.device, dtype=torch.int64).contiguous()

    def make_plan(self, fock, fock_block_offsets, atomic_numbers, rows, cols, orbital_template,
                  block_data_offsets=None):
        """BasisPlan for the atom pairs (rows[r], cols[r]) of ``fock`` (dense, or
        the block list of ``block_data_offsets``)."""
        _lib.require_cuda(fock)
        _check_pairs_on_host(fock_block_offsets, atomic_numbers, rows, cols)
        dev = fock.device
        tabs = self._template_tables(orbital_template)
        off, Z, r_, c_ = (_i32(x, dev) for x in (fock_block_offsets, atomic_numbers, rows, cols))
        ld, bdo = self._storage(fock, block_data_offsets)
        R = int(r_.shape[0])
        meta = torch.empty(max(R, 1), 4, device=dev, dtype=torch.int32)
        _lib.call("maloq_basis_row_meta", ld, _lib.ptr(bdo), _lib.ptr(off), _lib.ptr(Z), _lib.ptr(r_),
                  _lib.ptr(c_), R, _lib.ptr(tabs["pair_kind"]), tabs["maxe"], _lib.ptr(meta),
                  _lib.stream_of(dev))
        return BasisPlan(meta, R, ld, id(orbital_template))

    def _plan_for(self, plan, fock, fock_block_offsets, atomic_numbers, rows, cols, orbital_template,
                  block_data_offsets):
        if fock.dtype != torch.float32:
            raise ValueError("Unsupported dtype for the Fock matrix; only float32 is supported.")
        if plan is None:
            return self.make_plan(fock, fock_block_offsets, atomic_numbers, rows, cols, orbital_template,
                                  block_data_offsets)
        ld, _ = self._storage(fock, block_data_offsets)
        if plan.ld != ld or plan.template_key != id(orbital_template):
            raise ValueError("plan was built for another Fock storage or template")
        return plan

    def _pairs(self, fock, fock_block_offsets, atomic_numbers, rows, cols, block_data_offsets):
        """Device arguments of the plan-less entry points (the pair list itself)."""
        if fock.dtype != torch.float32:
            raise ValueError("Unsupported dtype for the Fock matrix; only float32 is supported.")
        _check_pairs_on_host(fock_block_offsets, atomic_numbers, rows, cols)
        dev = fock.device
        off, Z, r_, c_ = (_i32(x, dev) for x in (fock_block_offsets, atomic_numbers, rows, cols))
        if r_.shape != c_.shape:
            raise ValueError("rows and cols must have the same length")
        ld, bdo = self._storage(fock, block_data_offsets)
        return ld, bdo, off, Z, r_, c_

    def fock_to_irreps(self, fock, fock_block_offsets, atomic_numbers, rows, cols, orbital_template,
                       block_data_offsets=None, plan=None):
        """Labels in the irreps basis for every atom pair (rows[r], cols[r]):
        gather by template + get_net_out in one launch.  Without a plan the
        kernel describes the rows from the pair list itself (one launch, no
        plan); with one (make_plan, for a structure transformed many times) it
        reads the plan."""
        _lib.require_cuda(fock)
        tabs = self._template_tables(orbital_template)
        if plan is None:
            ld, bdo, off, Z, r_, c_ = self._pairs(fock, fock_block_offsets, atomic_numbers, rows, cols,
                                                 block_data_offsets)
            R = int(r_.shape[0])
            out = torch.empty(R, self.total_in_dim, device=fock.device, dtype=torch.float32)
            _lib.call("maloq_fock_to_irreps_pairs", _lib.ptr(fock), ld, _lib.ptr(bdo), _lib.ptr(off), _lib.ptr(Z),
                      _lib.ptr(r_), _lib.ptr(c_), R, _lib.ptr(tabs["pair_kind"]), _lib.ptr(tabs["raw"]),
                      tabs["maxe"], _lib.ptr(tabs["kind_blocks"]), _lib.ptr(out), _lib.ptr(self._perm),
                      self.total_in_dim, self.num_blocks, _lib.ptr(self._blocks_fwd), _lib.ptr(self._wk_fwd),
                      _lib.ptr(self._sched), _lib.stream_of(fock.device))
            return out
        plan = self._plan_for(plan, fock, fock_block_offsets, atomic_numbers, rows, cols, orbital_template,
                              block_data_offsets)
        out = torch.empty(plan.num_rows, self.total_in_dim, device=fock.device, dtype=torch.float32)
        _lib.call("maloq_fock_to_irreps", _lib.ptr(fock), plan.ld, _lib.ptr(plan.meta), plan.num_rows,
                  _lib.ptr(tabs["raw"]), tabs["maxe"], _lib.ptr(tabs["kind_blocks"]), _lib.ptr(out),
                  _lib.ptr(self._perm), self.total_in_dim, self.num_blocks, _lib.ptr(self._blocks_fwd),
                  _lib.ptr(self._wk_fwd), _lib.ptr(self._sched), _lib.stream_of(fock.device))
        return out

    def irreps_to_fock(self, net_out, fock, fock_block_offsets, atomic_numbers, rows, cols,
                       orbital_template, block_data_offsets=None, plan=None):
        """get_H per row, scattered into ``fock`` (in place) at the template's
        entries (without a plan: one launch from the pair list, as
        fock_to_irreps)."""
        self._check(net_out, self.total_in_dim)
        _lib.require_cuda(fock)
        tabs = self._template_tables(orbital_template)
        net_out = net_out.contiguous()
        if plan is None:
            ld, bdo, off, Z, r_, c_ = self._pairs(fock, fock_block_offsets, atomic_numbers, rows, cols,
                                                 block_data_offsets)
            R = int(r_.shape[0])
            if R != net_out.shape[0]:
                raise ValueError("net_out rows must match the atom-pair list")
            _lib.call("maloq_irreps_to_fock_pairs", _lib.ptr(net_out), _lib.ptr(self._perm), _lib.ptr(fock), ld,
                      _lib.ptr(bdo), _lib.ptr(off), _lib.ptr(Z), _lib.ptr(r_), _lib.ptr(c_), R,
                      _lib.ptr(tabs["pair_kind"]), _lib.ptr(tabs["raw"]), tabs["maxe"], _lib.ptr(tabs["kind_blocks"]),
                      self.total_in_dim, self.num_blocks, _lib.ptr(self._blocks_inv), _lib.ptr(self._wk_inv),
                      _lib.ptr(self._sched), _lib.stream_of(fock.device))
            return fock
        plan = self._plan_for(plan, fock, fock_block_offsets, atomic_numbers, rows, cols, orbital_template,
                              block_data_offsets)
        if plan.num_rows != net_out.shape[0]:
            raise ValueError("net_out rows must match the atom-pair list")
        _lib.call("maloq_irreps_to_fock", _lib.ptr(net_out), _lib.ptr(self._perm), _lib.ptr(fock), plan.ld,
                  _lib.ptr(plan.meta), plan.num_rows, _lib.ptr(tabs["raw"]), tabs["maxe"],
                  _lib.ptr(tabs["kind_blocks"]), self.total_in_dim, self.num_blocks, _lib.ptr(self._blocks_inv),
                  _lib.ptr(self._wk_inv), _lib.ptr(self._sched), _lib.stream_of(fock.device))
        return fock


def make_basis_transform(base_decomp, basis_transform_backend: str = "hip"):
    """The basis_transform_backend switch (fock_targets_batched.py:152-165) with 'hip'."""
    if basis_transform_backend == "hip":
        return HipE3TensorDecomp(base_decomp)
    if basis_transform_backend == "torch":
        return base_decomp
    raise ValueError(f"unknown basis_transform_backend '{basis_transform_backend}', "
                     f"expected 'torch' or 'hip'")
