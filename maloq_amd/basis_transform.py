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
        wms = [np.asarray(w.detach().cpu().double()) for w in decomp_obj.wms]
        wms_h = [np.asarray(w.detach().cpu().double()) for w in decomp_obj.wms_H]

        # block geometry
        self.block_n2 = np.array([(2 * (l2 % 10) + 1) for _, l2 in decomp_obj.out_js_list], np.int32)
        in_block = np.zeros(self.total_in_dim, np.int32)
        h_block = np.zeros(self.total_h_dim, np.int32)
        for b in range(self.num_blocks):
            in_block[ins[b]:ins[b + 1]] = b
            h_block[hs[b]:hs[b + 1]] = b
        self.h_block = h_block

        # net_out (unsorted column c) from H:  W row = wms_H[b][t, :]
        w_parts, src, ln, woff = [], [], [], []
        off = 0
        for c in range(self.total_in_dim):
            b = in_block[c]
            t = c - ins[b]
            row = wms_h[b].reshape(ins[b + 1] - ins[b], -1)[t]
            w_parts.append(row); src.append(hs[b]); ln.append(len(row)); woff.append(off)
            off += len(row)
        netout_tab = (np.array(src), np.array(ln), np.array(woff), np.concatenate(w_parts))
        # H column from net_out:  W row = wms[b][h, :]
        w_parts, src, ln, woff = [], [], [], []
        off = 0
        for c in range(self.total_h_dim):
            b = h_block[c]
            h = c - hs[b]
            row = wms[b].reshape(hs[b + 1] - hs[b], -1)[h]
            w_parts.append(row); src.append(ins[b]); ln.append(len(row)); woff.append(off)
            off += len(row)
        geth_tab = (np.array(src), np.array(ln), np.array(woff), np.concatenate(w_parts))
        # adjoint of get_H:  net_out grad column c = sum_h gH[h] wms[b][h, t]
        w_parts, src, ln, woff = [], [], [], []
        off = 0
        for c in range(self.total_in_dim):
            b = in_block[c]
            t = c - ins[b]
            col = wms[b].reshape(hs[b + 1] - hs[b], -1)[:, t]
            w_parts.append(col); src.append(hs[b]); ln.append(len(col)); woff.append(off)
            off += len(col)
        adj_tab = (np.array(src), np.array(ln), np.array(woff), np.concatenate(w_parts))

        perm = self.sort_perm
        dev = self.device

        def upload(tab, rows=None):
            s, l_, w_o, w = tab
            if rows is not None:
                s, l_, w_o = s[rows], l_[rows], w_o[rows]
            return (_i32(s, dev), _i32(l_, dev), _i32(w_o, dev),
                    torch.as_tensor(w.astype(np.float32), device=dev), int(np.max(l_)))

        self._netout = upload(netout_tab, perm)
        self._adj = upload(adj_tab, perm)
        self._geth = upload(geth_tab)
        # get_H reads sorted input: unsorted column c lives at sorted position inv[c]
        self._geth_in_map = _i32(np.argsort(perm), dev) if perm is not None else None
        self._netout_block = _i32(in_block if perm is None else in_block[perm], dev)
        self._h_tabs = None
        self.block_n2_dev = _i32(self.block_n2, dev)
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

    def _transform(self, x, tab, t_out, in_map=None):
        src, ln, woff, w, mx = tab
        x = x.contiguous()
        out = torch.empty(x.shape[0], t_out, device=x.device, dtype=torch.float32)
        if x.shape[0]:
            _lib.call("maloq_label_transform", _lib.ptr(x), x.shape[0], x.shape[1], _lib.ptr(in_map),
                      _lib.ptr(out), t_out, _lib.ptr(src), _lib.ptr(ln), _lib.ptr(woff), _lib.ptr(w),
                      mx, _lib.stream_of(x.device))
        return out

    def _get_H_impl(self, net_out):
        self._check(net_out, self.total_in_dim)
        return self._transform(net_out, self._geth, self.total_h_dim, self._geth_in_map)

    def _get_H_adjoint(self, grad):
        self._check(grad, self.total_h_dim)
        return self._transform(grad, self._adj, self.total_in_dim)

    def get_H(self, net_out):
        return _GetH.apply(net_out, self)

    def get_net_out(self, H):
        self._check(H, self.total_h_dim)
        return self._transform(H, self._netout, self.total_in_dim)

    # ------------------------------------------------ fused Fock <-> irreps
    def _template_tables(self, orbital_template):
        key = id(orbital_template)
        hit = self._templates.get(key)
        if hit is not None and hit[0] is orbital_template:
            return hit[1]
        starts = {int(s): b for b, s in enumerate(self._decomp_obj.H_slices[:-1])}
        pair_kind = np.full(MAX_ELEMENTS * MAX_ELEMENTS, -1, np.int32)
        origins = []
        for k, entries in enumerate(orbital_template):
            if not entries:
                continue
            org = np.full((self.num_blocks, 2), -1, np.int32)
            for rs, cs, os_ in entries:
                b = starts[int(os_.start)]
                org[b] = (rs.start, cs.start)
            pair_kind[k] = len(origins)
            origins.append(org)
        sub = np.stack(origins) if origins else np.full((1, self.num_blocks, 2), -1, np.int32)
        tabs = (_i32(pair_kind, self.device), _i32(sub.reshape(-1), self.device))
        self._templates[key] = (orbital_template, tabs)
        return tabs

    def _h_tables(self):
        if self._h_tabs is None:
            hs = self._decomp_obj.H_slices
            pos = np.arange(self.total_h_dim) - np.asarray(hs)[self.h_block]
            self._h_tabs = (_i32(self.h_block, self.device), _i32(pos, self.device))
        return self._h_tabs

    @staticmethod
    def _storage(fock, sparse_offsets):
        if sparse_offsets is None:
            if fock.dim() != 2 or fock.stride(1) != 1:
                raise ValueError("dense Fock matrix must be 2-D with unit column stride")
            return fock.stride(0), None
        return 0, sparse_offsets.to(torch.int64).contiguous()

    def fock_to_irreps(self, fock, fock_block_offsets, atomic_numbers, rows, cols, orbital_template,
                       block_data_offsets=None):
        """Labels in the irreps basis for every atom pair (rows[r], cols[r]):
        gather by template + get_net_out in one launch."""
        _lib.require_cuda(fock)
        if fock.dtype != torch.float32:
            raise ValueError("Unsupported dtype for the Fock matrix; only float32 is supported.")
        dev = fock.device
        pk, sub = self._template_tables(orbital_template)
        off = _i32(fock_block_offsets, dev)
        Z = _i32(atomic_numbers, dev)
        r_ = _i32(rows, dev)
        c_ = _i32(cols, dev)
        R = int(r_.shape[0])
        sizes = torch.diff(off) if torch.is_tensor(off) else np.diff(np.asarray(fock_block_offsets))
        maxe = int(sizes.max()) ** 2 if len(sizes) else 1
        ld, bdo = self._storage(fock, block_data_offsets)
        out = torch.empty(R, self.total_in_dim, device=dev, dtype=torch.float32)
        if R:
            src, ln, woff, w, mx = self._netout
            _lib.call("maloq_fock_to_irreps", _lib.ptr(fock), ld, _lib.ptr(bdo), _lib.ptr(off),
                      _lib.ptr(Z), _lib.ptr(r_), _lib.ptr(c_), R, _lib.ptr(pk), _lib.ptr(sub),
                      self.num_blocks, _lib.ptr(self.block_n2_dev), _lib.ptr(out), self.total_in_dim,
                      _lib.ptr(self._netout_block), _lib.ptr(ln), _lib.ptr(woff), _lib.ptr(w), maxe,
                      _lib.stream_of(dev))
        return out

    def irreps_to_fock(self, net_out, fock, fock_block_offsets, atomic_numbers, rows, cols,
                       orbital_template, block_data_offsets=None):
        """get_H per row, scattered into ``fock`` (in place) at the template's entries."""
        self._check(net_out, self.total_in_dim)
        _lib.require_cuda(fock)
        if fock.dtype != torch.float32:
            raise ValueError("Unsupported dtype for the Fock matrix; only float32 is supported.")
        dev = fock.device
        if self.sort_perm is not None:
            net_out = net_out[:, torch.as_tensor(np.argsort(self.sort_perm), device=dev)]
        net_out = net_out.contiguous()
        pk, sub = self._template_tables(orbital_template)
        hb, hp = self._h_tables()
        off = _i32(fock_block_offsets, dev)
        Z = _i32(atomic_numbers, dev)
        r_ = _i32(rows, dev)
        c_ = _i32(cols, dev)
        R = int(r_.shape[0])
        if R != net_out.shape[0]:
            raise ValueError("net_out rows must match the atom-pair list")
        ld, bdo = self._storage(fock, block_data_offsets)
        if R:
            src, ln, woff, w, mx = self._geth
            _lib.call("maloq_irreps_to_fock", _lib.ptr(net_out), R, self.total_in_dim, _lib.ptr(fock), ld,
                      _lib.ptr(bdo), _lib.ptr(off), _lib.ptr(Z), _lib.ptr(r_), _lib.ptr(c_), _lib.ptr(pk),
                      _lib.ptr(sub), self.num_blocks, _lib.ptr(self.block_n2_dev), self.total_h_dim,
                      _lib.ptr(hb), _lib.ptr(hp), _lib.ptr(src), _lib.ptr(ln), _lib.ptr(woff), _lib.ptr(w),
                      _lib.stream_of(dev))
        return fock


def make_basis_transform(base_decomp, basis_transform_backend: str = "hip"):
    """The basis_transform_backend switch (fock_targets_batched.py:152-165) with 'hip'."""
    if basis_transform_backend == "hip":
        return HipE3TensorDecomp(base_decomp)
    if basis_transform_backend == "torch":
        return base_decomp
    raise ValueError(f"unknown basis_transform_backend '{basis_transform_backend}', "
                     f"expected 'torch' or 'hip'")
