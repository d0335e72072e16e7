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


def _on_host(*arrs):
    return not any(torch.is_tensor(a) and a.is_cuda for a in arrs if a is not None)


def _host_np(a):
    return np.asarray(a.numpy() if torch.is_tensor(a) else a).reshape(-1)


def _check_pairs_on_host(off, Z, rows, cols, fock=None, block_data_offsets=None):
    """Range checks of the atom-pair structure where it is still on the host
    (numpy or CPU tensors, as the per-molecule callers hold it): the kernels
    index with these values unchecked.  With ``fock`` also the extent of every
    atom-pair block: inside the dense matrix (the last orbital offset within
    both dimensions), or, for block-list storage, one data offset per pair and
    every block n_i x n_j inside the flat data.  Device tensors are the caller's
    responsibility (checking them would read them back, a sync per call)."""
    if not _on_host(off, Z, rows, cols):
        return
    off, Z, rows, cols = (_host_np(a) for a in (off, Z, rows, cols))
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
    if fock is None or natoms == 0:
        return
    if block_data_offsets is None:
        if fock.dim() != 2 or off[-1] > fock.shape[0] or off[-1] > fock.shape[1]:
            raise ValueError(f"fock_block_offsets reach orbital {int(off[-1])}, outside the "
                             f"{tuple(fock.shape)} Fock matrix")
        return
    if not _on_host(block_data_offsets):
        return
    bdo = _host_np(block_data_offsets).astype(np.int64)
    if bdo.shape[0] < rows.shape[0]:
        raise ValueError(f"block_data_offsets has {bdo.shape[0]} entries for {rows.shape[0]} atom pairs")
    if rows.size:
        n = np.diff(off).astype(np.int64)
        ends = bdo[:rows.shape[0]] + n[rows] * n[cols]
        if bdo[:rows.shape[0]].min() < 0 or ends.max() > fock.numel():
            raise ValueError(f"an atom-pair block of block_data_offsets lies outside the {fock.numel()} "
                             f"elements of the block data")


# (2 l1 + 1)(2 l2 + 1) for l1, l2 <= 3: the block sizes the kernel is built for
_SUPPORTED_N = frozenset((2 * a + 1) * (2 * b + 1) for a in range(4) for b in range(4))
_WAVES = 4  # block lists of the transform kernel's schedule
# Column groups: at most this many CG blocks (the presence masks are 64 bits)
# and, by default, this many columns: a 64-row tile of 203-float rows and its
# 36-byte row descriptors lets three 8-wave workgroups share a CU (24 waves,
# the register budget of the kernels).
MAX_GROUP_BLOCKS = 64
GROUP_COLS = 203
MAX_GROUP_COLS = 1269  # a 32-row fp32 tile of one group and its row descriptors in 160 KB of LDS


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


def column_groups(widths, max_cols=GROUP_COLS, max_blocks=MAX_GROUP_BLOCKS, shell_rows=None):
    """Split the CG blocks (column widths in row order) into runs of
    consecutive blocks of at most ``max_cols`` columns and ``max_blocks``
    blocks: [(first column, width, first block, blocks), ...].  A row that fits
    is one group.

    ``shell_rows`` (the first shell of each block's pair, when the blocks are
    the full shell x shell grid) keeps a group inside one shell row, or makes it
    whole shell rows: its elements are then one rectangle of every atom-pair
    block (the rows of those shells, and all or a run of the columns)."""
    widths = [int(n) for n in widths]
    if max_cols < max(widths, default=1) or max_cols > MAX_GROUP_COLS:
        raise ValueError(f"column group width {max_cols} outside {max(widths, default=1)}..{MAX_GROUP_COLS}")
    rows = list(range(len(widths))) if shell_rows is None else list(shell_rows)
    segs = []  # runs of blocks of one shell row: (first block, end block)
    for b in range(len(widths)):
        if b == 0 or rows[b] != rows[b - 1]:
            segs.append([b, b])
        segs[-1][1] = b + 1
    groups = []
    col = 0
    cur = None  # [first column, width, first block, blocks]
    for b0, b1 in segs:
        w = sum(widths[b0:b1])
        if w <= max_cols and b1 - b0 <= max_blocks:
            if cur is not None and cur[1] + w <= max_cols and cur[3] + b1 - b0 <= max_blocks:
                cur[1] += w
                cur[3] += b1 - b0
            else:
                if cur is not None:
                    groups.append(tuple(cur))
                cur = [col, w, b0, b1 - b0]
        else:  # a shell row wider than a group: balanced runs of its blocks
            if cur is not None:
                groups.append(tuple(cur))
                cur = None
            groups += _balanced_runs(widths, b0, b1, col, max_cols, max_blocks)
        col += w
    if cur is not None:
        groups.append(tuple(cur))
    return groups


def _greedy_runs(widths, b0, b1, col, limit, max_blocks):
    runs = []
    c, width, g0, nb = col, 0, b0, 0
    for b in range(b0, b1):
        if nb and (width + widths[b] > limit or nb == max_blocks):
            runs.append((c, width, g0, nb))
            c, width, g0, nb = c + width, 0, b, 0
        width += widths[b]
        nb += 1
    runs.append((c, width, g0, nb))
    return runs


def _balanced_runs(widths, b0, b1, col, max_cols, max_blocks):
    """The fewest runs of blocks b0 .. b1-1 within max_cols / max_blocks, as
    even in width as a greedy split under the smallest limit allows."""
    best = _greedy_runs(widths, b0, b1, col, max_cols, max_blocks)
    total = sum(widths[b0:b1])
    lo = max(max(widths[b0:b1]), -(-total // len(best)))
    for limit in range(lo, max_cols + 1):
        runs = _greedy_runs(widths, b0, b1, col, limit, max_blocks)
        if len(runs) <= len(best):
            return runs
    return best


def shell_rows_of(out_js_list):
    """The first shell of each CG block when the blocks are the full n x n
    shell grid, row-major (as make_output_irreps builds them), else None."""
    nb = len(out_js_list)
    n = int(round(nb ** 0.5))
    if n * n != nb or nb == 0:
        return None
    ls = [out_js_list[b][1] for b in range(n)]
    for b, (l1, l2) in enumerate(out_js_list):
        if (l1, l2) != (ls[b // n], ls[b % n]):
            return None
    return [b // n for b in range(nb)]


def group_schedule(groups, costs):
    """The kernels' ``sched`` table: [G, G x (first column, width, first block,
    offset o_g)], then per group at o_g its _wave_schedule with global block
    ids."""
    G = len(groups)
    head = [G]
    body = []
    off = 1 + 4 * G
    for c0, width, b0, nb in groups:
        lists = _wave_schedule(costs[b0:b0 + nb]).astype(np.int64)
        lists[_WAVES + 1:] += b0
        head += [c0, width, b0, off]
        body.append(lists)
        off += len(lists)
    return np.concatenate([np.array(head, np.int64)] + body).astype(np.int32)


def cg_block_tables(decomp_obj, group_cols=GROUP_COLS):
    """Host tables of the transform kernels for an e3TensorDecomp (numpy):

    * ``blocks`` [nblocks, 3] = (n, first column, weight offset);
    * ``w_fwd`` / ``w_inv`` / ``w_adj``: the n x n block matrices, row-major
      [output column][input column], of get_net_out (W[t][h] = wms_H[b] as
      [n, n], utils_tensor_decomp.py:118), get_H (W[h][t] = wms[b] as [n, n],
      :117) and the transpose of get_H's block (its adjoint);
    * ``programs`` [3, nblocks]: per direction (fwd, inv, adj) the compiled CG
      program of libmaloq_hip.so whose matrix equals the block's exactly, or -1
      (the kernels then read the weights);
    * ``groups``: the column groups (column_groups, at most ``group_cols``
      columns each);
    * ``sched``: per group the per-wave block lists (group_schedule), costed by
      the nonzeros a compiled program computes or n^2 for a dense block.
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
    groups = column_groups([n for n, _, _ in blocks], group_cols, shell_rows=shell_rows_of(decomp_obj.out_js_list))
    return {"blocks": np.array(blocks, np.int32), "programs": programs, "groups": groups,
            "sched": group_schedule(groups, costs), "w_fwd": w[0], "w_inv": w[1], "w_adj": w[2]}


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


def template_slot_tables(orbital_template, h_slices, groups=None):
    """Per element-pair tables of a template (numpy):

    * ``pair_kind`` [100*100]: element-pair key Z_i*100+Z_j -> kind, or -1;
    * ``raw_slot`` [kinds, maxe]: element q = a * n_j + b of an atom-pair block of
      that kind (row-major, n_i x n_j orbitals) goes to label column
      raw_slot[kind, q], -1 if no shell pair of the template covers it.  The
      columns are those of the template's row-major copies
      (numpy_single_matrix2label, matrix2labels_kernels.py:1117-1170);
      maxe = the largest n_i * n_j;
    * ``slots``: the kernels' per (column group, kind) rectangles, built from
      raw_slot for ``groups`` (column_groups; one group over the whole row if
      None): [K, G, G x largest rectangle, G*K rectangles r0 | nr << 8 |
      c0 << 16 | nc << 24 (the bounding box of the kind's elements in the
      group; 0 if none), G*K table offsets, tables]; a table holds, row-major
      over the rectangle, each element's column relative to the group's first
      column, or -1.  With one group the rectangle is the whole template block
      and the tables are the rows of raw_slot (maxe entries each: the kernels
      find kind k's at a fixed offset);
    * ``kind_blocks`` [G*K, 2] uint32: bit i set if the kind has the group's
      i-th CG block (the block whose label columns start at h_slices[b]).
    """
    T = int(h_slices[-1])
    starts = {int(x): b for b, x in enumerate(h_slices[:-1])}
    nblocks = len(h_slices) - 1
    if groups is None:
        groups = [(0, T, 0, nblocks)]
    pair_kind = np.full(MAX_ELEMENTS * MAX_ELEMENTS, -1, np.int32)
    kinds, have, shapes = [], [], []
    for k, entries in enumerate(orbital_template):
        if not entries:
            continue
        ni = max(rs.stop for rs, _, _ in entries)
        nj = max(cs.stop for _, cs, _ in entries)
        if ni > 255 or nj > 255:
            raise ValueError("atom-pair blocks are limited to 255 x 255 orbitals")
        sl = np.full(ni * nj, -1, np.int64)
        hb = np.zeros(nblocks, bool)
        for rs, cs, os_ in entries:
            n1, n2 = rs.stop - rs.start, cs.stop - cs.start
            if os_.stop - os_.start != n1 * n2 or os_.stop > T or int(os_.start) not in starts:
                raise ValueError("orbital template entry does not match its CG block")
            a_, b_ = np.meshgrid(np.arange(rs.start, rs.stop), np.arange(cs.start, cs.stop), indexing="ij")
            sl[(a_ * nj + b_).reshape(-1)] = np.arange(os_.start, os_.stop)
            hb[starts[int(os_.start)]] = True
        pair_kind[k] = len(kinds)
        kinds.append(sl)
        have.append(hb)
        shapes.append((ni, nj))
    maxe = max([len(x) for x in kinds] + [1])
    K = max(len(kinds), 1)
    raw = np.full((K, maxe), -1, np.int32)
    for k, sl in enumerate(kinds):
        raw[k, :len(sl)] = sl
    G = len(groups)
    rects = np.zeros(G * K, np.int64)
    offs = np.zeros(G * K, np.int64)
    longest = []
    tables = []
    head = 2 + G + 2 * G * K
    pos = head
    kb = np.zeros((G * K, 2), np.uint32)
    for g, (c0, width, b0, nb) in enumerate(groups):
        if nb > MAX_GROUP_BLOCKS:
            raise ValueError(f"column group {g} has {nb} > {MAX_GROUP_BLOCKS} CG blocks")
        most = 0
        for k, sl in enumerate(kinds):
            nj = shapes[k][1]
            q = np.nonzero((sl >= c0) & (sl < c0 + width))[0]
            if k < len(have):
                m = sum(1 << i for i in range(nb) if have[k][b0 + i])
                kb[g * K + k] = (m & 0xFFFFFFFF, m >> 32)
            if G == 1:
                # one group: the whole block, tables as rows of maxe entries
                ni = shapes[k][0]
                rects[k] = 0 | ni << 8 | 0 << 16 | nj << 24
                offs[k] = head + k * maxe
                tables.append(raw[k].astype(np.int64) - c0 * (raw[k] >= 0))
                most = max(most, ni * nj)
                continue
            if len(q) == 0:
                continue
            r, c = q // nj, q % nj
            r0, nr, cc, nc = int(r.min()), int(r.max() - r.min() + 1), int(c.min()), int(c.max() - c.min() + 1)
            tab = np.full(nr * nc, -1, np.int64)
            tab[(r - r0) * nc + (c - cc)] = sl[q] - c0
            rects[g * K + k] = r0 | nr << 8 | cc << 16 | nc << 24
            offs[g * K + k] = pos
            tables.append(tab)
            pos += len(tab)
            most = max(most, nr * nc)
        longest.append(most)
    slots = np.concatenate([np.array([K, G] + longest, np.int64), rects, offs] + tables)
    slots = (slots.astype(np.uint32)).view(np.int32) if slots.max() >= 2 ** 31 else slots.astype(np.int32)
    return {"pair_kind": pair_kind, "raw_slot": raw, "maxe": maxe, "slots": slots, "kind_blocks": kb}


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


def _ops():
    """The C++ operators (maloq_amd.ops loads the extension on first use)."""
    from . import ops
    return ops


class HipE3TensorDecomp:
    """``group_cols``: the widest column group of the kernels' tiles (rows wider
    than that are split into groups of whole CG blocks; one group when the row
    fits)."""

    def __init__(self, decomp_obj, device=None, group_cols=GROUP_COLS):
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
        tabs = cg_block_tables(decomp_obj, group_cols)
        dev = self.device
        # one blocks table per direction: (n, col0, woff, compiled program or -1)
        self._blocks_fwd, self._blocks_inv, self._blocks_adj = (
            _i32(np.concatenate([tabs["blocks"], tabs["programs"][d][:, None]], axis=1).reshape(-1), dev)
            for d in range(3))
        self.cg_programs = tabs["programs"]
        self.groups = tabs["groups"]
        self.ngroups = len(self.groups)
        self.group_cols = max(w for _, w, _, _ in self.groups)
        self._sched = _i32(tabs["sched"], dev)
        f32 = lambda a: torch.as_tensor(a.astype(np.float32), device=dev)
        self._w_fwd, self._w_inv, self._w_adj = f32(tabs["w_fwd"]), f32(tabs["w_inv"]), f32(tabs["w_adj"])
        # the weights the kernels read: none in a direction where every block
        # runs a compiled program (the kernel variant without the dense loops)
        self._wk_fwd, self._wk_inv, self._wk_adj = (
            None if (self.cg_programs[d] >= 0).all() else w for d, w in enumerate(
                (self._w_fwd, self._w_inv, self._w_adj)))
        self._perm = _i32(self.sort_perm, dev) if self.sort_perm is not None else None
        self._perm_inv = None
        if self._perm is not None and self.ngroups > 1:
            # rows of several column groups are permuted by a separate column
            # gather: sorted <- unsorted (perm) and unsorted <- sorted (inverse)
            self._perm_inv = _i32(np.argsort(np.asarray(self.sort_perm)), dev)
            self._ones = torch.ones(self.total_in_dim, device=dev, dtype=torch.float32)
        self.block_n2 = np.array([(2 * (l2 % 10) + 1) for _, l2 in decomp_obj.out_js_list], np.int32)
        self._templates = {}

    @property
    def required_irreps_out(self):
        return self._decomp_obj.required_irreps_out

    def _layout(self):
        return self.ngroups, self.group_cols

    # ------------------------------------------------------------ labels
    def _check(self, x, width):
        _lib.require_cuda(x)
        if x.dtype != torch.float32:
            raise ValueError(f"HIP basis transform computes in fp32, got {x.dtype}")
        if x.dim() != 2 or x.shape[1] != width:
            raise ValueError(f"expected [R, {width}], got {tuple(x.shape)}")

    def _permute(self, x, src):
        """out[:, j] = x[:, src[j]] (maloq_gather_columns)."""
        out = torch.empty_like(x)
        _lib.call("maloq_gather_columns", _lib.ptr(x), x.shape[1], x.shape[0], _lib.ptr(src), _lib.ptr(self._ones),
                  x.shape[1], _lib.ptr(out), out.shape[1], _lib.stream_of(x.device))
        return out

    def _split_perms(self, perm_in, perm_out):
        """(perm_in, perm_out) for the kernels, and whether the input must be
        un-sorted before / the output sorted after them (several groups)."""
        if self.ngroups == 1:
            return perm_in, perm_out, False, False
        return None, None, perm_in is not None, perm_out is not None

    def _transform(self, x, blocks, w, perm_in=None, perm_out=None):
        """The registered operator maloq_hip::label_transform (the C++
        extension): for rows of several column groups it un-sorts the input
        through the inverse permutation and sorts the output after the kernel."""
        with torch.no_grad():  # differentiable through _GetH only, like the tables it is given
            return _ops().label_transform(x, blocks, w, self._sched, perm_in, perm_out, self.num_blocks,
                                          self.ngroups, self.group_cols, self._perm_inv)

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
        t = template_slot_tables(orbital_template, self._decomp_obj.H_slices, self.groups)
        dev = self.device
        tabs = {"pair_kind": _i32(t["pair_kind"], dev), "slots": _i32(t["slots"], dev), "maxe": t["maxe"],
                "kind_blocks": torch.as_tensor(t["kind_blocks"].reshape(-1).view(np.int32), device=dev)}
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
        _check_pairs_on_host(fock_block_offsets, atomic_numbers, rows, cols, fock, block_data_offsets)
        dev = fock.device
        tabs = self._template_tables(orbital_template)
        off, Z, r_, c_ = (_i32(x, dev) for x in (fock_block_offsets, atomic_numbers, rows, cols))
        ld, bdo = self._storage(fock, block_data_offsets)
        R = int(r_.shape[0])
        meta = _ops().basis_row_meta(ld, bdo, off, Z, r_, c_, tabs["pair_kind"], tabs["maxe"])
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
        _check_pairs_on_host(fock_block_offsets, atomic_numbers, rows, cols, fock, block_data_offsets)
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
        _, perm_out, _, post = self._split_perms(None, self._perm)
        if plan is None:
            ld, bdo, off, Z, r_, c_ = self._pairs(fock, fock_block_offsets, atomic_numbers, rows, cols,
                                                 block_data_offsets)
            meta, R = None, int(r_.shape[0])
        else:
            plan = self._plan_for(plan, fock, fock_block_offsets, atomic_numbers, rows, cols, orbital_template,
                                  block_data_offsets)
            ld, bdo, off, Z, r_, c_ = plan.ld, None, None, None, None, None
            meta, R = plan.meta, plan.num_rows
        with torch.no_grad():
            return _ops().fock_to_irreps(fock, ld, bdo, off, Z, r_, c_, meta, R, tabs["pair_kind"],
                                         tabs["slots"], tabs["maxe"], tabs["kind_blocks"], perm_out,
                                         self.total_in_dim, self.num_blocks, self._blocks_fwd, self._wk_fwd,
                                         self._sched, self.ngroups, self.group_cols,
                                         self._perm if post else None)

    def irreps_to_fock(self, net_out, fock, fock_block_offsets, atomic_numbers, rows, cols,
                       orbital_template, block_data_offsets=None, plan=None):
        """get_H per row, scattered into ``fock`` (in place) at the template's
        entries (without a plan: one launch from the pair list, as
        fock_to_irreps)."""
        self._check(net_out, self.total_in_dim)
        _lib.require_cuda(fock)
        tabs = self._template_tables(orbital_template)
        perm_in, _, pre, _ = self._split_perms(self._perm, None)
        if plan is None:
            ld, bdo, off, Z, r_, c_ = self._pairs(fock, fock_block_offsets, atomic_numbers, rows, cols,
                                                 block_data_offsets)
            meta, R = None, int(r_.shape[0])
        else:
            plan = self._plan_for(plan, fock, fock_block_offsets, atomic_numbers, rows, cols, orbital_template,
                                  block_data_offsets)
            ld, bdo, off, Z, r_, c_ = plan.ld, None, None, None, None, None
            meta, R = plan.meta, plan.num_rows
        if R != net_out.shape[0]:
            raise ValueError("net_out rows must match the atom-pair list")
        with torch.no_grad():
            _ops().irreps_to_fock(net_out, fock, ld, bdo, off, Z, r_, c_, meta, R, tabs["pair_kind"], tabs["slots"],
                                  tabs["maxe"], tabs["kind_blocks"], perm_in, self.total_in_dim, self.num_blocks,
                                  self._blocks_inv, self._wk_inv, self._sched, self.ngroups, self.group_cols,
                                  self._perm_inv if pre else None)
        return fock


def make_basis_transform(base_decomp, basis_transform_backend: str = "hip"):
    """The basis_transform_backend switch (fock_targets_batched.py:152-165) with 'hip'."""
    if basis_transform_backend == "hip":
        return HipE3TensorDecomp(base_decomp)
    if basis_transform_backend == "torch":
        return base_decomp
    raise ValueError(f"unknown basis_transform_backend '{basis_transform_backend}', "
                     f"expected 'torch' or 'hip'")
