"""Fock_Irreps_Head on the GPU: node and edge embeddings -> irreps labels.

The reference's output head (helm/esen_osh.py:522-1064) maps the backbone's
[rows, (lmax+1)^2, C] features to the label irreps of every orbital pair:
``stack_irreps`` regroups the features by degree, ``process`` applies

    s = Linear(C x 0e -> (C + L C) x 0e)(x_l=0)            (lin_scalars_learnable)
    g = [s[:C], Gate(sigmoid(s[C:]), x_l>=1)]                (e3nn Gate)
    y_l = Linear(C x le -> mul_l x le)(g_l),  l = 0..L       (lin_out_layers)

and the l-sorted result is permuted to the labels' irreps order (and, with
reduce_node, expanded from the node-reduced irreps by index and parity sign).

Here the features stay in the backbone's l-major layout (no stacked copy):
the scalar and per-l linears are plain GEMMs on the library (torch.matmul ->
hipBLASLt); the gate is ``maloq_irreps_gate_fwd`` / ``_bwd``; and one
``maloq_gather_columns`` does the per-l transpose to e3nn's channel-major
layout, the output permutation and the node expansion together (its gradient
is the fixed-order ``maloq_scatter_columns``).  Parameter names follow the
reference (e3nn Linear's flat ``weight`` [mul_in * mul_out] and ``bias``), so
state dicts load.

With reduce_edge (esen_osh.py:570-575, 894-944, 1090-1130) every edge pair
(i -> j, j -> i) is processed once as alpha = x_ij + x_ji and beta = x_ij - x_ji
(gates cst tanh(|s|), no biases but the node layers'), and the labels of both
directions are rebuilt as A + B and A - B, where A and B are two signed column
gathers of the alpha and beta GEMM outputs that carry the reference's
output permutations, the Vpa +- Vpb remix of the off-diagonal shell pairs, the
subspace remix and the parity flips.
"""
from __future__ import annotations

import math

import numpy as np
import torch
from torch import nn

from . import _lib


def _normalize2mom(act):
    """e3nn's normalize2mom constant: E[act(z)^2]^-1/2 over 10^6 float64 N(0, 1)
    draws of a CPU generator seeded 0 (as e3nn computes it)."""
    gen = torch.Generator(device="cpu").manual_seed(0)
    z = torch.randn(1_000_000, generator=gen, dtype=torch.float64)
    cst = act(z).pow(2).mean().pow(-0.5).item()
    return 1.0 if abs(cst - 1.0) < 1e-4 else cst


_CST = {}


def _cst(act):
    """act 0: sigmoid gates; act 1: tanh gates (reduce_edge)."""
    if act not in _CST:
        _CST[act] = _normalize2mom(torch.tanh if act else torch.sigmoid)
    return _CST[act]


def _irreps_ls(irreps):
    """The degree of every 1x le entry of an irreps (string "1x0e+1x1e+...",
    an e3nn / maloq_amd Irreps, or (mul, (l, p)) pairs), mul expanded."""
    if isinstance(irreps, str):
        out = []
        for term in irreps.replace(" ", "").split("+"):
            if not term:
                continue
            mul, ir = term.split("x") if "x" in term else ("1", term)
            out += [int(ir[:-1])] * int(mul)
        return out
    out = []
    for mul, ir in irreps:
        l = ir.l if hasattr(ir, "l") else int(ir[0])
        out += [int(l)] * int(mul)
    return out


def _product_ls(l1, l2, kind="all"):
    l3s = range(abs(l1 - l2), l1 + l2 + 1)
    if kind == "even":
        return [l for l in l3s if l % 2 == 0]
    if kind == "odd":
        return [l for l in l3s if l % 2 == 1]
    return list(l3s)


def _nodereduced_ls(ls_list, intra):
    """make_irreps_nodereduced (esen_osh.py:697-722): upper-triangle shell pairs,
    and on the diagonal the even irreps only with reduce_node_intra."""
    out = []
    for i, li in enumerate(ls_list):
        for j, lj in enumerate(ls_list):
            if i == j:
                out += _product_ls(li, lj, "even" if intra else "all")
            elif i < j:
                out += _product_ls(li, lj)
    return out


def _expand_tables(ls_list, intra):
    """get_reduced_to_all_indices / get_parity_multiplier (irreps_utils.py:163-211):
    label column -> node-reduced column (-1: zero) and its sign."""
    red, idx = {}, 0
    for i, li in enumerate(ls_list):
        for j, lj in enumerate(ls_list):
            if i <= j:
                for l in _product_ls(li, lj, "even" if (i == j and intra) else "all"):
                    red[(i, j, l)] = idx
                    idx += 2 * l + 1
    src, sign = [], []
    for i, li in enumerate(ls_list):
        for j, lj in enumerate(ls_list):
            for l in _product_ls(li, lj):
                n = 2 * l + 1
                key = (i, j, l) if i <= j else (j, i, l)
                if key not in red:  # odd self-interaction irreps removed by reduce_node_intra
                    src += [-1] * n
                    sign += [0.0] * n
                    continue
                flip = i > j and ((l % 2 == 0) if (li + lj) % 2 == 1 else (l % 2 == 1))
                src += range(red[key], red[key] + n)
                sign += [-1.0 if flip else 1.0] * n
    return np.asarray(src, np.int64), np.asarray(sign, np.float32)


def _label_to_z(ls, lmax):
    """For irreps entries 1x l e in the order ``ls`` (the labels'), the column of
    the GEMM output buffer Z each label column reads: Z holds per degree l the
    block [2l+1, mul_l] (m-major, straight from the GEMM), and the k-th entry of
    degree l (in label order) is copy k -- the l-sorted order of get_output_permutation
    (esen_osh.py:833-880)."""
    mul = [sum(1 for l in ls if l == k) for k in range(lmax + 1)]
    zoff = np.concatenate([[0], np.cumsum([(2 * l + 1) * mul[l] for l in range(lmax + 1)])])
    seen = [0] * (lmax + 1)
    cols = []
    for l in ls:
        v = seen[l]
        seen[l] += 1
        cols += [int(zoff[l] + m * mul[l] + v) for m in range(2 * l + 1)]
    return np.asarray(cols, np.int64), mul, int(zoff[-1])


def _edgereduced(ls_list):
    """make_irreps_edgereduced (esen_osh.py:733-835): the alpha (symmetric) and
    beta (antisymmetric) irreps, the parity-flip label columns, and the paired
    columns of the off-diagonal shell pairs: alpha (i, j) with beta (j, i), i < j."""
    alpha, beta, flips = [], [], []
    pos = 0
    ablk, bblk = {}, {}
    at = bt = 0
    for i, li in enumerate(ls_list):
        for j, lj in enumerate(ls_list):
            prod = _product_ls(li, lj)
            dim = sum(2 * l + 1 for l in prod)
            if i == j:
                ev, od = _product_ls(li, lj, "even"), _product_ls(li, lj, "odd")
                alpha += ev
                beta += od
                at += sum(2 * l + 1 for l in ev)
                bt += sum(2 * l + 1 for l in od)
                pos += dim
            elif i < j:
                alpha += prod
                ablk[(i, j)] = range(at, at + dim)
                at += dim
                for l in prod:
                    if (l + li + lj) % 2 == 1:   # odd l of an even pair, even l of an odd pair
                        flips += range(pos, pos + 2 * l + 1)
                    pos += 2 * l + 1
            else:
                beta += prod
                bblk[(i, j)] = range(bt, bt + dim)
                bt += dim
                pos += dim
    off_a = [k for (i, j), r in ablk.items() for k in r]
    off_b = [k for (i, j) in ablk for k in bblk[(j, i)]]
    return alpha, beta, set(flips), off_a, off_b


def _remix(ls_a, ls_b, ls_list):
    """get_subspace_remix_permutation (irreps_utils.py:46-103): label column ->
    column of cat(alpha, beta) (alpha: even irreps of diagonal pairs and the
    upper pairs; beta: odd irreps of diagonal pairs and the lower pairs, in order)."""
    def starts(ls, base):
        out, cur = [], base
        for l in ls:
            out.append(cur)
            cur += 2 * l + 1
        return out
    sa, sb = starts(ls_a, 0), starts(ls_b, sum(2 * l + 1 for l in ls_a))
    perm, ia, ib = [], 0, 0
    for i, li in enumerate(ls_list):
        for j, lj in enumerate(ls_list):
            for l in _product_ls(li, lj):
                if i < j or (i == j and l % 2 == 0):
                    perm += range(sa[ia], sa[ia] + 2 * l + 1)
                    ia += 1
                else:
                    perm += range(sb[ib], sb[ib] + 2 * l + 1)
                    ib += 1
    return perm


def _edge_pair_maps(ls_list, lmax):
    """Column gathers of the reduce_edge edge labels: for label column t,
    label = A[t] + B[t] on the canonical edge and A[t] - B[t] on its reverse,
    A[t] = sa[t] Za[:, ca[t]], B[t] = sb[t] Zb[:, cb[t]] (Za, Zb: the alpha and
    beta GEMM outputs).  Follows half_edges_to_full, the output permutations,
    the Vpa +- Vpb remix, the subspace remix and the parity flips
    (esen_osh.py:918-937)."""
    ls_a, ls_b, flips, off_a, off_b = _edgereduced(ls_list)
    za, _, wa = _label_to_z(ls_a, lmax)
    zb, _, wb = _label_to_z(ls_b, lmax)
    da = sum(2 * l + 1 for l in ls_a)
    pos_a = {k: n for n, k in enumerate(off_a)}
    pos_b = {k: n for n, k in enumerate(off_b)}
    remix = _remix(ls_a, ls_b, ls_list)
    ca, sa, cb, sb = [], [], [], []
    for t, c in enumerate(remix):
        f = -1.0 if t in flips else 1.0
        if c < da:
            ka, kb, beta_sign = c, (off_b[pos_a[c]] if c in pos_a else None), 1.0
        else:
            kb = c - da
            ka, beta_sign = (off_a[pos_b[kb]] if kb in pos_b else None), (-1.0 if kb in pos_b else 1.0)
        ca.append(int(za[ka]) if ka is not None else -1)
        sa.append(f if ka is not None else 0.0)
        cb.append(int(zb[kb]) if kb is not None else -1)
        sb.append(f * beta_sign if kb is not None else 0.0)
    return (ca, sa, wa), (cb, sb, wb), ls_a, ls_b


def _reverse_edges(edge_index):
    """create_half_antisym_edge_pairs (esen_osh.py:1090-1110): the reverse of
    every edge and the canonical half (index below its reverse's); every edge
    must have its reverse."""
    src, dst = edge_index[0].long(), edge_index[1].long()
    k = int(edge_index.max()) + 1 if edge_index.numel() else 1
    perm_orig = torch.sort(src * k + dst)[1]
    perm_flip = torch.sort(dst * k + src)[1]
    rev = perm_flip[torch.argsort(perm_orig)]
    if not bool(((src[rev] == dst) & (dst[rev] == src)).all()):
        raise ValueError("reduce_edge needs every edge (i, j) to come with its reverse (j, i)")
    half = torch.nonzero(torch.arange(src.numel(), device=src.device) < rev)[:, 0]
    return rev, half


class _ColumnMap:
    """Device tables of a signed column gather out[:, t] = sign[t] Z[:, src[t]]
    and the CSR of its transpose (for the fixed-order gradient)."""

    def __init__(self, src, sign, width, device):
        src = np.asarray(src, np.int64)
        sign = np.asarray(sign, np.float32)
        self.t, self.width = len(src), int(width)
        self.src = torch.as_tensor(src.astype(np.int32), device=device)
        self.sign = torch.as_tensor(sign, device=device)
        keep = np.nonzero((src >= 0) & (sign != 0))[0]
        order = keep[np.argsort(src[keep], kind="stable")]
        counts = np.bincount(src[order], minlength=self.width) if len(order) else np.zeros(self.width, np.int64)
        self.ptr = torch.as_tensor(np.concatenate([[0], np.cumsum(counts)]).astype(np.int32), device=device)
        self.cols = torch.as_tensor(order.astype(np.int32), device=device)
        self.csign = torch.as_tensor(sign[order], device=device)


class _Gather(torch.autograd.Function):
    @staticmethod
    def forward(ctx, z, cmap):
        z = z.contiguous()
        out = torch.empty(z.shape[0], cmap.t, device=z.device, dtype=torch.float32)
        _lib.call("maloq_gather_columns", z, z.shape[1], z.shape[0], cmap.src, cmap.sign, cmap.t, out, cmap.t,
                  _lib.stream_of(z.device))
        ctx.cmap = cmap
        return out

    @staticmethod
    def backward(ctx, g):
        cmap = ctx.cmap
        g = g.contiguous()
        dz = torch.empty(g.shape[0], cmap.width, device=g.device, dtype=torch.float32)
        _lib.call("maloq_scatter_columns", g, cmap.t, g.shape[0], cmap.ptr, cmap.cols, cmap.csign, cmap.width, dz,
                  cmap.width, _lib.stream_of(g.device))
        return dz, None


class _RowLinear(torch.autograd.Function):
    """y = x W (+ b) over many rows.  The weight gradient x^T dy is a reduction
    over all rows, which the library runs as one product on a few dozen
    workgroups (2.7 ms for 97 k rows); here it is summed over fixed chunks of
    rows by one batched product (deterministic: the chunking depends only on
    the row count)."""

    @staticmethod
    def forward(ctx, x, w, b):
        ctx.save_for_backward(x, w)
        ctx.has_b = b is not None
        return torch.addmm(b, x, w) if b is not None else x @ w

    @staticmethod
    def backward(ctx, gy):
        x, w = ctx.saved_tensors
        gx = gy @ w.t() if ctx.needs_input_grad[0] else None
        gw = None
        if ctx.needs_input_grad[1]:
            rows = x.shape[0]
            nc = max(1, min(256, rows // 2048))
            k = -(-rows // nc)
            pad = nc * k - rows
            xp = torch.nn.functional.pad(x, (0, 0, 0, pad)) if pad else x
            gp = torch.nn.functional.pad(gy, (0, 0, 0, pad)) if pad else gy
            gw = torch.bmm(xp.reshape(nc, k, x.shape[1]).transpose(1, 2).contiguous(),
                           gp.reshape(nc, k, gy.shape[1]).contiguous()).sum(0)
        gb = gy.sum(0) if ctx.has_b and ctx.needs_input_grad[2] else None
        return gx, gw, gb


class _GateFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, s, lmax, act):
        out = torch.empty_like(x)
        cst = _cst(act)
        _lib.call("maloq_irreps_gate_fwd", x, x.shape[0], lmax, x.shape[2], s, cst, act, out,
                  _lib.stream_of(x.device))
        ctx.save_for_backward(x, s)
        ctx.lmax, ctx.act = lmax, act
        return out

    @staticmethod
    def backward(ctx, g):
        x, s = ctx.saved_tensors
        g = g.contiguous()
        dx, ds = torch.empty_like(x), torch.empty_like(s)
        _lib.call("maloq_irreps_gate_bwd", x, x.shape[0], ctx.lmax, x.shape[2], s, _cst(ctx.act), ctx.act, g, dx,
                  ds, _lib.stream_of(x.device))
        return dx, ds, None, None


class E3Linear(nn.Module):
    """e3nn.o3.Linear for mul_in x le -> mul_out x le (one path): ``weight`` flat
    [mul_in * mul_out] (viewed [mul_in, mul_out], N(0, 1) init), output divided
    by sqrt(mul_in); ``bias`` [mul_out] (zeros) on scalar outputs, empty else."""

    def __init__(self, mul_in, mul_out, l, biases=True):
        super().__init__()
        self.mul_in, self.mul_out, self.l = mul_in, mul_out, l
        self.weight = nn.Parameter(torch.randn(mul_in * mul_out))
        self.bias = nn.Parameter(torch.zeros(mul_out if (biases and l == 0) else 0))

    def matrix(self):
        return self.weight.view(self.mul_in, self.mul_out) / math.sqrt(self.mul_in)


class _GateModule(nn.Module):
    """Placeholder for the reference's e3nn Gate (no parameters); the gate runs
    in ``maloq_irreps_gate_fwd``."""


class Fock_Irreps_Head(nn.Module):
    """esen_osh.py:522-1064.  forward(emb, batch) -> (node_outputs [spins, N, T],
    edge_outputs [spins, E, T]) from emb["node_embeddings"] [N, (lmax+1)^2, C]
    and emb["edge_embeddings"]; with reduce_edge, batch.edge_index [2, E] (every
    edge with its reverse)."""

    def __init__(self, irreps_in, irreps_out, lmax, sphere_channels, reduce_edge=False, ls_list=None,
                 open_shell=False, reduce_node=False, reduce_node_intra=False, orbital_basis=None):
        super().__init__()
        if reduce_edge and not reduce_node:
            raise NotImplementedError("The case of not reducing node irreps but reducing edge irreps is "
                                      "currently not implemented")
        C, L = int(sphere_channels), int(lmax)
        self.sphere_channels, self.lmax = C, L
        self.reduce_node, self.reduce_node_intra, self.reduce_edge = reduce_node, reduce_node_intra, bool(reduce_edge)
        self._act = 1 if reduce_edge else 0
        self.irreps_out = irreps_out
        self.ls_list = None if ls_list is None else [int(l) % 10 for l in ls_list]
        self.num_spins = 2 if open_shell else 1
        self._ls_out = _irreps_ls(irreps_out)
        if max(self._ls_out) > L:
            raise ValueError(f"irreps_out reaches l = {max(self._ls_out)} > lmax = {L}")
        in_ls = _irreps_ls(irreps_in)
        if sorted(set(in_ls)) != list(range(L + 1)) or any(in_ls.count(l) != C for l in range(L + 1)):
            raise ValueError("irreps_in must be sphere_channels x le for l = 0..lmax")
        if reduce_node:
            if self.ls_list is None:
                raise ValueError("reduce_node needs ls_list")
            self._ls_node = _nodereduced_ls(self.ls_list, reduce_node_intra)
        # with reduce_edge the scalar linear and the edge layers carry no bias
        # (odd data must stay odd: not_antisym, esen_osh.py:570-575, 622)
        self.lin_scalars_learnable = nn.ModuleList([E3Linear(C, C + L * C, 0, biases=not reduce_edge)
                                                    for _ in range(self.num_spins)])
        self.gate = nn.ModuleList([_GateModule() for _ in range(self.num_spins)])

        def layers(ls, biases=True):
            mul = [sum(1 for x in ls if x == l) for l in range(L + 1)]
            return nn.ModuleList([nn.ModuleList([E3Linear(C, mul[l], l, biases=biases) for l in range(L + 1)])
                                  for _ in range(self.num_spins)])
        if reduce_edge:
            (self._map_a, self._map_b, ls_a, ls_b) = _edge_pair_maps(self.ls_list, L)
            if len(self._map_a[0]) != sum(2 * l + 1 for l in self._ls_out):
                raise ValueError("the edge-pair irreps do not rebuild irreps_out (ls_list mismatch)")
            self.node_lin_out_layers = layers(self._ls_node)
            self.edge_lin_out_layers = nn.ModuleDict({"alpha": layers(ls_a, biases=False),
                                                      "beta": layers(ls_b, biases=False)})
        elif reduce_node:
            self.node_lin_out_layers = layers(self._ls_node)
            self.edge_lin_out_layers = layers(self._ls_out)
        else:
            self.lin_out_layers = layers(self._ls_out)
        self._maps = {}

    # ---------------------------------------------------------------- tables
    def _column_map(self, stream, device):
        key = (stream, str(device))
        if key not in self._maps:
            if stream == "node" and self.reduce_node:
                zcol, _, width = _label_to_z(self._ls_node, self.lmax)
                red_src, sign = _expand_tables(self.ls_list, self.reduce_node_intra)
                src = np.where(red_src >= 0, zcol[np.maximum(red_src, 0)], -1)
            else:
                src, _, width = _label_to_z(self._ls_out, self.lmax)
                sign = np.ones(len(src), np.float32)
            if len(src) != sum(2 * l + 1 for l in self._ls_out):
                raise ValueError("the reduced node irreps do not expand to irreps_out (ls_list mismatch)")
            self._maps[key] = _ColumnMap(src, sign, width, device)
        return self._maps[key]

    def _pair_maps(self, device):
        key = ("pairs", str(device))
        if key not in self._maps:
            self._maps[key] = tuple(_ColumnMap(c, s, w, device) for c, s, w in (self._map_a, self._map_b))
        return self._maps[key]

    # ---------------------------------------------------------------- compute
    def _z(self, x, lin_layers, spin):
        """s = lin_scalars(x_0), gate, per-l linear into Z [rows, sum_l (2l+1) mul_l]
        (m-major per degree)."""
        _lib.require_cuda(x)
        if x.dtype != torch.float32 or x.dim() != 3 or x.shape[1] != (self.lmax + 1) ** 2 \
                or x.shape[2] != self.sphere_channels:
            raise ValueError(f"embeddings must be float32 [rows, {(self.lmax + 1) ** 2}, {self.sphere_channels}]")
        x = x.contiguous()
        ls = self.lin_scalars_learnable[spin]
        s = _RowLinear.apply(x[:, 0, :], ls.matrix(), ls.bias if ls.bias.numel() else None)
        g = _GateFn.apply(x, s.contiguous(), self.lmax, self._act)
        # one flat [rows (2l+1), C] x [C, mul_l] GEMM per degree: split (its
        # backward is one concatenation) rather than slices of g (whose
        # gradients would each be a zero-filled full-size tensor, summed), and
        # no batched [2l+1, C] products per row
        gl = torch.split(g, [2 * l + 1 for l in range(self.lmax + 1)], dim=1)
        rows, C = x.shape[0], x.shape[2]
        zs = []
        for l, lin in enumerate(lin_layers):
            if lin.mul_out == 0:
                continue
            y = _RowLinear.apply(gl[l].reshape(rows * (2 * l + 1), C), lin.matrix(), None)   # [rows (2l+1), mul_l]
            if l == 0 and lin.bias.numel():
                y = y + lin.bias
            zs.append(y.view(rows, (2 * l + 1) * lin.mul_out))
        return torch.cat(zs, dim=1)

    def _process(self, x, lin_layers, spin, stream):
        """Z, then the label gather."""
        return _Gather.apply(self._z(x, lin_layers, spin), self._column_map(stream, x.device))

    def _edge_pairs(self, edge_x, edge_index, spin):
        """reduce_edge: alpha / beta of the canonical half, both directions' labels."""
        rev, half = edge_index
        xh, xr = edge_x[half], edge_x[rev[half]]
        za = self._z(xh + xr, self.edge_lin_out_layers["alpha"][spin], spin)
        zb = self._z(xh - xr, self.edge_lin_out_layers["beta"][spin], spin)
        ma, mb = self._pair_maps(edge_x.device)
        a, b = _Gather.apply(za, ma), _Gather.apply(zb, mb)
        out = torch.zeros(edge_x.shape[0], a.shape[1], device=a.device, dtype=a.dtype)
        return out.index_put((half,), a + b).index_put((rev[half],), a - b)

    def forward(self, emb, batch=None):
        node_x, edge_x = emb["node_embeddings"], emb["edge_embeddings"]
        if self.reduce_edge:
            ei = batch["edge_index"] if isinstance(batch, dict) else batch.edge_index
            pairs = _reverse_edges(ei.squeeze(0).reshape(2, -1).to(edge_x.device))
        node_out, edge_out = [], []
        for spin in range(self.num_spins):
            if self.reduce_edge:
                node_out.append(self._process(node_x, self.node_lin_out_layers[spin], spin, "node"))
                edge_out.append(self._edge_pairs(edge_x, pairs, spin))
            elif self.reduce_node:
                node_out.append(self._process(node_x, self.node_lin_out_layers[spin], spin, "node"))
                edge_out.append(self._process(edge_x, self.edge_lin_out_layers[spin], spin, "edge"))
            else:
                node_out.append(self._process(node_x, self.lin_out_layers[spin], spin, "common"))
                edge_out.append(self._process(edge_x, self.lin_out_layers[spin], spin, "common"))
        return torch.stack(node_out), torch.stack(edge_out)
