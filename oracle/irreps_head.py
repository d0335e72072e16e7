"""CPU restatement (fp64 torch) of the Fock irreps output head -- test
infrastructure only; the product is maloq_amd.irreps_head.

Reference: Fock_Irreps_Head (helm/esen_osh.py:522-1064), with the index helpers
of helm/common/irreps_utils.py:10-211, including reduce_edge (edge pairs
(i->j, j->i) as symmetric / antisymmetric combinations, :733-835, 894-944,
1090-1130).  e3nn is not
importable here, so its two building blocks are restated from their published
definitions (e3nn 0.5.x, e3nn.o3.Linear and e3nn.nn.Gate):

* Linear(mul_in x le -> mul_out x le): out[v, m] = sum_u W[u, v] x[u, m] /
  sqrt(mul_in), W the flat ``weight`` parameter viewed [mul_in, mul_out]; a
  ``bias`` of mul_out is added to scalar (0e) outputs only;
* Gate(irreps_gates = n x 0e, act = sigmoid, irreps_gated): each gated irrep
  copy times act(its gate), act normalised to unit second moment under
  N(0, 1) (normalize2mom: cst = E[act(z)^2]^-1/2 over 10^6 float64 normals
  drawn by a CPU generator seeded 0).

Parity unpinned: the values of those normalisation constants (sigmoid gates,
and tanh gates with reduce_edge) and e3nn's exact parameter shapes depend on
e3nn's own code, which no file here holds; the tests pin everything else
(closed forms, brute force, the CG labels of symmetric on-site blocks and of
transposed edge blocks, equivariance).
"""
from __future__ import annotations

import math

import numpy as np
import torch


def normalize2mom_constant(act=torch.sigmoid):
    gen = torch.Generator(device="cpu").manual_seed(0)
    z = torch.randn(1_000_000, generator=gen, dtype=torch.float64)
    cst = act(z).pow(2).mean().pow(-0.5).item()
    return 1.0 if abs(cst - 1.0) < 1e-4 else cst


def product_ls(l1, l2, kind="all"):
    """irreps_utils.py:32-43."""
    l3s = range(abs(l1 - l2), l1 + l2 + 1)
    if kind == "even":
        return [l for l in l3s if l % 2 == 0]
    if kind == "odd":
        return [l for l in l3s if l % 2 != 0]
    return list(l3s)


def all_ls(ls_list):
    """irreps_utils.py:106-111: the labels' irreps (every shell pair, row-major)."""
    return [l for li in ls_list for lj in ls_list for l in product_ls(li, lj)]


def nodereduced_ls(ls_list, reduce_node_intra):
    """esen_osh.py:697-722 (make_irreps_nodereduced) = irreps_utils.py:114-123."""
    ii = "even" if reduce_node_intra else "all"
    out = []
    for i, li in enumerate(ls_list):
        for j, lj in enumerate(ls_list):
            if i == j:
                out += product_ls(li, lj, ii)
            elif i < j:
                out += product_ls(li, lj)
    return out


def reduced_to_all(ls_list, reduce_node_intra):
    """(indices, parity multiplier) of expand_reduced_node: irreps_utils.py:163-211."""
    red, idx = {}, 0
    ii = "even" if reduce_node_intra else "all"
    for i, li in enumerate(ls_list):
        for j, lj in enumerate(ls_list):
            if i > j:
                continue
            for l in product_ls(li, lj, ii if i == j else "all"):
                red[(i, j, l)] = idx
                idx += 2 * l + 1
    indices, parity = [], []
    for i, li in enumerate(ls_list):
        for j, lj in enumerate(ls_list):
            for l in product_ls(li, lj):
                n = 2 * l + 1
                if (i, j, l) in red:
                    indices += range(red[(i, j, l)], red[(i, j, l)] + n)
                    parity += [1] * n
                elif i == j:  # odd self-interaction irreps removed by reduce_node_intra
                    indices += [-1] * n
                    parity += [0] * n
                else:  # lower triangle: the upper block's irreps, sign by parity
                    indices += range(red[(j, i, l)], red[(j, i, l)] + n)
                    flip = (l % 2 == 0) if (li + lj) % 2 == 1 else (l % 2 == 1)
                    parity += [-1 if flip else 1] * n
    return np.asarray(indices, np.int64), np.asarray(parity, np.float64)


def output_permutation(ls):
    """get_output_permutation (esen_osh.py:833-880) for irreps 1x l e in the order
    ``ls``: column k of the labels reads column perm[k] of the l-sorted output
    (stable sort by l; within an l, copies in their original order)."""
    order = sorted(range(len(ls)), key=lambda i: (ls[i], i))
    sorted_pos = {}
    pos = 0
    for i in order:
        sorted_pos[i] = pos
        pos += 2 * ls[i] + 1
    perm = []
    for i, l in enumerate(ls):
        perm += range(sorted_pos[i], sorted_pos[i] + 2 * l + 1)
    return np.asarray(perm, np.int64)


def mul_per_l(ls, lmax):
    return [sum(1 for l in ls if l == k) for k in range(lmax + 1)]


def stack_irreps(x):
    """esen_osh.py:971-984: [B, d, C] -> [B, C d] with each degree's block as
    [C, 2l+1] (channel-major)."""
    B, d, C = x.shape
    L = int(round(math.sqrt(d))) - 1
    return torch.cat([x[:, l * l:(l + 1) ** 2, :].transpose(1, 2).reshape(B, -1) for l in range(L + 1)], dim=1)


def process(xs, lmax, C, w_scalar, b_scalar, w_out, b_out0, cst, reduce_edge=False):
    """esen_osh.py:986-1052: lin_scalars -> Gate -> per-l Linear.
    xs: stacked [B, C d]; w_scalar [C (C + L C)] flat, b_scalar [C + L C] (None:
    no bias, as with reduce_edge); w_out[l] [C mul_l] flat, b_out0 [mul_0] or None.
    With reduce_edge the gates are tanh of the absolute gating scalars (:994-995,
    act_gates tanh at :625).  Returns [B, sum_l mul_l (2l+1)]."""
    B = xs.shape[0]
    xsc = xs[:, :C]
    s = xsc @ w_scalar.view(C, -1) / math.sqrt(C)
    if b_scalar is not None:
        s = s + b_scalar
    t0, gates = s[:, :C], s[:, C:]
    if reduce_edge:
        gates = torch.abs(gates)
    act = torch.tanh if reduce_edge else torch.sigmoid
    gated = []
    off = C
    for l in range(1, lmax + 1):
        n = 2 * l + 1
        blk = xs[:, off:off + C * n].view(B, C, n)
        g = cst * act(gates[:, (l - 1) * C:l * C])
        gated.append((blk * g.unsqueeze(-1)).reshape(B, -1))
        off += C * n
    xg = torch.cat([t0] + gated, dim=1)
    outs = []
    off = 0
    for l in range(lmax + 1):
        n = 2 * l + 1
        xl = xg[:, off:off + C * n].view(B, C, n)
        off += C * n
        mul = w_out[l].numel() // C
        y = torch.einsum("bum,uv->bvm", xl, w_out[l].view(C, mul)) / math.sqrt(C)
        if l == 0 and mul > 0 and b_out0 is not None:
            y = y + b_out0.view(1, mul, 1)
        outs.append(y.reshape(B, -1))
    return torch.cat(outs, dim=1)


def edgereduced(ls_list):
    """make_irreps_edgereduced (esen_osh.py:733-835): (ls_alpha, ls_beta,
    parity_flip_indices, off_diag alpha indices, off_diag beta indices)."""
    alpha, beta, flips = [], [], []
    ptr = 0
    for i, li in enumerate(ls_list):
        for j, lj in enumerate(ls_list):
            prod = product_ls(li, lj)
            if i == j:
                alpha += product_ls(li, lj, "even")
                beta += product_ls(li, lj, "odd")
                ptr += sum(2 * l + 1 for l in prod)
            if i < j:
                alpha += prod
                for l in prod:
                    n = 2 * l + 1
                    if ((li + lj) % 2 == 0 and l % 2 == 1) or ((li + lj) % 2 == 1 and l % 2 == 0):
                        flips += range(ptr, ptr + n)
                    ptr += n
            if j < i:
                beta += prod
                ptr += sum(2 * l + 1 for l in prod)
    a_blocks, b_blocks = {}, {}
    at = bt = 0
    for i, li in enumerate(ls_list):
        for j, lj in enumerate(ls_list):
            prod = product_ls(li, lj)
            dim = sum(2 * l + 1 for l in prod)
            if i == j:
                at += sum(2 * l + 1 for l in product_ls(li, lj, "even"))
                bt += sum(2 * l + 1 for l in product_ls(li, lj, "odd"))
            if i < j:
                a_blocks[(i, j)] = list(range(at, at + dim))
                at += dim
            if j < i:
                b_blocks[(i, j)] = list(range(bt, bt + dim))
                bt += dim
    off_a, off_b = [], []
    for (i, j), idx in a_blocks.items():
        off_a += idx
        off_b += b_blocks[(j, i)]
    return alpha, beta, np.asarray(flips, np.int64), np.asarray(off_a, np.int64), np.asarray(off_b, np.int64)


def subspace_remix(ls_alpha, ls_beta, ls_list):
    """get_subspace_remix_permutation (irreps_utils.py:46-103): label column ->
    column of cat(alpha, beta)."""
    def pool(ls, start):
        out, cur = [], start
        for l in ls:
            out.append(list(range(cur, cur + 2 * l + 1)))
            cur += 2 * l + 1
        return out
    pa = pool(ls_alpha, 0)
    pb = pool(ls_beta, sum(2 * l + 1 for l in ls_alpha))
    perm, ia, ib = [], 0, 0
    for i, li in enumerate(ls_list):
        for j, lj in enumerate(ls_list):
            for l in product_ls(li, lj):
                if (i == j and l % 2 == 0) or i < j:
                    perm += pa[ia]
                    ia += 1
                else:
                    perm += pb[ib]
                    ib += 1
    return np.asarray(perm, np.int64)


def reverse_edges(edge_index):
    """create_half_antisym_edge_pairs (esen_osh.py:1090-1110): the index of each
    edge's reverse, and the canonical half (index < its reverse's)."""
    src, dst = edge_index[0], edge_index[1]
    k = int(edge_index.max()) + 1
    perm_orig = torch.sort(src * k + dst)[1]
    perm_flip = torch.sort(dst * k + src)[1]
    rev = perm_flip[torch.argsort(perm_orig)]
    half = torch.arange(edge_index.shape[1]) < rev
    return rev, half


def head_forward(node_x, edge_x, ls_list, lmax, C, params, reduce_node, reduce_node_intra, num_spins=1,
                 reduce_edge=False, edge_index=None):
    """Fock_Irreps_Head.forward (esen_osh.py:894-969): (node_outputs [spins, N, T],
    edge_outputs [spins, E, T]).  ``params``: per spin a dict with "scalar" (w, b)
    and per stream ("node", "edge", or "common" when not reduce_node; with
    reduce_edge "node", "alpha", "beta") the list of (w_l) and the l = 0 bias
    (None where the reference has none: every bias of the reduce_edge streams
    but the node layers')."""
    cst = normalize2mom_constant(torch.tanh if reduce_edge else torch.sigmoid)
    ls_all = all_ls(ls_list)
    perm_all = output_permutation(ls_all)
    if reduce_node:
        ls_red = nodereduced_ls(ls_list, reduce_node_intra)
        perm_node = output_permutation(ls_red)
        idx, par = reduced_to_all(ls_list, reduce_node_intra)
    if reduce_edge:
        assert reduce_node, "reduce_edge needs reduce_node (esen_osh.py:597-598)"
        ls_a, ls_b, flips, off_a, off_b = edgereduced(ls_list)
        perm_a, perm_b = output_permutation(ls_a), output_permutation(ls_b)
        remix = subspace_remix(ls_a, ls_b, ls_list)
        rev, half = reverse_edges(edge_index)
        xh = edge_x[half]
        xf = edge_x[rev[half]]
        xa, xb = xh + xf, xh - xf
    node_out, edge_out = [], []
    for spin in range(num_spins):
        p = params[spin]
        ws, bs = p["scalar"]
        ns = "node" if reduce_node else "common"
        y = process(stack_irreps(node_x), lmax, C, ws, bs, p[ns][0], p[ns][1], cst, reduce_edge)
        y = y[:, torch.as_tensor(perm_node if reduce_node else perm_all)]
        if reduce_node:
            safe = torch.as_tensor(np.where(idx < 0, 0, idx))
            y = y[:, safe] * torch.as_tensor(par, dtype=y.dtype)
        if reduce_edge:
            oa = process(stack_irreps(xa), lmax, C, ws, bs, p["alpha"][0], p["alpha"][1], cst, True)
            ob = process(stack_irreps(xb), lmax, C, ws, bs, p["beta"][0], p["beta"][1], cst, True)
            E = edge_x.shape[0]
            fa = torch.zeros(E, oa.shape[1], dtype=oa.dtype)
            fb = torch.zeros(E, ob.shape[1], dtype=ob.dtype)
            fl = rev[half]
            fa = fa.index_put((torch.nonzero(half)[:, 0],), oa).index_put((fl,), oa)
            fb = fb.index_put((torch.nonzero(half)[:, 0],), ob).index_put((fl,), -ob)
            fa = fa[:, torch.as_tensor(perm_a)]
            fb = fb[:, torch.as_tensor(perm_b)]
            va = fa[:, torch.as_tensor(off_a)].clone()
            vb = fb[:, torch.as_tensor(off_b)].clone()
            fa, fb = fa.clone(), fb.clone()
            fa[:, torch.as_tensor(off_a)] = va + vb      # Vsp in place (esen_osh.py:931-932)
            fb[:, torch.as_tensor(off_b)] = va - vb      # Vps in place
            e = torch.cat([fa, fb], dim=1)[:, torch.as_tensor(remix)]
            sign = torch.ones(e.shape[1], dtype=e.dtype)
            sign[torch.as_tensor(flips)] = -1.0
            e = e * sign
        else:
            es = "edge" if reduce_node else "common"
            e = process(stack_irreps(edge_x), lmax, C, ws, bs, p[es][0], p[es][1], cst)
            e = e[:, torch.as_tensor(perm_all)]
        node_out.append(y)
        edge_out.append(e)
    return torch.stack(node_out), torch.stack(edge_out)
