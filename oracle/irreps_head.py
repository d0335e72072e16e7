"""CPU restatement (fp64 torch) of the Fock irreps output head -- test
infrastructure only; the product is maloq_amd.irreps_head.

Reference: Fock_Irreps_Head (helm/esen_osh.py:522-1064) for reduce_edge=False,
with the index helpers of helm/common/irreps_utils.py:10-211.  e3nn is not
importable here, so its two building blocks are restated from their published
definitions (e3nn 0.5.x, e3nn.o3.Linear and e3nn.nn.Gate):

* Linear(mul_in x le -> mul_out x le): out[v, m] = sum_u W[u, v] x[u, m] /
  sqrt(mul_in), W the flat ``weight`` parameter viewed [mul_in, mul_out]; a
  ``bias`` of mul_out is added to scalar (0e) outputs only;
* Gate(irreps_gates = n x 0e, act = sigmoid, irreps_gated): each gated irrep
  copy times act(its gate), act normalised to unit second moment under
  N(0, 1) (normalize2mom: cst = E[act(z)^2]^-1/2 over 10^6 float64 normals
  drawn by a CPU generator seeded 0).

Parity unpinned: the value of that normalisation constant and e3nn's exact
parameter shapes depend on e3nn's own code, which no file here holds; the
tests pin everything else (closed forms, brute force, equivariance).
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


def process(xs, lmax, C, w_scalar, b_scalar, w_out, b_out0, cst):
    """esen_osh.py:986-1052 (reduce_edge False): lin_scalars -> Gate -> per-l Linear.
    xs: stacked [B, C d]; w_scalar [C (C + L C)] flat, b_scalar [C + L C];
    w_out[l] [C mul_l] flat, b_out0 [mul_0].  Returns [B, sum_l mul_l (2l+1)]."""
    B = xs.shape[0]
    xsc = xs[:, :C]
    s = xsc @ w_scalar.view(C, -1) / math.sqrt(C) + b_scalar
    t0, gates = s[:, :C], s[:, C:]
    gated = []
    off = C
    for l in range(1, lmax + 1):
        n = 2 * l + 1
        blk = xs[:, off:off + C * n].view(B, C, n)
        g = cst * torch.sigmoid(gates[:, (l - 1) * C:l * C])
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
        if l == 0 and mul > 0:
            y = y + b_out0.view(1, mul, 1)
        outs.append(y.reshape(B, -1))
    return torch.cat(outs, dim=1)


def head_forward(node_x, edge_x, ls_list, lmax, C, params, reduce_node, reduce_node_intra, num_spins=1):
    """Fock_Irreps_Head.forward (esen_osh.py:894-969) for reduce_edge False:
    (node_outputs [spins, N, T], edge_outputs [spins, E, T]).  ``params``:
    per spin a dict with "scalar" (w, b) and per stream ("node", "edge", or
    "common" when not reduce_node) the list of (w_l) and the l = 0 bias."""
    cst = normalize2mom_constant()
    ls_all = all_ls(ls_list)
    perm_all = output_permutation(ls_all)
    if reduce_node:
        ls_red = nodereduced_ls(ls_list, reduce_node_intra)
        perm_node = output_permutation(ls_red)
        idx, par = reduced_to_all(ls_list, reduce_node_intra)
    node_out, edge_out = [], []
    for spin in range(num_spins):
        p = params[spin]
        ws, bs = p["scalar"]
        ns = "node" if reduce_node else "common"
        es = "edge" if reduce_node else "common"
        y = process(stack_irreps(node_x), lmax, C, ws, bs, p[ns][0], p[ns][1], cst)
        y = y[:, torch.as_tensor(perm_node if reduce_node else perm_all)]
        if reduce_node:
            safe = torch.as_tensor(np.where(idx < 0, 0, idx))
            y = y[:, safe] * torch.as_tensor(par, dtype=y.dtype)
        e = process(stack_irreps(edge_x), lmax, C, ws, bs, p[es][0], p[es][1], cst)
        e = e[:, torch.as_tensor(perm_all)]
        node_out.append(y)
        edge_out.append(e)
    return torch.stack(node_out), torch.stack(edge_out)
