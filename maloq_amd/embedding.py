"""EdgeDegreeEmbedding of the eSEN backbone on MI355X.

The reference (src/maloq/helm/nn/embedding.py:17-141) turns the edge scalars
into the initial node embedding: ``RadialMLP(x_edge)`` gives one coefficient
per degree l (the m = 0 rows), these are zero-padded to the m-major rows,
permuted to l-major (``einsum`` with ``to_m``), rotated back with
``bmm(wigner_inv)`` and summed into the destination nodes
(``x.index_add_(0, dst, emb / rescale_factor)``), or returned per edge.

Here the radial function is the fused HIP :class:`~maloq_amd.radial.RadialMLP`
and the rest is two launches, each a ``maloq_hip`` operator: ``edge_m0_rows``
(the m = 0 row of every block of D, the only part of ``wigner_inv`` that meets
a non-zero) and ``edge_degree_embed`` (each edge adds a rank-one product per degree; the
node sum runs per node in the stable dst-sorted order, deterministic, no
atomics).  ``wigner_inv`` may be the
reference's dense ``[E, d, d]`` tensor, or ``None`` with ``eulers=`` (the
Euler-angle triple of :func:`maloq_amd.wigner.extract_euler_angles`), in which
case no dense Wigner matrix is formed at all.  There is no CPU path.
"""
from __future__ import annotations

import copy

import torch
from torch import nn

from . import _lib
from .message import plan_for
from .radial import RadialMLP

DTYPE_CODE = {torch.float32: 0, torch.bfloat16: 1}


class EdgeDegreeEmbedding(nn.Module):
    """Drop-in for the reference's EdgeDegreeEmbedding (embedding.py:17-141):
    same constructor arguments, attributes and ``rad_func`` parameters."""

    def __init__(self, sphere_channels: int, lmax: int, mmax: int, max_num_elements: int,
                 edge_channels_list, rescale_factor, cutoff, mappingReduced, out_mask) -> None:
        super().__init__()
        self.sphere_channels = sphere_channels
        self.lmax = lmax
        self.mmax = mmax
        self.mappingReduced = mappingReduced
        self.m_0_num_coefficients: int = self.mappingReduced.m_size[0]
        self.m_all_num_coefficents: int = len(self.mappingReduced.l_harmonic)
        self.max_num_elements = max_num_elements
        self.edge_channels_list = copy.deepcopy(edge_channels_list)
        self.edge_channels_list.append(self.m_0_num_coefficients * self.sphere_channels)
        self.rad_func = RadialMLP(self.edge_channels_list)
        self.rescale_factor = rescale_factor
        self.out_mask = out_mask

    def forward(self, x, x_edge, edge_distance, edge_index, wigner_inv, node_or_edge="node",
                partition=None, eulers=None, plan=None):
        if partition:
            raise NotImplementedError("partitioned (multi-GPU) graphs are not supported on one GPU")
        u = self.rad_func(x_edge)
        return edge_degree_embed(x, u, edge_index, wigner_inv, self.lmax, self.rescale_factor,
                                 node_or_edge, eulers=eulers, plan=plan)


def edge_degree_embed(x, u, edge_index, wigner_inv, lmax, rescale_factor, node_or_edge="node",
                      eulers=None, plan=None):
    """The embedding of the radial rows ``u [E, (lmax+1) C]``.

    node: ``x.index_add_(0, edge_index[1], emb / rescale_factor)``, returning x
    (updated in place when no gradient is needed, as the reference does).
    edge: ``emb [E, d, C]`` in the dtype of x.  ``plan``: a MessagePlan of the
    graph (built here when not given)."""
    _lib.require_cuda(u)
    if node_or_edge not in ("node", "edge"):
        raise ValueError("node_or_edge must be 'node' or 'edge'")
    if (wigner_inv is None) == (eulers is None):
        raise ValueError("give exactly one of wigner_inv and eulers")
    d = (lmax + 1) ** 2
    E = u.shape[0]
    if u.dim() != 2 or u.shape[1] % (lmax + 1):
        raise ValueError(f"u must be [E, {lmax + 1} * C]")
    C = u.shape[1] // (lmax + 1)
    if x.dtype not in DTYPE_CODE or u.dtype not in DTYPE_CODE:
        raise ValueError("x and u must be fp32 or bf16")
    if x.dim() != 3 or x.shape[1] != d or x.shape[2] != C:
        raise ValueError(f"x must be [N, {d}, {C}]")
    if wigner_inv is not None:
        wigner_inv = wigner_inv.float().contiguous()
        if tuple(wigner_inv.shape) != (E, d, d):
            raise ValueError(f"wigner_inv must be [{E}, {d}, {d}]")
        eul = None
    else:
        eul = eulers.float().contiguous()
        if tuple(eul.shape) != (E, 3):
            raise ValueError(f"eulers must be [{E}, 3]")
    node = node_or_edge == "node"
    if node and plan is None:
        plan = plan_for(edge_index, x.shape[0])
    rows = _m0_rows(wigner_inv, eul, lmax, E, u.device)
    need = torch.is_grad_enabled() and (u.requires_grad or (node and x.requires_grad))
    if not need:
        with torch.no_grad():
            return _forward(x, u.contiguous(), rows, lmax, C, float(rescale_factor), node, plan, in_place=node)
    dst = edge_index[1].long().contiguous() if node else None
    return _EmbedFn.apply(x, u, rows, lmax, C, float(rescale_factor), node, plan, dst)


def _m0_rows(wigner_inv, eul, lmax, E, dev):
    """rows [E, d]: the m = 0 row of every block of D."""
    from . import ops
    return ops.edge_m0_rows(wigner_inv, eul, lmax, E)


def _forward(x, u, rows, lmax, C, rescale, node, plan, in_place):
    from . import ops
    if node and in_place and x.is_contiguous():
        ops.edge_degree_embed_(x, u, rows, plan.seg_ptr, plan.perm, lmax, C, rescale)
        return x
    out = ops.edge_degree_embed(x, u, rows, plan.seg_ptr if node else None, plan.perm if node else None,
                                lmax, C, rescale, node)
    if node and in_place:
        x.copy_(out)
        return x
    return out


class _EmbedFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, u, rows, lmax, C, rescale, node, plan, dst):
        out = _forward(x, u.contiguous(), rows, lmax, C, rescale, node, plan, in_place=False)
        ctx.lmax, ctx.C, ctx.rescale, ctx.node, ctx.u_dtype = lmax, C, rescale, node, u.dtype
        ctx.dst = dst
        ctx.save_for_backward(rows)
        return out

    @staticmethod
    def backward(ctx, g):
        from . import ops
        (rows,) = ctx.saved_tensors
        grad_u = None
        if ctx.needs_input_grad[1]:
            grad_u = ops.edge_degree_embed_bwd(g, ctx.dst, rows, ctx.lmax, ctx.C,
                                               1.0 / ctx.rescale if ctx.node else 1.0).to(ctx.u_dtype)
        grad_x = g if (ctx.node and ctx.needs_input_grad[0]) else None
        return grad_x, grad_u, None, None, None, None, None, None, None
