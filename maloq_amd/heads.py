"""The energy and force heads' message pass on the fused kernels.

The reference's HELM_Energy_Head and HELM_Force_Head
(src/maloq/helm/esen_osh.py:1137-1254, :1257-1342) each run one more message
block over the backbone's node embeddings: cat(x[src], x[dst]), rotate into
the edge frame, so2_conv_1 (radial scales from x_edge) + GateActivation,
so2_conv_2, rotate back, index_add_ per destination.  The energy head keeps
the l = 0 row and maps it to per-atom energies with a two-layer MLP, summed
per molecule; the force head keeps the three l = 1 rows of its single output
channel.

Here the message block is the fused two-convolution kernel chain
(``maloq_message_edgewise_fwd`` and its backward), with the reference's dense
``wigner`` (its kept rows gathered in-kernel) or Euler angles; the per-molecule
energy sum is the deterministic segment sum (``maloq_segment_sum``) instead
of ``scatter_add``.  The kernels' second convolution writes as many channels
as the node features have: the force head's one output channel is carried as
``sphere_channels`` zero-padded channels (its real weights scattered into a
zero matrix, so gradients reach only them), and channel 0 is returned.
Parameter names match the reference, so state dicts load.
"""
from __future__ import annotations

import torch
from torch import nn

from . import _lib
from .edgewise import SO2_Convolution
from .message import CB, edgewise_block, plan_for
from .so3 import CoefficientMapping


def _check_backbone(backbone):
    if not _lib.load().maloq_message_supported(backbone.lmax, backbone.mmax):
        raise ValueError(f"no message kernels for lmax={backbone.lmax}, mmax={backbone.mmax}")
    if backbone.sphere_channels % 32 or backbone.hidden_channels % 32:
        raise ValueError("sphere_channels and hidden_channels must be multiples of 32")


def _pad_out_channels(conv, lmax, mmax, c_out, c_pad):
    """(w0, b0, [wm]) of ``conv`` with its c_out output channels per row block
    placed in the first c_out of c_pad (the rest zero); differentiable."""
    w0, b0, wm = conv.weights()
    dev = w0.device

    def rows(nblocks):
        return torch.cat([torch.arange(c_out, device=dev) + k * c_pad for k in range(nblocks)])
    w0p = torch.zeros((lmax + 1) * c_pad, w0.shape[1], device=dev, dtype=w0.dtype).index_copy(0, rows(lmax + 1), w0)
    b0p = torch.zeros((lmax + 1) * c_pad, device=dev, dtype=b0.dtype).index_copy(0, rows(lmax + 1), b0)
    wmp = []
    for m, w in zip(range(1, mmax + 1), wm):
        n = 2 * (lmax - m + 1)   # (Wr, Wi) halves of (lmax - m + 1) row blocks each
        wmp.append(torch.zeros(n * c_pad, w.shape[1], device=dev, dtype=w.dtype).index_copy(0, rows(n), w))
    return w0p, b0p, wmp


class _HeadBase(nn.Module):
    def __init__(self, backbone, out_channels):
        super().__init__()
        _check_backbone(backbone)
        self.sphere_channels = backbone.sphere_channels
        self.hidden_channels = backbone.hidden_channels
        self.lmax, self.mmax = backbone.lmax, backbone.mmax
        self.mappingReduced = CoefficientMapping(self.lmax, self.mmax)
        self.edge_channels_list = backbone.edge_channels_list
        self.so2_conv_1 = SO2_Convolution(2 * self.sphere_channels, self.hidden_channels, self.lmax, self.mmax,
                                          self.mappingReduced, internal_weights=False,
                                          edge_channels_list=self.edge_channels_list,
                                          extra_m0_output_channels=self.lmax * self.hidden_channels)
        self.so2_conv_2 = SO2_Convolution(self.hidden_channels, out_channels, self.lmax, self.mmax,
                                          self.mappingReduced, internal_weights=True)
        self.out_channels = out_channels

    def message_pass(self, emb, edge_index, plan=None, eulers=None):
        """sum over in-edges of the rotated-back two-convolution messages,
        [N, d, out_channels] (esen_osh.py:1210-1238 / :1310-1338)."""
        nodes = emb["node_embeddings"]
        x_edge = emb["x_edge"]
        if plan is None:
            plan = plan_for(edge_index, nodes.shape[0])
        wigner = emb.get("wigner") if eulers is None else None
        rad = self.so2_conv_1.rad_func(plan.sort_edges(x_edge.float()), out_dtype=nodes.dtype)
        # the kernels write output channels in blocks of 32: a head with fewer
        # (the force head's one) pads its conv2 to one block, not to sphere_channels
        pad = -(-self.out_channels // CB) * CB
        if self.out_channels == pad:
            conv2 = self.so2_conv_2.weights()
        else:
            conv2 = _pad_out_channels(self.so2_conv_2, self.lmax, self.mmax, self.out_channels, pad)
        out = edgewise_block(nodes, plan, plan.sort_edges(eulers.float()) if eulers is not None else None, rad,
                             self.so2_conv_1.weights(), conv2, self.lmax, self.mmax, wigner=wigner)
        return out[:, :, :self.out_channels]


class HELM_Energy_Head(_HeadBase):
    """esen_osh.py:1137-1254: per-molecule energies from the l = 0 row of one
    more message pass, mapped by Linear(C, 2C) -> SiLU -> Linear(2C, 1)."""

    def __init__(self, backbone):
        super().__init__(backbone, backbone.sphere_channels)
        h = 2 * self.sphere_channels
        self.linear = nn.Sequential(nn.Linear(self.sphere_channels, h, bias=True), nn.SiLU(),
                                    nn.Linear(h, 1, bias=True))

    def forward(self, emb, batch, plan=None, eulers=None):
        edge_index = batch.edge_index.squeeze(0).reshape(2, -1)
        new_embedding = self.message_pass(emb, edge_index, plan, eulers)
        energies = self.linear(new_embedding.narrow(1, 0, 1).float()).squeeze(-1).squeeze(-1)
        counts = torch.as_tensor(batch.num_atoms_in_molecule, device=energies.device).long()
        seg_ptr = torch.cat([torch.zeros(1, dtype=torch.int64, device=energies.device), torch.cumsum(counts, 0)])
        return {"energies": _MoleculeSum.apply(energies, seg_ptr)}


class HELM_Force_Head(_HeadBase):
    """esen_osh.py:1257-1342: per-atom forces, the l = 1 rows of one more
    message pass with a single output channel."""

    def __init__(self, backbone):
        super().__init__(backbone, 1)

    def forward(self, emb, batch, plan=None, eulers=None):
        edge_index = batch.edge_index.squeeze(0).reshape(2, -1)
        new_embedding = self.message_pass(emb, edge_index, plan, eulers)
        return {"forces": new_embedding.narrow(1, 1, 3).squeeze(-1)}


class _MoleculeSum(torch.autograd.Function):
    """Per-molecule sums of per-atom values (atoms grouped by molecule, seg_ptr
    the CSR of the groups): scatter_add in a fixed order."""

    @staticmethod
    def forward(ctx, values, seg_ptr):
        nseg = seg_ptr.shape[0] - 1
        v = values.float().contiguous().reshape(-1, 1)
        out = torch.empty(nseg, 1, device=v.device, dtype=torch.float32)
        if nseg:
            perm = torch.arange(v.shape[0], device=v.device)
            seg = seg_ptr.contiguous()          # alive across the launch
            _lib.call("maloq_segment_sum", _lib.ptr(v), _lib.ptr(perm), _lib.ptr(seg), nseg, 1,
                      _lib.ptr(out), _lib.stream_of(v.device))
        counts = seg_ptr[1:] - seg_ptr[:-1]
        ctx.save_for_backward(counts)
        ctx.n, ctx.dtype = values.shape[0], values.dtype
        return out.reshape(-1)

    @staticmethod
    def backward(ctx, g):
        (counts,) = ctx.saved_tensors
        return torch.repeat_interleave(g, counts, output_size=ctx.n).to(ctx.dtype), None
