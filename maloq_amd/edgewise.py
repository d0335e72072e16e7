"""Edgewise message block of the eSEN backbone (two SO(2) convolutions) on MI355X.

The reference (src/maloq/helm/esen_block.py:37-258) forms the message
``cat(x[src], x[dst])``, rotates it into the edge frame, runs
``so2_conv_1`` (radial scales from ``x_edge``, lmax * hidden extra m = 0
outputs), ``GateActivation``, ``so2_conv_2`` (internal weights), rotates back
and sums per destination node (``forward_node``) or returns the per-edge
messages (``forward_edge``).

Here the whole chain is one C-ABI call, ``maloq_message_edgewise_fwd``: the
prep kernel gathers both halves of the message and rotates them, the first
GEMM applies the gate in its epilogue and leaves the rows in the edge frame,
the second GEMM rotates back and sums per segment.  The backward
(``maloq_message_edgewise_bwd_dx`` plus the weight-gradient kernels) gives
the gradients of x, of both convolutions' weights and of the radial
function's parameters (through ``rad_func``).  The Wigner rows come from the
reference's own dense ``wigner`` argument (its kept rows gathered once per
call, ``maloq_message_wigner_rows``; ``wigner_inv``, its transpose, is not
read) or, with ``eulers=`` (as from
:func:`maloq_amd.wigner.extract_euler_angles`), are built inside the prep
kernel with no dense [E, d, d] in HBM.  Built for (lmax, mmax) in (2, 2),
(4, 2), (4, 4), (6, 2), (6, 6); the reference's models use mmax = lmax
(training_workflow.py:510-511).
"""
from __future__ import annotations

import copy
import math

import torch
from torch import nn

from . import _lib
from .message import edgewise_block, plan_for, rad_width
from .radial import RadialMLP


class SO2_m_Conv(nn.Module):
    """Weights of one order m (so2_layers.py:19-68): ``fc`` [2 (lmax-m+1) c_out,
    (lmax-m+1) c_in], no bias, initialised scaled by 1/sqrt(2) as there."""

    def __init__(self, m, sphere_channels, m_output_channels, lmax, mmax) -> None:
        super().__init__()
        self.m, self.sphere_channels, self.m_output_channels = m, sphere_channels, m_output_channels
        self.lmax, self.mmax = lmax, mmax
        assert mmax >= m
        n = lmax - m + 1
        self.out_channels_half = m_output_channels * n
        self.fc = nn.Linear(n * sphere_channels, 2 * self.out_channels_half, bias=False)
        self.fc.weight.data.mul_(1 / math.sqrt(2))


class SO2_Convolution(nn.Module):
    """Weights of one SO(2) convolution (so2_layers.py:71-214): ``fc_m0``
    (with the extra m = 0 outputs first), ``so2_m_conv``, and ``rad_func``
    when the radial scales come from the edge features (internal_weights
    False).  The arithmetic runs in the fused kernels."""

    def __init__(self, sphere_channels, m_output_channels, lmax, mmax, mappingReduced, internal_weights=True,
                 edge_channels_list=None, extra_m0_output_channels=None) -> None:
        super().__init__()
        self.sphere_channels, self.m_output_channels = sphere_channels, m_output_channels
        self.lmax, self.mmax, self.mappingReduced = lmax, mmax, mappingReduced
        self.internal_weights = internal_weights
        self.edge_channels_list = copy.deepcopy(edge_channels_list)
        self.extra_m0_output_channels = extra_m0_output_channels
        n0 = (lmax + 1) * sphere_channels
        self.fc_m0 = nn.Linear(n0, m_output_channels * (lmax + 1) + (extra_m0_output_channels or 0), bias=True)
        self.so2_m_conv = nn.ModuleList(
            [SO2_m_Conv(m, sphere_channels, m_output_channels, lmax, mmax) for m in range(1, mmax + 1)])
        self.rad_func = None
        if not internal_weights:
            assert self.edge_channels_list is not None
            self.edge_channels_list.append(rad_width(lmax, mmax, sphere_channels))
            self.rad_func = RadialMLP(self.edge_channels_list)

    def weights(self):
        return (self.fc_m0.weight, self.fc_m0.bias, [c.fc.weight for c in self.so2_m_conv])


class Edgewise(nn.Module):
    """Drop-in for the reference's Edgewise (esen_block.py:37-258): same
    constructor arguments and parameter names (``so2_conv_1.*``,
    ``so2_conv_2.*``); message_type "source-target" or "source-target-message"
    (then ``x_message_edge`` [E, d, sphere_channels] is the third part)."""

    def __init__(self, sphere_channels, hidden_channels, lmax, mmax, edge_channels_list, mappingReduced, SO3_grid,
                 cutoff, message_type, act_type="gate", include_edges=True) -> None:
        super().__init__()
        self.sphere_channels, self.hidden_channels = sphere_channels, hidden_channels
        self.lmax, self.mmax = lmax, mmax
        self.mappingReduced, self.SO3_grid = mappingReduced, SO3_grid
        self.edge_channels_list = copy.deepcopy(edge_channels_list)
        self.act_type, self.include_edges = act_type, include_edges
        if act_type != "gate":
            raise ValueError(f"Unknown activation type {act_type}")
        # Refuse at construction what the kernels are not built for (instead of
        # a C-ABI error at the first forward).
        if not _lib.load().maloq_message_supported(lmax, mmax):
            raise ValueError(f"no message kernels for lmax={lmax}, mmax={mmax} "
                             "(built: (2, 2), (4, 2), (4, 4), (6, 2), (6, 6))")
        if sphere_channels % 32 or hidden_channels % 32:
            raise ValueError("sphere_channels and hidden_channels must be multiples of 32")
        if message_type == "source-target-message":
            self.concat_size = 3
        elif message_type == "source-target":
            self.concat_size = 2
        else:
            raise ValueError(f"Unknown message type {message_type}")
        self.so2_conv_1 = SO2_Convolution(self.concat_size * sphere_channels, hidden_channels, lmax, mmax,
                                          mappingReduced, internal_weights=False,
                                          edge_channels_list=self.edge_channels_list,
                                          extra_m0_output_channels=lmax * hidden_channels)
        self.so2_conv_2 = SO2_Convolution(hidden_channels, sphere_channels, lmax, mmax, mappingReduced,
                                          internal_weights=True)

    def forward(self, x, x_message_edge, x_edge, edge_index, wigner, wigner_inv, node_or_edge="node",
                partition=None, eulers=None, plan=None):
        """Node sums [N, d, sphere_channels] (node) or per-edge messages
        [E, d, sphere_channels] (edge), in the dtype of x.  ``eulers`` [E, 3]:
        the edges' Euler angles in the original edge order; ``plan``: the
        graph's MessagePlan (the cached plan of edge_index when not given)."""
        if partition:
            raise NotImplementedError("partitioned (multi-GPU) graphs are not supported on one GPU")
        if self.concat_size == 3 and x_message_edge is None:
            raise ValueError("message_type 'source-target-message' needs x_message_edge")
        if eulers is None and wigner is None:
            raise ValueError("pass the reference's dense wigner [E, d, d] or eulers= [E, 3]")
        _lib.require_cuda(x, x_edge, eulers, wigner)
        if plan is None:
            plan = plan_for(edge_index, x.shape[0])
        rad = self.so2_conv_1.rad_func(plan.sort_edges(x_edge.float()), out_dtype=x.dtype)
        # The kept rows of the dense wigner are gathered in-kernel; wigner_inv is
        # its transpose (esen_osh.py:294) and is not read.
        out = edgewise_block(x, plan, plan.sort_edges(eulers.float()) if eulers is not None else None, rad,
                             self.so2_conv_1.weights(), self.so2_conv_2.weights(), self.lmax, self.mmax,
                             node_or_edge=node_or_edge,
                             x_message_edge=x_message_edge if self.concat_size == 3 else None,
                             wigner=wigner if eulers is None else None)
        return out.to(x.dtype)
