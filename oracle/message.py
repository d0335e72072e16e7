"""CPU restatement of the Edgewise message block (test oracle only).

Follows ``Edgewise.forward_node`` / ``forward_edge`` (esen_block.py:146-258):
gather -> bmm(wigner) -> einsum(to_m) -> SO(2) conv [-> gate -> SO(2) conv]
-> einsum(to_m^T) -> bmm(wigner_inv) -> index_add_ on dst.

The reference only runs mmax == lmax.  For mmax < lmax this restatement keeps
the rows ``coefficient_idx(lmax, mmax)`` of D x (the eSCN rule the reference
half-carries, so3.py:126-159 / esen_block.py:108) and rotates back with the
matching columns of D^T; for mmax == lmax it is exactly the reference.
"""
from __future__ import annotations

import torch

from .rotation import eulers_to_wigner
from .so2 import gate_activation_m, gate_expand_index, so2_convolution
from .so3 import CoefficientMapping


def rotate_in(x_message, wigner, mapping, out_mask):
    """bmm(wigner[:, mask, :], x) then l-major -> m-major (esen_block.py:181,184)."""
    y = torch.bmm(wigner[:, out_mask, :], x_message)
    return torch.einsum("nac,ba->nbc", y, mapping.to_m.to(y.dtype))


def rotate_out(x_m, wigner_inv, mapping, out_mask):
    """m-major -> l-major, then bmm(wigner_inv[:, :, mask], x) (esen_block.py:188,191)."""
    y = torch.einsum("nac,ab->nbc", x_m, mapping.to_m.to(x_m.dtype))
    return torch.bmm(wigner_inv[:, :, out_mask].contiguous(), y)


def message_block(
    x,
    edge_index,
    eulers,
    Jd,
    lmax,
    mmax,
    conv1,
    rad=None,
    conv2=None,
    gate=False,
    concat="source",
    x_message_edge=None,
    reduce=True,
):
    """One fused block.  ``conv1``/``conv2`` are dicts with w0, b0, wm, c_out.

    concat: "source" (x[src]), "source-target" (cat(x[src], x[dst])), or
    "source-target-message" (plus x_message_edge), esen_block.py:170-178.
    Returns node output [N, d, C_out] (reduce=True) or the per-edge message.
    """
    src, dst = edge_index[0], edge_index[1]
    parts = [x[src]]
    if concat in ("source-target", "source-target-message"):
        parts.append(x[dst])
    if concat == "source-target-message":
        parts.append(x_message_edge)
    msg = torch.cat(parts, dim=2) if len(parts) > 1 else parts[0]
    wigner = eulers_to_wigner(eulers, 0, lmax, Jd)
    wigner_inv = wigner.transpose(1, 2).contiguous()
    mapping = CoefficientMapping(lmax, mmax)
    full = CoefficientMapping(lmax, lmax)
    out_mask = full.coefficient_idx(lmax, mmax)
    y = rotate_in(msg, wigner, mapping, out_mask)
    extra = lmax * conv1["c_out"] if gate else None
    r = so2_convolution(y, rad, conv1["w0"], conv1.get("b0"), conv1["wm"], mapping.m_size,
                        conv1["c_out"], extra=extra)
    if gate:
        y, g = r
        y = gate_activation_m(g, y, gate_expand_index(mapping), lmax)
    else:
        y = r
    if conv2 is not None:
        y = so2_convolution(y, None, conv2["w0"], conv2.get("b0"), conv2["wm"], mapping.m_size,
                            conv2["c_out"])
    m = rotate_out(y, wigner_inv, mapping, out_mask)
    if not reduce:
        return m
    out = torch.zeros((x.shape[0],) + m.shape[1:], dtype=m.dtype)
    out.index_add_(0, dst, m)
    return out
