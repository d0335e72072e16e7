"""CPU restatement of the SO(2) layers and the gate (test oracle only).

* ``so2_m_conv``        so2_layers.py:61-67 (complex +-m mix of one Linear)
* ``so2_convolution``   so2_layers.py:139-214 (radial output supplied by caller)
* ``gate_activation_m`` activation.py:39-77 (outer_dim='m'), expand index from
                        esen_block.py:66-75
* ``gaussian_smearing`` radial.py:44-60
"""
from __future__ import annotations

import torch


def so2_m_conv(x_m, weight):
    """x_m [E, 2, K]; weight [2*half, K] (fc.weight, no bias)."""
    y = x_m @ weight.T
    half = weight.shape[0] // 2
    x_r, x_i = y[..., :half], y[..., half:]
    y_r = x_r[:, 0:1] - x_i[:, 1:2]
    y_i = x_r[:, 1:2] + x_i[:, 0:1]
    return torch.cat((y_r, y_i), dim=1)


def so2_convolution(x, rad, w0, b0, wm, m_size, c_out, extra=None):
    """x [E, d', C_in] m-major; rad [E, sum K] or None; w0 [N0, K0]; b0 [N0] or None;
    wm[m-1] [2*(L-m+1)*c_out, (L-m+1)*C_in].  Returns out [E, d', c_out] (and the
    extra m=0 outputs when ``extra``)."""
    E = x.shape[0]
    out = []
    x0 = x[:, : m_size[0]].reshape(E, -1)
    k0 = x0.shape[1]
    if rad is not None:
        x0 = x0 * rad[:, :k0]
    y0 = x0 @ w0.T
    if b0 is not None:
        y0 = y0 + b0
    y0_extra = None
    if extra:
        y0_extra = y0[:, :extra]
        y0 = y0[:, extra:]
    out.append(y0.reshape(E, -1, c_out))
    offset, offset_rad = m_size[0], k0
    for m in range(1, len(m_size)):
        xm = x[:, offset: offset + 2 * m_size[m]].reshape(E, 2, -1)
        km = xm.shape[2]
        if rad is not None:
            xm = xm * rad[:, offset_rad: offset_rad + km].reshape(E, 1, km)
        ym = so2_m_conv(xm, wm[m - 1])
        out.append(ym.reshape(E, -1, c_out))
        offset += 2 * m_size[m]
        offset_rad += km
    out = torch.cat(out, dim=1)
    return (out, y0_extra) if extra else out


def gate_expand_index(mapping):
    """l of every m-major row (minus 1), skipping row 0 (esen_block.py:66-75, activation.py:39-47)."""
    l_to_m = mapping.l_harmonic[torch.argmax(mapping.to_m, dim=1)]
    return (l_to_m[1:] - 1).long()


def gate_activation_m(gating, x, expand_index, lmax):
    """activation.py:57-77: silu on row 0, tanh(gate)[l-1] on the other rows."""
    E, _, H = x.shape
    g = torch.tanh(gating).reshape(E, lmax, H)
    g = torch.index_select(g, 1, expand_index)
    s = torch.nn.functional.silu(x[:, 0:1])
    return torch.cat((s, x[:, 1:] * g), dim=1)


def gaussian_smearing(dist, start, stop, num, width=1.0):
    """radial.py:44-60."""
    offset = torch.linspace(start, stop, num, dtype=torch.float64)
    coeff = -0.5 / (width * (offset[1] - offset[0])).item() ** 2
    d = dist.reshape(-1, 1).to(torch.float64) - offset.reshape(1, -1)
    return torch.exp(coeff * d ** 2)


def radial_mlp(x, hidden, w_out, b_out, eps=1e-5):
    """radial.py:115-142 (RadialMLP): per hidden layer (W, b, gamma, beta)
    z = x W^T + b; LayerNorm over the last axis with the biased variance,
    (z - mean) / sqrt(var + eps) * gamma + beta; SiLU(a) = a / (1 + exp(-a));
    then the output Linear.  Written out in fp64 (differentiable by autograd)."""
    u = x.to(torch.float64)
    for w, b, g, bt in hidden:
        z = u @ w.to(torch.float64).T + b.to(torch.float64)
        mean = z.mean(dim=-1, keepdim=True)
        var = ((z - mean) ** 2).mean(dim=-1, keepdim=True)
        a = (z - mean) / torch.sqrt(var + eps) * g.to(torch.float64) + bt.to(torch.float64)
        u = a / (1.0 + torch.exp(-a))
    return u @ w_out.to(torch.float64).T + b_out.to(torch.float64)
