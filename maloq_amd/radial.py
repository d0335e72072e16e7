"""RadialMLP of the SO(2) convolution on MI355X.

The reference builds the radial function of every SO2_Convolution as
``RadialMLP(edge_channels_list + [num_channels_rad])`` (helm/nn/radial.py:115-142,
helm/nn/so2_layers.py:133-137) and applies it to the edge features before the
per-m linears (so2_layers.py:152-154):

    Linear(c_0, c_1) -> LayerNorm(c_1) -> SiLU -> ... -> Linear(c_H, c_out)

:class:`RadialMLP` keeps that module structure (``net`` is the same
``nn.Sequential`` of Linear / LayerNorm / SiLU, so state dicts are
interchangeable) but its forward and backward are the fused HIP kernels of
``maloq_radial_fwd`` / ``maloq_radial_bwd``: one launch for the whole forward
(the output written directly in the message rows' dtype), three for the
backward (per-tile hidden gradients, split-K output-layer gradient, fixed-order
sums).  There is no CPU path: tensors must live on the GPU.
"""
from __future__ import annotations

import ctypes

import torch
import torch.nn.functional as F
from torch import nn

from . import _lib

DTYPE_CODE = {torch.float32: 0, torch.bfloat16: 1}


def _layers(channels_list):
    layers = []
    n = len(channels_list)
    for i in range(1, n):
        layers.append(nn.Linear(channels_list[i - 1], channels_list[i], bias=True))
        if i < n - 1:
            layers += [nn.LayerNorm(channels_list[i]), nn.SiLU()]
    return layers


class RadialMLP(nn.Module):
    """Drop-in for the reference's RadialMLP (radial.py:115-142).

    ``forward(inputs, out_dtype=None)``: inputs [E, c_0] fp32 on the GPU; the
    result is [E, c_out] in ``out_dtype`` (default fp32; bfloat16 when it
    feeds a bf16 message block)."""

    def __init__(self, channels_list) -> None:
        super().__init__()
        self.channels_list = [int(c) for c in channels_list]
        if len(self.channels_list) < 3:
            raise ValueError("RadialMLP needs at least one hidden layer: [c_0, c_1, ..., c_out]")
        self.net = nn.Sequential(*_layers(self.channels_list))

    def forward(self, inputs: torch.Tensor, out_dtype: torch.dtype | None = None) -> torch.Tensor:
        return radial_mlp(inputs, self, out_dtype)


def _params(mod: RadialMLP):
    mods = list(mod.net)
    lin = [m for m in mods if isinstance(m, nn.Linear)]
    lns = [m for m in mods if isinstance(m, nn.LayerNorm)]
    if len(lns) != len(lin) - 1:
        raise ValueError("unexpected RadialMLP structure")
    eps = lns[0].eps
    for ln in lns:
        if ln.weight is None or ln.bias is None:
            raise ValueError("RadialMLP's LayerNorms must be affine")
        if ln.eps != eps:
            raise ValueError("RadialMLP's LayerNorms must share eps")
    hidden = []
    for li, ln in zip(lin[:-1], lns):
        hidden += [li.weight, li.bias, ln.weight, ln.bias]
    return eps, hidden + [lin[-1].weight, lin[-1].bias]


def fused_supported(widths) -> bool:
    """True if the fused kernels take this channels_list: they stage one
    workgroup's layer weights, gradients and activations in LDS, which holds
    inputs up to 128 wide with small hidden layers (the benchmark's
    [8, 64, 64, out]) but not the reference's models'
    [num_distance_basis + 2 edge_channels, edge_channels, edge_channels, out]
    = [384, 128, 128, out] (esen_osh.py:189-192)."""
    widths = tuple(int(c) for c in widths)
    if len(widths) < 3:
        return False
    arr = _widths_array(widths)
    return _lib.load().maloq_radial_bwd_partials_floats(0, len(widths) - 2, arr, 1) >= 0


def radial_mlp(inputs: torch.Tensor, mod: RadialMLP, out_dtype: torch.dtype | None = None):
    """Forward (differentiable) of ``mod`` on ``inputs``.

    The leading hidden layers the fused kernels cannot hold (see
    :func:`fused_supported`) run as Linear (a plain library GEMM) ->
    LayerNorm -> SiLU in torch, as the reference's own module does; the rest,
    when any is left, are the fused kernels, which hand the gradient of their
    input to autograd.  When no hidden layer is left for them, the output
    Linear runs as a library GEMM in the output dtype (bf16 operands, fp32
    accumulation for a bf16 block), like the fused kernels' output layer."""
    dt = out_dtype or torch.float32
    if dt not in DTYPE_CODE:
        raise ValueError(f"unsupported output dtype {dt}")
    _lib.require_cuda(inputs)
    eps, params = _params(mod)
    widths = tuple(mod.channels_list)
    if inputs.dim() != 2 or inputs.shape[1] != widths[0]:
        raise ValueError(f"inputs must be [E, {widths[0]}]")
    while len(widths) >= 3 and not fused_supported(widths):
        w1, b1, g1, bt1 = params[:4]
        inputs = F.silu(F.layer_norm(F.linear(inputs.float(), w1, b1), (widths[1],), g1, bt1, eps))
        widths, params = widths[1:], params[4:]
    if len(widths) < 3:    # no hidden layer left: the output Linear alone
        if dt == torch.bfloat16:
            # in the message dtype with fp32 accumulation, as the fused kernels
            # run their output layer (hidden layers stay fp32)
            return F.linear(inputs.to(dt), params[0].to(dt), params[1].to(dt))
        return F.linear(inputs, params[0], params[1]).to(dt)
    return _RadialFn.apply(inputs, dt, widths, eps, *params)


def _widths_array(widths):
    return (ctypes.c_int * len(widths))(*widths)


class _RadialFn(torch.autograd.Function):
    """Autograd of the fused MLP through the registered operators
    maloq_hip::radial_fwd / radial_bwd."""

    @staticmethod
    def forward(ctx, x, dt, widths, eps, *params):
        from . import ops
        need = any(ctx.needs_input_grad[:1] + ctx.needs_input_grad[4:])
        out, wpack, save = ops.radial_fwd(x, list(params), list(widths), float(eps), dt == torch.bfloat16, need)
        ctx.widths, ctx.eps, ctx.dt = widths, eps, dt
        ctx.param_dtypes = [p.dtype for p in params]
        if need:
            ctx.save_for_backward(x, wpack, save, *params)
        return out

    @staticmethod
    def backward(ctx, g):
        from . import ops
        x, wpack, save, *ps = ctx.saved_tensors
        widths = ctx.widths
        nh = len(widths) - 2
        dx, gh, dwo, dbo = ops.radial_bwd(g, x, wpack, save, list(ps), list(widths), float(ctx.eps),
                                          bool(ctx.needs_input_grad[0]))
        grads = []
        off = 0
        for i in range(nh):
            c, ci = widths[i + 1], widths[i]
            grads.append(gh[off: off + c * ci].view(c, ci))
            off += c * ci
            for _ in range(3):  # bias, LayerNorm weight, LayerNorm bias
                grads.append(gh[off: off + c])
                off += c
        grads += [dwo, dbo]
        grads = [gr.to(d) for gr, d in zip(grads, ctx.param_dtypes)]
        return (dx.to(x.dtype) if ctx.needs_input_grad[0] else None, None, None, None, *grads)
