"""PyTorch custom ops (namespace ``maloq_hip``) over the C ABI.

The reference's hot path is PyTorch code, so its replacement is exposed to
PyTorch's dispatcher as registered operators rather than opaque Python calls:
``torch.compile`` and other graph capture see them as single ops with known
output shapes (each has a fake implementation), and autograd goes through the
registered backward formulas.  Each op enqueues HIP kernels of
``libmaloq_hip.so`` on the current stream; there is no CPU implementation.

    maloq_hip::edge_euler(edge_vec, seed)                 extract_euler_angles
    maloq_hip::wigner_from_euler(eulers, lmax, inverse)   eulers_to_wigner (dense D or D^T)
    maloq_hip::rotate(x, eulers, gather?, lmax, inverse)  bmm(wigner, x[src]) / bmm(wigner_inv, z)
    maloq_hip::segment_sum(msg, perm, seg_ptr, n)         index_add_ in a fixed order
    maloq_hip::label_transform(x, ..)                     get_net_out / get_H on label rows
    maloq_hip::message_block(x, rad?, w0, b0?, wm, plan tensors, eulers, lmax, mmax, gate)
                                                          Edgewise.forward_node with one convolution

Reference interfaces: helm/triton_kernels/wigner_fused.py:383-486,
helm/common/rotation.py:19-39, helm/esen_block.py:146-208,
fock_utils/utils_tensor_decomp.py:154-169.
"""
from __future__ import annotations

from typing import List, Optional

import torch
from torch import Tensor
from torch.library import custom_op, register_fake

from . import _lib
from . import message as M
from .rotate import _scatter_rows, rotate as _rotate


# ------------------------------------------------------------------ Wigner
@custom_op("maloq_hip::edge_euler", mutates_args=())
def edge_euler(edge_vec: Tensor, seed: int) -> Tensor:
    from .wigner import extract_euler_angles
    return extract_euler_angles(edge_vec, seed)


@register_fake("maloq_hip::edge_euler")
def _(edge_vec, seed):
    return edge_vec.new_empty(edge_vec.shape[0], 3)


@custom_op("maloq_hip::wigner_from_euler", mutates_args=())
def wigner_from_euler(eulers: Tensor, lmax: int, inverse: bool) -> Tensor:
    from .wigner import wigner_from_eulers
    return wigner_from_eulers(eulers, None, lmax, inverse=inverse)


@register_fake("maloq_hip::wigner_from_euler")
def _(eulers, lmax, inverse):
    d = (lmax + 1) ** 2
    return eulers.new_empty(eulers.shape[0], d, d)


# ---------------------------------------------------------------- rotation
@custom_op("maloq_hip::rotate", mutates_args=())
def rotate(x: Tensor, eulers: Tensor, gather: Optional[Tensor], lmax: int, inverse: bool) -> Tensor:
    return _rotate(x, lmax, eulers=eulers, gather=gather, inverse=inverse)


@register_fake("maloq_hip::rotate")
def _(x, eulers, gather, lmax, inverse):
    return x.new_empty(eulers.shape[0], x.shape[1], x.shape[2])


def _rotate_setup(ctx, inputs, output):
    x, eulers, gather, lmax, inverse = inputs
    ctx.save_for_backward(eulers, gather)
    ctx.lmax, ctx.inverse, ctx.n_x, ctx.x_dtype = lmax, inverse, x.shape[0], x.dtype


def _rotate_backward(ctx, grad):
    eulers, gather = ctx.saved_tensors
    back = _rotate(grad.contiguous(), ctx.lmax, eulers=eulers, inverse=not ctx.inverse, out_dtype=torch.float32)
    gx = back if gather is None else _scatter_rows(back, gather, ctx.n_x)
    return gx.to(ctx.x_dtype), None, None, None, None


rotate.register_autograd(_rotate_backward, setup_context=_rotate_setup)


# ------------------------------------------------------------ segment sum
@custom_op("maloq_hip::segment_sum", mutates_args=())
def segment_sum(msg: Tensor, perm: Tensor, seg_ptr: Tensor, num_segments: int) -> Tensor:
    _lib.require_cuda(msg, perm, seg_ptr)
    m = msg.float().contiguous()
    out = torch.empty((num_segments,) + tuple(msg.shape[1:]), device=msg.device, dtype=torch.float32)
    width = m[0].numel() if m.shape[0] > 0 else int(torch.tensor(msg.shape[1:]).prod())
    perm_d, seg_d = perm.long().contiguous(), seg_ptr.long().contiguous()   # alive across the launch
    _lib.call("maloq_segment_sum", _lib.ptr(m), _lib.ptr(perm_d), _lib.ptr(seg_d), num_segments, width,
              _lib.ptr(out), _lib.stream_of(msg.device))
    return out


@register_fake("maloq_hip::segment_sum")
def _(msg, perm, seg_ptr, num_segments):
    return msg.new_empty((num_segments,) + tuple(msg.shape[1:]), dtype=torch.float32)


# --------------------------------------------------------- basis transform
@custom_op("maloq_hip::label_transform", mutates_args=())
def label_transform(x: Tensor, blocks: Tensor, w: Optional[Tensor], sched: Tensor, perm_in: Optional[Tensor],
                    perm_out: Optional[Tensor], num_blocks: int, ngroups: int, group_cols: int,
                    perm_inv: Optional[Tensor]) -> Tensor:
    """Rows of several column groups (``ngroups`` > 1) are permuted by a
    separate column gather: the input through ``perm_inv`` (the inverse of
    ``perm_in``), the output through ``perm_out``."""
    _lib.require_cuda(x)
    xc = x.contiguous()
    pre = ngroups > 1 and perm_in is not None
    post = ngroups > 1 and perm_out is not None
    if pre or post:
        ones = torch.ones(xc.shape[1], device=xc.device, dtype=torch.float32)

    def gather(y, src):
        o = torch.empty_like(y)
        _lib.call("maloq_gather_columns", _lib.ptr(y), y.shape[1], y.shape[0], _lib.ptr(src), _lib.ptr(ones),
                  y.shape[1], _lib.ptr(o), o.shape[1], _lib.stream_of(y.device))
        return o

    if pre:
        if perm_inv is None:
            raise ValueError("rows of several column groups need the inverse input permutation")
        xc = gather(xc, perm_inv)
    out = torch.empty_like(xc)
    _lib.call("maloq_label_transform", _lib.ptr(xc), _lib.ptr(None if pre else perm_in), _lib.ptr(out),
              _lib.ptr(None if post else perm_out), xc.shape[0], xc.shape[1], num_blocks, _lib.ptr(blocks),
              _lib.ptr(w), _lib.ptr(sched), ngroups, group_cols, _lib.stream_of(x.device))
    return gather(out, perm_out) if post else out


@register_fake("maloq_hip::label_transform")
def _(x, blocks, w, sched, perm_in, perm_out, num_blocks, ngroups, group_cols, perm_inv):
    return torch.empty_like(x)


def _layout(d):
    return d.num_blocks, d.ngroups, d.group_cols, getattr(d, "_perm_inv", None)


def get_net_out(decomp, H: Tensor) -> Tensor:
    """``e3TensorDecomp.get_net_out`` (utils_tensor_decomp.py:163-169) as the op,
    with the tables of a :class:`maloq_amd.basis_transform.HipE3TensorDecomp`."""
    decomp._check(H, decomp.total_h_dim)
    return label_transform(H, decomp._blocks_fwd, decomp._wk_fwd, decomp._sched, None, decomp._perm,
                           *_layout(decomp))


def get_H(decomp, net_out: Tensor) -> Tensor:
    """``e3TensorDecomp.get_H`` (utils_tensor_decomp.py:154-161) as the op
    (differentiable: the adjoint tables give the gradient)."""
    decomp._check(net_out, decomp.total_in_dim)
    return _GetHOp.apply(net_out, decomp)


class _GetHOp(torch.autograd.Function):
    @staticmethod
    def forward(ctx, net_out, decomp):
        ctx.decomp = decomp
        return label_transform(net_out, decomp._blocks_inv, decomp._wk_inv, decomp._sched, decomp._perm, None,
                               *_layout(decomp))

    @staticmethod
    def backward(ctx, g):
        d = ctx.decomp
        return label_transform(g.contiguous(), d._blocks_adj, d._wk_adj, d._sched, None, d._perm,
                               *_layout(d)), None


# ----------------------------------------------------------- message block
@custom_op("maloq_hip::message_block_fwd", mutates_args=())
def message_block_fwd(x: Tensor, rad: Optional[Tensor], w0: Tensor, b0: Optional[Tensor], wm: List[Tensor],
                      src: Tensor, dst: Tensor, seg_ptr: Tensor, eulers: Tensor, lmax: int, mmax: int,
                      gate: bool) -> List[Tensor]:
    """Node output and the workspaces the backward reads: [out, y, r, dk, g]
    (r empty without radial scales, g empty ungated)."""
    plan = _PlanView(src, dst, seg_ptr, x.shape[0])
    saved = {}
    out = M.message_forward(x, plan, eulers, rad, w0, b0, list(wm), lmax, mmax, gate=gate, save=saved)
    empty = x.new_empty(0)
    return [out, saved["y"], saved["r"] if saved["r"] is not None else empty, saved["dk"],
            saved["g"] if saved["g"] is not None else empty]


@register_fake("maloq_hip::message_block_fwd")
def _(x, rad, w0, b0, wm, src, dst, seg_ptr, eulers, lmax, mmax, gate):
    N, d, c_in = x.shape
    E = src.shape[0]
    c_out = w0.shape[0] // (lmax + 1 + (lmax if gate else 0))
    kr = M.kept_rows(lmax, mmax)
    rows = int(_lib.load().maloq_message_edge_rows(E))  # the saved rows' padding, as the forward allocates them
    out = x.new_empty(N, d, c_out, dtype=torch.float32)
    y = x.new_empty(rows, kr, c_in)
    r = x.new_empty(max(E, 1), kr, c_in) if rad is not None else x.new_empty(0)
    dk = x.new_empty(max(E, 1), M.wigner_floats(lmax, mmax), dtype=torch.float32)
    g = x.new_empty(max(E, 1), kr + lmax, c_out) if gate else x.new_empty(0)
    return [out, y, r, dk, g]


class _PlanView:
    """The tensors of a MessagePlan the forward kernels read."""

    def __init__(self, src, dst, seg_ptr, num_nodes):
        self.src, self.dst, self.seg_ptr = src, dst, seg_ptr
        self.num_nodes, self.num_edges = int(seg_ptr.shape[0]) - 1, int(src.shape[0])
        self.perm = None


def message_block(x, plan, eulers, rad, w0, b0, wm, lmax, mmax, gate=False):
    """The fused block through the registered op (forward) and
    :func:`maloq_amd.message.message_backward_dx` / ``message_weight_grad``
    (backward): same results as :func:`maloq_amd.message.message_block`."""
    return _MessageOp.apply(x, rad, w0, b0, plan, eulers, lmax, mmax, bool(gate), *wm[:mmax])


class _MessageOp(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, rad, w0, b0, plan, eulers, lmax, mmax, gate, *wm):
        out, y, r, dk, g = message_block_fwd(x, rad, w0, b0, list(wm), plan.src, plan.dst, plan.seg_ptr, eulers,
                                             lmax, mmax, gate)
        ctx.plan, ctx.lmax, ctx.mmax, ctx.gate = plan, lmax, mmax, gate
        ctx.x_shape, ctx.dt, ctx.has_b0 = tuple(x.shape), x.dtype, b0 is not None
        ctx.save_for_backward(rad, w0, y, dk, r if r.numel() else None, g if g.numel() else None, *wm)
        return out

    @staticmethod
    def backward(ctx, gout):
        rad, w0, y, dk, r, g, *wm = ctx.saved_tensors
        plan, lmax, mmax, gate = ctx.plan, ctx.lmax, ctx.mmax, ctx.gate
        gx, grad_rad, dz = M.message_backward_dx(gout, ctx.x_shape, ctx.dt, plan, {"dk": dk, "r": r, "g": g}, rad,
                                                 w0, wm, lmax, mmax, need_rad_grad=ctx.needs_input_grad[1],
                                                 gate=gate)
        dw0 = db0 = None
        dwm = [None] * len(wm)
        if plan.num_edges > 0:
            dw0, dwm, db0 = M.message_weight_grad(dz, y, lmax, mmax, gout.shape[2], ctx.x_shape[2],
                                                  num_edges=plan.num_edges, gate=gate)
        else:
            dw0, dwm = torch.zeros_like(w0), [torch.zeros_like(w) for w in wm]
            db0 = torch.zeros(w0.shape[0], device=w0.device)
        return (gx.to(ctx.dt), grad_rad, dw0.to(w0.dtype), db0 if ctx.has_b0 else None, None, None, None, None,
                None, *[d.to(w.dtype) for d, w in zip(dwm, wm)])
