"""PyTorch custom ops (namespace ``maloq_hip``) of the HIP path.

The operators are defined and implemented in C++ (``csrc/torch_ops.cpp``,
built into ``_maloq_torch.so``, a thin extension over ``libmaloq_hip.so``):
each checks its arguments, allocates its outputs and calls the C ABI on the
current HIP stream; there is no CPU implementation.  This module loads the
extension and registers, from Python, each operator's fake (meta)
implementation, so that ``torch.compile`` and other graph capture see single
ops with known output shapes, and the autograd formulas.

    maloq_hip::edge_euler(edge_vec, seed)                 extract_euler_angles
    maloq_hip::edge_vec_to_wigner(edge_vec, jd, ..)       edge_vec_to_wigner_fused, (wigner, wigner_inv)
    maloq_hip::wigner_from_euler(eulers, lmax, inverse)   eulers_to_wigner (dense D or D^T)
    maloq_hip::rotate(x, eulers, gather?, lmax, inverse)  bmm(wigner, x[src]) / bmm(wigner_inv, z)
    maloq_hip::segment_sum(msg, perm, seg_ptr, n)         index_add_ in a fixed order
    maloq_hip::label_transform(x, ..)                     get_net_out / get_H on label rows
    maloq_hip::message_block_fwd(x, rad?, w0, b0?, wm, plan tensors, eulers, lmax, mmax, gate)
                                                          Edgewise.forward_node with one convolution
    maloq_hip::edgewise_fwd / edgewise_bwd(..)            the two-convolution Edgewise, both modes
    maloq_hip::radial_fwd / radial_bwd(..)                the fused RadialMLP
    maloq_hip::edge_m0_rows / edge_degree_embed[_] / edge_degree_embed_bwd(..)
                                                          EdgeDegreeEmbedding (node or edge mode)

Reference interfaces: helm/triton_kernels/wigner_fused.py:383-486,
helm/common/rotation.py:19-39, helm/esen_block.py:146-208,
helm/nn/radial.py:115-142, helm/nn/embedding.py:17-141,
fock_utils/utils_tensor_decomp.py:154-169.
"""
from __future__ import annotations

import os

import torch
from torch import Tensor
from torch.library import register_autograd, register_fake

from . import _lib
from . import message as M
from .rotate import _scatter_rows, rotate as _rotate

EXT_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_maloq_torch.so")


def _load_extension():
    if not os.path.exists(EXT_PATH):
        raise _lib.MaloqHipError(f"{EXT_PATH} is missing: build it with `python -m maloq_amd.build` "
                                 "(the operators have no Python implementation)")
    _lib.load()  # the HIP library the extension links, loaded once
    torch.ops.load_library(EXT_PATH)


_load_extension()
_ops = torch.ops.maloq_hip

# ------------------------------------------------------------------ Wigner
edge_euler = _ops.edge_euler
wigner_from_euler = _ops.wigner_from_euler
edge_vec_to_wigner = _ops.edge_vec_to_wigner
edge_vec_to_wigner_out = _ops.edge_vec_to_wigner_out


@register_fake("maloq_hip::edge_vec_to_wigner")
def _(edge_vec, jd, lmax, seed, with_inverse, with_eulers):
    E, d = edge_vec.shape[0], (lmax + 1) ** 2
    res = [edge_vec.new_empty(E, d, d)]
    if with_inverse:
        res.append(edge_vec.new_empty(E, d, d))
    if with_eulers:
        res.append(edge_vec.new_empty(E, 3))
    return res


@register_fake("maloq_hip::edge_vec_to_wigner_out")
def _(edge_vec, jd, lmax, seed, out):
    return None


@register_fake("maloq_hip::edge_euler")
def _(edge_vec, seed):
    return edge_vec.new_empty(edge_vec.shape[0], 3)


@register_fake("maloq_hip::wigner_from_euler")
def _(eulers, lmax, inverse):
    d = (lmax + 1) ** 2
    return eulers.new_empty(eulers.shape[0], d, d)


# ---------------------------------------------------------------- rotation
rotate = _ops.rotate


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


register_autograd("maloq_hip::rotate", _rotate_backward, setup_context=_rotate_setup)


# ------------------------------------------------------------ segment sum
segment_sum = _ops.segment_sum


@register_fake("maloq_hip::segment_sum")
def _(msg, perm, seg_ptr, num_segments):
    return msg.new_empty((num_segments,) + tuple(msg.shape[1:]), dtype=torch.float32)


# --------------------------------------------------------- basis transform
label_transform = _ops.label_transform


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
# Node output and the workspaces the backward reads: [out, y, r, dk, g, wpt]
# (r empty without radial scales, g empty ungated, wpt the transposed weight
# packing of the backward with save_tr, else empty).
message_block_fwd = _ops.message_block_fwd


@register_fake("maloq_hip::message_block_fwd")
def _(x, rad, w0, b0, wm, src, dst, seg_ptr, eulers, lmax, mmax, gate, save_tr=False):
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
    if save_tr:
        code = 1 if x.dtype == torch.bfloat16 else 0
        nb = int(_lib.load().maloq_message_wpack_bytes(code, lmax, mmax, int(gate), c_out, c_in))
        wpt = x.new_empty(nb // x.element_size())
    else:
        wpt = x.new_empty(0)
    return [out, y, r, dk, g, wpt]


message_block_bwd = _ops.message_block_bwd


@register_fake("maloq_hip::message_block_bwd")
def _(grad_out, rad, w0, wm, bwd_src, bwd_dst, bwd_eidx, seg_ptr_src, y, dk, r, g, num_nodes, c_in, lmax, mmax,
      gate, need_rad_grad, dst=None, wpack_t=None):
    d = (lmax + 1) ** 2
    c_out = grad_out.shape[2]
    f32 = dict(dtype=torch.float32)
    extra = lmax * c_out if gate else 0
    gx = grad_out.new_empty(num_nodes, d, c_in, **f32)
    grad_rad = rad.new_empty(rad.shape, dtype=y.dtype) if (rad is not None and need_rad_grad) \
        else grad_out.new_empty(0, **f32)
    dw0 = grad_out.new_empty(extra + (lmax + 1) * c_out, (lmax + 1) * c_in, **f32)
    db0 = grad_out.new_empty(extra + (lmax + 1) * c_out, **f32)
    dwm = [grad_out.new_empty(2 * (lmax - m + 1) * c_out, (lmax - m + 1) * c_in, **f32) for m in range(1, mmax + 1)]
    return [gx, grad_rad, dw0, db0] + dwm


def message_block(x, plan, eulers, rad, w0, b0, wm, lmax, mmax, gate=False):
    """The fused block through the registered operators (message_block_fwd,
    message_block_bwd): same results as :func:`maloq_amd.message.message_block`."""
    return _MessageOp.apply(x, rad, w0, b0, plan, eulers, lmax, mmax, bool(gate), *wm[:mmax])


class _MessageOp(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, rad, w0, b0, plan, eulers, lmax, mmax, gate, *wm):
        # both weight packings from one launch when a backward will run
        out, y, r, dk, g, wpt = message_block_fwd(x, rad, w0, b0, list(wm), plan.src, plan.dst, plan.seg_ptr,
                                                  eulers, lmax, mmax, gate, any(ctx.needs_input_grad))
        ctx.plan, ctx.lmax, ctx.mmax, ctx.gate = plan, lmax, mmax, gate
        ctx.x_shape, ctx.dt, ctx.has_b0 = tuple(x.shape), x.dtype, b0 is not None
        ctx.save_for_backward(rad, w0, y, dk, r if r.numel() else None, g if g.numel() else None,
                              wpt if wpt.numel() else None, *wm)
        return out

    @staticmethod
    def backward(ctx, gout):
        rad, w0, y, dk, r, g, wpt, *wm = ctx.saved_tensors
        plan, lmax, mmax, gate = ctx.plan, ctx.lmax, ctx.mmax, ctx.gate
        need_rad = rad is not None and ctx.needs_input_grad[1]
        gx, grad_rad, dw0, db0, *dwm = message_block_bwd(
            gout, rad, w0, list(wm), plan.bwd_src, plan.bwd_dst, plan.bwd_eidx, plan.seg_ptr_src, y, dk, r, g,
            ctx.x_shape[0], ctx.x_shape[2], lmax, mmax, gate, need_rad, plan.dst, wpt)
        return (gx.to(ctx.dt), grad_rad if need_rad else None, dw0.to(w0.dtype), db0 if ctx.has_b0 else None,
                None, None, None, None, None, *[d.to(w.dtype) for d, w in zip(dwm, wm)])


# --------------------------------------------------------------- radial MLP
# Fused RadialMLP: [out, wpack, u_H] forward, [dx, hidden grads (flat), dW_o,
# db_o] backward (maloq_amd.radial holds the autograd wiring).
radial_fwd = _ops.radial_fwd
radial_bwd = _ops.radial_bwd


@register_fake("maloq_hip::radial_fwd")
def _(x, params, widths, eps, bf16, save):
    E = x.shape[0]
    dt = torch.bfloat16 if bf16 else torch.float32
    nb = int(_lib.load().maloq_radial_pack_bytes(1 if bf16 else 0, widths[-1], widths[-2]))
    return [x.new_empty(E, widths[-1], dtype=dt), x.new_empty(nb, dtype=torch.uint8),
            x.new_empty(E, widths[-2], dtype=dt) if save else x.new_empty(0, dtype=dt)]


@register_fake("maloq_hip::radial_bwd")
def _(grad, x, wpack, save, params, widths, eps, need_dx):
    E = x.shape[0]
    n_hid = sum(widths[i + 1] * (widths[i] + 3) for i in range(len(widths) - 2))
    f32 = dict(dtype=torch.float32)
    return [grad.new_empty(E, widths[0], **f32) if need_dx else grad.new_empty(0, **f32),
            grad.new_empty(n_hid, **f32), grad.new_empty(widths[-1], widths[-2], **f32),
            grad.new_empty(widths[-1], **f32)]


# ---------------------------------------------------- edge-degree embedding
# EdgeDegreeEmbedding: m = 0 rows [E, d] fp32, the embedding (node: a copy of
# x with the edges summed in, or in place; edge: [E, d, C]) and the gradient
# wrt the radial rows (maloq_amd.embedding holds the autograd wiring).
edge_m0_rows = _ops.edge_m0_rows
edge_degree_embed = _ops.edge_degree_embed
edge_degree_embed_ = _ops.edge_degree_embed_
edge_degree_embed_bwd = _ops.edge_degree_embed_bwd


@register_fake("maloq_hip::edge_m0_rows")
def _(wigner_inv, eulers, lmax, num_edges):
    ref = wigner_inv if wigner_inv is not None else eulers
    return ref.new_empty(num_edges, (lmax + 1) ** 2, dtype=torch.float32)


@register_fake("maloq_hip::edge_degree_embed")
def _(x, u, rows, seg_ptr, perm, lmax, channels, rescale, node):
    if node:
        return torch.empty_like(x, memory_format=torch.contiguous_format)
    return x.new_empty(u.shape[0], (lmax + 1) ** 2, channels)


@register_fake("maloq_hip::edge_degree_embed_")
def _(x, u, rows, seg_ptr, perm, lmax, channels, rescale):
    return None


@register_fake("maloq_hip::edge_degree_embed_bwd")
def _(grad, grad_rows, rows, lmax, channels, scale):
    return grad.new_empty(rows.shape[0], (lmax + 1) * channels, dtype=torch.float32)


# -------------------------------------------------- two-convolution Edgewise
edgewise_fwd = _ops.edgewise_fwd
edgewise_bwd = _ops.edgewise_bwd


@register_fake("maloq_hip::edgewise_fwd")
def _(x, rad, w01, b01, wm1, w02, b02, wm2, src, dst, seg_ptr, perm, eulers, wigner, x_message_edge, wpack1, wpack2,
      lmax, mmax, edge_mode, save):
    N, d, c_x = x.shape
    E = src.shape[0]
    E1 = max(E, 1)
    npart = 2 if x_message_edge is None else 3
    c_hidden, c_out = w01.shape[0] // (2 * lmax + 1), w02.shape[0] // (lmax + 1)
    kr = M.kept_rows(lmax, mmax)
    rows_y = int(_lib.load().maloq_message_edge_rows(E)) if save else E1
    lib = _lib.load()
    out = x.new_empty(E if edge_mode else seg_ptr.shape[0] - 1, d, c_out, dtype=torch.float32)
    y = x.new_empty(rows_y, kr, npart * c_x)
    z = x.new_empty(rows_y, kr, c_hidden)
    r = x.new_empty(E1, kr, npart * c_x) if (save and rad is not None) else x.new_empty(0)
    dk = x.new_empty(E1, M.wigner_floats(lmax, mmax), dtype=torch.float32)
    g = x.new_empty(E1, kr + lmax, c_hidden) if save else x.new_empty(0)
    code = M.DTYPE_CODE[x.dtype]
    el = x.element_size()
    wp1t = x.new_empty(lib.maloq_message_wpack_bytes(code, lmax, mmax, 1, c_hidden, npart * c_x) // el) \
        if save else x.new_empty(0)
    wp2t = x.new_empty(lib.maloq_message_wpack_bytes(code, lmax, mmax, 0, c_out, c_hidden) // el) \
        if save else x.new_empty(0)
    return [out, y, r, z, dk, g, wp1t, wp2t]


@register_fake("maloq_hip::edgewise_bwd")
def _(grad_out, rad, w01, wm1, w02, wm2, dst, bwd_src, bwd_eidx, perm, seg_ptr, seg_ptr_src, y, r, z, dk, g,
      wpack1_t, wpack2_t, num_nodes, c_x, lmax, mmax, edge_mode, parts, need_rad_grad, need_w1, need_w2):
    d = (lmax + 1) ** 2
    E = dst.shape[0]
    f32 = dict(dtype=torch.float32)
    c_hidden = w01.shape[0] // (2 * lmax + 1)
    res = [grad_out.new_empty(num_nodes, d, c_x, **f32),
           rad.new_empty(rad.shape, dtype=y.dtype) if (rad is not None and need_rad_grad) else grad_out.new_empty(0, **f32),
           grad_out.new_empty(E, d, c_x, **f32) if parts == 3 else grad_out.new_empty(0, **f32)]
    for need, co, ci, gate in ((need_w1, c_hidden, parts * c_x, True), (need_w2, c_x, c_hidden, False)):
        extra = lmax * co if gate else 0
        if need:
            res += [grad_out.new_empty(extra + (lmax + 1) * co, (lmax + 1) * ci, **f32),
                    grad_out.new_empty(extra + (lmax + 1) * co, **f32)]
            res += [grad_out.new_empty(2 * (lmax - m + 1) * co, (lmax - m + 1) * ci, **f32)
                    for m in range(1, mmax + 1)]
        else:
            res += [grad_out.new_empty(0, **f32) for _ in range(2 + mmax)]
    return res


# ------------------------------------------------- fused Fock <-> irreps
basis_row_meta = _ops.basis_row_meta
fock_to_irreps = _ops.fock_to_irreps
irreps_to_fock = _ops.irreps_to_fock


@register_fake("maloq_hip::basis_row_meta")
def _(ld, block_data_offsets, off, Z, rows, cols, pair_kind, maxe):
    return rows.new_empty(max(rows.shape[0], 1), 4, dtype=torch.int32)


@register_fake("maloq_hip::fock_to_irreps")
def _(fock, ld, block_data_offsets, off, Z, rows, cols, meta, num_rows, pair_kind, slots, maxe, kind_blocks,
      perm_out, t, num_blocks, blocks, w, sched, ngroups, group_cols, perm_post):
    return fock.new_empty(num_rows, t)


@register_fake("maloq_hip::irreps_to_fock")
def _(net_out, fock, ld, block_data_offsets, off, Z, rows, cols, meta, num_rows, pair_kind, slots, maxe,
      kind_blocks, perm_in, t, num_blocks, blocks, w, sched, ngroups, group_cols, perm_pre):
    return None
