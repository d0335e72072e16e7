"""Rotation of irreps features into and out of the edge frame (``maloq_rotate``).

Drop-in for the reference's ``torch.bmm(wigner, x_message)`` and
``torch.bmm(wigner_inv, x_message)`` (src/maloq/helm/esen_block.py:181,191;
the heads at src/maloq/helm/esen_osh.py:1218,1228,1318,1328) where the rotated
rows themselves are wanted rather than the fused message block:

* ``rotate(x, lmax, eulers=..., gather=src)``  -> ``D_e x[src[e]]``  ([E, d, C])
* ``rotate(z, lmax, eulers=..., inverse=True)`` -> ``D_e^T z[e]``

The Wigner blocks come from the Euler triples of
:func:`maloq_amd.wigner.extract_euler_angles` (built inside the kernel, no
dense [E, d, d] in HBM) or from the block-diagonal part of a dense ``wigner``
[E, d, d] (the reference's own input).  ``rotate_block`` is the differentiable
form (gradient with respect to x: the inverse rotation, summed per gathered
row in a fixed order).
"""
from __future__ import annotations

import torch

from . import _lib
from .message import DTYPE_CODE, _csr, _jd_dev


def rotate(x, lmax, eulers=None, wigner=None, gather=None, inverse=False, out_dtype=None, Jd=None):
    """[E, d, C] rows ``D_e x[g(e)]`` (``inverse``: ``D_e^T x[g(e)]``), fp32
    arithmetic, output in ``out_dtype`` (default: the dtype of x)."""
    if x.dtype not in DTYPE_CODE:
        raise ValueError(f"unsupported dtype {x.dtype}")
    od = x.dtype if out_dtype is None else out_dtype
    if od not in DTYPE_CODE:
        raise ValueError(f"unsupported output dtype {od}")
    if not 0 <= lmax <= 8:
        raise ValueError(f"lmax must be 0-8, got {lmax}")
    d = (lmax + 1) ** 2
    if x.dim() != 3 or x.shape[1] != d:
        raise ValueError(f"x must be [*, {d}, C], got {tuple(x.shape)}")
    C = x.shape[2]
    if C % 4:
        raise ValueError("channels must be a multiple of 4")
    if (eulers is None) == (wigner is None):
        raise ValueError("give exactly one of eulers= and wigner=")
    _lib.require_cuda(x, eulers, wigner, gather)
    E = (eulers if eulers is not None else wigner).shape[0]
    if wigner is not None:
        if tuple(wigner.shape) != (E, d, d):
            raise ValueError(f"wigner must be [E, {d}, {d}]")
        wigner = wigner.float().contiguous()
    else:
        if tuple(eulers.shape) != (E, 3):
            raise ValueError("eulers must be [E, 3]")
        eulers = eulers.float().contiguous()
    g = None
    if gather is not None:
        if gather.shape != (E,):
            raise ValueError("gather must be [E]")
        if E > 0 and (int(gather.min()) < 0 or int(gather.max()) >= x.shape[0]):
            raise ValueError("gather holds rows outside x")
        g = gather.to(torch.int32).contiguous()
    elif x.shape[0] != E:
        raise ValueError("without gather, x must have one row per edge")
    out = torch.empty(E, d, C, device=x.device, dtype=od)
    if E == 0:
        return out
    xc = x.contiguous()
    if Jd is None:
        jd = _jd_dev(lmax, x.device) if eulers is not None else None
    else:
        from .wigner import _packed_jd
        jd = _packed_jd(Jd, lmax, x.device)
    _lib.call("maloq_rotate", DTYPE_CODE[x.dtype], DTYPE_CODE[od], lmax, _lib.ptr(xc), C, _lib.ptr(g), E,
              _lib.ptr(eulers), _lib.ptr(wigner), _lib.ptr(jd), int(bool(inverse)), _lib.ptr(out),
              _lib.stream_of(x.device))
    return out


def _scatter_rows(rows, gather, num_rows):
    """sum over e with gather[e] = r of rows[e] -> [num_rows, ...] fp32, in edge
    order per row (maloq_segment_sum over the stable gather-sorted order)."""
    E = rows.shape[0]
    width = rows[0].numel() if E > 0 else 0
    out = torch.empty((num_rows,) + tuple(rows.shape[1:]), device=rows.device, dtype=torch.float32)
    if num_rows == 0:
        return out
    if E == 0:
        return out.zero_()
    g = gather.long()
    perm = torch.sort(g, stable=True).indices.contiguous()
    seg_ptr = _csr(g[perm], num_rows)
    msg = rows.float().contiguous()
    _lib.call("maloq_segment_sum", _lib.ptr(msg), _lib.ptr(perm), _lib.ptr(seg_ptr), num_rows, width,
              _lib.ptr(out), _lib.stream_of(rows.device))
    return out


class _RotateFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, lmax, eulers, wigner, gather, inverse):
        ctx.lmax, ctx.inverse, ctx.n_x = lmax, inverse, x.shape[0]
        ctx.x_dtype = x.dtype
        ctx.save_for_backward(eulers, wigner, gather)
        return rotate(x, lmax, eulers=eulers, wigner=wigner, gather=gather, inverse=inverse)

    @staticmethod
    def backward(ctx, g):
        eulers, wigner, gather = ctx.saved_tensors
        if not ctx.needs_input_grad[0]:
            return None, None, None, None, None, None
        back = rotate(g.contiguous(), ctx.lmax, eulers=eulers, wigner=wigner, inverse=not ctx.inverse,
                      out_dtype=torch.float32)
        gx = back if gather is None else _scatter_rows(back, gather, ctx.n_x)
        return gx.to(ctx.x_dtype), None, None, None, None, None


def rotate_block(x, lmax, eulers=None, wigner=None, gather=None, inverse=False):
    """Differentiable :func:`rotate` (gradient with respect to x)."""
    return _RotateFn.apply(x, lmax, eulers, wigner, gather, bool(inverse))
