"""maloq_message_fwd_noalloc (the message forward whose workspace is the
library's own device array) against maloq_message_fwd with caller-allocated
workspaces: the same kernels, so the node outputs must be bitwise equal.  Two
calls in a row, the second on a smaller graph (the array keeps the first call's
contents), and a call too large for the array is refused."""
import math

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _case(device, N, E, lmax, mmax, C, dtype, gate, seed):
    from maloq_amd import message as M
    from maloq_amd.wigner import extract_euler_angles
    gen = torch.Generator().manual_seed(seed)
    d = (lmax + 1) ** 2
    x = torch.randn(N, d, C, generator=gen).to(device=device, dtype=dtype)
    ei = torch.stack([torch.randint(0, N, (E,), generator=gen), torch.randint(0, max(1, N - 2), (E,), generator=gen)])
    plan = M.MessagePlan(ei.to(device), N)
    k0 = (lmax + 1) * C
    extra = lmax * C if gate else 0
    w0 = (torch.randn(k0 + extra, k0, generator=gen) / math.sqrt(k0)).to(device)
    b0 = (torch.randn(k0 + extra, generator=gen) * 0.1).to(device)
    wm = [(torch.randn(2 * (lmax - m + 1) * C, (lmax - m + 1) * C, generator=gen) / math.sqrt((lmax - m + 1) * C))
          .to(device) for m in range(1, mmax + 1)]
    rad = (torch.rand(E, M.rad_width(lmax, mmax, C), generator=gen) + 0.5).to(device=device, dtype=dtype)
    eul = plan.sort_edges(extract_euler_angles(torch.randn(E, 3, generator=gen).to(device), seed=seed))
    rad = plan.sort_edges(rad)
    return x, plan, eul, rad, w0, b0, wm


def _noalloc(x, plan, eul, rad, w0, b0, wm, lmax, mmax, gate, wpack):
    from maloq_amd import _lib
    from maloq_amd import message as M
    N, d, C = x.shape
    out = torch.empty(N, d, C, device=x.device)
    _lib.call("maloq_message_fwd_noalloc", M.DTYPE_CODE[x.dtype], lmax, mmax, int(gate), _lib.ptr(x), C,
              _lib.ptr(plan.src), _lib.ptr(plan.dst), plan.num_edges, _lib.ptr(eul), _lib.ptr(rad), _lib.ptr(wpack),
              _lib.ptr(b0), _lib.ptr(M._jd_dev(lmax, x.device)), _lib.ptr(out), N, C, _lib.ptr(plan.seg_ptr),
              _lib.stream_of(x.device))
    return out


@pytest.mark.parametrize("lmax,mmax,dtype,gate", [(4, 2, torch.bfloat16, False), (2, 2, torch.float32, True),
                                                  (4, 4, torch.bfloat16, True)])
def test_noalloc_forward_equals_allocating_forward(lmax, mmax, dtype, gate, device):
    from maloq_amd import message as M
    print(f"noalloc case lmax={lmax} mmax={mmax} dtype={dtype} gate={gate}", flush=True)
    C = 64
    for N, E, seed in ((200, 5000, 1), (37, 600, 2)):     # the second call is smaller
        x, plan, eul, rad, w0, b0, wm = _case(device, N, E, lmax, mmax, C, dtype, gate, seed)
        wpack = M.pack_weights(w0, wm, lmax, mmax, gate, C, C, dtype, 0)
        want = M.message_forward(x, plan, eul, rad, w0, b0, wm, lmax, mmax, gate=gate, wpack=wpack)
        got = _noalloc(x, plan, eul, rad, w0, b0, wm, lmax, mmax, gate, wpack)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"N={N} E={E}: max diff {(got - want).abs().max().item()}"


def test_noalloc_refuses_oversized_graph(device):
    from maloq_amd import _lib
    from maloq_amd import message as M
    lmax, mmax, C = 4, 2, 128
    x, plan, eul, rad, w0, b0, wm = _case(device, 300, 20000, lmax, mmax, C, torch.bfloat16, False, 3)
    wpack = M.pack_weights(w0, wm, lmax, mmax, False, C, C, torch.bfloat16, 0)
    with pytest.raises(_lib.MaloqHipError, match="scratch array holds"):
        _noalloc(x, plan, eul, rad, w0, b0, wm, lmax, mmax, False, wpack)
