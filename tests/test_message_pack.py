"""CPU check of the SO(2) weight packing and of the kernel's complex mix.

The fused GEMM reads packed B fragments (the MFMA B operand's lane order:
lane i holds B[k][n = i % 32] for k = 8 (i // 32) + j, j < 8, in bf16; in fp32
each lane's four floats feed four 32x32x2 MFMAs, float j of lane i being
channel 4 (i // 32) + j) and forms, per m > 0,
    forward:         y+ = Wr x+ - Wi x-,      y- = Wi x+ + Wr x-
    input gradient:  dx+ = Wr^T dy+ + Wi^T dy-,  dx- = -Wi^T dy+ + Wr^T dy-.
This test walks the packed buffer exactly as the kernel does (channel block,
kernel-input degree, K step, fragment list) in fp64 numpy and compares the
result with the oracle's SO(2) convolution (so2_layers.py:139-214) and, for
the transposed mode, with fp64 autograd through it.
"""
import math

import numpy as np
import pytest
import torch

from maloq_amd import message as M
from oracle import so2 as oso2


def _decode(dtype_code):
    fe = 512 if dtype_code == 1 else 256
    e = np.arange(fe)
    if dtype_code == 1:
        lane, j = e // 8, e % 8
        k = 8 * (lane // 32) + j
    else:
        lane, j = e // 4, e % 4
        k = 4 * (lane // 32) + j
    return fe, k, lane % 32


def _model(packed, dtype_code, lmax, mmax, gate, c_k, c_n, rows, mode, grows=None):
    """Kernel-order GEMM: rows [E, d', c_k] m-major -> [E, d' (+gate), c_n].
    Transposed gated mode: grows [E, lmax, c_k] are the dL/dgate input rows."""
    fe, k_of, n_of = _decode(dtype_code)
    kc = 16 if dtype_code == 1 else 8
    E = rows.shape[0]
    P = M.kept_rows(lmax, mmax)

    def mrow(q, l):
        if q == 0:
            return l
        m = (q + 1) // 2
        base = lmax + 1 + sum(2 * (lmax - k + 1) for k in range(1, m))
        return base + (0 if q % 2 else lmax - m + 1) + (l - m)

    out = np.zeros((E, P, c_n))
    gate_out = np.zeros((E, lmax, c_n))
    pos = 0
    for cb in range(c_n // 32):
        for l_k in range(lmax + 1):
            flist = M._frag_list(lmax, mmax, gate and mode == 0, l_k, gate_in=gate and mode == 1)
            for ks in range(c_k // kc):
                B = {}
                for kind, m, l_n in flist:
                    blk = np.zeros((kc, 32))
                    blk[k_of, n_of] = packed[pos: pos + fe]
                    pos += fe
                    B[(kind, m, l_n)] = blk
                cs = slice(ks * kc, (ks + 1) * kc)
                ns = slice(cb * 32, (cb + 1) * 32)
                for (kind, m, l_n), blk in B.items():
                    if kind == "g0":
                        out[:, mrow(0, l_n), ns] += rows[:, mrow(0, l_k), cs] @ blk
                    elif kind == "gate" and mode == 0:
                        gate_out[:, l_n - 1, ns] += rows[:, mrow(0, l_k), cs] @ blk
                    elif kind == "gate":
                        out[:, mrow(0, l_n), ns] += grows[:, l_k - 1, cs] @ blk
                    elif kind == "wr":
                        wr, wi = blk, B[("wi", m, l_n)]
                        ap = rows[:, mrow(2 * m - 1, l_k), cs]
                        am = rows[:, mrow(2 * m, l_k), cs]
                        sp, sm = mrow(2 * m - 1, l_n), mrow(2 * m, l_n)
                        if mode == 0:
                            out[:, sp, ns] += ap @ wr - am @ wi
                            out[:, sm, ns] += ap @ wi + am @ wr
                        else:
                            out[:, sp, ns] += ap @ wr + am @ wi
                            out[:, sm, ns] += -(ap @ wi) + am @ wr
    assert pos == packed.size
    return out, gate_out


def _weights(lmax, mmax, c_in, c_out, gate, gen):
    extra = lmax * c_out if gate else 0
    k0 = (lmax + 1) * c_in
    w0 = torch.randn(extra + (lmax + 1) * c_out, k0, generator=gen, dtype=torch.float64) / math.sqrt(k0)
    wm = [torch.randn(2 * (lmax - m + 1) * c_out, (lmax - m + 1) * c_in, generator=gen, dtype=torch.float64)
          for m in range(1, mmax + 1)]
    return w0, wm


@pytest.mark.parametrize("dtype_code", [0, 1])
@pytest.mark.parametrize("lmax,mmax,gate", [(2, 2, False), (4, 2, False), (4, 2, True), (3, 1, False)])
def test_forward_packing_matches_so2_convolution(dtype_code, lmax, mmax, gate):
    gen = torch.Generator().manual_seed(lmax * 7 + mmax + int(gate))
    c_in, c_out, E = 32, 64, 5
    w0, wm = _weights(lmax, mmax, c_in, c_out, gate, gen)
    idx, total = M._pack_index(dtype_code, lmax, mmax, gate, c_in, c_out, 0)
    flat = torch.cat([w0.reshape(-1)] + [w.reshape(-1) for w in wm]).numpy()
    assert flat.size == total
    packed = flat[idx]
    m_size = [lmax - m + 1 for m in range(mmax + 1)]
    x = torch.randn(E, M.kept_rows(lmax, mmax), c_in, generator=gen, dtype=torch.float64)
    got, got_gate = _model(packed, dtype_code, lmax, mmax, gate, c_in, c_out, x.numpy(), 0)
    extra = lmax * c_out if gate else None
    ref = oso2.so2_convolution(x, None, w0, None, wm, m_size, c_out, extra=extra)
    if gate:
        ref, ref_gate = ref
        np.testing.assert_allclose(got_gate, ref_gate.reshape(E, lmax, c_out).numpy(), rtol=0, atol=1e-12)
    np.testing.assert_allclose(got, ref.numpy(), rtol=0, atol=1e-12)


@pytest.mark.parametrize("dtype_code", [0, 1])
@pytest.mark.parametrize("lmax,mmax", [(2, 2), (4, 2)])
def test_transposed_packing_matches_autograd(dtype_code, lmax, mmax):
    gen = torch.Generator().manual_seed(50 + lmax)
    c_in, c_out, E = 64, 32, 4
    w0, wm = _weights(lmax, mmax, c_in, c_out, False, gen)
    idx, total = M._pack_index(dtype_code, lmax, mmax, False, c_in, c_out, 1)
    packed = torch.cat([w0.reshape(-1)] + [w.reshape(-1) for w in wm]).numpy()[idx]
    m_size = [lmax - m + 1 for m in range(mmax + 1)]
    x = torch.randn(E, M.kept_rows(lmax, mmax), c_in, generator=gen, dtype=torch.float64, requires_grad=True)
    dy = torch.randn(E, M.kept_rows(lmax, mmax), c_out, generator=gen, dtype=torch.float64)
    (oso2.so2_convolution(x, None, w0, None, wm, m_size, c_out) * dy).sum().backward()
    got, _ = _model(packed, dtype_code, lmax, mmax, False, c_out, c_in, dy.numpy(), 1)
    np.testing.assert_allclose(got, x.grad.numpy(), rtol=0, atol=1e-12)


def test_packed_size_matches_library():
    from maloq_amd import _lib
    lib = _lib.load()
    for code, fe in ((0, 256), (1, 512)):
        for lmax, mmax, gate, c_in, c_out, mode in [(4, 2, False, 128, 128, 0), (4, 2, True, 64, 32, 0),
                                                    (6, 2, False, 128, 128, 1), (2, 2, False, 32, 64, 1)]:
            idx, _ = M._pack_index(code, lmax, mmax, gate, c_in, c_out, mode)
            c_k, c_n = (c_in, c_out) if mode == 0 else (c_out, c_in)
            want = lib.maloq_message_wpack_bytes(code, lmax, mmax, int(gate), c_k, c_n)
            assert idx.size * (2 if code == 1 else 4) == want


@pytest.mark.parametrize("dtype_code", [0, 1])
@pytest.mark.parametrize("lmax,mmax", [(2, 2), (4, 2)])
def test_transposed_gated_packing_matches_autograd(dtype_code, lmax, mmax):
    """Input gradient of a gated SO(2) convolution with respect to its input,
    given dL/dy (kept rows) and dL/dgate: the kernel's transposed walk over the
    packed gate and SO(2) weights equals fp64 autograd."""
    gen = torch.Generator().manual_seed(70 + lmax)
    c_in, c_out, E = 64, 32, 4
    w0, wm = _weights(lmax, mmax, c_in, c_out, True, gen)
    idx, total = M._pack_index(dtype_code, lmax, mmax, True, c_in, c_out, 1)
    packed = torch.cat([w0.reshape(-1)] + [w.reshape(-1) for w in wm]).numpy()[idx]
    m_size = [lmax - m + 1 for m in range(mmax + 1)]
    x = torch.randn(E, M.kept_rows(lmax, mmax), c_in, generator=gen, dtype=torch.float64, requires_grad=True)
    dy = torch.randn(E, M.kept_rows(lmax, mmax), c_out, generator=gen, dtype=torch.float64)
    dg = torch.randn(E, lmax * c_out, generator=gen, dtype=torch.float64)
    y, g = oso2.so2_convolution(x, None, w0, None, wm, m_size, c_out, extra=lmax * c_out)
    ((y * dy).sum() + (g * dg).sum()).backward()
    got, _ = _model(packed, dtype_code, lmax, mmax, True, c_out, c_in, dy.numpy(), 1,
                    grows=dg.reshape(E, lmax, c_out).numpy())
    np.testing.assert_allclose(got, x.grad.numpy(), rtol=0, atol=1e-12)


@pytest.mark.parametrize("lmax,mmax", [(2, 2), (4, 2), (4, 4), (6, 2), (6, 6)])
@pytest.mark.parametrize("gate", [False, True])
@pytest.mark.parametrize("dtype_code", [0, 1])
@pytest.mark.parametrize("mode", [0, 1])
def test_pack_index_places_every_weight_once(lmax, mmax, gate, dtype_code, mode):
    """The packed buffer is a permutation of cat(W0, W1, ..) for every built
    shape: each weight element (gate rows included) lands in exactly one slot,
    so no element is dropped or read twice by the GEMM, for channel counts that
    differ on the two sides."""
    for c_in, c_out in ((32, 32), (64, 32), (32, 96)):
        r = M._pack_index(dtype_code, lmax, mmax, gate, c_in, c_out, mode)
        idx = np.asarray(r[0] if isinstance(r, tuple) else r)
        extra = lmax * c_out if gate else 0
        total = (extra + (lmax + 1) * c_out) * (lmax + 1) * c_in + sum(
            2 * (lmax - m + 1) * c_out * (lmax - m + 1) * c_in for m in range(1, mmax + 1))
        assert idx.size == total and idx.min() >= 0
        assert np.array_equal(np.bincount(idx, minlength=total), np.ones(total, np.int64)), (c_in, c_out)
