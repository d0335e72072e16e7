"""GPU parity of the standalone rotation op (maloq_rotate) against the CPU
oracle: the reference's torch.bmm(wigner, x[src]) / bmm(wigner_inv, z)
(esen_block.py:181,191) with the oracle's Wigner-D (rotation.py:19-39,189-225)
at the kernel's own Euler angles.

Bars: fp32 within 1e-5 of the output scale; bf16 within 2e-2 (oracle in fp64 on
the bf16-rounded input).  Config 1 of the benchmark: the round trip
D^T (D x) = x, and equivariance under a global rotation R (positions by R,
features by D(R)): the edge-frame rows change only by a roll about the edge
axis, so the m = 0 rows are unchanged and the (+m, -m) pair norms are too.
"""
import math

import numpy as np
import pytest
import torch

from oracle import rotation as orot

pytestmark = pytest.mark.gpu


def _ref_blocks(eul, lmax):
    e = eul.cpu().double()
    return orot.eulers_to_wigner((e[:, 0], e[:, 1], e[:, 2]), 0, lmax, orot.load_jd())


@pytest.mark.parametrize("lmax", list(range(0, 9)))
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_rotate_matches_oracle(lmax, dtype, device):
    from maloq_amd.rotate import rotate
    from maloq_amd.wigner import extract_euler_angles
    print(f"rotate lmax={lmax} dtype={dtype}", flush=True)
    gen = torch.Generator().manual_seed(lmax)
    d, C, N, E = (lmax + 1) ** 2, 12, 17, 203
    x = torch.randn(N, d, C, generator=gen, dtype=torch.float64)
    src = torch.randint(0, N, (E,), generator=gen)
    eul = extract_euler_angles(torch.randn(E, 3, generator=gen).to(device), seed=lmax)
    Dm = _ref_blocks(eul, lmax)
    xq = x.to(dtype).double()
    ref_in = torch.bmm(Dm, xq[src])
    ref_out = torch.bmm(Dm.transpose(1, 2), xq[src])
    xd = x.to(device=device, dtype=dtype)
    sd = src.to(device)
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    for inv, ref in ((False, ref_in), (True, ref_out)):
        got = rotate(xd, lmax, eulers=eul, gather=sd, inverse=inv, out_dtype=torch.float32).cpu().double()
        err = (got - ref).abs().max().item() / ref.abs().max().item()
        assert err < tol, f"inverse={inv} err {err}"


@pytest.mark.parametrize("lmax", [2, 4])
@pytest.mark.parametrize("C", [4, 1024])
def test_rotate_channel_widths(lmax, C, device):
    """Edges per workgroup follow the width: min(256 / d, 256 / (C / 4)), so
    C = 4 packs 256 / d edges and C = 1024 one edge per workgroup."""
    from maloq_amd.rotate import rotate
    from maloq_amd.wigner import extract_euler_angles
    print(f"rotate widths lmax={lmax} C={C}", flush=True)
    gen = torch.Generator().manual_seed(C + lmax)
    d, N, E = (lmax + 1) ** 2, 11, 97
    x = torch.randn(N, d, C, generator=gen, dtype=torch.float64)
    src = torch.randint(0, N, (E,), generator=gen)
    eul = extract_euler_angles(torch.randn(E, 3, generator=gen).to(device), seed=C)
    Dm = _ref_blocks(eul, lmax)
    xd, sd = x.to(device=device, dtype=torch.float32), src.to(device)
    for inv in (False, True):
        ref = torch.bmm(Dm.transpose(1, 2) if inv else Dm, x.float().double()[src])
        got = rotate(xd, lmax, eulers=eul, gather=sd, inverse=inv, out_dtype=torch.float32).cpu().double()
        assert (got - ref).abs().max().item() / ref.abs().max().item() < 1e-5, inv


@pytest.mark.parametrize("lmax", [2, 4, 6])
def test_rotate_dense_wigner_equals_euler_path(lmax, device):
    """The dense-wigner input (the reference's argument) gives bit-identical rows
    to the Euler path when the matrices come from the same angles."""
    from maloq_amd.rotate import rotate
    from maloq_amd.wigner import extract_euler_angles, wigner_from_eulers
    gen = torch.Generator().manual_seed(7)
    d, C, E = (lmax + 1) ** 2, 32, 300
    z = torch.randn(E, d, C, generator=gen).to(device)
    eul = extract_euler_angles(torch.randn(E, 3, generator=gen).to(device), seed=3)
    w = wigner_from_eulers(eul, None, lmax)
    for inv in (False, True):
        a = rotate(z, lmax, eulers=eul, inverse=inv)
        b = rotate(z, lmax, wigner=w, inverse=inv)
        assert torch.equal(a, b)


def test_rotate_gradient_matches_oracle(device):
    """d/dx of sum(G * D_e x[src[e]]) = sum over edges of D_e^T G_e, per source."""
    from maloq_amd.rotate import rotate_block
    from maloq_amd.wigner import extract_euler_angles
    lmax, C, N, E = 4, 16, 23, 410
    gen = torch.Generator().manual_seed(11)
    d = (lmax + 1) ** 2
    x = torch.randn(N, d, C, generator=gen, dtype=torch.float64)
    G = torch.randn(E, d, C, generator=gen, dtype=torch.float64)
    src = torch.randint(0, N - 2, (E,), generator=gen)   # the last rows get no gradient
    eul = extract_euler_angles(torch.randn(E, 3, generator=gen).to(device), seed=5)
    xr = x.float().double().requires_grad_()
    (torch.bmm(_ref_blocks(eul, lmax), xr[src]) * G).sum().backward()
    xd = x.float().to(device).requires_grad_()
    y = rotate_block(xd, lmax, eulers=eul, gather=src.to(device))
    (y.double() * G.to(device)).sum().backward()
    got = xd.grad.cpu().double()
    err = (got - xr.grad).abs().max().item() / xr.grad.abs().max().item()
    assert err < 1e-5, err
    assert torch.all(got[-2:] == 0)


def test_rotate_edge_cases(device):
    from maloq_amd.rotate import rotate
    eul = torch.zeros(0, 3, device=device)
    x = torch.randn(5, 9, 8, device=device)
    assert rotate(x, 2, eulers=eul, gather=torch.zeros(0, dtype=torch.int64, device=device)).shape == (0, 9, 8)
    with pytest.raises(ValueError):
        rotate(x, 2, eulers=torch.zeros(3, 3, device=device), gather=torch.tensor([0, 1, 5], device=device))
    with pytest.raises(ValueError):
        rotate(x[:, :, :6], 2, eulers=torch.zeros(5, 3, device=device))
    with pytest.raises(ValueError):
        rotate(x, 2)


def _config1(device, seed=0):
    from maloq_amd import synth
    g = synth.config1_graph()
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(g.num_nodes, 9, 32, generator=gen)
    return g, x


def _rot(a, b, c):
    ca, sa, cb, sb, cc, sc = math.cos(a), math.sin(a), math.cos(b), math.sin(b), math.cos(c), math.sin(c)
    Ry = lambda co, si: np.array([[co, 0, si], [0, 1, 0], [-si, 0, co]])
    Rx = np.array([[1, 0, 0], [0, cb, -sb], [0, sb, cb]])
    return Ry(ca, sa) @ Rx @ Ry(cc, sc)


def test_config1_round_trip_identity(device):
    """Config 1 (12 atoms, lmax 2, 32 channels, fp32): D^T (D x[src]) = x[src]."""
    from maloq_amd.rotate import rotate
    from maloq_amd.wigner import extract_euler_angles
    g, x = _config1(device)
    eul = extract_euler_angles(torch.from_numpy(g.edge_distance_vec()).float().to(device), seed=0)
    src = torch.from_numpy(g.src).to(device)
    xd = x.to(device)
    y = rotate(xd, 2, eulers=eul, gather=src)
    back = rotate(y, 2, eulers=eul, inverse=True)
    err = (back - xd[src]).abs().max().item() / xd.abs().max().item()
    assert err < 1e-5, err
    # the edge frame aligns the edge with the y axis: D^1 v = (0, |v|, 0)
    v = torch.from_numpy(g.edge_distance_vec()).float().to(device)
    v1 = rotate(torch.cat([torch.zeros(len(v), 1, 4, device=device),
                           v[:, :, None].expand(-1, 3, 4)], 1), 1, eulers=eul)[:, 1:, 0]
    assert (v1[:, 0].abs().max() / v.norm(dim=1).max()).item() < 1e-5
    assert (v1[:, 2].abs().max() / v.norm(dim=1).max()).item() < 1e-5
    assert torch.allclose(v1[:, 1], v.norm(dim=1), rtol=1e-5)


def test_config1_global_rotation_equivariance(device):
    """Positions rotated by R and features by D(R): each edge-frame row block
    changes by a roll about the edge axis only."""
    from maloq_amd.rotate import rotate
    from maloq_amd.wigner import extract_euler_angles
    g, x = _config1(device)
    Jd = orot.load_jd()
    a, b, c = 0.3, 1.1, -0.7
    R = torch.from_numpy(_rot(a, b, c))
    t = lambda v: torch.tensor([v], dtype=torch.float64)
    Dfull = torch.block_diag(*[orot.wigner_D(l, t(a), t(b), t(c), Jd)[0] for l in range(3)])
    vec = torch.from_numpy(g.edge_distance_vec())
    src = torch.from_numpy(g.src).to(device)
    y = rotate(x.to(device), 2, eulers=extract_euler_angles(vec.float().to(device), seed=0), gather=src)
    xr = torch.einsum("ij,njc->nic", Dfull, x.double()).float()
    yr = rotate(xr.to(device), 2, eulers=extract_euler_angles((vec @ R.T).float().to(device), seed=0), gather=src)
    y, yr = y.cpu().double(), yr.cpu().double()
    scale = y.abs().max().item()
    for l in range(3):
        m0 = l * l + l
        assert (yr[:, m0] - y[:, m0]).abs().max().item() / scale < 1e-5, f"m = 0 row of l = {l}"
        for m in range(1, l + 1):
            n = lambda z: (z[:, m0 + m] ** 2 + z[:, m0 - m] ** 2).sqrt()
            assert (n(yr) - n(y)).abs().max().item() / scale < 1e-5, f"l = {l}, |m| = {m}"
