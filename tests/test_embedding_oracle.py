"""The EdgeDegreeEmbedding oracle (oracle.embedding, a restatement of
embedding.py:82-141), pinned by what the mathematics fixes rather than by a
retyping of its formula:

* l = 0 block: D^0 = 1, so emb[e, 0, c] = u[e, 0, c] exactly;
* an edge along +y (beta = 0): D^l = X(a) J J X(c) = X(a + c) (J_l is an
  involution), whose m = 0 row is the unit vector, so only the (l, m = 0)
  entries are non-zero and equal u[e, l];
* orthogonality: per (edge, l, channel) the 2l + 1 entries have the norm |u|;
* the random roll gamma enters D through X(a), a = -gamma, whose m = 0 row is
  fixed, so the embedding does not depend on it (using D instead of D^T, a
  plausible transposition mistake, breaks this);
* node mode equals a brute-force loop x[dst] += emb / rescale in edge order;
* mmax < lmax gives the same result as mmax = lmax (only m = 0 columns meet a
  non-zero).
The module mirrors the reference's constructor and parameter names; the HIP
path refuses CPU tensors."""
import math

import pytest
import torch

from oracle import embedding as oemb
from oracle import rotation as orot
from oracle.so3 import CoefficientMapping


def _setup(lmax, mmax, E, C, seed, vec=None, gamma=None):
    gen = torch.Generator().manual_seed(seed)
    Jd = orot.load_jd(torch.float64)
    if vec is None:
        vec = torch.randn(E, 3, generator=gen, dtype=torch.float64)
    if gamma is None:
        gamma = torch.rand(E, generator=gen, dtype=torch.float64)
    eul = orot.init_edge_rot_euler_angles(vec, gamma)
    wig = orot.eulers_to_wigner(eul, 0, lmax, Jd)
    winv = wig.transpose(1, 2).contiguous()
    mapping = CoefficientMapping(lmax, mmax)
    full = CoefficientMapping(lmax, lmax)
    mask = full.coefficient_idx(lmax, mmax)
    u = torch.randn(E, (lmax + 1) * C, generator=gen, dtype=torch.float64)
    return winv, mapping, mask, u


def _edge(lmax, mmax, winv, mapping, mask, u):
    x = torch.zeros(1, (lmax + 1) ** 2, u.shape[1] // (lmax + 1), dtype=torch.float64)
    ei = torch.zeros(2, u.shape[0], dtype=torch.long)
    return oemb.edge_degree_embedding(x, u, ei, winv, mapping, mask, 5.0, "edge")


@pytest.mark.parametrize("lmax,mmax", [(2, 2), (4, 2), (6, 2)])
def test_l0_block_is_the_radial_row(lmax, mmax):
    winv, mapping, mask, u = _setup(lmax, mmax, 40, 8, 1)
    emb = _edge(lmax, mmax, winv, mapping, mask, u)
    assert torch.equal(emb[:, 0, :], u.reshape(40, lmax + 1, 8)[:, 0, :])


@pytest.mark.parametrize("lmax", [2, 4])
def test_edge_along_y_has_only_m0_entries(lmax):
    E, C = 6, 4
    vec = torch.tensor([[0.0, 1.0, 0.0]] * E, dtype=torch.float64) * torch.rand(E, 1, dtype=torch.float64).add(0.5)
    winv, mapping, mask, u = _setup(lmax, 2, E, C, 2, vec=vec)
    emb = _edge(lmax, 2, winv, mapping, mask, u)
    want = torch.zeros_like(emb)
    uu = u.reshape(E, lmax + 1, C)
    for l in range(lmax + 1):
        want[:, l * l + l, :] = uu[:, l, :]
    assert torch.allclose(emb, want, atol=1e-12)


@pytest.mark.parametrize("lmax,mmax", [(4, 2), (6, 2)])
def test_norm_per_degree_is_preserved(lmax, mmax):
    E, C = 30, 5
    winv, mapping, mask, u = _setup(lmax, mmax, E, C, 3)
    emb = _edge(lmax, mmax, winv, mapping, mask, u)
    uu = u.reshape(E, lmax + 1, C)
    for l in range(lmax + 1):
        nrm = emb[:, l * l: (l + 1) ** 2, :].norm(dim=1)
        assert torch.allclose(nrm, uu[:, l, :].abs(), rtol=1e-10, atol=1e-12)


def test_independent_of_the_random_roll():
    lmax, E, C = 4, 25, 3
    gen = torch.Generator().manual_seed(4)
    vec = torch.randn(E, 3, generator=gen, dtype=torch.float64)
    w1, mapping, mask, u = _setup(lmax, 2, E, C, 5, vec=vec, gamma=torch.rand(E, generator=gen, dtype=torch.float64))
    w2, _, _, _ = _setup(lmax, 2, E, C, 5, vec=vec, gamma=torch.rand(E, generator=gen, dtype=torch.float64))
    assert not torch.allclose(w1, w2)
    e1 = _edge(lmax, 2, w1, mapping, mask, u)
    e2 = _edge(lmax, 2, w2, mapping, mask, u)
    assert torch.allclose(e1, e2, atol=1e-12)
    # planted mistake: D in place of D^T depends on the roll
    t1 = _edge(lmax, 2, w1.transpose(1, 2), mapping, mask, u)
    t2 = _edge(lmax, 2, w2.transpose(1, 2), mapping, mask, u)
    assert not torch.allclose(t1, t2, atol=1e-6)


def test_node_mode_is_the_edge_order_sum():
    lmax, mmax, N, E, C = 2, 2, 5, 17, 3
    winv, mapping, mask, u = _setup(lmax, mmax, E, C, 6)
    gen = torch.Generator().manual_seed(7)
    ei = torch.stack([torch.randint(0, N, (E,), generator=gen), torch.randint(0, N - 1, (E,), generator=gen)])
    x = torch.randn(N, (lmax + 1) ** 2, C, generator=gen, dtype=torch.float64)
    got = oemb.edge_degree_embedding(x, u, ei, winv, mapping, mask, 5.0, "node")
    emb = _edge(lmax, mmax, winv, mapping, mask, u)
    want = x.clone()
    for e in range(E):
        want[ei[1, e]] += emb[e] / 5.0
    assert torch.allclose(got, want, atol=1e-12)
    assert torch.equal(got[N - 1], x[N - 1])   # no in-edges: unchanged


def test_mmax_below_lmax_matches_full():
    lmax, E, C = 4, 20, 4
    winv, mapping, mask, u = _setup(lmax, 2, E, C, 8)
    full = CoefficientMapping(lmax, lmax)
    a = _edge(lmax, 2, winv, mapping, mask, u)
    b = _edge(lmax, lmax, winv, full, full.coefficient_idx(lmax, lmax), u)
    assert torch.allclose(a, b, atol=1e-12)


def test_module_mirrors_reference_structure():
    from maloq_amd.embedding import EdgeDegreeEmbedding
    from maloq_amd.so3 import CoefficientMapping as CM
    m = CM(4, 2)
    mod = EdgeDegreeEmbedding(16, 4, 2, 90, [8, 32, 32], 5.0, 6.0, m, None)
    assert mod.m_0_num_coefficients == 5 and mod.m_all_num_coefficents == 19
    assert mod.edge_channels_list == [8, 32, 32, 80]
    names = sorted(k for k, _ in mod.named_parameters())
    assert names == sorted(["rad_func.net.0.weight", "rad_func.net.0.bias", "rad_func.net.1.weight",
                            "rad_func.net.1.bias", "rad_func.net.3.weight", "rad_func.net.3.bias",
                            "rad_func.net.4.weight", "rad_func.net.4.bias", "rad_func.net.6.weight",
                            "rad_func.net.6.bias"])


def test_hip_path_refuses_cpu_tensors():
    from maloq_amd.embedding import edge_degree_embed
    from maloq_amd import _lib
    x = torch.zeros(3, 9, 4)
    u = torch.zeros(5, 12)
    with pytest.raises((_lib.MaloqHipError, RuntimeError, ValueError)):
        edge_degree_embed(x, u, torch.zeros(2, 5, dtype=torch.long), torch.zeros(5, 9, 9), 2, 5.0)
