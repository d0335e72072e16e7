"""The output head's CPU restatement (oracle/irreps_head.py) against what the
mathematics fixes: the reduce_node expansion reproduces the labels of a
symmetric on-site block (parity signs from the CG tensors' exchange symmetry,
odd self-interaction irreps zero), the output permutation is the stable
l-sort, the head is SO(3)-equivariant, and the gate is the normalised sigmoid."""
import math

import numpy as np
import pytest
import torch

from oracle import irreps_head as oh
from oracle import rotation as orot
from oracle import tensor_decomp as otd

LS_CASES = [[0, 0, 1], [0, 0, 0, 1, 1, 2], [0, 1, 1, 2, 3]]


def _onsite_labels(ls_list, seed):
    """Irreps labels (unsorted, every shell pair) of a random symmetric on-site
    block with shells ls_list, through the oracle's CG decomposition."""
    rng = np.random.default_rng(seed)
    n = sum(2 * l + 1 for l in ls_list)
    H = rng.standard_normal((n, n))
    H = H + H.T
    off = np.concatenate([[0], np.cumsum([2 * l + 1 for l in ls_list])])
    row = np.concatenate([H[off[i]:off[i + 1], off[j]:off[j + 1]].reshape(-1)
                          for i in range(len(ls_list)) for j in range(len(ls_list))])
    js = [(li, lj) for li in ls_list for lj in ls_list]
    o = otd.E3TensorDecomp(js, dtype=torch.float64)
    return o.get_net_out(torch.from_numpy(row)[None])[0].numpy()


@pytest.mark.parametrize("ls_list", LS_CASES)
@pytest.mark.parametrize("intra", [False, True])
def test_reduce_node_expansion_reproduces_symmetric_block_labels(ls_list, intra):
    lab = _onsite_labels(ls_list, seed=len(ls_list))
    idx, par = oh.reduced_to_all(ls_list, intra)
    # the reduced columns: every label column some label column reads with sign +1 from itself
    ls_all = oh.all_ls(ls_list)
    assert len(idx) == len(lab) == sum(2 * l + 1 for l in ls_all)
    red_len = sum(2 * l + 1 for l in oh.nodereduced_ls(ls_list, intra))
    reduced = np.zeros(red_len)
    for t, (i, p) in enumerate(zip(idx, par)):
        if i >= 0 and p == 1 and reduced[i] == 0:
            reduced[i] = lab[t]
    expanded = np.where(idx >= 0, reduced[np.maximum(idx, 0)], 0.0) * par
    assert np.allclose(expanded, lab, atol=1e-12), "parity signs / indices disagree with the CG labels"
    if intra:
        assert np.all(np.abs(lab[par == 0]) < 1e-12), "odd self-interaction irreps of a symmetric block are zero"


def test_expansion_detects_a_wrong_sign():
    """Planted mistake: one flipped parity sign fails the symmetric-block check."""
    ls_list = [0, 1, 1, 2]
    lab = _onsite_labels(ls_list, seed=3)
    idx, par = oh.reduced_to_all(ls_list, True)
    par = par.copy()
    k = int(np.nonzero(par == -1)[0][0])
    par[k] = 1.0
    red = np.zeros(sum(2 * l + 1 for l in oh.nodereduced_ls(ls_list, True)))
    for t, (i, p) in enumerate(zip(idx, oh.reduced_to_all(ls_list, True)[1])):
        if i >= 0 and p == 1:
            red[i] = lab[t]
    expanded = np.where(idx >= 0, red[np.maximum(idx, 0)], 0.0) * par
    assert not np.allclose(expanded, lab, atol=1e-9)


def test_output_permutation_is_the_stable_l_sort():
    ls = [1, 0, 2, 1, 0, 3, 2]
    perm = oh.output_permutation(ls)
    # the sorted layout: for l ascending, copies in original order, each 2l+1 wide
    sorted_tags = []
    for l in sorted(set(ls)):
        for i, li in enumerate(ls):
            if li == l:
                sorted_tags += [(i, m) for m in range(2 * l + 1)]
    label_tags = [(i, m) for i, l in enumerate(ls) for m in range(2 * l + 1)]
    assert [sorted_tags[p] for p in perm] == label_tags


def test_normalize2mom_constant():
    cst = oh.normalize2mom_constant()
    # E[sigmoid(z)^2] for z ~ N(0, 1) by quadrature
    z = np.linspace(-12, 12, 200001)
    w = np.exp(-z * z / 2) / math.sqrt(2 * math.pi)
    m2 = np.trapezoid(w / (1 + np.exp(-z)) ** 2, z)
    assert abs(cst - m2 ** -0.5) < 2e-3   # sampled estimate (10^6 draws)
    assert abs(cst - 1.8467) < 5e-3


def _params(lmax, C, ls_out, ls_node, spins, gen, reduce_node):
    mul = lambda ls: [sum(1 for x in ls if x == l) for l in range(lmax + 1)]
    out = []
    for _ in range(spins):
        p = {"scalar": (torch.randn(C * (C + lmax * C), generator=gen, dtype=torch.float64),
                        torch.randn(C + lmax * C, generator=gen, dtype=torch.float64))}
        streams = {"node": ls_node, "edge": ls_out} if reduce_node else {"common": ls_out}
        for name, ls in streams.items():
            m = mul(ls)
            p[name] = ([torch.randn(C * m[l], generator=gen, dtype=torch.float64) for l in range(lmax + 1)],
                       torch.randn(m[0], generator=gen, dtype=torch.float64))
        out.append(p)
    return out


@pytest.mark.parametrize("reduce_node", [False, True])
def test_head_is_equivariant(reduce_node):
    ls_list = [0, 0, 1, 2]
    lmax, C = 4, 6
    gen = torch.Generator().manual_seed(11)
    ls_out = oh.all_ls(ls_list)
    ls_node = oh.nodereduced_ls(ls_list, True)
    params = _params(lmax, C, ls_out, ls_node, 1, gen, reduce_node)
    d = (lmax + 1) ** 2
    xn = torch.randn(5, d, C, generator=gen, dtype=torch.float64)
    xe = torch.randn(7, d, C, generator=gen, dtype=torch.float64)
    Jd = orot.load_jd(torch.float64)
    a, b, c = 0.7, 1.1, -0.4
    D = [orot.wigner_D(l, torch.tensor(a, dtype=torch.float64), torch.tensor(b, dtype=torch.float64),
                       torch.tensor(c, dtype=torch.float64), Jd).reshape(2 * l + 1, 2 * l + 1) for l in range(lmax + 1)]

    def rot_feat(x):
        return torch.cat([torch.einsum("ij,bjc->bic", D[l], x[:, l * l:(l + 1) ** 2]) for l in range(lmax + 1)], 1)

    def rot_labels(y, ls):
        out, o = [], 0
        for l in ls:
            out.append(y[:, o:o + 2 * l + 1] @ D[l].T)
            o += 2 * l + 1
        return torch.cat(out, 1)

    n0, e0 = oh.head_forward(xn, xe, ls_list, lmax, C, params, reduce_node, True)
    n1, e1 = oh.head_forward(rot_feat(xn), rot_feat(xe), ls_list, lmax, C, params, reduce_node, True)
    assert torch.allclose(n1[0], rot_labels(n0[0], ls_out), atol=1e-10)
    assert torch.allclose(e1[0], rot_labels(e0[0], ls_out), atol=1e-10)


# ------------------------------------------------------------- reduce_edge
def _decode_block(labels, ls_list):
    """Labels of one orbital-pair block row -> the n x n block, through the
    oracle's CG tensors (the inverse of _onsite_labels)."""
    js = [(li, lj) for li in ls_list for lj in ls_list]
    o = otd.E3TensorDecomp(js, dtype=torch.float64)
    row = o.get_H(torch.as_tensor(labels, dtype=torch.float64)[None])[0].numpy()
    n = sum(2 * l + 1 for l in ls_list)
    off = np.concatenate([[0], np.cumsum([2 * l + 1 for l in ls_list])])
    H = np.zeros((n, n))
    k = 0
    for i in range(len(ls_list)):
        for j in range(len(ls_list)):
            ni, nj = off[i + 1] - off[i], off[j + 1] - off[j]
            H[off[i]:off[i + 1], off[j]:off[j + 1]] = row[k:k + ni * nj].reshape(ni, nj)
            k += ni * nj
    return H


def _pair_labels(ls_list, seed, flips=None):
    """Labels of an edge pair (0 -> 1, 1 -> 0) from random alpha / beta outputs,
    through head_forward's assembly (process outputs replaced by random ones)."""
    ls_a, ls_b, fl, off_a, off_b = oh.edgereduced(ls_list)
    if flips is not None:
        fl = flips
    rng = np.random.default_rng(seed)
    ta, tb = sum(2 * l + 1 for l in ls_a), sum(2 * l + 1 for l in ls_b)
    oa, ob = rng.standard_normal(ta), rng.standard_normal(tb)
    # half_edges_to_full: edge 0 canonical, edge 1 its reverse
    fa = np.stack([oa, oa])[:, oh.output_permutation(ls_a)]
    fb = np.stack([ob, -ob])[:, oh.output_permutation(ls_b)]
    va, vb = fa[:, off_a].copy(), fb[:, off_b].copy()
    fa[:, off_a], fb[:, off_b] = va + vb, va - vb
    e = np.concatenate([fa, fb], 1)[:, oh.subspace_remix(ls_a, ls_b, ls_list)]
    e[:, fl] *= -1
    return e


@pytest.mark.parametrize("ls_list", LS_CASES)
def test_reduce_edge_pairs_decode_to_transposed_blocks(ls_list):
    """The edge-pair construction gives the reverse edge the labels of the
    transposed Fock block (H_ji = H_ij^T), for any alpha / beta outputs."""
    for seed in range(3):
        e = _pair_labels(ls_list, seed)
        H01, H10 = _decode_block(e[0], ls_list), _decode_block(e[1], ls_list)
        assert np.allclose(H10, H01.T, atol=1e-10), "reverse-edge labels are not the transposed block"
        assert np.abs(H01).max() > 1e-3


def test_reduce_edge_detects_a_wrong_sign():
    """Planted mistake: one parity flip dropped breaks the transpose property."""
    ls_list = [0, 1, 1, 2]
    fl = oh.edgereduced(ls_list)[2]
    assert len(fl) > 0
    e = _pair_labels(ls_list, 1, flips=fl[1:])
    H01, H10 = _decode_block(e[0], ls_list), _decode_block(e[1], ls_list)
    assert not np.allclose(H10, H01.T, atol=1e-6)


@pytest.mark.parametrize("ls_list", LS_CASES)
def test_reduce_edge_remix_keeps_degree_and_m(ls_list):
    """Every label column reads the alpha or beta column of the same degree and
    the same m (so the remix is a relabelling of whole irreps)."""
    ls_a, ls_b, _, _, _ = oh.edgereduced(ls_list)
    tag = lambda ls: [(l, m) for l in ls for m in range(2 * l + 1)]
    src = tag(ls_a) + tag(ls_b)
    remix = oh.subspace_remix(ls_a, ls_b, ls_list)
    assert [src[c] for c in remix] == tag(oh.all_ls(ls_list))
    assert sorted(remix) == list(range(len(src)))


def test_reduce_edge_head_is_equivariant():
    ls_list = [0, 0, 1, 2]
    lmax, C = 4, 6
    gen = torch.Generator().manual_seed(13)
    ls_out = oh.all_ls(ls_list)
    ls_node = oh.nodereduced_ls(ls_list, True)
    ls_a, ls_b, _, _, _ = oh.edgereduced(ls_list)
    mul = lambda ls: [sum(1 for x in ls if x == l) for l in range(lmax + 1)]
    rw = lambda n: torch.randn(n, generator=gen, dtype=torch.float64)
    p = {"scalar": (rw(C * (C + lmax * C)), None),
         "node": ([rw(C * m) for m in mul(ls_node)], rw(mul(ls_node)[0])),
         "alpha": ([rw(C * m) for m in mul(ls_a)], None),
         "beta": ([rw(C * m) for m in mul(ls_b)], None)}
    d = (lmax + 1) ** 2
    ei = torch.tensor([[0, 1, 1, 2, 0, 2], [1, 0, 2, 1, 2, 0]])
    xn = torch.randn(3, d, C, generator=gen, dtype=torch.float64)
    xe = torch.randn(6, d, C, generator=gen, dtype=torch.float64)
    Jd = orot.load_jd(torch.float64)
    a, b, c = 0.3, 1.7, -0.9
    D = [orot.wigner_D(l, *(torch.tensor(v, dtype=torch.float64) for v in (a, b, c)), Jd).reshape(2 * l + 1, 2 * l + 1)
         for l in range(lmax + 1)]
    rot_feat = lambda x: torch.cat([torch.einsum("ij,bjc->bic", D[l], x[:, l * l:(l + 1) ** 2])
                                    for l in range(lmax + 1)], 1)

    def rot_labels(y):
        out, o = [], 0
        for l in ls_out:
            out.append(y[:, o:o + 2 * l + 1] @ D[l].T)
            o += 2 * l + 1
        return torch.cat(out, 1)

    n0, e0 = oh.head_forward(xn, xe, ls_list, lmax, C, [p], True, True, reduce_edge=True, edge_index=ei)
    n1, e1 = oh.head_forward(rot_feat(xn), rot_feat(xe), ls_list, lmax, C, [p], True, True, reduce_edge=True,
                             edge_index=ei)
    assert torch.allclose(n1[0], rot_labels(n0[0]), atol=1e-10)
    assert torch.allclose(e1[0], rot_labels(e0[0]), atol=1e-10)
    assert e0.abs().max() > 1e-3
