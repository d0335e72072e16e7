"""Host tables of the GPU output head (maloq_amd.irreps_head) against the CPU
restatement of the reference (oracle/irreps_head.py): the reduce_edge column
gathers rebuild both directions of an edge pair exactly as the reference's
half_edges_to_full -> output permutations -> Vpa +- Vpb -> subspace remix ->
parity flips (helm/esen_osh.py:918-937)."""
import numpy as np
import pytest

from maloq_amd import irreps_head as ih
from oracle import irreps_head as oh

LS_CASES = [[0, 0, 1], [0, 0, 0, 1, 1, 2], [0, 1, 1, 2, 3]]


def _sorted_to_z(v, ls, lmax):
    """A process output in the l-sorted e3nn layout (per degree: copies, then m)
    -> the GEMM buffer Z (per degree: m, then copies)."""
    mul = [sum(1 for x in ls if x == l) for l in range(lmax + 1)]
    out, o = [], 0
    for l in range(lmax + 1):
        n = (2 * l + 1) * mul[l]
        out.append(v[o:o + n].reshape(mul[l], 2 * l + 1).T.reshape(-1))
        o += n
    return np.concatenate(out)


@pytest.mark.parametrize("ls_list", LS_CASES)
def test_tables_match_reference_restatement(ls_list):
    a, b, f, oa, ob = ih._edgereduced(ls_list)
    A, B, F, OA, OB = oh.edgereduced(ls_list)
    assert (a, b) == (A, B) and sorted(f) == sorted(F.tolist()) and oa == list(OA) and ob == list(OB)
    assert ih._remix(a, b, ls_list) == list(oh.subspace_remix(a, b, ls_list))


@pytest.mark.parametrize("ls_list", LS_CASES)
def test_edge_pair_gathers_rebuild_both_directions(ls_list):
    lmax = max(oh.all_ls(ls_list))
    (ca, sa, _), (cb, sb, _), ls_a, ls_b = ih._edge_pair_maps(ls_list, lmax)
    _, _, flips, off_a, off_b = oh.edgereduced(ls_list)
    rng = np.random.default_rng(len(ls_list))
    oa = rng.standard_normal(sum(2 * l + 1 for l in ls_a))   # l-sorted process outputs
    ob = rng.standard_normal(sum(2 * l + 1 for l in ls_b))
    # the reference's assembly, edge 0 canonical and edge 1 its reverse
    fa = np.stack([oa, oa])[:, oh.output_permutation(ls_a)]
    fb = np.stack([ob, -ob])[:, oh.output_permutation(ls_b)]
    va, vb = fa[:, off_a].copy(), fb[:, off_b].copy()
    fa[:, off_a], fb[:, off_b] = va + vb, va - vb
    ref = np.concatenate([fa, fb], 1)[:, oh.subspace_remix(ls_a, ls_b, ls_list)]
    ref[:, flips] *= -1
    # the product's two signed gathers of the GEMM buffers
    za, zb = _sorted_to_z(oa, ls_a, lmax), _sorted_to_z(ob, ls_b, lmax)
    ca, cb = np.asarray(ca), np.asarray(cb)
    A = np.where(ca >= 0, za[np.maximum(ca, 0)], 0.0) * np.asarray(sa)
    Bv = np.where(cb >= 0, zb[np.maximum(cb, 0)], 0.0) * np.asarray(sb)
    assert np.array_equal(A + Bv, ref[0])
    assert np.array_equal(A - Bv, ref[1])
