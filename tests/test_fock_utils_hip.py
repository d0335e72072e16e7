"""GPU parity of the label-side hooks (maloq_amd.fock_utils) against the CPU
restatements (oracle/fock_utils.py): scale-shift and its undo, the padding
mask, sort_by_m and the CSR export are exact (a subtraction per element, a
copy, a signed permutation, a scatter); make_targets within 1e-5 of the row
scale (the fp32 transform against the fp64 oracle)."""
import os

import numpy as np
import pytest
import torch

from oracle import fock_utils as ofu
from oracle import matrix2labels as om2l
from oracle import tensor_decomp as otd

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _nabla():
    z = np.load(os.path.join(GOLDEN, "scale_shifts_nabladft.npz"))
    means = {int(Z): z["means"][k].tolist() for k, Z in enumerate(z["Z"])}
    return {"element_scalar_means": means, "element_scalar_stds": None,
            "scalar_irrep_indices": z["scalar_irrep_indices"].tolist()}


def test_scale_shift_matches_oracle(device):
    from maloq_amd.fock_utils import ScaleShift
    data = _nabla()
    ss = ScaleShift(data, device)
    Zs = np.array([1, 6, 8, 7, 6, 16, 9, 35, 17, 1])
    x = torch.randn(len(Zs), 1024, generator=torch.Generator().manual_seed(0))
    means32 = {z: np.asarray(v, np.float32).tolist() for z, v in data["element_scalar_means"].items()}
    want = ofu.scale_shift_node_blocks(x, Zs, means32, data["scalar_irrep_indices"])
    xd = x.to(device)
    got = ss.scale_shift_node_blocks(xd, Zs)
    assert got is xd
    assert torch.equal(got.cpu(), want)
    back = ss.undo_scale_shift(got, Zs)
    assert torch.equal(back.cpu(), ofu.unscale_shift_node_blocks(want, Zs, means32, data["scalar_irrep_indices"]))
    with pytest.raises(IndexError):
        ss.scale_shift_node_blocks(xd, np.full(len(Zs), 90))


CFG3 = {1: [0, 0, 1], 6: [0, 0, 0, 1, 1, 2], 7: [0, 0, 0, 1, 1, 2], 8: [0, 0, 0, 1, 1, 2]}


def test_make_targets_and_mask_match_oracle(device):
    from maloq_amd import tensor_decomp as ptd
    from maloq_amd.basis_transform import HipE3TensorDecomp
    from maloq_amd.fock_utils import ScaleShift, create_label_unpadding_mask, make_targets
    from maloq_amd.synth import sphere_molecule, radius_graph, dense_hamiltonian
    t = ptd.BasisTables(CFG3)
    hip = HipE3TensorDecomp(ptd.e3TensorDecomp(t.req_output_irreps, t.out_js_list, torch.float32,
                                               device_torch=device))
    T = hip.total_h_dim
    z, p = sphere_molecule(24, ["H", "C", "N", "O"], [0.45, 0.3, 0.1, 0.1], seed=3)
    H, off = dense_hamiltonian(z, p, t.orbitals_per_atom(z), seed=4)
    src, dst, _ = radius_graph(p, 6.0)
    # scale-shift data on this basis' label width: random means for H/C/N/O
    rng = np.random.default_rng(5)
    idx = sorted(rng.choice(T, 12, replace=False).tolist())
    means = {int(e): rng.standard_normal(12).tolist() for e in (1, 6, 7, 8)}
    ss = ScaleShift({"element_scalar_means": means, "scalar_irrep_indices": idx}, device)
    node, edge = make_targets(hip, torch.from_numpy(H).to(device), z, (src, dst), t.orbitals_per_atom(z),
                              t.orbital_template, scale_shift=ss)
    rows = np.concatenate([src, np.arange(len(z))]).astype(np.int32)
    cols = np.concatenate([dst, np.arange(len(z))]).astype(np.int32)
    lab = np.zeros((len(rows), T), np.float32)
    om2l.single_matrix2label(t.orbital_template, off, z, rows, cols, H, lab, True)
    irr = otd.E3TensorDecomp(t.out_js_list).get_net_out(torch.from_numpy(lab).double())
    want_node = ofu.scale_shift_node_blocks(irr[len(src):], z, means, idx)
    scale = irr.abs().max().item()
    assert node.shape == (1, len(z), T) and edge.shape == (1, len(src), T)
    assert (edge[0].cpu().double() - irr[:len(src)]).abs().max().item() < 1e-5 * scale
    assert (node[0].cpu().double() - want_node).abs().max().item() < 1e-5 * scale
    # open shell: two spins through the same call
    node2, edge2 = make_targets(hip, torch.stack([torch.from_numpy(H), 2 * torch.from_numpy(H)]).to(device), z,
                                (src, dst), t.orbitals_per_atom(z), t.orbital_template)
    assert node2.shape[0] == 2 and torch.allclose(edge2[1], 2 * edge2[0], rtol=1e-6, atol=1e-6)
    em, nm = create_label_unpadding_mask(t.orbital_template, z, src, dst, T, device)
    wem, wnm = ofu.create_label_unpadding_mask(t.orbital_template, z, src, dst, T)
    assert torch.equal(em.cpu(), wem) and torch.equal(nm.cpu(), wnm)


BASIS = {1: [0, 0, 1], 6: [0, 0, 0, 1, 1, 2], 8: [0, 0, 0, 1, 1, 2], 16: [0, 0, 0, 1, 1, 2, 3]}


@pytest.mark.parametrize("direction", ["orca_to_e3nn", "e3nn_to_orca", "e3nn_to_pyscf", "pyscf_to_e3nn"])
def test_sort_by_m_matches_oracle(direction, device):
    from maloq_amd.fock_utils import sort_by_m
    Z = [8, 1, 16, 6, 1, 6, 8]
    n = sum(sum(2 * (l % 10) + 1 for l in BASIS[z]) for z in Z)
    a = np.random.default_rng(1).standard_normal((n, n)).astype(np.float32)
    got = sort_by_m(torch.from_numpy(a).to(device), BASIS, Z, direction).cpu().numpy()
    assert np.array_equal(got, ofu.sort_by_m(a.astype(np.float64), BASIS, Z, direction).astype(np.float32))


def test_csr_export_matches_scipy(device):
    from maloq_amd.fock_utils import sparse_block_matrix_to_scipy_csr
    from maloq_amd.matrix2labels import SparseBlockMatrix
    from maloq_amd.synth import sio2_cell, radius_graph, atom_pair_rows
    Z, pos, L = sio2_cell(n_atoms=90, seed=2, iters=100)
    src, dst, _ = radius_graph(pos, 5.0, cell=L)
    rows, cols = atom_pair_rows(src, dst, len(Z))
    perm = np.random.default_rng(0).permutation(len(rows))     # any block order
    rows, cols = rows[perm], cols[perm]
    off = np.concatenate([[0], np.cumsum(np.where(Z == 14, 13, 9))]).astype(np.int32)
    bdo = om2l.block_data_offsets(off, rows, cols)
    data = np.random.default_rng(1).standard_normal(int(bdo[-1])).astype(np.float32)
    sbm = SparseBlockMatrix(data=torch.from_numpy(data).to(device), block_data_offsets=torch.from_numpy(bdo).to(device),
                            fock_block_rows=torch.from_numpy(rows).to(device),
                            fock_block_cols=torch.from_numpy(cols).to(device),
                            fock_block_offsets=torch.from_numpy(off).to(device))
    got = sparse_block_matrix_to_scipy_csr(sbm)
    want = ofu.sparse_block_matrix_to_scipy_csr(data, bdo, rows, cols, off)
    want.sort_indices()
    assert got.has_sorted_indices or got.sorted_indices().nnz == got.nnz
    assert np.array_equal(got.indptr, want.indptr)
    assert np.array_equal(got.indices, want.indices)
    assert np.array_equal(got.data, want.data)
    # a (row atom, column atom) pair listed twice is refused before any launch
    dup = SparseBlockMatrix(data=sbm.data,
                            block_data_offsets=torch.cat([sbm.block_data_offsets[:-1], sbm.block_data_offsets[:1],
                                                          sbm.block_data_offsets[-1:]]),
                            fock_block_rows=torch.cat([sbm.fock_block_rows, sbm.fock_block_rows[:1]]),
                            fock_block_cols=torch.cat([sbm.fock_block_cols, sbm.fock_block_cols[:1]]),
                            fock_block_offsets=sbm.fock_block_offsets)
    with pytest.raises(ValueError, match="appears twice"):
        sparse_block_matrix_to_scipy_csr(dup)


# def2-TZVPD shells (src/maloq/fock_utils/basis_sets.py:28): with Ga and I the template is the
# whole dictionary's (4096 columns), the width of the OMol scale-shift data.
TZVPD = {1: [0, 0, 0, 1, 1], 6: [0, 0, 0, 0, 0, 1, 1, 1, 2, 2, 3, 0, 2],
         7: [0, 0, 0, 0, 0, 1, 1, 1, 2, 2, 3, 0, 2], 8: [0, 0, 0, 0, 0, 1, 1, 1, 2, 2, 3, 0, 1, 2],
         31: [0, 0, 0, 0, 0, 0, 1, 1, 1, 1, 1, 2, 2, 2, 2, 3, 0, 2],
         53: [0, 0, 0, 0, 0, 0, 1, 1, 1, 1, 1, 2, 2, 2, 3, 3, 0, 1, 2]}


def _omol():
    z = np.load(os.path.join(GOLDEN, "scale_shifts_omol.npz"))
    means = {int(Z): z["means"][k].tolist() for k, Z in enumerate(z["Z"])}
    return {"element_scalar_means": means, "element_scalar_stds": None,
            "scalar_irrep_indices": z["scalar_irrep_indices"].tolist()}


def test_make_targets_def2_tzvpd_with_omol_scale_shift(device):
    """The OMol workflow's label side at its real width: make_targets over the
    4096-column def2-TZVPD template (several column groups) with the reference's
    OMol element means (114 scalar columns, f-f on-site pairs included), against
    the oracle's gather, fp64 get_net_out and scale-shift (1e-5 of the row
    scale); the undo equals the oracle's fp32 undo bit for bit and the
    unshifted labels within one rounding."""
    from maloq_amd import tensor_decomp as ptd
    from maloq_amd.basis_transform import HipE3TensorDecomp
    from maloq_amd.fock_utils import ScaleShift, make_targets
    from maloq_amd.synth import sphere_molecule, radius_graph, dense_hamiltonian
    t = ptd.BasisTables(TZVPD)
    hip = HipE3TensorDecomp(ptd.e3TensorDecomp(t.req_output_irreps, t.out_js_list, torch.float32,
                                               device_torch=device))
    T = hip.total_h_dim
    assert T == 4096 and hip.ngroups > 1
    data = _omol()
    ss = ScaleShift(data, device)
    z, p = sphere_molecule(16, ["H", "C", "N", "O"], [0.45, 0.3, 0.1, 0.15], seed=11)
    H, off = dense_hamiltonian(z, p, t.orbitals_per_atom(z), seed=12)
    src, dst, _ = radius_graph(p, 6.0)
    node, edge = make_targets(hip, torch.from_numpy(H).to(device), z, (src, dst), t.orbitals_per_atom(z),
                              t.orbital_template, scale_shift=ss)
    rows = np.concatenate([src, np.arange(len(z))]).astype(np.int32)
    cols = np.concatenate([dst, np.arange(len(z))]).astype(np.int32)
    lab = np.zeros((len(rows), T), np.float32)
    om2l.single_matrix2label(t.orbital_template, off, z, rows, cols, H, lab, True)
    irr = otd.E3TensorDecomp(t.out_js_list).get_net_out(torch.from_numpy(lab).double())
    idx = data["scalar_irrep_indices"]
    means32 = {k: np.asarray(v, np.float32).tolist() for k, v in data["element_scalar_means"].items()}
    want_node = ofu.scale_shift_node_blocks(irr[len(src):], z, means32, idx)
    scale = irr.abs().max().item()
    assert (edge[0].cpu().double() - irr[:len(src)]).abs().max().item() < 1e-5 * scale
    assert (node[0].cpu().double() - want_node).abs().max().item() < 1e-5 * scale
    back = ss.undo_scale_shift(node[0], z)
    assert torch.equal(back.cpu(), ofu.unscale_shift_node_blocks(node[0].cpu(), z, means32, idx))
    unshifted = hip.fock_to_irreps(torch.from_numpy(H).to(device), off, z, rows, cols, t.orbital_template)
    assert (back - unshifted[len(src):]).abs().max().item() < 1e-6 * scale
