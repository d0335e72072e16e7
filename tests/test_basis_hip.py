"""GPU parity of the HIP basis transform and the Fock <-> label copy.

Oracle: the restated numpy gather (numpy_single_matrix2label) and the dense
fp64 e3TensorDecomp transforms.  Bars: copies bit-exact; transforms within
1e-5 relative to the row scale (fp32 dot products of <= 25 terms); round trip
get_H(get_net_out(H)) within 1e-6 of H's scale.
"""
import copy

import numpy as np
import pytest
import torch

from oracle import matrix2labels as om2l
from oracle import tensor_decomp as otd

pytestmark = pytest.mark.gpu

CFG3 = {1: [0, 0, 1], 6: [0, 0, 0, 1, 1, 2], 7: [0, 0, 0, 1, 1, 2], 8: [0, 0, 0, 1, 1, 2]}
MOCK = {1: [0], 6: [0, 0, 1], 8: [0, 0, 1]}
SIO2 = {14: [0, 0, 1, 1, 2], 8: [0, 0, 1, 1, 2]}
# def2-TZVPD shells (src/maloq/fock_utils/basis_sets.py:28): H/C/N/O rows are 1600
# columns wide; with Ga and I the template has the whole dictionary's 64 orbitals
# (4096 columns, 400 CG blocks), as get_loader.py:106-107 builds it for OMol.
TZVPD_HCNO = {1: [0, 0, 0, 1, 1], 6: [0, 0, 0, 0, 0, 1, 1, 1, 2, 2, 3, 0, 2],
              7: [0, 0, 0, 0, 0, 1, 1, 1, 2, 2, 3, 0, 2], 8: [0, 0, 0, 0, 0, 1, 1, 1, 2, 2, 3, 0, 1, 2]}
TZVPD = {**TZVPD_HCNO, 31: [0, 0, 0, 0, 0, 0, 1, 1, 1, 1, 1, 2, 2, 2, 2, 3, 0, 2],
         53: [0, 0, 0, 0, 0, 0, 1, 1, 1, 1, 1, 2, 2, 2, 3, 3, 0, 1, 2]}


def _tables(basis, if_sort=False):
    from maloq_amd import tensor_decomp as ptd
    t = ptd.BasisTables(basis)
    base = ptd.e3TensorDecomp(t.simplified_irreps if if_sort else t.req_output_irreps, t.out_js_list,
                              torch.float32, if_sort=if_sort, device_torch="cuda:0")
    ora = otd.E3TensorDecomp(t.out_js_list, if_sort=if_sort)
    return t, base, ora


def _molecules(n, basis_tables, seed0=0, sizes=(6, 14)):
    from maloq_amd.synth import sphere_molecule, radius_graph, dense_hamiltonian, atom_pair_rows
    out = []
    rng = np.random.default_rng(seed0)
    for m in range(n):
        na = int(rng.integers(*sizes))
        els = [k for k in basis_tables.orbital_basis]
        z, p = sphere_molecule(na, ["H", "C", "N", "O"], [0.45, 0.3, 0.1, 0.1], seed=seed0 + m)
        z = np.array([els[int(x) % len(els)] if int(x) not in els else int(x) for x in z])
        H, off = dense_hamiltonian(z, p, basis_tables.orbitals_per_atom(z), seed=100 + m)
        src, dst, _ = radius_graph(p, 8.0)
        rows, cols = atom_pair_rows(src, dst, na)
        out.append((z, H, off, rows, cols))
    return out


def _oracle_labels(t, z, H, off, rows, cols, T):
    lab = np.zeros((len(rows), T), np.float32)
    om2l.single_matrix2label(t.orbital_template, off, z, rows, cols, H, lab, True)
    return lab


def test_matrix2label_dense_bit_exact(device):
    from maloq_amd.matrix2labels import hip_single_matrix2label
    t, base, ora = _tables(CFG3)
    for z, H, off, rows, cols in _molecules(3, t):
        ref = _oracle_labels(t, z, H, off, rows, cols, 196)
        Hd = torch.from_numpy(H).to(device)
        lab = torch.zeros(len(rows), 196, device=device)
        hip_single_matrix2label(t.orbital_template, off, z, rows, cols, Hd, lab, None, forward=True)
        torch.cuda.synchronize()
        assert np.array_equal(lab.cpu().numpy(), ref)
        # inverse: scatter into a zero matrix, compare with the oracle scatter
        H2 = torch.zeros_like(Hd)
        hip_single_matrix2label(t.orbital_template, off, z, rows, cols, H2, lab, None, forward=False)
        H2r = np.zeros_like(H)
        om2l.single_matrix2label(t.orbital_template, off, z, rows, cols, H2r, ref.copy(), False)
        assert np.array_equal(H2.cpu().numpy(), H2r)


def test_matrix2label_dtype_errors(device):
    from maloq_amd.matrix2labels import hip_single_matrix2label
    t, _, _ = _tables(MOCK)
    with pytest.raises(ValueError):
        hip_single_matrix2label(t.orbital_template, [0, 1], [1], [0], [0],
                                torch.zeros(1, 1, device=device, dtype=torch.float64),
                                torch.zeros(1, 1, device=device, dtype=torch.float64), None, True)


def test_sparse_block_list_bit_exact(device):
    from maloq_amd.matrix2labels import hip_single_matrix2label_sparse, SparseBlockMatrix, block_data_offsets_for
    t, _, _ = _tables(CFG3)
    for z, H, off, rows, cols in _molecules(2, t, seed0=7):
        bdo = om2l.block_data_offsets(off, rows, cols)
        data = np.concatenate([H[off[i]:off[i + 1], off[j]:off[j + 1]].reshape(-1) for i, j in zip(rows, cols)])
        ref = np.zeros((len(rows), 196), np.float32)
        om2l.single_matrix2label_sparse(t.orbital_template, off, z, rows, cols, data, bdo, ref, True)
        assert np.array_equal(ref, _oracle_labels(t, z, H, off, rows, cols, 196))
        offd = torch.as_tensor(off, dtype=torch.int32, device=device)
        rr = torch.as_tensor(rows, device=device)
        cc = torch.as_tensor(cols, device=device)
        sm = SparseBlockMatrix(torch.from_numpy(data).to(device), block_data_offsets_for(offd, rr, cc), rr, cc, offd)
        lab = torch.zeros(len(rows), 196, device=device)
        hip_single_matrix2label_sparse(t.orbital_template, off, z, rows, cols, lab, None, True, sparse_matrix=sm)
        assert np.array_equal(lab.cpu().numpy(), ref)
        back = hip_single_matrix2label_sparse(t.orbital_template, off, z, rows, cols, lab, None, False)
        covered = back.data.cpu().numpy() != 0
        assert np.array_equal(back.data.cpu().numpy()[covered], data[covered])


@pytest.mark.parametrize("basis,if_sort", [(MOCK, True), (MOCK, False), (CFG3, False), (SIO2, False),
                                           (TZVPD_HCNO, False), (TZVPD_HCNO, True), (TZVPD, False)])
def test_label_transforms_match_oracle(basis, if_sort, device):
    """get_net_out / get_H against the dense fp64 oracle; the def2-TZVPD rows
    (1600 and 4096 columns) run as several column groups, sorted ones through
    the separate column permutation."""
    from maloq_amd.basis_transform import HipE3TensorDecomp
    t, base, ora = _tables(basis, if_sort)
    hip = HipE3TensorDecomp(base)
    T = ora.H_slices[-1]
    assert (hip.ngroups > 1) == (T > 204)
    g = torch.Generator().manual_seed(0)
    for R in ((0, 1, 77, 1000) if T <= 204 else (0, 1, 77, 300)):
        Hh = torch.randn(R, T, generator=g)
        x = torch.randn(R, ora.in_slices[-1], generator=g)
        got = hip.get_net_out(Hh.float().to(device)).cpu().double()
        ref = ora.get_net_out(Hh.double())
        assert got.shape == ref.shape
        if R:
            assert (got - ref).abs().max() / ref.abs().max() < 1e-5
        got = hip.get_H(x.float().to(device)).cpu().double()
        ref = ora.get_H(x.double())
        if R:
            assert (got - ref).abs().max() / ref.abs().max() < 1e-5


def test_reference_mock_triton_case(device):
    """tests/test_basis_transform_triton_backend.py:11-54: if_sort=True, 256 rows,
    get_H vs the dense re-assembly of wms (atol = rtol = 1e-4)."""
    from maloq_amd.basis_transform import HipE3TensorDecomp
    t, base, ora = _tables(MOCK, if_sort=True)
    hip = HipE3TensorDecomp(base)
    x = torch.randn((256, base.in_slices[-1]), device=device)
    out_rows = sum(w.shape[2] for w in base.wms)
    cols = [w.shape[0] * w.shape[1] for w in base.wms]
    wms = torch.zeros((sum(cols), out_rows), device=device)
    oc = 0
    for i in range(len(base.out_js_list)):
        s = slice(base.in_slices[i], base.in_slices[i + 1])
        wms[oc:oc + cols[i], s] = base.wms[i].reshape(-1, s.stop - s.start)
        oc += cols[i]
    y_ref = base.sort.inverse(x) @ wms.T
    assert torch.allclose(hip.get_H(x), y_ref, atol=1e-4, rtol=1e-4)


@pytest.mark.parametrize("basis,if_sort", [(CFG3, False), (TZVPD, False), (TZVPD_HCNO, True)])
def test_get_H_backward_is_adjoint(basis, if_sort, device):
    from maloq_amd.basis_transform import HipE3TensorDecomp
    t, base, ora = _tables(basis, if_sort)
    hip = HipE3TensorDecomp(base)
    T = int(ora.H_slices[-1])
    x = torch.randn(300, T, device=device, requires_grad=True)
    gH = torch.randn(300, T, device=device)
    hip.get_H(x).backward(gH)
    ref = gH.cpu().double() @ ora.W_global.T  # gradient wrt the unsorted rows get_H multiplies
    if if_sort:
        ref = ora.sort(ref)  # get_H un-sorts its input first, so the gradient is sorted back
    assert (x.grad.cpu().double() - ref).abs().max() / ref.abs().max() < 1e-5


@pytest.mark.parametrize("basis", [CFG3, {1: [0, 1], 6: [0, 0, 1, 2, 3], 8: [0, 1, 1, 2, 3]}])
def test_compiled_programs_equal_dense_blocks(basis, device):
    """Every direction through the compiled CG programs (no weights passed)
    and through the dense loops (program column -1, weights passed) gives the
    same bits, label rows and fused Fock side, f shells included."""
    from maloq_amd import _lib
    from maloq_amd.basis_transform import HipE3TensorDecomp
    t, base, ora = _tables(basis)
    hip = HipE3TensorDecomp(base)
    assert (hip.cg_programs >= 0).all() and hip._wk_fwd is None
    T = hip.total_in_dim
    x = torch.randn(517, T, device=device)

    def rows(blocks, w, perm_in, perm_out):
        out = torch.empty_like(x)
        _lib.call("maloq_label_transform", x, perm_in, out, perm_out, x.shape[0], T, hip.num_blocks, blocks, w,
                  hip._sched, *hip._layout(), _lib.stream_of(device))
        return out

    for blocks, w, pin, pout in ((hip._blocks_fwd, hip._w_fwd, None, hip._perm),
                                 (hip._blocks_inv, hip._w_inv, hip._perm, None),
                                 (hip._blocks_adj, hip._w_adj, None, hip._perm)):
        dense = blocks.clone().reshape(-1, 4)
        dense[:, 3] = -1
        a = rows(blocks, None, pin, pout)
        b = rows(dense.reshape(-1), w, pin, pout)
        assert torch.equal(a, b)
    # Fock side: the fused gather + get_net_out and get_H + scatter
    z, H, off, r_, c_ = _molecules(1, t, seed0=7)[0]
    Hd = torch.from_numpy(H).to(device)
    lab = hip.fock_to_irreps(Hd, off, z, r_, c_, t.orbital_template)
    hip._wk_fwd, hip._blocks_fwd = hip._w_fwd, hip._blocks_fwd.reshape(-1, 4).clone()
    hip._blocks_fwd[:, 3] = -1
    hip._blocks_fwd = hip._blocks_fwd.reshape(-1)
    assert torch.equal(lab, hip.fock_to_irreps(Hd, off, z, r_, c_, t.orbital_template))


def test_fused_fock_to_irreps_and_back(device):
    from maloq_amd.basis_transform import HipE3TensorDecomp
    t, base, ora = _tables(CFG3)
    hip = HipE3TensorDecomp(base)
    for z, H, off, rows, cols in _molecules(3, t, seed0=20):
        lab = _oracle_labels(t, z, H, off, rows, cols, 196)
        ref = ora.get_net_out(torch.from_numpy(lab).double())
        Hd = torch.from_numpy(H).to(device)
        got = hip.fock_to_irreps(Hd, off, z, rows, cols, t.orbital_template).cpu().double()
        scale = ref.abs().max()
        assert (got - ref).abs().max() / scale < 1e-5
        # inverse: scatter back into a zero matrix
        H2 = torch.zeros_like(Hd)
        hip.irreps_to_fock(got.float().to(device), H2, off, z, rows, cols, t.orbital_template)
        mask = np.zeros(H.shape, bool)
        for i, j in zip(rows, cols):
            mask[off[i]:off[i + 1], off[j]:off[j + 1]] = True
        diff = np.abs(H2.cpu().numpy() - H)[mask].max()
        assert diff / np.abs(H).max() < 1e-6
        assert np.all(H2.cpu().numpy()[~mask] == 0)


def test_fused_sparse_storage(device):
    from maloq_amd.basis_transform import HipE3TensorDecomp
    t, base, ora = _tables(SIO2)
    hip = HipE3TensorDecomp(base)
    from maloq_amd.synth import sio2_cell, radius_graph, atom_pair_rows
    Z, pos, L = sio2_cell(n_atoms=120, seed=1, iters=200)
    src, dst, vec = radius_graph(pos, 5.0, cell=L)
    rows, cols = atom_pair_rows(src, dst, len(Z))
    off = np.concatenate([[0], np.cumsum(t.orbitals_per_atom(Z))]).astype(np.int32)
    rng = np.random.default_rng(0)
    bdo = om2l.block_data_offsets(off, rows, cols)
    data = rng.standard_normal(int(bdo[-1])).astype(np.float32)
    lab = np.zeros((len(rows), 169), np.float32)
    om2l.single_matrix2label_sparse(t.orbital_template, off, Z, rows, cols, data, bdo, lab, True)
    ref = ora.get_net_out(torch.from_numpy(lab).double())
    dd = torch.from_numpy(data).to(device)
    bd = torch.from_numpy(bdo).to(device)
    got = hip.fock_to_irreps(dd, off, Z, rows, cols, t.orbital_template, block_data_offsets=bd).cpu().double()
    assert (got - ref).abs().max() / ref.abs().max() < 1e-5
    back = torch.zeros_like(dd)
    hip.irreps_to_fock(got.float().to(device), back, off, Z, rows, cols, t.orbital_template, block_data_offsets=bd)
    assert np.abs(back.cpu().numpy() - data).max() / np.abs(data).max() < 1e-6


def test_config3_full_scale_round_trip(device):
    """All 64 molecules of the benchmark's config 3: bit-exact gather against the
    oracle and round trip within 1e-6."""
    from maloq_amd.basis_transform import HipE3TensorDecomp
    from maloq_amd.matrix2labels import hip_single_matrix2label
    from maloq_amd.synth import config3_molecules, radius_graph, dense_hamiltonian, atom_pair_rows
    t, base, ora = _tables(CFG3)
    hip = HipE3TensorDecomp(base)
    mols = config3_molecules()
    worst = 0.0
    for m, (z, p) in enumerate(mols):
        H, off = dense_hamiltonian(z, p, t.orbitals_per_atom(z), seed=m, cutoff=8.0)
        src, dst, _ = radius_graph(p, 8.0)
        rows, cols = atom_pair_rows(src, dst, len(z))
        Hd = torch.from_numpy(H).to(device)
        if m < 4:
            ref = _oracle_labels(t, z, H, off, rows, cols, 196)
            lab = torch.zeros(len(rows), 196, device=device)
            hip_single_matrix2label(t.orbital_template, off, z, rows, cols, Hd, lab, None, True)
            assert np.array_equal(lab.cpu().numpy(), ref)
        irr = hip.fock_to_irreps(Hd, off, z, rows, cols, t.orbital_template)
        H2 = torch.zeros_like(Hd)
        hip.irreps_to_fock(irr, H2, off, z, rows, cols, t.orbital_template)
        worst = max(worst, ((H2 - Hd).abs().max() / Hd.abs().max()).item())
    assert worst < 1e-6


def test_row_plan_reuse_and_mismatch(device):
    """A prebuilt row plan (rows in their original order) gives the same labels
    as the per-call plan; a plan for another storage is refused."""
    from maloq_amd.basis_transform import HipE3TensorDecomp
    t, base, ora = _tables(CFG3)
    hip = HipE3TensorDecomp(base)
    z, H, off, rows, cols = _molecules(1, t, seed0=40)[0]
    Hd = torch.from_numpy(H).to(device)
    plan = hip.make_plan(Hd, off, z, rows, cols, t.orbital_template)
    a = hip.fock_to_irreps(Hd, off, z, rows, cols, t.orbital_template)
    b = hip.fock_to_irreps(Hd, off, z, rows, cols, t.orbital_template, plan=plan)
    assert torch.equal(a, b)
    assert plan.meta[:, 2].cpu().tolist() == list(range(len(rows)))
    wide = torch.zeros(H.shape[0], H.shape[1] + 3, device=device)[:, :H.shape[1]]  # other row stride
    with pytest.raises(ValueError):
        hip.fock_to_irreps(wide, off, z, rows, cols, t.orbital_template, plan=plan)


def test_pair_list_calls_equal_planned_calls(device):
    """Without a plan the fused transforms describe their rows from the pair
    list inside the kernel (maloq_fock_to_irreps_pairs /
    maloq_irreps_to_fock_pairs): the same bits as with a prebuilt plan, both
    directions, block-list and dense storage; block offsets given on the host
    are moved to the device."""
    from maloq_amd.basis_transform import HipE3TensorDecomp
    from maloq_amd.synth import sio2_cell, radius_graph, atom_pair_rows
    t, base, ora = _tables(SIO2)
    hip = HipE3TensorDecomp(base)
    Z, pos, L = sio2_cell(n_atoms=150, seed=3, iters=200)
    src, dst, vec = radius_graph(pos, 5.0, cell=L)
    rows, cols = atom_pair_rows(src, dst, len(Z))
    off = np.concatenate([[0], np.cumsum(t.orbitals_per_atom(Z))]).astype(np.int32)
    bdo = om2l.block_data_offsets(off, rows, cols)
    data = np.random.default_rng(1).standard_normal(int(bdo[-1])).astype(np.float32)
    dd = torch.from_numpy(data).to(device)
    bd = torch.from_numpy(bdo).to(device)
    plan = hip.make_plan(dd, off, Z, rows, cols, t.orbital_template, block_data_offsets=bd)
    a = hip.fock_to_irreps(dd, off, Z, rows, cols, t.orbital_template, block_data_offsets=bd, plan=plan)
    for offsets in (bd, bdo, torch.from_numpy(bdo)):  # device tensor, numpy, host tensor
        b = hip.fock_to_irreps(dd, off, Z, rows, cols, t.orbital_template, block_data_offsets=offsets)
        assert torch.equal(a, b)
    back_a, back_b = torch.zeros_like(dd), torch.zeros_like(dd)
    hip.irreps_to_fock(a, back_a, off, Z, rows, cols, t.orbital_template, block_data_offsets=bd, plan=plan)
    hip.irreps_to_fock(a, back_b, off, Z, rows, cols, t.orbital_template, block_data_offsets=bdo)
    assert torch.equal(back_a, back_b)
    assert np.abs(back_b.cpu().numpy() - data).max() / np.abs(data).max() < 1e-6
    # dense storage, the inverse direction (the forward is compared in the test above)
    t3, base3, _ = _tables(CFG3)
    hip3 = HipE3TensorDecomp(base3)
    z, H, off3, r3, c3 = _molecules(1, t3, seed0=41)[0]
    Hd = torch.from_numpy(H).to(device)
    plan3 = hip3.make_plan(Hd, off3, z, r3, c3, t3.orbital_template)
    irr = hip3.fock_to_irreps(Hd, off3, z, r3, c3, t3.orbital_template)
    H_a, H_b = torch.zeros_like(Hd), torch.zeros_like(Hd)
    hip3.irreps_to_fock(irr, H_a, off3, z, r3, c3, t3.orbital_template, plan=plan3)
    hip3.irreps_to_fock(irr, H_b, off3, z, r3, c3, t3.orbital_template)
    assert torch.equal(H_a, H_b)


def _wide_molecule(t, elements, seed, n=12):
    from maloq_amd.synth import sphere_molecule, radius_graph, dense_hamiltonian, atom_pair_rows
    z, p = sphere_molecule(n, elements, [1.0] * len(elements), seed=seed)
    H, off = dense_hamiltonian(z, p, t.orbitals_per_atom(z), seed=seed + 1)
    src, dst, _ = radius_graph(p, 8.0)
    rows, cols = atom_pair_rows(src, dst, n)
    return z, H, off, rows, cols


@pytest.mark.parametrize("basis,elements", [(TZVPD_HCNO, ["H", "C", "N", "O"]), (TZVPD, ["H", "C", "N", "O"]),
                                            (TZVPD, ["H", "C", "O", "Ga", "I"])])
def test_wide_fused_fock_transforms(basis, elements, device):
    """def2-TZVPD widths, dense and block-list storage, with and without a row
    plan.  The gather and the scatter are bit-exact: fock_to_irreps(F) equals
    get_net_out of the oracle's gathered labels bit for bit (the same CG
    programs on the same tile), and irreps_to_fock(x) equals the oracle's
    scatter of get_H(x).  Against the fp64 oracle: 1e-5; round trip: 1e-6."""
    from maloq_amd.basis_transform import HipE3TensorDecomp
    t, base, ora = _tables(basis)
    hip = HipE3TensorDecomp(base)
    T = hip.total_in_dim
    assert hip.ngroups > 1
    for seed in (0, 1):
        z, H, off, rows, cols = _wide_molecule(t, elements, 50 + seed)
        lab = _oracle_labels(t, z, H, off, rows, cols, T)
        Hd = torch.from_numpy(H).to(device)
        want = hip.get_net_out(torch.from_numpy(lab).to(device))
        ref = ora.get_net_out(torch.from_numpy(lab).double())
        bdo = om2l.block_data_offsets(off, rows, cols)
        data = np.concatenate([H[off[i]:off[i + 1], off[j]:off[j + 1]].reshape(-1) for i, j in zip(rows, cols)])
        dd = torch.from_numpy(data).to(device)
        plan = hip.make_plan(Hd, off, z, rows, cols, t.orbital_template)
        for got in (hip.fock_to_irreps(Hd, off, z, rows, cols, t.orbital_template),
                    hip.fock_to_irreps(Hd, off, z, rows, cols, t.orbital_template, plan=plan),
                    hip.fock_to_irreps(dd, off, z, rows, cols, t.orbital_template, block_data_offsets=bdo)):
            assert torch.equal(got, want)
            assert (got.cpu().double() - ref).abs().max() / ref.abs().max() < 1e-5
        # inverse: scatter into zeros, compare with the oracle scatter of get_H
        Hx = hip.get_H(want).cpu().numpy()
        H_ref = np.zeros_like(H)
        om2l.single_matrix2label(t.orbital_template, off, z, rows, cols, H_ref, Hx.copy(), False)
        H2 = torch.zeros_like(Hd)
        hip.irreps_to_fock(want, H2, off, z, rows, cols, t.orbital_template)
        assert np.array_equal(H2.cpu().numpy(), H_ref)
        H3 = torch.zeros_like(Hd)
        hip.irreps_to_fock(want, H3, off, z, rows, cols, t.orbital_template, plan=plan)
        assert torch.equal(H2, H3)
        back = torch.zeros_like(dd)
        hip.irreps_to_fock(want, back, off, z, rows, cols, t.orbital_template, block_data_offsets=bdo)
        assert np.abs(back.cpu().numpy() - data).max() / np.abs(data).max() < 1e-6
        mask = np.zeros(H.shape, bool)
        for i, j in zip(rows, cols):
            mask[off[i]:off[i + 1], off[j]:off[j + 1]] = True
        assert np.abs(H2.cpu().numpy() - H)[mask].max() / np.abs(H).max() < 1e-6
        assert np.all(H2.cpu().numpy()[~mask] == 0)


def test_wide_sorted_fock_transforms(device):
    """Sorted irreps rows wider than one column group: the fused transforms
    permute in a separate column gather, and give the sorted rows of the
    unsorted decomposition exactly."""
    from maloq_amd.basis_transform import HipE3TensorDecomp
    t, base_s, _ = _tables(TZVPD_HCNO, if_sort=True)
    _, base_u, _ = _tables(TZVPD_HCNO)
    hs, hu = HipE3TensorDecomp(base_s), HipE3TensorDecomp(base_u)
    z, H, off, rows, cols = _wide_molecule(t, ["H", "C", "N", "O"], 60)
    Hd = torch.from_numpy(H).to(device)
    perm = torch.as_tensor(np.asarray(hs.sort_perm), device=device)
    a = hs.fock_to_irreps(Hd, off, z, rows, cols, t.orbital_template)
    b = hu.fock_to_irreps(Hd, off, z, rows, cols, t.orbital_template)
    assert torch.equal(a, b[:, perm])
    Ha, Hb = torch.zeros_like(Hd), torch.zeros_like(Hd)
    hs.irreps_to_fock(a, Ha, off, z, rows, cols, t.orbital_template)
    hu.irreps_to_fock(b, Hb, off, z, rows, cols, t.orbital_template)
    assert torch.equal(Ha, Hb)
