"""Host tables of the HIP basis transform, checked on the CPU.

A numpy model of what the kernels do with the tables (drop every element of
an atom-pair block into its label column through raw_slot, contract every CG
block in place with its n x n matrix, store through the sort permutation) is compared with the oracle: the gather
bit-exactly with numpy_single_matrix2label, the transforms with the dense
fp64 e3TensorDecomp within 1e-12.
"""
import numpy as np
import pytest
import torch

from oracle import matrix2labels as om2l
from oracle import tensor_decomp as otd

CFG3 = {1: [0, 0, 1], 6: [0, 0, 0, 1, 1, 2], 7: [0, 0, 0, 1, 1, 2], 8: [0, 0, 0, 1, 1, 2]}
MOCK = {1: [0], 6: [0, 0, 1], 8: [0, 0, 1]}
SIO2 = {14: [0, 0, 1, 1, 2], 8: [0, 0, 1, 1, 2]}
FSHELL = {1: [0, 0, 1], 6: [0, 0, 1, 1, 2, 3]}


def _setup(basis, if_sort=False):
    from maloq_amd import tensor_decomp as ptd
    t = ptd.BasisTables(basis)
    base = ptd.e3TensorDecomp(t.simplified_irreps if if_sort else t.req_output_irreps, t.out_js_list,
                              torch.float64, if_sort=if_sort, device_torch="cpu")
    ora = otd.E3TensorDecomp(t.out_js_list, if_sort=if_sort)
    return t, base, ora


def _model(x, tabs, w, perm_in=None, perm_out=None):
    """The contraction phase of the transform kernel on a [R, T] tile."""
    tile = np.zeros_like(x)
    if perm_in is None:
        tile[:] = x
    else:
        tile[:, perm_in] = x
    for n, c0, wo in tabs["blocks"]:
        W = w[wo:wo + n * n].reshape(n, n)
        tile[:, c0:c0 + n] = tile[:, c0:c0 + n] @ W.T
    return tile if perm_out is None else tile[:, perm_out]


@pytest.mark.parametrize("basis,if_sort", [(MOCK, True), (MOCK, False), (CFG3, False), (SIO2, False),
                                           (FSHELL, False)])
def test_block_tables_reproduce_dense_transforms(basis, if_sort):
    from maloq_amd.basis_transform import cg_block_tables
    t, base, ora = _setup(basis, if_sort)
    tabs = cg_block_tables(base)
    perm = getattr(base, "sort_perm", None)
    T = int(ora.H_slices[-1])
    rng = np.random.default_rng(1)
    H = rng.standard_normal((50, T))
    x = rng.standard_normal((50, T))
    ref = ora.get_net_out(torch.from_numpy(H)).numpy()
    assert np.abs(_model(H, tabs, tabs["w_fwd"], perm_out=perm) - ref).max() < 1e-12
    ref = ora.get_H(torch.from_numpy(x)).numpy()
    assert np.abs(_model(x, tabs, tabs["w_inv"], perm_in=perm) - ref).max() < 1e-12
    # adjoint of get_H: <get_H(x), g> == <x, adj(g)>
    g = rng.standard_normal((50, T))
    lhs = np.sum(_model(x, tabs, tabs["w_inv"], perm_in=perm) * g)
    rhs = np.sum(x * _model(g, tabs, tabs["w_adj"], perm_out=perm))
    assert abs(lhs - rhs) < 1e-9 * abs(lhs)


@pytest.mark.parametrize("basis", [MOCK, CFG3, SIO2, FSHELL])
def test_wave_schedule_covers_every_block_once(basis):
    from maloq_amd.basis_transform import cg_block_tables
    t, base, ora = _setup(basis)
    tabs = cg_block_tables(base)
    s = tabs["sched"]
    nb = len(tabs["blocks"])
    assert s[0] == 0 and s[4] == nb and np.all(np.diff(s[:5]) >= 0)
    assert sorted(s[5:].tolist()) == list(range(nb))
    cost = [sum(int(tabs["blocks"][b][0]) ** 2 for b in s[5 + s[w]:5 + s[w + 1]]) for w in range(4)]
    assert max(cost) <= sum(cost) / 4 + max(int(n) ** 2 for n, _, _ in tabs["blocks"])


def _gather_model(H, off, Z, rows, cols, pair_kind, raw, bdo=None):
    """The kernel's gather: walk every atom-pair block in memory order and drop
    element q into label column raw[kind, q]."""
    T = 196 if raw.max() < 196 else int(raw.max()) + 1
    lab = np.zeros((len(rows), T), H.dtype)
    for r, (i, j) in enumerate(zip(rows, cols)):
        k = pair_kind[Z[i] * 100 + Z[j]]
        if k < 0:
            continue
        ni, nj = off[i + 1] - off[i], off[j + 1] - off[j]
        for q in range(ni * nj):
            c = int(raw[k, q])
            if c < 0:
                continue
            a, b = divmod(q, nj)
            lab[r, c] = H[off[i] + a, off[j] + b] if bdo is None else H[bdo[r] + q]
    return lab


def _check_kind_blocks(raw, kb, h_slices):
    """Bit b of a kind's mask is set exactly when some element lands in block b."""
    hs = np.asarray(h_slices)
    for k in range(raw.shape[0]):
        cols = raw[k][raw[k] >= 0]
        have = set(np.searchsorted(hs, cols, side="right") - 1)
        mask = int(kb[k, 0]) | (int(kb[k, 1]) << 32)
        assert have == {b for b in range(len(hs) - 1) if mask >> b & 1}


def test_slot_tables_gather_bit_exact():
    from maloq_amd.basis_transform import template_slot_tables
    from maloq_amd.synth import sphere_molecule, radius_graph, dense_hamiltonian, atom_pair_rows
    t, base, ora = _setup(CFG3)
    pk, raw, kb = template_slot_tables(t.orbital_template, base.H_slices)
    _check_kind_blocks(raw, kb, base.H_slices)
    z, p = sphere_molecule(14, ["H", "C", "N", "O"], [0.45, 0.3, 0.15, 0.1], seed=3)
    H, off = dense_hamiltonian(z, p, t.orbitals_per_atom(z), seed=4)
    src, dst, _ = radius_graph(p, 8.0)
    rows, cols = atom_pair_rows(src, dst, len(z))
    ref = np.zeros((len(rows), 196), np.float32)
    om2l.single_matrix2label(t.orbital_template, off, z, rows, cols, H, ref, True)
    got = _gather_model(H.astype(np.float32), off, z, rows, cols, pk, raw)
    assert np.array_equal(got, ref)


def test_slot_tables_sparse_gather_bit_exact():
    from maloq_amd.basis_transform import template_slot_tables
    from maloq_amd.synth import sio2_cell, radius_graph, atom_pair_rows
    t, base, ora = _setup(SIO2)
    pk, raw, kb = template_slot_tables(t.orbital_template, base.H_slices)
    _check_kind_blocks(raw, kb, base.H_slices)
    Z, pos, L = sio2_cell(n_atoms=30, seed=2, iters=100)
    src, dst, _ = radius_graph(pos, 5.0, cell=L)
    rows, cols = atom_pair_rows(src, dst, len(Z))
    off = np.concatenate([[0], np.cumsum(t.orbitals_per_atom(Z))]).astype(np.int32)
    bdo = om2l.block_data_offsets(off, rows, cols)
    data = np.random.default_rng(0).standard_normal(int(bdo[-1])).astype(np.float32)
    ref = np.zeros((len(rows), 169), np.float32)
    om2l.single_matrix2label_sparse(t.orbital_template, off, Z, rows, cols, data, bdo, ref, True)
    got = _gather_model(data, off, Z, rows, cols, pk, raw, bdo=bdo)[:, :169]
    assert np.array_equal(got, ref)


def test_unsupported_block_size_rejected():
    from maloq_amd.basis_transform import cg_block_tables
    t, base, ora = _setup({1: [0, 4]})   # a g shell: 9 x 9 = 81 > 49
    with pytest.raises(ValueError):
        cg_block_tables(base)


def test_pair_structure_checked_on_host():
    """Index arrays given on the host are range-checked before any launch (the
    kernels index with them unchecked)."""
    import numpy as np
    import pytest
    import torch
    from maloq_amd.basis_transform import _check_pairs_on_host
    off = np.array([0, 5, 19, 33], np.int32)
    Z = np.array([1, 6, 8], np.int32)
    rows, cols = np.array([0, 1, 2, 2]), np.array([0, 2, 1, 2])
    _check_pairs_on_host(off, Z, rows, cols)
    _check_pairs_on_host(torch.from_numpy(off), torch.from_numpy(Z), torch.from_numpy(rows), torch.from_numpy(cols))
    with pytest.raises(IndexError):
        _check_pairs_on_host(off, Z, rows, np.array([0, 3, 1, 2]))
    with pytest.raises(IndexError):
        _check_pairs_on_host(off, Z, np.array([-1, 1, 2, 2]), cols)
    with pytest.raises(ValueError):
        _check_pairs_on_host(off, np.array([1, 6, 100], np.int32), rows, cols)
    with pytest.raises(ValueError):
        _check_pairs_on_host(np.array([0, 5, 4, 33], np.int32), Z, rows, cols)
    with pytest.raises(ValueError):
        _check_pairs_on_host(off, Z, rows, cols[:3])
