"""Host tables of the HIP basis transform, checked on the CPU.

A numpy model of what the kernels do with the tables (per column group: drop
every listed element of an atom-pair block into its column, contract the
group's CG blocks in place with their n x n matrices, store through the sort
permutation) is compared with the oracle: the gather bit-exactly with
numpy_single_matrix2label, the transforms with the dense fp64 e3TensorDecomp
within 1e-12, at the config widths and at the def2-TZVPD widths (1600 and 4096
columns, several groups).
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
# def2-TZVPD shells (src/maloq/fock_utils/basis_sets.py:28, keyed by Z as get_loader.py:106-107
# does): H/C/N/O gives 1600-column rows; with Ga (4 d shells) and I (2 f shells) the
# template reaches the 64 orbitals of the whole dictionary, 4096 columns and 400 CG blocks.
TZVPD_HCNO = {1: [0, 0, 0, 1, 1], 6: [0, 0, 0, 0, 0, 1, 1, 1, 2, 2, 3, 0, 2],
              7: [0, 0, 0, 0, 0, 1, 1, 1, 2, 2, 3, 0, 2], 8: [0, 0, 0, 0, 0, 1, 1, 1, 2, 2, 3, 0, 1, 2]}
TZVPD = {**TZVPD_HCNO, 31: [0, 0, 0, 0, 0, 0, 1, 1, 1, 1, 1, 2, 2, 2, 2, 3, 0, 2],
         53: [0, 0, 0, 0, 0, 0, 1, 1, 1, 1, 1, 2, 2, 2, 3, 3, 0, 1, 2]}


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


def _groups_of(sched):
    G = int(sched[0])
    return [tuple(int(v) for v in sched[1 + 4 * g:5 + 4 * g]) for g in range(G)]


@pytest.mark.parametrize("basis", [MOCK, CFG3, SIO2, FSHELL, TZVPD_HCNO, TZVPD])
def test_wave_schedule_covers_every_block_once(basis):
    """Column groups partition the row into runs of whole CG blocks (at most 64
    blocks and GROUP_COLS columns each), and every group's 4 wave lists hold
    each of its blocks once, balanced to within one block."""
    from maloq_amd.basis_transform import cg_block_tables, GROUP_COLS
    t, base, ora = _setup(basis)
    tabs = cg_block_tables(base)
    s = tabs["sched"]
    blocks = tabs["blocks"]
    nb, T = len(blocks), int(base.in_slices[-1])
    groups = _groups_of(s)
    assert [g[:3] for g in groups] == [g[:3] for g in tabs["groups"]]
    col = blk = 0
    for c0, width, b0, off in groups:
        assert c0 == col and b0 == blk and width <= max(GROUP_COLS, 1)
        ls = s[off:off + 5]
        ids = s[off + 5:off + 5 + ls[4]]
        assert ls[0] == 0 and np.all(np.diff(ls) >= 0) and len(ids) <= 64
        assert sorted(ids.tolist()) == list(range(b0, b0 + len(ids)))
        assert int(blocks[b0][1]) == c0 and sum(int(blocks[b][0]) for b in ids) == width
        cost = [sum(int(blocks[b][0]) ** 2 for b in ids[ls[w]:ls[w + 1]]) for w in range(4)]
        assert max(cost) <= sum(cost) / 4 + max(int(blocks[b][0]) ** 2 for b in ids)
        col, blk = col + width, blk + len(ids)
    assert col == T and blk == nb
    if T <= GROUP_COLS:
        assert len(groups) == 1


def _rect(slots, g, k):
    """Rectangle (r0, nr, c0, nc) of (group g, kind k) and its column table."""
    K, G = int(slots[0]), int(slots[1])
    rect = int(slots[2 + G + g * K + k]) & 0xFFFFFFFF
    r0, nr, c0, nc = rect & 255, (rect >> 8) & 255, (rect >> 16) & 255, rect >> 24
    off = int(slots[2 + G + G * K + g * K + k])
    return r0, nr, c0, nc, slots[off:off + nr * nc].astype(np.int64)


def _slot_entries(slots, g, k, nj):
    """(element q, group column) pairs of (group g, kind k) from its rectangle,
    nj the kind's block width."""
    r0, nr, c0, nc, tab = _rect(slots, g, k)
    i, j = np.divmod(np.arange(nr * nc), max(nc, 1))
    q = (r0 + i) * nj + c0 + j
    keep = tab >= 0
    return q[keep], tab[keep]


def _gather_model(H, off, Z, rows, cols, pair_kind, slots, groups, T, bdo=None):
    """The kernel's gather: per column group, walk the (group, kind) rectangle
    of every atom-pair block (row-major, memory order) and drop each element
    into its column of the group."""
    lab = np.zeros((len(rows), T), H.dtype)
    for r, (i, j) in enumerate(zip(rows, cols)):
        k = pair_kind[Z[i] * 100 + Z[j]]
        if k < 0:
            continue
        ni, nj = off[i + 1] - off[i], off[j + 1] - off[j]
        for g, (c0, width, _, _) in enumerate(groups):
            r0, nr, cc, nc, tab = _rect(slots, g, k)
            if nr == 0 or r0 + nr > ni or cc + nc > nj:
                continue
            assert np.all(tab < width)
            for e in range(nr * nc):
                if tab[e] < 0:
                    continue
                a, b = r0 + e // nc, cc + e % nc
                lab[r, c0 + tab[e]] = H[off[i] + a, off[j] + b] if bdo is None else H[bdo[r] + a * nj + b]
    return lab


def _check_slot_tables(t, raw, kb, h_slices, groups):
    """The rectangles cover exactly each kind's raw_slot entries of the group
    (the largest one in the header), and bit i of a (group, kind) mask is set
    exactly when some element lands in the group's i-th block."""
    slots = t["slots"]
    K, G = int(slots[0]), int(slots[1])
    assert G == len(groups) and K == raw.shape[0]
    hs = np.asarray(h_slices)
    pk = t["pair_kind"]
    nj_of = {}
    for key in np.nonzero(pk >= 0)[0]:
        nj_of[int(pk[key])] = None
    for g, (c0, width, b0, nb) in enumerate(groups):
        largest = 0
        for k in range(K):
            r0, nr, cc, nc, tab = _rect(slots, g, k)
            largest = max(largest, nr * nc)
            want = np.nonzero((raw[k] >= c0) & (raw[k] < c0 + width))[0]
            got_cols = np.sort(tab[tab >= 0] + c0)
            assert np.array_equal(got_cols, np.sort(raw[k][want]))
            have = set(np.searchsorted(hs, got_cols, side="right") - 1 - b0)
            mask = int(kb[g * K + k, 0]) | (int(kb[g * K + k, 1]) << 32)
            assert have == {i for i in range(nb) if mask >> i & 1}
        assert int(slots[2 + g]) == largest


def _contract_model(x, tabs, w, perm_in=None, perm_out=None):
    """The contraction as the kernel schedules it: per column group, the blocks
    of its wave lists in place on the group's columns."""
    s = tabs["sched"]
    tile = np.zeros_like(x)
    if perm_in is None:
        tile[:] = x
    else:
        tile[:, perm_in] = x
    for c0, width, b0, off in _groups_of(s):
        part = tile[:, c0:c0 + width].copy()
        for b in s[off + 5:off + 5 + s[off + 4]]:
            n, bc, wo = (int(v) for v in tabs["blocks"][b])
            W = w[wo:wo + n * n].reshape(n, n)
            part[:, bc - c0:bc - c0 + n] = part[:, bc - c0:bc - c0 + n] @ W.T
        tile[:, c0:c0 + width] = part
    return tile if perm_out is None else tile[:, perm_out]


@pytest.mark.parametrize("basis", [TZVPD_HCNO, TZVPD])
def test_grouped_contraction_matches_dense_transforms(basis):
    """def2-TZVPD widths (1600 and 4096 columns, several column groups): the
    grouped contraction equals the dense fp64 e3TensorDecomp, both directions
    and the adjoint."""
    from maloq_amd.basis_transform import cg_block_tables
    t, base, ora = _setup(basis)
    tabs = cg_block_tables(base)
    assert len(tabs["groups"]) > 1
    T = int(ora.H_slices[-1])
    rng = np.random.default_rng(5)
    H = rng.standard_normal((12, T))
    ref = ora.get_net_out(torch.from_numpy(H)).numpy()
    assert np.abs(_contract_model(H, tabs, tabs["w_fwd"]) - ref).max() < 1e-12
    x = rng.standard_normal((12, T))
    ref = ora.get_H(torch.from_numpy(x)).numpy()
    assert np.abs(_contract_model(x, tabs, tabs["w_inv"]) - ref).max() < 1e-12
    g = rng.standard_normal((12, T))
    lhs = np.sum(_contract_model(x, tabs, tabs["w_inv"]) * g)
    rhs = np.sum(x * _contract_model(g, tabs, tabs["w_adj"]))
    assert abs(lhs - rhs) < 1e-9 * abs(lhs)


@pytest.mark.parametrize("basis,elements", [(CFG3, ["H", "C", "N", "O"]), (TZVPD_HCNO, ["H", "C", "N", "O"]),
                                            (TZVPD, ["H", "C", "O", "Ga", "I"])])
def test_slot_tables_gather_bit_exact(basis, elements):
    from maloq_amd.basis_transform import template_slot_tables, cg_block_tables
    from maloq_amd.synth import sphere_molecule, radius_graph, dense_hamiltonian, atom_pair_rows
    t, base, ora = _setup(basis)
    groups = cg_block_tables(base)["groups"]
    tabs = template_slot_tables(t.orbital_template, base.H_slices, groups)
    _check_slot_tables(tabs, tabs["raw_slot"], tabs["kind_blocks"], base.H_slices, groups)
    # groups of whole shell rows or runs of one shell row: every rectangle is
    # exactly its kind's elements (no lanes spent on holes)
    K = int(tabs["slots"][0])
    for g in range(len(groups)):
        for k in range(K):
            assert np.all(_rect(tabs["slots"], g, k)[4] >= 0)
    T = int(base.H_slices[-1])
    z, p = sphere_molecule(9, elements, [1.0 / len(elements)] * len(elements), seed=3)
    H, off = dense_hamiltonian(z, p, t.orbitals_per_atom(z), seed=4)
    src, dst, _ = radius_graph(p, 8.0)
    rows, cols = atom_pair_rows(src, dst, len(z))
    ref = np.zeros((len(rows), T), np.float32)
    om2l.single_matrix2label(t.orbital_template, off, z, rows, cols, H, ref, True)
    got = _gather_model(H.astype(np.float32), off, z, rows, cols, tabs["pair_kind"], tabs["slots"], groups, T)
    assert np.array_equal(got, ref)


def test_slot_tables_sparse_gather_bit_exact():
    from maloq_amd.basis_transform import template_slot_tables
    from maloq_amd.synth import sio2_cell, radius_graph, atom_pair_rows
    t, base, ora = _setup(SIO2)
    tabs = template_slot_tables(t.orbital_template, base.H_slices)
    groups = [(0, 169, 0, len(base.out_js_list))]
    _check_slot_tables(tabs, tabs["raw_slot"], tabs["kind_blocks"], base.H_slices, groups)
    Z, pos, L = sio2_cell(n_atoms=30, seed=2, iters=100)
    src, dst, _ = radius_graph(pos, 5.0, cell=L)
    rows, cols = atom_pair_rows(src, dst, len(Z))
    off = np.concatenate([[0], np.cumsum(t.orbitals_per_atom(Z))]).astype(np.int32)
    bdo = om2l.block_data_offsets(off, rows, cols)
    data = np.random.default_rng(0).standard_normal(int(bdo[-1])).astype(np.float32)
    ref = np.zeros((len(rows), 169), np.float32)
    om2l.single_matrix2label_sparse(t.orbital_template, off, Z, rows, cols, data, bdo, ref, True)
    got = _gather_model(data, off, Z, rows, cols, tabs["pair_kind"], tabs["slots"], groups, 169, bdo=bdo)
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


def test_fock_extent_checked_on_host():
    """With the Fock storage given, the host also checks every atom-pair block's
    extent: orbital offsets one orbital past a dense matrix, and a block list
    whose offsets are too few or reach past the flat data, are refused."""
    from maloq_amd.basis_transform import _check_pairs_on_host
    off = np.array([0, 5, 19, 33], np.int32)
    Z = np.array([1, 6, 8], np.int32)
    rows, cols = np.array([0, 1, 2, 2]), np.array([0, 2, 1, 2])
    _check_pairs_on_host(off, Z, rows, cols, torch.zeros(33, 33))
    with pytest.raises(ValueError, match="outside"):
        _check_pairs_on_host(np.array([0, 5, 19, 34], np.int32), Z, rows, cols, torch.zeros(33, 33))
    with pytest.raises(ValueError, match="outside"):
        _check_pairs_on_host(off, Z, rows, cols, torch.zeros(33, 32))
    n = np.diff(off)
    sizes = n[rows] * n[cols]
    bdo = np.concatenate([[0], np.cumsum(sizes)[:-1]]).astype(np.int64)
    data = torch.zeros(int(sizes.sum()))
    _check_pairs_on_host(off, Z, rows, cols, data, bdo)
    _check_pairs_on_host(off, Z, rows, cols, data, torch.from_numpy(bdo))
    with pytest.raises(ValueError, match="entries for 4 atom pairs"):
        _check_pairs_on_host(off, Z, rows, cols, data, bdo[:3])
    with pytest.raises(ValueError, match="outside"):
        _check_pairs_on_host(off, Z, rows, cols, data, bdo + 1)
    with pytest.raises(ValueError, match="outside"):
        _check_pairs_on_host(off, Z, rows, cols, data, bdo - 1)
