"""Seeded synthetic inputs for the benchmark configurations.

Geometry follows the generator described for the reference's headline
benchmarks: atoms uniform in a sphere at a fixed number density with a
minimum separation (rejection sampling, one seed per molecule), an all-ordered
-pairs radius graph, edge vectors ``pos[src] - pos[dst]`` stored as
``edge_attr = [dist, x, y, z]`` (fock_targets_batched.py:218-220) and fed to the
Wigner path as ``edge_attr[:, [2, 3, 1]]`` (esen_osh.py:318).  Synthetic
Hamiltonians: atom-pair blocks N(0,1) * exp(-r/2), symmetric, on-site blocks
shifted by -10.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

SYMBOL_Z = {"H": 1, "C": 6, "N": 7, "O": 8, "F": 9, "Si": 14, "S": 16, "Ga": 31, "I": 53}


@dataclass
class Graph:
    Z: np.ndarray            # [N] int
    pos: np.ndarray          # [N, 3] float64
    src: np.ndarray          # [E] int64 (sorted by src, then dst)
    dst: np.ndarray          # [E] int64
    vec: np.ndarray          # [E, 3] pos[src] - pos[dst] (minimum image if periodic)
    mol: np.ndarray          # [N] molecule id
    cell: float | None = None

    @property
    def num_nodes(self):
        return len(self.Z)

    @property
    def num_edges(self):
        return len(self.src)

    def edge_attr(self):
        d = np.linalg.norm(self.vec, axis=1, keepdims=True)
        return np.concatenate([d, self.vec], axis=1)

    def edge_distance_vec(self):
        """The e3nn-frame vectors the Wigner path consumes (esen_osh.py:318)."""
        return self.edge_attr()[:, [2, 3, 1]]


def sphere_molecule(n_atoms, symbols, probs, seed, density=0.1, min_sep=0.9):
    rng = np.random.default_rng(seed)
    radius = (3.0 * n_atoms / (4.0 * math.pi * density)) ** (1.0 / 3.0)
    pos = []
    while len(pos) < n_atoms:
        p = rng.uniform(-radius, radius, 3)
        if np.dot(p, p) > radius * radius:
            continue
        if pos and np.min(np.linalg.norm(np.asarray(pos) - p, axis=1)) < min_sep:
            continue
        pos.append(p)
    z = rng.choice([SYMBOL_Z[s] for s in symbols], size=n_atoms, p=np.asarray(probs) / np.sum(probs))
    return z.astype(np.int64), np.asarray(pos)


def radius_graph(pos, cutoff, mol=None, cell=None):
    """All ordered pairs i != j with 0 < r < cutoff inside each molecule (or
    under the minimum image in a cubic cell of side ``cell``)."""
    n = len(pos)
    if mol is None:
        mol = np.zeros(n, np.int64)
    src_all, dst_all, vec_all = [], [], []
    for m in np.unique(mol):
        idx = np.nonzero(mol == m)[0]
        p = pos[idx]
        v = p[:, None, :] - p[None, :, :]
        if cell is not None:
            v -= cell * np.round(v / cell)
        r = np.linalg.norm(v, axis=-1)
        ok = (r < cutoff) & (r > 0)
        s, d = np.nonzero(ok)
        src_all.append(idx[s]); dst_all.append(idx[d]); vec_all.append(v[s, d])
    src = np.concatenate(src_all).astype(np.int64)
    dst = np.concatenate(dst_all).astype(np.int64)
    vec = np.concatenate(vec_all)
    o = np.lexsort((dst, src))
    return src[o], dst[o], vec[o]


def config1_graph():
    """12 atoms (6 H, 4 C, 2 O) uniform in a 6 A cube (seed 0), min 0.9 A, 5 A cutoff."""
    rng = np.random.default_rng(0)
    pos = []
    while len(pos) < 12:
        p = rng.uniform(0.0, 6.0, 3)
        if pos and np.min(np.linalg.norm(np.asarray(pos) - p, axis=1)) < 0.9:
            continue
        pos.append(p)
    pos = np.asarray(pos)
    Z = np.array([1] * 6 + [6] * 4 + [8] * 2, np.int64)
    src, dst, vec = radius_graph(pos, 5.0)
    return Graph(Z, pos, src, dst, vec, np.zeros(12, np.int64))


def batch_of_molecules(n_mol, n_atoms, symbols, probs, cutoff, seed0=0, spacing=1000.0):
    Zs, ps, mols = [], [], []
    for m in range(n_mol):
        na = n_atoms(m) if callable(n_atoms) else n_atoms
        z, p = sphere_molecule(na, symbols, probs, seed=seed0 + m)
        Zs.append(z); ps.append(p + np.array([spacing * m, 0.0, 0.0])); mols.append(np.full(na, m))
    Z, pos, mol = np.concatenate(Zs), np.concatenate(ps), np.concatenate(mols)
    src, dst, vec = radius_graph(pos, cutoff, mol)
    return Graph(Z, pos, src, dst, vec, mol)


def config2_graph():
    """32 molecules x 40 atoms, H/C/N/O/F/S .45/.30/.10/.10/.03/.02, 6 A cutoff."""
    return batch_of_molecules(32, 40, ["H", "C", "N", "O", "F", "S"],
                              [0.45, 0.30, 0.10, 0.10, 0.03, 0.02], 6.0)


def config3_molecules(n_mol=64, seed0=0):
    """64 molecules of 30-50 atoms, H/C/N/O (config-2 probabilities renormalised)."""
    rng = np.random.default_rng(12345)
    sizes = rng.integers(30, 51, size=n_mol)
    probs = np.array([0.45, 0.30, 0.10, 0.10])
    out = []
    for m in range(n_mol):
        z, p = sphere_molecule(int(sizes[m]), ["H", "C", "N", "O"], probs / probs.sum(), seed=seed0 + m)
        out.append((z, p))
    return out


def config4_graph():
    """8 molecules x 150 atoms, H/C/N/O/S .5/.3/.08/.1/.02, 8 A cutoff."""
    return batch_of_molecules(8, 150, ["H", "C", "N", "O", "S"], [0.5, 0.3, 0.08, 0.1, 0.02], 8.0)


def sio2_cell(n_atoms=2000, density_g_cm3=2.2, seed=0, iters=400):
    """Amorphous SiO2-like cubic cell: Si:O = 1:2, min separations Si-O 1.5 A and
    others 2.4 A, from random positions relaxed by pairwise push-apart."""
    n_si = n_atoms // 3
    Z = np.array([14] * n_si + [8] * (n_atoms - n_si), np.int64)
    mass = (n_si * 28.0855 + (n_atoms - n_si) * 15.999) * 1.66053906660e-24
    L = (mass / density_g_cm3 * 1e24) ** (1.0 / 3.0)
    rng = np.random.default_rng(seed)
    pos = rng.uniform(0.0, L, (n_atoms, 3))
    is_si = Z == 14
    # Pairwise push-apart over a pair list (pairs closer than 2.4 + skin A at
    # the last rebuild; an atom moves far less than skin / 2 between rebuilds,
    # so no pair outside the list can come within 2.4 A).
    skin, rebuild = 1.2, 8
    pi = pj = dmin = None
    since = rebuild
    for _ in range(iters):
        if since >= rebuild:
            v = pos[:, None, :] - pos[None, :, :]
            v -= L * np.round(v / L)
            r = np.linalg.norm(v, axis=-1)
            pi, pj = np.nonzero(np.triu(r < 2.4 + skin, 1))
            dmin = np.where(is_si[pi] ^ is_si[pj], 1.5, 2.4)
            since = 0
        fresh = since == 0
        since += 1
        v = pos[pi] - pos[pj]
        v -= L * np.round(v / L)
        r = np.linalg.norm(v, axis=-1)
        viol = np.clip(dmin - r, 0.0, None)
        if viol.size == 0 or viol.max() < 1e-9:
            if fresh:       # converged on a list that holds every close pair
                break
            since = rebuild
            continue
        f = (viol / np.maximum(r, 1e-9))[:, None] * v * 0.5
        push = np.zeros_like(pos)
        for k in range(3):
            push[:, k] = np.bincount(pi, f[:, k], n_atoms) - np.bincount(pj, f[:, k], n_atoms)
        pos = (pos + push) % L
    return Z, pos, L


def config5_graph(cutoff=6.0):
    Z, pos, L = sio2_cell()
    src, dst, vec = radius_graph(pos, cutoff, cell=L)
    return Graph(Z, pos, src, dst, vec, np.zeros(len(Z), np.int64), cell=L)


# ------------------------------------------------------------- Hamiltonians
def dense_hamiltonian(Z, pos, orbitals_per_atom, seed, cutoff=None):
    """Symmetric [n, n]: block (i, j) ~ N(0,1) exp(-r_ij/2), H_ji = H_ij^T,
    on-site blocks symmetrised and shifted by -10."""
    rng = np.random.default_rng(seed)
    off = np.concatenate([[0], np.cumsum(orbitals_per_atom)]).astype(np.int64)
    n = int(off[-1])
    H = np.zeros((n, n), np.float64)
    na = len(Z)
    for i in range(na):
        for j in range(i, na):
            r = float(np.linalg.norm(pos[i] - pos[j]))
            if cutoff is not None and i != j and r >= cutoff:
                continue
            blk = rng.standard_normal((off[i + 1] - off[i], off[j + 1] - off[j])) * math.exp(-r / 2.0)
            if i == j:
                blk = 0.5 * (blk + blk.T) - 10.0 * np.eye(blk.shape[0])
            H[off[i]:off[i + 1], off[j]:off[j + 1]] = blk
            H[off[j]:off[j + 1], off[i]:off[i + 1]] = blk.T
    return H.astype(np.float32), off


def atom_pair_rows(src, dst, num_atoms):
    """Rows [edges..., on-site...] as in make_targets (fock_targets_batched.py:392-396)."""
    rows = np.concatenate([np.asarray(src), np.arange(num_atoms)])
    cols = np.concatenate([np.asarray(dst), np.arange(num_atoms)])
    return rows.astype(np.int32), cols.astype(np.int32)
