"""Host-side tables of the Fock <-> irreps basis transform.

Mirrors the reference's table builders with the same names and return values:
``l1l2_to_l3s``, ``e3TensorDecomp``, ``make_output_irreps``, ``process_targets``
(src/maloq/fock_utils/utils_tensor_decomp.py:12-373) and ``get_orbital_template``
(src/maloq/fock_utils/matrix2labels_kernels.py:1232-1271).  e3nn is not a
dependency: irreps are represented by the small ``Irreps`` class below and the
CG tensors come from ``maloq_amd.so3.wigner_3j``.

``e3TensorDecomp.get_H`` / ``get_net_out`` keep the reference's dense torch
matmuls (its 'torch' backend); the HIP backend is
``maloq_amd.basis_transform.HipE3TensorDecomp``.
"""
from __future__ import annotations

import copy
from collections import namedtuple

import numpy as np
import torch

from .so3 import wigner_3j

MAX_ELEMENTS = 100

Irrep = namedtuple("Irrep", ["l", "p"])


class Irreps(tuple):
    """Minimal e3nn-style irreps: a tuple of (mul, Irrep(l, p)) pairs."""

    def __new__(cls, items=()):
        if items is None:
            items = ()
        out = []
        for mul, ir in items:
            if not isinstance(ir, Irrep):
                ir = Irrep(int(ir[0]), int(ir[1]))
            out.append((int(mul), ir))
        return super().__new__(cls, out)

    @property
    def dim(self) -> int:
        return sum(mul * (2 * ir.l + 1) for mul, ir in self)

    @property
    def ls(self) -> list:
        return [ir.l for mul, ir in self for _ in range(mul)]

    def __add__(self, other):
        return Irreps(list(self) + list(Irreps(other)))

    def sort(self):
        """Stable sort by (l, p); returns (irreps, p, inv) like e3nn's Irreps.sort()."""
        order = sorted(range(len(self)), key=lambda i: (self[i][1].l, self[i][1].p, i))
        inv = tuple(order)
        p = [0] * len(order)
        for new, old in enumerate(order):
            p[old] = new
        Ret = namedtuple("sort", ["irreps", "p", "inv"])
        return Ret(Irreps([self[i] for i in order]), tuple(p), inv)

    def simplify(self):
        out = []
        for mul, ir in self:
            if out and out[-1][1] == ir:
                out[-1] = (out[-1][0] + mul, ir)
            elif mul > 0:
                out.append((mul, ir))
        return Irreps(out)

    def __repr__(self):
        return "+".join(f"{mul}x{ir.l}{'e' if ir.p == 1 else 'o'}" for mul, ir in self)


def l1l2_to_l3s(l1, l2) -> Irreps:
    """Even irreps l3 = |l1-l2|..l1+l2 (utils_tensor_decomp.py:12-22); diffuse l kept mod 10."""
    l1, l2 = l1 % 10, l2 % 10
    return Irreps([(1, (l, 1)) for l in range(abs(l1 - l2), l1 + l2 + 1)])


class e3TensorDecomp:  # noqa: N801  (reference name)
    """Coupled <-> uncoupled basis tables (utils_tensor_decomp.py:51-137).

    wms[i]   : [2l1+1, 2l2+1, n_irr]   w3j(l1, l2, l3) concatenated over l3
    wms_H[i] : [n_irr, 2l1+1, 2l2+1]   (2l3+1) * w3j(l3, l1, l2) concatenated over l3
    """

    def __init__(self, net_irreps_out, out_js_list, default_dtype_torch=torch.float32,
                 if_sort=False, device_torch="cpu"):
        self.dtype = default_dtype_torch
        self.device = device_torch
        self.out_js_list = [tuple(x) for x in out_js_list]
        required = Irreps()
        self.in_slices, self.H_slices = [0], [0]
        self.wms, self.wms_H = [], []
        for l1, l2 in self.out_js_list:
            l1, l2 = l1 % 10, l2 % 10
            single = l1l2_to_l3s(l1, l2)
            required = required + single
            self.in_slices.append(required.dim)
            self.H_slices.append(self.H_slices[-1] + (2 * l1 + 1) * (2 * l2 + 1))
            l3s = [ir.l for _, ir in single]
            wm = np.concatenate([wigner_3j(l1, l2, l3) for l3 in l3s], axis=-1)
            wm_h = np.concatenate([wigner_3j(l3, l1, l2) * (2 * l3 + 1) for l3 in l3s], axis=0)
            self.wms.append(torch.from_numpy(wm).to(device=device_torch, dtype=default_dtype_torch))
            self.wms_H.append(torch.from_numpy(wm_h).to(device=device_torch, dtype=default_dtype_torch))
        if net_irreps_out is not None:
            want = required.sort().irreps.simplify() if if_sort else required
            assert Irreps(net_irreps_out) == want, f"requires {want} but got {net_irreps_out}"
        T_in, T_h = self.in_slices[-1], self.H_slices[-1]
        self.W_global = torch.zeros(T_in, T_h, device=device_torch, dtype=default_dtype_torch)
        self.W_global_inv = torch.zeros(T_h, T_in, device=device_torch, dtype=default_dtype_torch)
        for i in range(len(self.out_js_list)):
            a, b = self.in_slices[i], self.in_slices[i + 1]
            c, d = self.H_slices[i], self.H_slices[i + 1]
            self.W_global[a:b, c:d] = self.wms[i].reshape(d - c, b - a).T
            self.W_global_inv[c:d, a:b] = self.wms_H[i].reshape(b - a, d - c).T
        self._required = required
        self.sort = None
        self.sort_perm = None  # sorted column k holds unsorted column sort_perm[k]
        if if_sort:
            srt = required.sort()
            starts = np.cumsum([0] + [mul * (2 * ir.l + 1) for mul, ir in required])
            perm = []
            for i in srt.inv:
                perm.extend(range(starts[i], starts[i + 1]))
            self.sort_perm = np.asarray(perm, dtype=np.int64)
            self.sort = _SortIrreps(self.sort_perm)
            self.required_irreps_out = srt.irreps.simplify()
        else:
            self.required_irreps_out = required

    def get_H(self, net_out):
        if self.sort is not None:
            net_out = self.sort.inverse(net_out)
        return torch.matmul(net_out, self.W_global)

    def get_net_out(self, H):
        out = torch.matmul(H, self.W_global_inv)
        if self.sort is not None:
            out = self.sort(out)
        return out


class _SortIrreps:
    """Column permutation of sort_irreps (utils_tensor_decomp.py:24-49)."""

    def __init__(self, perm):
        self.perm = np.asarray(perm)
        self.inv = np.argsort(self.perm)

    def __call__(self, x):
        return x[..., torch.as_tensor(self.perm, device=x.device)]

    def inverse(self, x):
        return x[..., torch.as_tensor(self.inv, device=x.device)]


_ORB_TYPES = {0: "s_", 1: "p_", 2: "d_", 3: "f_", 4: "g_", 10: "sd_", 11: "pd_", 12: "dd_"}


def _shell_names(shells):
    seen: dict = {}
    names = []
    for s in shells:
        names.append(f"{_ORB_TYPES[s]}{seen.get(s, 0)}")
        seen[s] = seen.get(s, 0) + 1
    return names


def make_output_irreps(orbital_basis):
    """utils_tensor_decomp.py:206-306.  Like the reference, shells after the first
    decrease in l are flagged diffuse (+10) in ``orbital_basis`` in place."""
    for el, shells in orbital_basis.items():
        cut = next((i for i in range(1, len(shells)) if shells[i] < shells[i - 1]), len(shells))
        shells[cut:] = [s + 10 for s in shells[cut:]]
    ls_list = []
    for l in range(20):
        ls_list += [l] * max(list(shells).count(l) for shells in orbital_basis.values())
    req = Irreps()
    out_slices = [0]
    for l1 in ls_list:
        for l2 in ls_list:
            req = req + l1l2_to_l3s(l1, l2)
            out_slices.append(np.int32(out_slices[-1] + (2 * (l1 % 10) + 1) * (2 * (l2 % 10) + 1)))
    pair_keys = {}
    for z1, s1 in orbital_basis.items():
        n1 = _shell_names(s1)
        for z2, s2 in orbital_basis.items():
            n2 = _shell_names(s2)
            pair_keys[f"{z1} {z2}"] = [a + "-" + b for a in n1 for b in n2]
    names = _shell_names(ls_list)
    full = [a + "-" + b for a in names for b in names]
    n = len(ls_list)
    targets, out_js_list = [], []
    for bi, blk in enumerate(full):
        t = {}
        for key, keys in pair_keys.items():
            if blk in keys:
                k = keys.index(blk)
                t[key] = [k // n, k % n]
        out_js_list.append((ls_list[bi // n], ls_list[bi % n]))
        if t:
            targets.append(t)
    return targets, req, req.sort()[0].simplify(), ls_list, out_js_list, out_slices, full


def process_targets(orbital_basis, targets, ls_list=None, out_js_list=None,
                    full_orb_interaction_list=None):
    """utils_tensor_decomp.py:309-373: [r0, r1, c0, c1] of every target in every
    element-pair block."""
    code = {v: k for k, v in _ORB_TYPES.items()}
    blocks = []
    for ti, target in enumerate(targets):
        a, b = full_orb_interaction_list[ti].split("-")
        ta, na = a.rstrip("0123456789"), int(a[len(a.rstrip("0123456789")):])
        tb, nb = b.rstrip("0123456789"), int(b[len(b.rstrip("0123456789")):])
        eb = {}
        for key in target:
            z1, z2 = (int(v) for v in key.split())
            s1 = np.asarray(orbital_basis[z1])
            s2 = np.asarray(orbital_basis[z2])
            i1 = np.nonzero(s1 == code[ta])[0][na]
            i2 = np.nonzero(s2 == code[tb])[0][nb]
            r0 = int(np.sum(2 * (s1[:i1] % 10) + 1))
            c0 = int(np.sum(2 * (s2[:i2] % 10) + 1))
            eb[key] = [r0, r0 + int(2 * (s1[i1] % 10) + 1), c0, c0 + int(2 * (s2[i2] % 10) + 1)]
        blocks.append(eb)
    return blocks


def get_orbital_template(equivariant_blocks, orbital_starts):
    """matrix2labels_kernels.py:1232-1271: list of 100*100 lists of
    (row slice, col slice, output slice), keyed Zi*100 + Zj."""
    template = [[] for _ in range(MAX_ELEMENTS ** 2)]
    for ti, eb in enumerate(equivariant_blocks):
        for key, (r0, r1, c0, c1) in eb.items():
            z1, z2 = (int(v) for v in key.split())
            template[z1 * MAX_ELEMENTS + z2].append(
                (slice(r0, r1), slice(c0, c1), slice(int(orbital_starts[ti]), int(orbital_starts[ti + 1])))
            )
    return template


class BasisTables:
    """Everything derived from an orbital basis, built the way Fock_Targets does
    (fock_targets_batched.py:100-150) without mutating the caller's dict."""

    def __init__(self, orbital_basis):
        basis = copy.deepcopy({k: list(v) for k, v in orbital_basis.items()})
        (targets, self.req_output_irreps, self.simplified_irreps, ls_list, self.out_js_list,
         self.orbital_starts, full) = make_output_irreps(basis)
        blocks = process_targets(basis, targets, ls_list, self.out_js_list, full)
        self.orbital_template = get_orbital_template(blocks, self.orbital_starts)
        self.ls_list = [l % 10 for l in ls_list]
        self.orbital_basis = {k: [s % 10 for s in v] for k, v in basis.items()}

    def orbitals_per_atom(self, atomic_numbers):
        return [sum(2 * l + 1 for l in self.orbital_basis[int(z)]) for z in atomic_numbers]
