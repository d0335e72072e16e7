"""CPU restatement of the Fock <-> irreps basis transform tables (test oracle only).

* ``wigner_3j``           e3nn 0.5.x o3.wigner_3j (called at utils_tensor_decomp.py:93-94):
                          e3nn's own Racah sum form, complex -> real basis, real part,
                          unit Frobenius norm.  e3nn is absent here, so the published
                          algorithm is restated; see the package docstring for pins.
* ``E3TensorDecomp``      e3TensorDecomp (utils_tensor_decomp.py:51-169)
* ``make_output_irreps``  utils_tensor_decomp.py:206-306
* ``process_targets``     utils_tensor_decomp.py:309-373
* ``get_orbital_template``matrix2labels_kernels.py:1232-1271
"""
from __future__ import annotations

import math
from fractions import Fraction

import numpy as np
import torch


# ----------------------------------------------------------------- CG tables
def _cg_e3nn_form(j1, m1, j2, m2, j3, m3):
    if m3 != m1 + m2:
        return 0.0
    f = math.factorial
    vmin = max(-j1 + j2 + m3, -j1 + m1, 0)
    vmax = min(j2 + j3 + m1, j3 - j1 + j2, j3 + m3)
    pre = (2 * j3 + 1) * Fraction(
        f(j3 + j1 - j2) * f(j3 - j1 + j2) * f(j1 + j2 - j3) * f(j3 + m3) * f(j3 - m3),
        f(j1 + j2 + j3 + 1) * f(j1 - m1) * f(j1 + m1) * f(j2 - m2) * f(j2 + m2),
    )
    s = Fraction(0)
    for v in range(vmin, vmax + 1):
        s += (-1) ** (v + j2 + m2) * Fraction(
            f(j2 + j3 + m1 - v) * f(j1 - m1 + v),
            f(v) * f(j3 - j1 + j2 - v) * f(j3 + m3 - v) * f(v + j1 - j2 - m3),
        )
    return math.sqrt(float(pre)) * float(s)


def _q_real_to_complex(l):
    q = torch.zeros(2 * l + 1, 2 * l + 1, dtype=torch.complex128)
    r2 = 2 ** -0.5
    for m in range(-l, 0):
        q[l + m, l + abs(m)] = r2
        q[l + m, l - abs(m)] = -1j * r2
    q[l, l] = 1
    for m in range(1, l + 1):
        q[l + m, l + abs(m)] = (-1) ** m * r2
        q[l + m, l - abs(m)] = 1j * (-1) ** m * r2
    return (-1j) ** l * q


def wigner_3j(l1, l2, l3):
    c = torch.zeros(2 * l1 + 1, 2 * l2 + 1, 2 * l3 + 1, dtype=torch.float64)
    if abs(l1 - l2) <= l3 <= l1 + l2:
        for m1 in range(-l1, l1 + 1):
            for m2 in range(-l2, l2 + 1):
                if abs(m1 + m2) <= l3:
                    c[l1 + m1, l2 + m2, l3 + m1 + m2] = _cg_e3nn_form(l1, m1, l2, m2, l3, m1 + m2)
    q1, q2, q3 = _q_real_to_complex(l1), _q_real_to_complex(l2), _q_real_to_complex(l3)
    out = torch.einsum("ij,kl,mn,ikn->jlm", q1, q2, torch.conj(q3.T), c.to(torch.complex128))
    assert torch.all(out.imag.abs() < 1e-10)
    out = out.real
    return out / torch.norm(out)


# --------------------------------------------------------- e3TensorDecomp
class E3TensorDecomp:
    """Tables and dense transforms of e3TensorDecomp (utils_tensor_decomp.py:51-169)."""

    def __init__(self, out_js_list, if_sort=False, dtype=torch.float64):
        self.out_js_list = out_js_list
        self.in_slices, self.H_slices = [0], [0]
        self.wms, self.wms_H = [], []
        self.irreps_ls = []          # required_irreps_out as a list of l (mul 1, even)
        for l1, l2 in out_js_list:
            l1, l2 = l1 % 10, l2 % 10
            l3s = list(range(abs(l1 - l2), l1 + l2 + 1))
            self.irreps_ls += l3s
            self.in_slices.append(self.in_slices[-1] + sum(2 * l + 1 for l in l3s))
            self.H_slices.append(self.H_slices[-1] + (2 * l1 + 1) * (2 * l2 + 1))
            self.wms.append(torch.cat([wigner_3j(l1, l2, l3) for l3 in l3s], dim=-1).to(dtype))
            self.wms_H.append(torch.cat([wigner_3j(l3, l1, l2) * (2 * l3 + 1) for l3 in l3s], dim=0).to(dtype))
        T_in, T_h = self.in_slices[-1], self.H_slices[-1]
        self.W_global = torch.zeros(T_in, T_h, dtype=dtype)
        self.W_global_inv = torch.zeros(T_h, T_in, dtype=dtype)
        for i in range(len(out_js_list)):
            a, b = self.in_slices[i], self.in_slices[i + 1]
            c, d = self.H_slices[i], self.H_slices[i + 1]
            self.W_global[a:b, c:d] = self.wms[i].reshape(d - c, b - a).T
            self.W_global_inv[c:d, a:b] = self.wms_H[i].reshape(b - a, d - c).T
        self.sort_perm = None
        if if_sort:
            # e3nn Irreps.sort(): stable by (l, parity); all parities even here.
            order = sorted(range(len(self.irreps_ls)), key=lambda i: (self.irreps_ls[i], i))
            starts = np.cumsum([0] + [2 * l + 1 for l in self.irreps_ls])
            perm = []
            for i in order:
                perm += list(range(starts[i], starts[i + 1]))
            self.sort_perm = torch.tensor(perm)            # sorted column k <- unsorted perm[k]

    def sort(self, x):
        return x[:, self.sort_perm]

    def sort_inverse(self, x):
        out = torch.empty_like(x)
        out[:, self.sort_perm] = x
        return out

    def get_H(self, net_out):                         # utils_tensor_decomp.py:154-161
        if self.sort_perm is not None:
            net_out = self.sort_inverse(net_out)
        return net_out @ self.W_global.to(net_out.dtype)

    def get_net_out(self, H):                         # utils_tensor_decomp.py:163-169
        out = H @ self.W_global_inv.to(H.dtype)
        if self.sort_perm is not None:
            out = self.sort(out)
        return out


# ------------------------------------------------ integer / template tables
_ORB = {0: "s_", 1: "p_", 2: "d_", 3: "f_", 4: "g_", 10: "sd_", 11: "pd_", 12: "dd_"}


def make_output_irreps(orbital_basis):
    """utils_tensor_decomp.py:206-306.  Mutates orbital_basis (diffuse +10) like the reference."""
    for el, orbs in orbital_basis.items():
        cut = len(orbs)
        for i in range(1, len(orbs)):
            if orbs[i] < orbs[i - 1]:
                cut = i
                break
        orbs[cut:] = [o + 10 for o in orbs[cut:]]
    ls_list = []
    for l in range(20):
        ls_list += [l] * max(sum(1 for o in orbs if o == l) for orbs in orbital_basis.values())
    out_slices = [0]
    for l1 in ls_list:
        for l2 in ls_list:
            out_slices.append(out_slices[-1] + (2 * (l1 % 10) + 1) * (2 * (l2 % 10) + 1))

    def labels(orbs):
        res = []
        for i, o in enumerate(orbs):
            res.append(_ORB[o] + str(sum(1 for k in range(i) if orbs[k] == o)))
        return res

    inter = {}
    for a1, o1 in orbital_basis.items():
        for a2, o2 in orbital_basis.items():
            l1s, l2s = labels(o1), labels(o2)
            inter[f"{a1} {a2}"] = [x + "-" + y for x in l1s for y in l2s]
    full = []
    lab = labels(ls_list)
    for x in lab:
        for y in lab:
            full.append(x + "-" + y)
    n = len(ls_list)
    targets, out_js_list = [], []
    for bi, blk in enumerate(full):
        t = {}
        for key, keys in inter.items():
            if blk in keys:
                k = keys.index(blk)
                t[key] = [k // n, k % n]
        out_js_list.append((ls_list[bi // n], ls_list[bi % n]))
        if t:
            targets.append(t)
    return targets, ls_list, out_js_list, out_slices, full


def process_targets(orbital_basis, targets, full_orb_interaction_list):
    """utils_tensor_decomp.py:309-373: per target, per element pair, [r0, r1, c0, c1]."""
    rev = {v: k for k, v in _ORB.items()}
    keys = list(orbital_basis.keys())
    z_to_idx = {z: i for i, z in enumerate(keys)}
    kinds = [orbital_basis[z] for z in keys]
    blocks = []
    for ti, t in enumerate(targets):
        a, b = full_orb_interaction_list[ti].split("-")
        def split(s):
            i = len(s) - 1
            while s[i].isdigit():
                i -= 1
            return s[: i + 1], int(s[i + 1:])
        (t1, n1), (t2, n2) = split(a), split(b)
        eb = {}
        for key in t:
            zi, zj = (int(v) for v in key.split())
            b1 = np.array(kinds[z_to_idx[zi]])
            b2 = np.array(kinds[z_to_idx[zj]])
            i1 = np.where(b1 == rev[t1])[0][n1]
            i2 = np.where(b2 == rev[t2])[0][n2]
            r0 = int(sum(2 * (o % 10) + 1 for o in b1[:i1]))
            c0 = int(sum(2 * (o % 10) + 1 for o in b2[:i2]))
            eb[key] = [r0, r0 + 2 * (b1[i1] % 10) + 1, c0, c0 + 2 * (b2[i2] % 10) + 1]
        blocks.append(eb)
    return blocks


def get_orbital_template(equivariant_blocks, orbital_starts, max_elements=100):
    """matrix2labels_kernels.py:1232-1271: template[Zi*100+Zj] = [(rows, cols, out)]."""
    tmpl = [[] for _ in range(max_elements ** 2)]
    for ti, eb in enumerate(equivariant_blocks):
        for key, s in eb.items():
            zi, zj = (int(v) for v in key.split())
            tmpl[zi * max_elements + zj].append(
                (slice(s[0], s[1]), slice(s[2], s[3]), slice(orbital_starts[ti], orbital_starts[ti + 1]))
            )
    return tmpl
