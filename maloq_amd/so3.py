"""Host-side SO(3) tables for the MI355X hot path.

Everything here is small, integer or fp64, computed once on the host and
uploaded to the device by the callers:

* ``CoefficientMapping``: the l-major <-> m-major coefficient permutation
  (reference ``src/maloq/helm/common/so3.py:15-133``).
* ``jd_matrices``: the per-degree involutions ``J_l`` that the reference ships as
  ``src/maloq/helm/Jd.pt`` (loaded at ``esen_osh.py:125-127``).  They are rebuilt
  here in closed form, ``J_l = (-1)^l D^l(R_pi)``, with ``R_pi`` the half turn
  about the (1,1,0)/sqrt2 axis of the e3nn frame, so the product does not need
  the reference's data file at run time.
* ``wigner_3j``: real Clebsch-Gordan tensors in the same real basis, following
  e3nn 0.5.x ``o3.wigner_3j`` (called at ``utils_tensor_decomp.py:93-94``):
  Racah's formula in the complex basis, change to the real basis with
  ``change_basis_real_to_complex`` (including its ``(-i)^l`` phase), real part,
  unit Frobenius norm.
"""

from __future__ import annotations

import functools
import math
from fractions import Fraction

import numpy as np


# ---------------------------------------------------------------------------
# Real <-> complex spherical-harmonic basis (e3nn convention)
# ---------------------------------------------------------------------------
@functools.lru_cache(maxsize=None)
def change_basis_real_to_complex(l: int) -> np.ndarray:
    """Rows: complex m = -l..l; columns: real index 0..2l.  Includes (-i)^l."""
    q = np.zeros((2 * l + 1, 2 * l + 1), dtype=np.complex128)
    s = 1.0 / math.sqrt(2.0)
    for m in range(-l, 0):
        q[l + m, l - m] = s
        q[l + m, l + m] = -1j * s
    q[l, l] = 1.0
    for m in range(1, l + 1):
        sign = (-1.0) ** m
        q[l + m, l + m] = sign * s
        q[l + m, l - m] = 1j * sign * s
    q = ((-1j) ** l) * q
    q.setflags(write=False)
    return q


@functools.lru_cache(maxsize=None)
def so3_generators(l: int) -> np.ndarray:
    """Real generators [3, 2l+1, 2l+1] of rotations about the e3nn-frame x, y, z."""
    m = np.arange(-l, l, dtype=np.float64)
    raising = np.diag(-np.sqrt(l * (l + 1) - m * (m + 1)), k=-1)
    m = np.arange(-l + 1, l + 1, dtype=np.float64)
    lowering = np.diag(np.sqrt(l * (l + 1) - m * (m - 1)), k=1)
    m = np.arange(-l, l + 1, dtype=np.float64)
    su2 = np.stack(
        [0.5 * (raising + lowering), np.diag(1j * m), -0.5j * (raising - lowering)]
    ).astype(np.complex128)
    q = change_basis_real_to_complex(l)
    gens = np.einsum("ji,ajk,kl->ail", q.conj(), su2, q)
    assert np.abs(gens.imag).max() < 1e-12
    out = np.ascontiguousarray(gens.real)
    out.setflags(write=False)
    return out


def _expm_antisymmetric(a: np.ndarray, t: float) -> np.ndarray:
    """exp(t*A) for real antisymmetric A via the Hermitian eigenproblem of iA."""
    w, v = np.linalg.eigh(1j * a)
    r = (v * np.exp(-1j * t * w)) @ v.conj().T
    return r.real


@functools.lru_cache(maxsize=None)
def _jd_single(l: int) -> np.ndarray:
    if l == 0:
        j = np.ones((1, 1))
    else:
        g = so3_generators(l)
        axis = (g[0] + g[1]) / math.sqrt(2.0)
        j = ((-1.0) ** l) * _expm_antisymmetric(axis, math.pi)
        j[np.abs(j) < 1e-14] = 0.0
    j.setflags(write=False)
    return j


def jd_matrices(lmax: int) -> list[np.ndarray]:
    """[J_0, ..., J_lmax] as fp64 arrays (the content of the reference's Jd.pt)."""
    return [_jd_single(l) for l in range(lmax + 1)]


def pack_jd(jd_list, lmax: int) -> np.ndarray:
    """Concatenate J_0..J_lmax row-major into one fp32 vector (device layout).

    Block l starts at ``sum_{k<l} (2k+1)^2``.
    """
    parts = []
    for l in range(lmax + 1):
        j = np.asarray(jd_list[l], dtype=np.float64)
        assert j.shape == (2 * l + 1, 2 * l + 1), f"J_{l} has shape {j.shape}"
        parts.append(j.reshape(-1))
    return np.concatenate(parts).astype(np.float32)


# ---------------------------------------------------------------------------
# Clebsch-Gordan / Wigner 3j (real basis)
# ---------------------------------------------------------------------------
def _su2_cg(j1: int, m1: int, j2: int, m2: int, j3: int, m3: int) -> float:
    """Condon-Shortley <j1 m1; j2 m2 | j3 m3> by Racah's closed form (exact)."""
    if m3 != m1 + m2:
        return 0.0
    if not (abs(j1 - j2) <= j3 <= j1 + j2):
        return 0.0
    if abs(m1) > j1 or abs(m2) > j2 or abs(m3) > j3:
        return 0.0
    f = math.factorial
    pre = Fraction(
        (2 * j3 + 1) * f(j3 + j1 - j2) * f(j3 - j1 + j2) * f(j1 + j2 - j3),
        f(j1 + j2 + j3 + 1),
    ) * Fraction(f(j3 + m3) * f(j3 - m3) * f(j1 - m1) * f(j1 + m1) * f(j2 - m2) * f(j2 + m2))
    total = Fraction(0)
    kmin = max(0, j2 - j3 - m1, j1 + m2 - j3)
    kmax = min(j1 + j2 - j3, j1 - m1, j2 + m2)
    for k in range(kmin, kmax + 1):
        den = (
            f(k)
            * f(j1 + j2 - j3 - k)
            * f(j1 - m1 - k)
            * f(j2 + m2 - k)
            * f(j3 - j2 + m1 + k)
            * f(j3 - j1 - m2 + k)
        )
        total += Fraction((-1) ** k, den)
    return float(total) * math.sqrt(float(pre))


@functools.lru_cache(maxsize=None)
def _su2_cg_tensor(l1: int, l2: int, l3: int) -> np.ndarray:
    t = np.zeros((2 * l1 + 1, 2 * l2 + 1, 2 * l3 + 1))
    for m1 in range(-l1, l1 + 1):
        for m2 in range(-l2, l2 + 1):
            m3 = m1 + m2
            if abs(m3) <= l3:
                t[l1 + m1, l2 + m2, l3 + m3] = _su2_cg(l1, m1, l2, m2, l3, m3)
    return t


@functools.lru_cache(maxsize=None)
def _wigner_3j_cached(l1: int, l2: int, l3: int) -> np.ndarray:
    q1 = change_basis_real_to_complex(l1)
    q2 = change_basis_real_to_complex(l2)
    q3 = change_basis_real_to_complex(l3)
    c = _su2_cg_tensor(l1, l2, l3).astype(np.complex128)
    # out[a, b, c] = sum_{i,k,n} q1[i,a] q2[k,b] conj(q3[n,c]) C[i,k,n]
    out = np.einsum("ia,kb,nc,ikn->abc", q1, q2, q3.conj(), c)
    assert np.abs(out.imag).max() < 1e-10, "CG tensor is not real"
    out = out.real
    out = out / np.linalg.norm(out)
    out.setflags(write=False)
    return out


def wigner_3j(l1: int, l2: int, l3: int) -> np.ndarray:
    """Real-basis coupling tensor [2l1+1, 2l2+1, 2l3+1], unit Frobenius norm."""
    if not (abs(l1 - l2) <= l3 <= l1 + l2):
        raise ValueError(f"({l1},{l2},{l3}) violates the triangle rule")
    return _wigner_3j_cached(int(l1), int(l2), int(l3))


# ---------------------------------------------------------------------------
# l-major <-> m-major coefficient mapping
# ---------------------------------------------------------------------------
class CoefficientMapping:
    """Integer tables for the l-major / m-major coefficient orders.

    Mirrors ``CoefficientMapping`` (reference ``so3.py:25-133``) without torch
    buffers.  The l-major layout lists, for l = 0..lmax, the orders
    m = -min(l, mmax)..min(l, mmax).  The m-major layout lists m = 0 for
    l = 0..lmax, then +1 for l = 1..lmax, -1 for l = 1..lmax, +2, -2, ...
    (``so3.py:52-64``).

    ``to_m_index[i]`` is the l-major position of m-major row i, so a tensor in
    l-major order ``x`` becomes ``x[to_m_index]`` in m-major order.
    """

    def __init__(self, lmax: int, mmax: int):
        assert 0 <= mmax <= lmax
        self.lmax = lmax
        self.mmax = mmax
        l_h, m_h, m_c = [], [], []
        for l in range(lmax + 1):
            mm = min(mmax, l)
            for m in range(-mm, mm + 1):
                l_h.append(l)
                m_c.append(m)
                m_h.append(abs(m))
        self.l_harmonic = np.array(l_h, dtype=np.int64)
        self.m_harmonic = np.array(m_h, dtype=np.int64)
        self.m_complex = np.array(m_c, dtype=np.int64)
        self.res_size = len(l_h)
        order = []
        self.m_size = [0] * (mmax + 1)
        for m in range(mmax + 1):
            plus = [i for i in range(self.res_size) if self.m_complex[i] == m]
            order.extend(plus)
            self.m_size[m] = len(plus)
            if m != 0:
                order.extend(i for i in range(self.res_size) if self.m_complex[i] == -m)
        self.to_m_index = np.array(order, dtype=np.int64)
        to_m = np.zeros((self.res_size, self.res_size), dtype=np.float32)
        to_m[np.arange(self.res_size), self.to_m_index] = 1.0
        self.to_m = to_m

    def coefficient_idx(self, lmax: int, mmax: int) -> np.ndarray:
        """l-major positions with l <= lmax and |m| <= mmax (``so3.py:126-133``)."""
        mask = (self.l_harmonic <= lmax) & (self.m_harmonic <= mmax)
        return np.nonzero(mask)[0].astype(np.int64)

    def __repr__(self) -> str:
        return f"{self.__class__.__name__}(lmax={self.lmax}, mmax={self.mmax})"


def kept_rows(lmax: int, mmax: int) -> list[tuple[int, int]]:
    """(l, i) for every kept row of the full (lmax+1)^2 l-major layout, in
    m-major order: i is the row inside the l block (order m = i - l)."""
    rows = [(l, l) for l in range(lmax + 1)]
    for m in range(1, mmax + 1):
        rows += [(l, l + m) for l in range(m, lmax + 1)]
        rows += [(l, l - m) for l in range(m, lmax + 1)]
    return rows
