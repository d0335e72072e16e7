"""CPU restatement of the reference's torch Wigner path (test oracle only).

Follows ``src/maloq/helm/common/rotation.py``:
* ``init_edge_rot_euler_angles``  rotation.py:68-83 (gamma drawn by the caller),
* ``_z_rot_mat``                  rotation.py:204-225,
* ``wigner_D``                    rotation.py:189-201,
* ``eulers_to_wigner``            rotation.py:19-39.
All arithmetic is float64 torch on the CPU.
"""
from __future__ import annotations

import math
import os

import numpy as np
import torch

_GOLDEN = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "tests", "golden")


def load_jd(dtype=torch.float64):
    """J_0..J_11 as stored in the reference's src/maloq/helm/Jd.pt (fixture copy)."""
    z = np.load(os.path.join(_GOLDEN, "jd_reference.npz"))
    return [torch.from_numpy(z[f"J{l}"]).to(dtype) for l in range(len(z.files))]


def init_edge_rot_euler_angles(edge_distance_vec: torch.Tensor, gamma_uniform: torch.Tensor):
    """rotation.py:68-83 with the random roll supplied: gamma = u * 2*pi."""
    xyz = torch.nn.functional.normalize(edge_distance_vec).clamp(-1.0, 1.0)
    x, y, z = xyz[:, 0], xyz[:, 1], xyz[:, 2]
    beta = torch.acos(y)
    alpha = torch.atan2(x, z)
    gamma = gamma_uniform.to(alpha.dtype) * 2 * math.pi
    return -gamma, -beta, -alpha


def z_rot_mat(angle: torch.Tensor, lv: int) -> torch.Tensor:
    """rotation.py:204-225: sin on the anti-diagonal, then cos on the diagonal."""
    M = angle.new_zeros((*angle.shape, 2 * lv + 1, 2 * lv + 1))
    freqs = list(range(lv, -lv - 1, -1))
    for i, f in enumerate(freqs):
        M[..., i, 2 * lv - i] = torch.sin(f * angle)
        M[..., i, i] = torch.cos(f * angle)
    return M


def wigner_D(lv, alpha, beta, gamma, Jd):
    """rotation.py:189-201: X(alpha) J X(beta) J X(gamma)."""
    alpha, beta, gamma = torch.broadcast_tensors(alpha, beta, gamma)
    J = Jd[lv].to(alpha.dtype)
    return z_rot_mat(alpha, lv) @ J @ z_rot_mat(beta, lv) @ J @ z_rot_mat(gamma, lv)


def eulers_to_wigner(eulers, start_lmax, end_lmax, Jd):
    """rotation.py:19-39: block-diagonal [E, d, d]."""
    alpha, beta, gamma = eulers
    size = (end_lmax + 1) ** 2 - start_lmax ** 2
    w = torch.zeros(len(alpha), size, size, dtype=alpha.dtype)
    start = 0
    for l in range(start_lmax, end_lmax + 1):
        b = wigner_D(l, alpha, beta, gamma, Jd)
        end = start + b.shape[1]
        w[:, start:end, start:end] = b
        start = end
    return w
