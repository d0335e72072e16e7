"""GPU: deterministic sorted-segment sum vs fp64 index_add_ (esen_block.py:194-206)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _csr(dst, n):
    perm = np.argsort(dst, kind="stable")
    counts = np.bincount(dst, minlength=n)
    return perm, np.concatenate([[0], np.cumsum(counts)])


@pytest.mark.parametrize("E,N,W", [(0, 5, 16), (1, 3, 8), (1000, 37, 3200), (5000, 200, 7), (30000, 1280, 3200)])
def test_segment_sum_matches_fp64_and_is_deterministic(E, N, W, device):
    from maloq_amd import _lib
    rng = np.random.default_rng(E + N)
    dst = rng.integers(0, N, E)
    perm, ptr = _csr(dst, N)
    msg = torch.from_numpy(rng.standard_normal((E, W)).astype(np.float32)).to(device)
    p = torch.from_numpy(perm).to(device)
    sp = torch.from_numpy(ptr).to(device)
    outs = []
    for _ in range(2):
        out = torch.empty(N, W, device=device)
        _lib.call("maloq_segment_sum", _lib.ptr(msg), _lib.ptr(p), _lib.ptr(sp), N, W, _lib.ptr(out),
                  _lib.stream_of(device))
        outs.append(out)
    assert torch.equal(outs[0], outs[1])
    ref = torch.zeros(N, W, dtype=torch.float64).index_add_(0, torch.from_numpy(dst), msg.cpu().double())
    tol = 1e-5 * max(1.0, float(np.sqrt(max(1, E / max(N, 1)))))
    assert (outs[0].cpu().double() - ref).abs().max() < tol
