"""The compiled CG programs of the basis transform (cg_blocks.h), on the CPU:
the committed header is what the generator writes, every compiled block
equals the oracle's e3nn-restated block for its shell pair, and the host
matches programs only where a decomposition's block is the same matrix."""
import ctypes

import numpy as np
import pytest
import torch

from maloq_amd import _lib
from maloq_amd import tensor_decomp as ptd
from maloq_amd.basis_transform import cg_block_tables
from maloq_amd.csrc import gen_cg_blocks
from oracle import tensor_decomp as otd

CFG3 = {1: [0, 0, 1], 6: [0, 0, 0, 1, 1, 2], 7: [0, 0, 0, 1, 1, 2], 8: [0, 0, 0, 1, 1, 2]}
WITH_F = {1: [0, 1], 6: [0, 0, 1, 2, 3], 8: [0, 1, 1, 2, 3]}


def _compiled(p, n):
    buf = np.empty(n * n, np.float32)
    rc = _lib.load().maloq_basis_cg_block(p, buf.ctypes.data_as(ctypes.c_void_p).value, n)
    assert rc == 0, _lib.load().maloq_last_error()
    return buf.reshape(n, n)


def test_header_is_current():
    with open(gen_cg_blocks.HEADER) as f:
        assert f.read() == gen_cg_blocks.render(), "regenerate: python -m maloq_amd.csrc.gen_cg_blocks"


@pytest.mark.parametrize("l1", range(4))
@pytest.mark.parametrize("l2", range(4))
def test_compiled_blocks_match_oracle(l1, l2):
    """Program (dir, l1, l2) against the oracle's float64 wms_H / wms / wms^T
    (utils_tensor_decomp.py:85-99 restated): same zero pattern, values to fp32
    rounding."""
    n = (2 * l1 + 1) * (2 * l2 + 1)
    o = otd.E3TensorDecomp([(l1, l2)], dtype=torch.float64)
    inv = o.wms[0].numpy().reshape(n, n)
    want = {0: o.wms_H[0].numpy().reshape(n, n), 1: inv, 2: inv.T}
    for d in range(3):
        got = _compiled(d * 16 + l1 * 4 + l2, n).astype(np.float64)
        ref = want[d]
        nz = np.abs(ref) > 1e-12
        assert np.array_equal(got != 0, nz), f"zero pattern of program ({d}, {l1}, {l2})"
        assert np.allclose(got, ref, rtol=2e-7, atol=1e-7), f"values of program ({d}, {l1}, {l2})"


def test_about_a_fifth_of_the_entries_are_nonzero():
    mats = gen_cg_blocks.block_matrices()
    dense = sum(m.size for (d, _, _), m in mats.items() if d == 0)
    nnz = sum(int(np.count_nonzero(m)) for (d, _, _), m in mats.items() if d == 0)
    assert nnz < 0.25 * dense


@pytest.mark.parametrize("basis", [CFG3, WITH_F])
def test_host_matches_every_block_of_a_decomposition(basis):
    t = ptd.BasisTables(basis)
    base = ptd.e3TensorDecomp(t.req_output_irreps, t.out_js_list, torch.float32, device_torch="cpu")
    tabs = cg_block_tables(base)
    progs = tabs["programs"]
    assert progs.shape == (3, len(base.out_js_list))
    for b, (l1, l2) in enumerate(base.out_js_list):
        for d in range(3):
            assert progs[d, b] == d * 16 + (l1 % 10) * 4 + (l2 % 10)


def test_host_falls_back_to_dense_on_any_difference():
    """A block whose matrix differs from the compiled one in one entry by one
    ulp keeps the dense path in that direction only."""
    t = ptd.BasisTables(CFG3)
    base = ptd.e3TensorDecomp(t.req_output_irreps, t.out_js_list, torch.float32, device_torch="cpu")
    b = next(i for i, (l1, l2) in enumerate(base.out_js_list) if (l1, l2) == (1, 1))
    w = base.wms_H[b].clone().reshape(-1)
    k = int(torch.nonzero(w)[0])
    w[k] = float(np.nextafter(np.float32(w[k]), np.float32(np.inf)))
    base.wms_H[b] = w.reshape(base.wms_H[b].shape)
    progs = cg_block_tables(base)["programs"]
    assert progs[0, b] == -1
    assert progs[1, b] >= 0 and progs[2, b] >= 0
    assert (np.delete(progs[0], b) >= 0).all()


def test_program_query_rejects_bad_arguments():
    lib = _lib.load()
    buf = np.empty(49 * 49, np.float32)
    ptr = buf.ctypes.data_as(ctypes.c_void_p).value
    assert lib.maloq_basis_cg_block(48, ptr, 1) != 0
    assert lib.maloq_basis_cg_block(-1, ptr, 1) != 0
    assert lib.maloq_basis_cg_block(5, ptr, 3) != 0      # (1, 1) is 9 x 9
    assert lib.maloq_basis_cg_block(5, None, 9) != 0
