"""The C++ operator layer (_maloq_torch.so, csrc/torch_ops.cpp), on the CPU:
the operators are defined by the extension with a GPU kernel each, the
committed J table is what its generator writes and equals the packing the
Python path uploads, and the weight-packing index the extension builds equals
the Python one for every mode, dtype and gate setting."""
import numpy as np
import pytest
import torch

from maloq_amd import message as M
from maloq_amd import ops
from maloq_amd.csrc import gen_jd_table
from maloq_amd.so3 import jd_matrices, pack_jd

OPS = ("edge_euler", "wigner_from_euler", "edge_vec_to_wigner", "edge_vec_to_wigner_out", "rotate", "segment_sum", "label_transform", "message_block_fwd",
       "message_block_bwd", "edgewise_fwd", "edgewise_bwd", "basis_row_meta", "fock_to_irreps", "irreps_to_fock",
       "radial_fwd", "radial_bwd", "edge_m0_rows", "edge_degree_embed", "edge_degree_embed_", "edge_degree_embed_bwd")


def test_operators_come_from_the_extension():
    maps = open("/proc/self/maps").read()
    assert "_maloq_torch.so" in maps and "libmaloq_hip.so" in maps
    for name in OPS:
        op = getattr(torch.ops.maloq_hip, name).default
        assert torch._C._dispatch_has_kernel_for_dispatch_key(op.name(), "CUDA"), name
        assert not torch._C._dispatch_has_kernel_for_dispatch_key(op.name(), "CPU"), name
        assert getattr(ops, name) is getattr(torch.ops.maloq_hip, name)


def test_cpu_tensors_are_refused():
    with pytest.raises(NotImplementedError):
        torch.ops.maloq_hip.edge_euler(torch.zeros(4, 3), 0)


def test_jd_header_is_current():
    with open(gen_jd_table.HEADER) as f:
        assert f.read() == gen_jd_table.render(), "regenerate: python -m maloq_amd.csrc.gen_jd_table"


def test_jd_table_is_every_lmax_prefix():
    t = torch.ops.maloq_hip._jd_table().numpy()
    assert np.array_equal(t.view(np.uint32), pack_jd(jd_matrices(8), 8).view(np.uint32))
    for lmax in range(8):
        p = pack_jd(jd_matrices(lmax), lmax)
        assert np.array_equal(t[:p.size].view(np.uint32), p.view(np.uint32)), lmax


@pytest.mark.parametrize("code", [0, 1])
@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("lmax,mmax,gate,c_in,c_out", [(2, 2, False, 32, 32), (4, 2, True, 64, 32),
                                                       (4, 4, False, 32, 64), (6, 2, True, 32, 32)])
def test_pack_index_matches_python(code, mode, lmax, mmax, gate, c_in, c_out):
    want, total = M._pack_index(code, lmax, mmax, gate, c_in, c_out, mode)
    got = torch.ops.maloq_hip._pack_index(code, lmax, mmax, gate, c_in, c_out, mode).numpy()
    assert got.shape == want.shape and np.array_equal(got, want)
    assert got.min() >= 0 and got.max() < total
