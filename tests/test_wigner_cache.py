"""The packed J-table cache of the Wigner entry points (host logic, no GPU):
the same tensor objects are served without a host copy, an in-place edit is
seen, and equal content from other objects reuses the packed tables."""
import torch

from maloq_amd import wigner
from maloq_amd.so3 import jd_matrices


def _js(lmax):
    return [torch.tensor(j, dtype=torch.float32) for j in jd_matrices(lmax)]


def test_same_tensors_hit_identity_path():
    js = _js(2)
    a = wigner._packed_jd(js, 2, "cpu")
    b = wigner._packed_jd(js, 2, "cpu")
    assert a is b
    key = ("ident", 2, "cpu", tuple((id(j), j._version) for j in js))
    assert key in wigner._JD_IDENT


def test_in_place_edit_is_seen():
    js = _js(2)
    a = wigner._packed_jd(js, 2, "cpu").clone()
    with torch.no_grad():
        js[1].mul_(2.0)  # bumps the version counter
    b = wigner._packed_jd(js, 2, "cpu")
    assert not torch.equal(a, b)


def test_equal_content_reuses_tables():
    a = wigner._packed_jd(_js(3), 3, "cpu")
    b = wigner._packed_jd(_js(3), 3, "cpu")  # other objects, same values
    assert a is b
