"""The C-ABI library loads and exports every symbol include/maloq_hip.h declares
(no compute calls: runs without a GPU)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "maloq_amd", "libmaloq_hip.so")


def declared_symbols():
    txt = open(os.path.join(ROOT, "include", "maloq_hip.h")).read()
    return re.findall(r"^(?:int|int64_t|const char\*)\s+(maloq_\w+)\(", txt, re.M)


def test_header_declares_symbols():
    assert len(declared_symbols()) >= 10


def test_library_exports_every_declared_symbol():
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} not built; run python -m maloq_amd.build")
    import torch  # noqa: F401  (bind to torch's HIP runtime first)
    lib = ctypes.CDLL(LIB)
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing
    lib.maloq_abi_version.restype = ctypes.c_int
    assert lib.maloq_abi_version() == 3


def test_ctypes_signatures_cover_header():
    from maloq_amd import _lib
    assert sorted(_lib.SIGNATURES) == sorted(declared_symbols())


def test_error_path_without_gpu():
    """Argument validation happens on the host before any launch."""
    from maloq_amd import _lib
    with pytest.raises(_lib.MaloqHipError, match="lmax must be 0-8"):
        _lib.call("maloq_wigner_from_euler", None, 0, 9, None, None, None, 1, None)


def test_supported_shapes_and_rotate_validation_without_gpu():
    """Shape queries and the rotation's argument checks run on the host."""
    from maloq_amd import _lib
    lib = _lib.load()
    built = {(l, m) for l in range(9) for m in range(l + 1) if lib.maloq_message_supported(l, m)}
    assert built == {(2, 2), (4, 2), (4, 4), (6, 2), (6, 6)}
    with pytest.raises(_lib.MaloqHipError, match="lmax must be 0-8"):
        _lib.call("maloq_rotate", 0, 0, 9, None, 4, None, 1, None, None, None, 0, None, None)
    with pytest.raises(_lib.MaloqHipError, match="multiple of 4"):
        _lib.call("maloq_rotate", 0, 0, 2, None, 6, None, 1, None, None, None, 0, None, None)
    with pytest.raises(_lib.MaloqHipError, match="no message kernels"):
        _lib.call("maloq_message_wigner_rows", 4, 3, None, None, 1, None, None)


def test_label_width_limit_without_gpu():
    """A 32-row fp32 tile of the widest column group and its 40-byte row
    descriptors must fit one CU's 160 KB of LDS: 1269 columns is the widest
    group accepted.  Wider rows are split into groups (any width, 0 rows launch
    nothing); a column permutation needs one group (checked on the host)."""
    import numpy as np
    from maloq_amd import _lib
    blocks = np.array([[1, 0, 0, 0]], dtype=np.int32)
    sched = np.array([1, 0, 1, 0, 5, 0, 1, 1, 1, 1, 0], dtype=np.int32)
    bp, sp = blocks.ctypes.data, sched.ctypes.data
    _lib.call("maloq_label_transform", None, None, None, None, 0, 1269, 1, bp, None, sp, 1, 1269, None)
    with pytest.raises(_lib.MaloqHipError, match="column group of 1270 columns too wide"):
        _lib.call("maloq_label_transform", None, None, None, None, 0, 1270, 1, bp, None, sp, 1, 1270, None)
    # 4096 columns as 21 groups of at most 204 (400 blocks)
    _lib.call("maloq_label_transform", None, None, None, None, 0, 4096, 400, bp, None, sp, 21, 204, None)
    with pytest.raises(_lib.MaloqHipError, match="does not fit the row width"):
        _lib.call("maloq_label_transform", None, None, None, None, 0, 4096, 400, bp, None, sp, 1, 204, None)
    with pytest.raises(_lib.MaloqHipError, match="needs rows of one column group"):
        _lib.call("maloq_label_transform", None, sp, None, None, 0, 4096, 400, bp, None, sp, 21, 204, None)
    with pytest.raises(_lib.MaloqHipError, match="column groups 401 outside"):
        _lib.call("maloq_label_transform", None, None, None, None, 0, 4096, 400, bp, None, sp, 401, 204, None)
