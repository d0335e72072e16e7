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
    assert lib.maloq_abi_version() == 1


def test_ctypes_signatures_cover_header():
    from maloq_amd import _lib
    assert sorted(_lib.SIGNATURES) == sorted(declared_symbols())


def test_error_path_without_gpu():
    """Argument validation happens on the host before any launch."""
    from maloq_amd import _lib
    with pytest.raises(_lib.MaloqHipError, match="lmax must be 0-8"):
        _lib.call("maloq_wigner_from_euler", None, 0, 9, None, None, None, 1, None)
