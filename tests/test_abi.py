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


def test_library_binds_its_own_functions():
    """The library is linked with -Bsymbolic: its calls to its own C++
    functions (the per-shape launch templates, kernel stubs) are bound inside
    it, with no PLT slot a second build loaded into the same process could
    take over."""
    import shutil
    import subprocess
    readelf = shutil.which("readelf")
    if readelf is None:
        pytest.skip("readelf is not installed")
    dyn = subprocess.run([readelf, "-dW", LIB], capture_output=True, text=True, check=True).stdout
    assert "SYMBOLIC" in dyn
    rel = subprocess.run([readelf, "-rW", LIB], capture_output=True, text=True, check=True).stdout
    own = [ln for ln in rel.splitlines() if "JUMP_SLOT" in ln and "_ZN5maloq" in ln]
    assert not own, own[:3]


def test_second_build_in_one_process_runs_its_own_templates(tmp_path):
    """Why the library binds its own functions.  Two builds that explicitly
    instantiate the same launch template with different tile sizes, both loaded
    with RTLD_GLOBAL as maloq_amd/_lib.py loads the library: without
    -Bsymbolic the second build's entry point runs the first build's template
    (it would size the grid for one tile and launch the other's kernel); with
    it, its own."""
    import shutil
    import subprocess
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ is not installed")
    (tmp_path / "t.h").write_text("template <int MODE> int launch(int e);\nextern template int launch<0>(int);\n")
    for te in (64, 32):
        (tmp_path / f"i{te}.cpp").write_text(
            '#include "t.h"\ntemplate <int MODE> int launch(int e) { return (e + %d - 1) / %d * 1000 + %d; }\n'
            "template int launch<0>(int);\n" % (te, te, te))
        (tmp_path / f"e{te}.cpp").write_text('#include "t.h"\nextern "C" int entry(int e) { return launch<0>(e); }\n')

    def build(te, name, flags):
        out = str(tmp_path / name)
        subprocess.run([gxx, "-O2", "-fPIC", "-shared", *flags, str(tmp_path / f"i{te}.cpp"),
                        str(tmp_path / f"e{te}.cpp"), "-o", out], check=True)
        return ctypes.CDLL(out, mode=ctypes.RTLD_GLOBAL)

    first = build(64, "first.so", [])
    plain = build(32, "plain.so", [])
    symbolic = build(32, "symbolic.so", ["-Wl,-Bsymbolic"])
    assert first.entry(100) == 2064        # 2 tiles of 64 edges
    assert plain.entry(100) == 2064        # the 32-edge build ran the 64-edge template
    assert symbolic.entry(100) == 4032     # 4 tiles of 32 edges: its own
