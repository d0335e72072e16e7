"""ctypes binding of libmaloq_hip.so (the C ABI declared in include/maloq_hip.h).

The product path has no fallback: if the library is missing or cannot be
loaded, every op raises.  torch is imported first so that the library binds to
the HIP runtime torch already loaded (same SONAME), which makes torch's device
pointers and streams valid arguments.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (load torch's HIP runtime before ours)

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmaloq_hip.so")

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_u64 = ctypes.c_uint64

# name -> argtypes (every symbol declared in include/maloq_hip.h)
SIGNATURES = {
    "maloq_abi_version": [],
    "maloq_last_error": [],
    "maloq_edge_euler": [_p, _i64, _u64, _p, _p],
    "maloq_edge_vec_to_wigner": [_p, _i64, _u64, _i32, _p, _p, _p, _p, _i32, _p],
    "maloq_wigner_from_euler": [_p, _i64, _i32, _p, _p, _p, _i32, _p],
    "maloq_rotate": [_i32, _i32, _i32, _p, _i32, _p, _i64, _p, _p, _p, _i32, _p, _p],
    "maloq_label_transform": [_p, _p, _p, _p, _i64, _i32, _i32, _p, _p, _p, _i32, _i32, _p],
    "maloq_basis_cg_block": [_i32, _p, _i32],
    "maloq_irreps_gate_fwd": [_p, _i64, _i32, _i32, _p, ctypes.c_float, _i32, _p, _p],
    "maloq_irreps_gate_bwd": [_p, _i64, _i32, _i32, _p, ctypes.c_float, _i32, _p, _p, _p, _p],
    "maloq_gather_columns": [_p, _i64, _i64, _p, _p, _i32, _p, _i64, _p],
    "maloq_scatter_columns": [_p, _i64, _i64, _p, _p, _p, _i32, _p, _i64, _p],
    "maloq_basis_row_meta": [_i64, _p, _p, _p, _p, _p, _i64, _p, _i32, _p, _p],
    "maloq_fock_to_irreps": [_p, _i64, _p, _i64, _p, _i32, _p, _p, _p, _i32, _i32, _p, _p, _p, _i32, _i32, _p],
    "maloq_irreps_to_fock": [_p, _p, _p, _i64, _p, _i64, _p, _i32, _p, _i32, _i32, _p, _p, _p, _i32, _i32, _p],
    "maloq_fock_to_irreps_pairs": [_p, _i64, _p, _p, _p, _p, _p, _i64, _p, _p, _i32, _p, _p, _p, _i32, _i32, _p,
                                   _p, _p, _i32, _i32, _p],
    "maloq_irreps_to_fock_pairs": [_p, _p, _p, _i64, _p, _p, _p, _p, _p, _i64, _p, _p, _i32, _p, _i32, _i32, _p,
                                   _p, _p, _i32, _i32, _p],
    "maloq_matrix2label": [_p, _i64, _p, _p, _p, _p, _p, _i64, _p, _p, _p, _i64, _i32, _p],
    "maloq_segment_sum": [_p, _p, _p, _i64, _i64, _p, _p],
    "maloq_label_scalar_shift": [_p, _i64, _i64, _p, _p, _p, _i32, ctypes.c_float, _p],
    "maloq_label_mask": [_p, _p, _p, _p, _p, _i32, _i64, _p, _p],
    "maloq_signed_permute": [_p, _i64, _i64, _p, _p, _p, _i64, _p],
    "maloq_blocks_to_csr": [_p, _p, _p, _p, _p, _p, _p, _i64, _p, _p, _p],
    "maloq_message_partials_floats": [_i32, _i32, _i64, _i32],
    "maloq_message_wpack_bytes": [_i32, _i32, _i32, _i32, _i32, _i32],
    "maloq_message_kept_rows": [_i32, _i32],
    "maloq_message_wigner_floats": [_i32, _i32],
    "maloq_message_fwd": [_i32, _i32, _i32, _i32, _p, _i32, _p, _p, _i64, _p, _p, _p, _p, _p, _p,
                          _i64, _i32, _p, _p, _p, _p, _p, _p, _p],
    "maloq_message_edgewise_fwd": [_i32, _i32, _i32, _p, _i32, _p, _p, _p, _i64, _p, _p, _p, _p, _i32, _p, _p,
                                   _p, _p, _i64, _i32, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p],
    "maloq_message_edgewise_bwd_dx": [_i32, _i32, _i32, _p, _i32, _p, _p, _p, _p, _i64, _p, _p, _p, _p, _p, _p,
                                      _i32, _p, _p, _p, _p, _i64, _p, _p, _p, _p, _p, _p, _p, _p],
    "maloq_message_bwd_dx": [_i32, _i32, _i32, _i32, _p, _i32, _p, _p, _p, _i64, _p, _p, _p, _p, _p,
                             _p, _p, _i64, _i32, _p, _p, _p, _p, _p, _p],
    "maloq_message_edge_rows": [_i64],
    "maloq_message_dw_partials_floats": [_i32, _i32, _i32, _i32, _i32, _i32],
    "maloq_message_dw": [_i32, _i32, _i32, _i32, _p, _p, _i64, _i32, _i32, _i32, _p, _p, _p, _p],
    "maloq_message_supported": [_i32, _i32],
    "maloq_message_fwd_noalloc": [_i32, _i32, _i32, _i32, _p, _i32, _p, _p, _i64, _p, _p, _p, _p, _p, _p, _i64,
                                  _i32, _p, _p],
    "maloq_message_wigner_rows": [_i32, _i32, _p, _p, _i64, _p, _p],
    "maloq_message_pack": [_i32, _i32, _p, _p, _p, _i64, _p, _p],
    "maloq_message_colsum_partials_floats": [_i32, _i32, _i64],
    "maloq_message_colsum": [_i32, _p, _i32, _i32, _i32, _i32, _i64, _p, _p, _p],
    "maloq_edge_m0_rows": [_i32, _i64, _p, _p, _p, _p, _p],
    "maloq_edge_degree_embed": [_i32, _i32, _i32, _p, _i64, _i32, _p, _p, _p, _i64, ctypes.c_float, _p, _p, _p],
    "maloq_edge_degree_embed_bwd": [_i32, _i32, _p, _p, _i64, _i32, _p, ctypes.c_float, _p, _p],
    "maloq_radial_pack_bytes": [_i32, _i32, _i32],
    "maloq_radial_fwd": [_i32, _i32, _p, _p, _i64, _p, _p, _p, _p, ctypes.c_float, _p, _p, _p, _p, _p, _p],
    "maloq_radial_bwd_partials_floats": [_i32, _i32, _p, _i64],
    "maloq_radial_bwd": [_i32, _i32, _p, _p, _i64, _p, _p, _p, _p, ctypes.c_float, _p, _p, _p, _p,
                         _p, _p, _p, _p, _p],
}
RESTYPES = {
    "maloq_last_error": ctypes.c_char_p,
    "maloq_message_partials_floats": ctypes.c_int64,
    "maloq_message_wpack_bytes": ctypes.c_int64,
    "maloq_message_dw_partials_floats": ctypes.c_int64,
    "maloq_message_edge_rows": ctypes.c_int64,
    "maloq_message_colsum_partials_floats": ctypes.c_int64,
    "maloq_radial_pack_bytes": ctypes.c_int64,
    "maloq_radial_bwd_partials_floats": ctypes.c_int64,
}

_lib = None


class MaloqHipError(RuntimeError):
    pass


def load():
    """Load (once) and return the ctypes library; raise if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise MaloqHipError(
            f"{LIB_PATH} is missing: build it with `python -m maloq_amd.build` "
            "(there is no CPU fallback for the HIP path)"
        )
    lib = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_GLOBAL)
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = RESTYPES.get(name, ctypes.c_int)
    _lib = lib
    return lib


def call(name: str, *args) -> None:
    """Call entry point ``name``; a tensor argument is passed as its device
    pointer and, being held by ``args``, stays allocated until the call has
    enqueued its kernels."""
    lib = load()
    rc = getattr(lib, name)(*(a.data_ptr() if isinstance(a, torch.Tensor) else a for a in args))
    if rc != 0:
        msg = lib.maloq_last_error().decode(errors="replace")
        raise MaloqHipError(f"{name} failed ({rc}): {msg}")


def ptr(t) -> int | None:
    """Device pointer of a tensor (None for None).  The caller must keep the
    tensor referenced until the kernels reading it are enqueued: the pointer of
    a temporary is released to the caching allocator as soon as this returns,
    and the next allocation of that size receives the same block."""
    if t is None:
        return None
    return t.data_ptr()


def stream_of(device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def require_cuda(*tensors):
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError("maloq_amd HIP ops need tensors on a ROCm GPU device")
