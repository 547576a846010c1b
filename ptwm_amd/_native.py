"""ctypes binding of libptwm_mi355x.so (declarations: include/ptwm_mi355x.h).

The library is built in-tree by ``ptwm_amd.build``.  Loading fails loudly
when it is missing: there is no CPU fallback for any entry point.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libptwm_mi355x.so")

# negative return codes (crates/ptwm-core/src/flavor/native.rs:634-657)
RC_INVALID_INPUT = -1
RC_BUFFER_TOO_SMALL = -2
RC_MISSING_CAPABILITY = -3
RC_MISSING_NATIVE_DEP = -4
RC_UNSUPPORTED = -5

_RC_NAMES = {
    -1: "InvalidInput",
    -2: "BufferTooSmall",
    -3: "MissingCapability",
    -4: "MissingNativeDep",
    -5: "Unsupported",
}

# every symbol the header declares, with its ctypes signature
_u8p = C.c_void_p
_SIGS = {
    "ptwm_plane_codec_v1_encode": (C.c_int64, [_u8p, C.c_size_t, _u8p, C.c_size_t]),
    "ptwm_plane_codec_v1_decode": (C.c_int64, [_u8p, C.c_size_t, _u8p, C.c_size_t]),
    "ptwm_plane_codec_v1_decode_stateful": (
        C.c_int64, [C.c_uint8, _u8p, C.c_size_t, _u8p, C.c_size_t, _u8p, C.c_size_t]),
    "ptwm_plane_codec_v1_cuda_stream_handle": (C.c_uint64, [C.c_uint32]),
    "ptwm_plane_codec_v1_decode_cuda": (
        C.c_int64, [C.c_uint8, _u8p, C.c_size_t, _u8p, C.c_size_t, C.c_uint64, C.c_size_t, C.c_uint64,
                    C.c_size_t, C.c_uint32]),
    "ptwm_plane_codec_v1_encode_cuda": (
        C.c_int64, [C.c_uint8, _u8p, C.c_size_t, _u8p, C.c_size_t, C.c_uint64, C.c_size_t, C.c_uint64,
                    C.c_size_t, C.POINTER(C.c_uint64), C.c_uint32]),
    "ptwm_hardware_backend_v1_cuda_stream_handle": (C.c_uint64, [C.c_uint32]),
    "ptwm_hardware_backend_v1_dispatch_decode_cuda": (
        C.c_int64, [C.c_uint8, _u8p, C.c_size_t, _u8p, C.c_size_t, C.c_uint64, C.c_size_t, C.c_uint64,
                    C.c_size_t, C.c_uint32]),
    "ptwm_mi355x_abi_version": (C.c_uint32, []),
    "ptwm_mi355x_canonical_id": (C.c_int64, [C.c_uint32, _u8p]),
    "ptwm_mi355x_encode_tensor_cuda": (
        C.c_int64, [C.c_uint32, C.c_uint64, C.c_size_t, C.c_uint64, C.c_size_t, _u8p, C.c_size_t,
                    C.POINTER(C.c_size_t), C.POINTER(C.c_uint64), C.c_uint32]),
    "ptwm_mi355x_encode_tensors_cuda": (
        C.c_int64, [C.c_uint32, C.c_uint32, C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint64, C.c_size_t, C.c_void_p,
                    C.c_size_t, C.POINTER(C.c_size_t), C.POINTER(C.c_uint64), C.c_uint32]),
    "ptwm_mi355x_encode_tensor_rans_cuda": (
        C.c_int64, [C.c_uint32, C.c_uint64, C.c_size_t, C.c_uint64, C.c_size_t, _u8p, C.c_size_t,
                    C.POINTER(C.c_size_t), C.POINTER(C.c_uint64), C.c_uint32]),
    "ptwm_mi355x_encode_tensor_ref_cuda": (
        C.c_int64, [C.c_uint32, C.POINTER(C.c_uint16), C.c_uint32, C.c_uint32, C.c_uint64, C.c_size_t, C.c_uint64,
                    C.c_size_t, _u8p, C.c_size_t, C.POINTER(C.c_size_t), C.POINTER(C.c_uint64), C.c_uint32]),
    "ptwm_mi355x_encode_tensor_ref_ops_cuda": (
        C.c_int64, [C.c_uint32, C.POINTER(C.c_uint16), C.POINTER(C.c_uint16), C.c_uint32, C.c_uint32, C.c_uint32,
                    C.c_uint64, C.c_size_t, C.c_uint64, C.c_size_t, _u8p, C.c_size_t, C.POINTER(C.c_size_t),
                    C.POINTER(C.c_uint64), C.POINTER(C.c_uint16), C.c_uint32]),
    "ptwm_mi355x_plane_crc32_cuda": (
        C.c_int64, [C.c_uint32, C.c_uint64, C.c_size_t, C.POINTER(C.c_uint32), C.c_uint32, C.c_uint32]),
    "ptwm_mi355x_xxh64_cuda": (C.c_int64, [C.c_uint64, C.c_size_t, C.POINTER(C.c_uint64), C.c_uint32]),
    "ptwm_mi355x_huffman_code_lengths": (C.c_int64, [_u8p, _u8p]),
    "ptwm_mi355x_stream_wait": (C.c_int64, [C.c_uint64, C.c_uint32]),
    "ptwm_mi355x_use_stream": (C.c_int64, [C.c_uint64, C.c_uint32, C.c_uint32]),
    "ptwm_mi355x_set_encode_batch_bytes": (C.c_int64, [C.c_uint64, C.c_uint32]),
    "ptwm_mi355x_dispatch_decode_noalloc_cuda": (
        C.c_int64, [C.c_uint8, _u8p, C.c_size_t, _u8p, C.c_size_t, C.c_uint64, C.c_size_t, C.c_uint64, C.c_size_t,
                    C.c_uint32]),
    "ptwm_mi355x_container_plan": (
        C.c_int64, [_u8p, C.c_size_t, _u8p, C.c_size_t, C.POINTER(C.c_size_t), C.c_void_p, C.c_size_t,
                    C.POINTER(C.c_size_t), C.POINTER(C.c_uint64)]),
    "ptwm_mi355x_device_init": (C.c_int64, [C.c_uint32]),
    "ptwm_mi355x_container_rewrite": (C.c_int64, [_u8p, C.c_size_t, _u8p, C.c_size_t, C.POINTER(C.c_size_t)]),
    "ptwm_mi355x_container_write": (
        C.c_int64, [_u8p, C.c_size_t, _u8p, C.c_size_t, _u8p, C.c_size_t, C.POINTER(C.c_size_t)]),
    "ptwm_mi355x_alloc_calls": (C.c_uint64, []),
    "ptwm_mi355x_decode_stats": (C.c_int64, [C.c_uint32, C.POINTER(C.c_uint64), C.c_size_t]),
    "ptwm_mi355x_set_profiling": (C.c_int64, [C.c_uint32, C.c_uint32]),
    "ptwm_mi355x_last_kernel_ms": (C.c_int64, [C.c_uint32, C.POINTER(C.c_float)]),
    "ptwm_mi355x_split_cuda": (
        C.c_int64, [C.c_uint32, C.c_uint64, C.c_size_t, C.POINTER(C.c_uint64), C.c_uint32, C.c_uint32]),
    "ptwm_mi355x_merge_cuda": (
        C.c_int64, [C.c_uint32, C.POINTER(C.c_uint64), C.c_uint32, C.c_size_t, C.c_uint64, C.c_size_t,
                    C.c_uint32]),
}


class NativeError(RuntimeError):
    """A negative return code from the native library."""

    def __init__(self, rc: int, what: str):
        super().__init__(f"{what}: {_RC_NAMES.get(rc, 'InternalError')} (rc={rc})")
        self.rc = rc


_lib = None


class ContainerTensor(C.Structure):
    """ptwm_mi355x_container_tensor (include/ptwm_mi355x.h)."""
    _fields_ = [
        ("name_offset", C.c_uint64), ("orig_size", C.c_uint64), ("out_offset", C.c_uint64),
        ("record_offset", C.c_uint64), ("record_len", C.c_uint64), ("name_len", C.c_uint32),
        ("dtype_code", C.c_uint16), ("input_format", C.c_uint8), ("chain", C.c_uint8),
        ("status", C.c_int32), ("plan_index", C.c_int32), ("flags", C.c_uint32), ("reserved", C.c_uint32),
    ]


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m ptwm_amd.build` "
                "(the MI355X path has no CPU fallback)")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def symbol_names() -> list[str]:
    return list(_SIGS)


def check(rc: int, what: str) -> int:
    if rc < 0:
        raise NativeError(rc, what)
    return rc
