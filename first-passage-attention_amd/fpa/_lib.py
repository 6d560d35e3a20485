"""ctypes binding of libfpa.so (the C ABI declared in include/fpa.h).

The library is built in-tree by ``first-passage-attention_amd/build.py`` and lives
next to this file.  Loading it never compiles anything; a missing or stale
library raises, so ``impl="hip"`` can never run on anything but the HIP kernels.
"""
import ctypes
import os
import struct
import warnings

import torch

from ._srchash import source_hash

ABI_VERSION = 5
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libfpa.so")

FPA_F16, FPA_F32 = 0, 1
FPA_OK, FPA_ERR_INVALID, FPA_ERR_UNSUPPORTED, FPA_ERR_HIP = 0, 1, 2, 3
FPA_FWD_STATS, FPA_FWD_MAIN, FPA_FWD_MERGE = 1, 2, 4
FPA_BWD_DELTA, FPA_BWD_KEYS, FPA_BWD_QUERIES, FPA_BWD_PHI, FPA_BWD_BETA = 1, 2, 4, 8, 16
NOALLOC_SCRATCH_BYTES = 64 << 20  # FPA_NOALLOC_SCRATCH_BYTES of include/fpa.h

_i64 = ctypes.c_int64
_vp = ctypes.c_void_p
_S4 = _i64 * 4
_S3 = _i64 * 3


class FpaFwdArgs(ctypes.Structure):
    _fields_ = [("B", _i64), ("H", _i64), ("T", _i64), ("D", _i64),
                ("dtype", ctypes.c_int32), ("tau", ctypes.c_float),
                ("q", _vp), ("sq", _S4), ("k", _vp), ("sk", _S4), ("v", _vp), ("sv", _S4),
                ("phi", _vp), ("sphi", _S3), ("psi", _vp), ("spsi", _S3),
                ("beta", _vp), ("o", _vp), ("so", _S4), ("lse", _vp), ("state", _vp),
                ("phases", ctypes.c_int32), ("workspace", _vp)]


class FpaBwdArgs(ctypes.Structure):
    _fields_ = [("B", _i64), ("H", _i64), ("T", _i64), ("D", _i64),
                ("dtype", ctypes.c_int32), ("tau", ctypes.c_float),
                ("q", _vp), ("sq", _S4), ("k", _vp), ("sk", _S4), ("v", _vp), ("sv", _S4),
                ("beta", _vp), ("o", _vp), ("so", _S4), ("dout", _vp), ("sdo", _S4),
                ("lse", _vp), ("state", _vp),
                ("dq", _vp), ("sdq", _S4), ("dk", _vp), ("sdk", _S4), ("dv", _vp), ("sdv", _S4),
                ("dphi", _vp), ("dpsi", _vp), ("dbeta", _vp), ("workspace", _vp),
                ("phases", ctypes.c_int32)]


# Byte images of the two argument structs, field after field as include/fpa.h lays them out (64-bit
# host: 8-byte pointers and int64, 4-byte int32 and float, the struct padded to 8 bytes): one pack call
# fills a struct instead of one ctypes assignment per field.
FWD_PACK = struct.Struct("=qqqqif" + "q4q" * 3 + "q3q" * 2 + "q" + "q4q" + "qq" + "i4x" + "q")
BWD_PACK = struct.Struct("=qqqqif" + "q4q" * 3 + "q" + "q4q" * 2 + "qq" + "q4q" * 3 + "qqqq" + "i4x")
assert FWD_PACK.size == ctypes.sizeof(FpaFwdArgs) and BWD_PACK.size == ctypes.sizeof(FpaBwdArgs)

_S2 = _i64 * 2


class FpaFieldFwdArgs(ctypes.Structure):
    _fields_ = [("B", _i64), ("T", _i64), ("C", _i64), ("H", _i64), ("dtype", ctypes.c_int32),
                ("x", _vp), ("sx", _S2), ("weight", _vp), ("bias", _vp), ("phi", _vp), ("psi", _vp),
                ("workspace", _vp)]


class FpaFieldBwdArgs(ctypes.Structure):
    _fields_ = [("B", _i64), ("T", _i64), ("C", _i64), ("H", _i64), ("dtype", ctypes.c_int32),
                ("x", _vp), ("sx", _S2), ("weight", _vp), ("dphi", _vp), ("dpsi", _vp),
                ("dx", _vp), ("sdx", _S2), ("dweight", _vp), ("dbias", _vp), ("workspace", _vp)]


class FpaError(RuntimeError):
    """A failed libfpa call (status code and message of fpa_last_error)."""

    def __init__(self, code, msg):
        super().__init__(msg)
        self.code = code


_LIB = None


def lib():
    """The loaded library; raises if it is not built or has the wrong ABI."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"libfpa.so is not built ({LIB_PATH}); run first-passage-attention_amd/build.py "
                           "or __graft_entry__.build()")
    L = ctypes.CDLL(LIB_PATH)
    L.fpa_abi_version.restype = ctypes.c_int
    L.fpa_last_error.restype = ctypes.c_char_p
    for name in ("fpa_state_floats", "fpa_lse_floats"):
        getattr(L, name).restype = _i64
        getattr(L, name).argtypes = [_i64, _i64, _i64]
    for name in ("fpa_fwd_workspace_bytes", "fpa_bwd_workspace_bytes"):
        getattr(L, name).restype = _i64
        getattr(L, name).argtypes = [_i64, _i64, _i64, _i64, ctypes.c_int32]
    L.fpa_fwd.restype = ctypes.c_int
    L.fpa_fwd.argtypes = [ctypes.POINTER(FpaFwdArgs), _vp]
    L.fpa_bwd.restype = ctypes.c_int
    L.fpa_bwd.argtypes = [ctypes.POINTER(FpaBwdArgs), _vp]
    L.fpa_bwd_noalloc.restype = ctypes.c_int
    L.fpa_bwd_noalloc.argtypes = [ctypes.POINTER(FpaBwdArgs), _vp]
    L.fpa_field_workspace_bytes.restype = _i64
    L.fpa_field_workspace_bytes.argtypes = [_i64, _i64, _i64, _i64]
    L.fpa_field_fwd.restype = ctypes.c_int
    L.fpa_field_fwd.argtypes = [ctypes.POINTER(FpaFieldFwdArgs), _vp]
    L.fpa_field_bwd.restype = ctypes.c_int
    L.fpa_field_bwd.argtypes = [ctypes.POINTER(FpaFieldBwdArgs), _vp]
    if L.fpa_abi_version() != ABI_VERSION:
        raise RuntimeError(f"libfpa.so ABI {L.fpa_abi_version()} != {ABI_VERSION}: rebuild it")
    L.fpa_source_hash.restype = ctypes.c_char_p
    built, here = L.fpa_source_hash().decode(), source_hash()
    if here is not None and built != here:
        tuned = built.startswith(here + "+")  # these sources, built with extra FPA_HIPCC_FLAGS
        if not (tuned and os.environ.get("FPA_ALLOW_TUNING_BUILD") == "1"):
            why = ("was built with extra FPA_HIPCC_FLAGS (a tuning build; set FPA_ALLOW_TUNING_BUILD=1 to use it)"
                   if tuned else f"was built from other sources (hash {built}, sources {here})")
            raise RuntimeError(f"libfpa.so {why}: rebuild it with first-passage-attention_amd/build.py")
        warnings.warn(f"libfpa.so is a tuning build ({built}): FPA_HIPCC_FLAGS were set when it was built")
    _LIB = L
    return L


def check(rc):
    if rc != FPA_OK:
        msg = lib().fpa_last_error().decode()
        if rc == FPA_ERR_INVALID:
            raise ValueError(msg)
        raise FpaError(rc, msg)


def dtype_code(dt):
    if dt == torch.float16:
        return FPA_F16
    if dt == torch.float32:
        return FPA_F32
    raise ValueError("q, k and v must all be fp16 or all fp32")


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(device):
    """torch's current stream on `device`, as the C ABI's stream argument."""
    if _raw_stream is not None:
        idx = device.index if device.index is not None else torch.cuda.current_device()
        return ctypes.c_void_p(_raw_stream(idx))
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def ptr(t):
    """Device address of t for a pointer field of an argument struct (an int: ctypes converts it)."""
    return t.data_ptr()
