"""ctypes binding of the HIP library (include/jeff_mlora.h). The structs below mirror the header field for field.

There is no fallback: if jeff_amd/libjeff_mlora.so is missing, every product raises LibraryMissing."""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIBRARY = Path(__file__).resolve().with_name("libjeff_mlora.so")
ABI_VERSION = 2
MAX_MATS = 8
MAX_REQUESTS = 8192
MAX_POOL_ROWS = 262144
READOUT_MAX_DIM = 2048
READOUT_MAX_OPTIONS = 256
EPILOGUE_MAX_N = 8192
NOALLOC_SCRATCH_BYTES = 64 << 20

OK, EINVAL, EALIGN, EOVERFLOW, EWORKSPACE, EUNSUPPORTED, ELAUNCH = 0, -1, -2, -3, -4, -5, -6
ERRORS = {EINVAL: "invalid argument (a null pointer, a bad size or shape)",
          EALIGN: "a pointer, stride or offset is not 16-byte aligned",
          EOVERFLOW: "sizes beyond the kernels' index range",
          EWORKSPACE: "the workspace is too small",
          EUNSUPPORTED: "a shape this build does not run",
          ELAUNCH: "the HIP kernel launch failed"}

ROUTE_BAD_ADAPTER = 1
ROUTE_BAD_SEQLENS = 2
FORCE_BASE_GEMV, FORCE_BASE_MFMA, FORCE_SHRINK_SEGMENT, FORCE_SHRINK_MFMA, FORCE_BASE_SPLIT = 1, 2, 4, 8, 16
FORCE_BASE_NARROW = 32
EPILOGUE_SILU_MUL = 64
EPILOGUE_RESIDUAL = 128


def force_ranges(s: int) -> int:
    """MLORA_FORCE_RANGES(s): a narrow product over s input ranges."""
    return s << 8


EXPORTS = ("mlora_abi_version", "mlora_capture_id", "mlora_workspace_bytes", "mlora_int4_partials_bytes",
           "mlora_int4_partials_bound", "mlora_route", "mlora_dequant", "mlora_int4_plan", "mlora_shrink", "mlora_int4_linear",
           "mlora_int4_linear_noalloc", "mlora_int4_base_expand", "mlora_lora_add", "mlora_readout_logits",
           "mlora_option_softmax", "mlora_add_rms", "mlora_silu_mul")

c_i32, c_i64, c_vp = ctypes.c_int32, ctypes.c_int64, ctypes.c_void_p


class Int4(ctypes.Structure):
    _fields_ = [("words", c_vp), ("scales", c_vp), ("zeros", c_vp),
                ("k", c_i32), ("columns", c_i32), ("out", c_i32), ("group", c_i32)]


class Lora(ctypes.Structure):
    _fields_ = [("pool", c_vp), ("ranks", c_vp), ("pool_stride", c_i64), ("off_a", c_i64),
                ("off_b", c_i64 * MAX_MATS), ("ranks_stride", c_i32), ("pool_rows", c_i32), ("n_mats", c_i32),
                ("rank_cap", c_i32), ("cap", c_i32 * MAX_MATS), ("cols", c_i32 * MAX_MATS)]


class Route(ctypes.Structure):
    _fields_ = [("req_order", c_vp), ("tok_perm", c_vp), ("last_of", c_vp), ("seg_of", c_vp),
                ("seg_start", c_vp),
                ("seg_adapter", c_vp), ("num_segs", c_vp), ("status", c_vp), ("tokens", c_i64),
                ("requests", c_i32), ("max_segs", c_i32)]


class LibraryMissing(RuntimeError):
    pass


class HipError(RuntimeError):
    pass


_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """The loaded library, with every signature declared. LibraryMissing when it has not been built."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIBRARY.is_file():
            raise LibraryMissing(f"{LIBRARY} is not built (python -m jeff_amd.build); the multi-LoRA INT4 linear has "
                                 "no CPU or PyTorch fallback")
        h = ctypes.CDLL(str(LIBRARY))
        P = ctypes.POINTER
        h.mlora_abi_version.restype = c_i32
        h.mlora_abi_version.argtypes = []
        h.mlora_capture_id.restype = c_i32
        h.mlora_capture_id.argtypes = [c_vp, P(ctypes.c_uint64)]
        h.mlora_workspace_bytes.restype = ctypes.c_size_t
        h.mlora_workspace_bytes.argtypes = [c_i64, c_i32]
        h.mlora_route.restype = c_i32
        h.mlora_route.argtypes = [c_vp, c_vp, c_i32, P(Route), c_i32, c_vp]
        h.mlora_int4_plan.restype = c_i32
        h.mlora_int4_plan.argtypes = [c_i32, c_i32, c_i32, c_i64, c_i32, c_i32, c_i32, c_i32, P(c_i32), P(c_i32),
                                      P(c_i32)]
        h.mlora_dequant.restype = c_i32
        h.mlora_dequant.argtypes = [P(Int4), c_vp, c_vp]
        h.mlora_shrink.restype = c_i32
        h.mlora_shrink.argtypes = [P(Lora), P(Route), c_vp, c_i64, c_i32, c_vp, c_i32, c_vp]
        h.mlora_int4_linear.restype = c_i32
        h.mlora_int4_linear.argtypes = [P(Int4), P(Lora), P(Route), c_vp, c_i64, c_vp, c_i64, c_vp, c_vp,
                                        ctypes.c_size_t, c_vp, ctypes.c_size_t, c_i32, c_vp]
        h.mlora_int4_linear_noalloc.restype = c_i32
        h.mlora_int4_linear_noalloc.argtypes = [P(Int4), P(Lora), P(Route), c_vp, c_i64, c_vp, c_i64, c_vp, c_i32,
                                                c_vp]
        h.mlora_int4_base_expand.restype = c_i32
        h.mlora_int4_base_expand.argtypes = [P(Int4), P(Lora), P(Route), c_vp, c_i64, c_vp, c_i64, c_vp, c_vp, c_vp,
                                             ctypes.c_size_t, c_i32, c_vp]
        h.mlora_readout_logits.restype = c_i32
        h.mlora_readout_logits.argtypes = [c_vp, c_i64, c_i32, c_vp, c_i64, c_i32, c_i32, c_vp, c_i32, c_vp, c_vp]
        h.mlora_option_softmax.restype = c_i32
        h.mlora_option_softmax.argtypes = [c_vp, c_i32, c_vp, c_vp, c_vp, c_i32, c_i32, c_vp, c_vp]
        h.mlora_add_rms.restype = c_i32
        h.mlora_add_rms.argtypes = [c_vp, c_i64, c_vp, c_i64, c_vp, c_vp, c_i64, c_vp, c_i64, c_i64, c_i32,
                                    ctypes.c_float, c_vp]
        h.mlora_silu_mul.restype = c_i32
        h.mlora_silu_mul.argtypes = [c_vp, c_i64, c_vp, c_i64, c_i64, c_i32, c_vp]
        h.mlora_int4_partials_bytes.restype = ctypes.c_size_t
        h.mlora_int4_partials_bytes.argtypes = [P(Int4), P(Lora), P(Route), c_i32]
        h.mlora_int4_partials_bound.restype = ctypes.c_size_t
        h.mlora_int4_partials_bound.argtypes = [c_i32, c_i32, c_i32, c_i64]
        h.mlora_lora_add.restype = c_i32
        h.mlora_lora_add.argtypes = [P(Lora), P(Route), c_vp, c_i64, c_i32, c_vp, c_i64, c_i32, c_vp,
                                     ctypes.c_size_t, c_i32, c_vp]
        version = h.mlora_abi_version()
        if version != ABI_VERSION:
            raise LibraryMissing(f"{LIBRARY} has ABI version {version}; this package needs {ABI_VERSION} (rebuild)")
        _lib = h
        return h


def capture_id(stream: int) -> int:
    """HIP's capture sequence id of `stream` (a hipStream_t as an int) while it captures a graph, else 0."""
    cid = ctypes.c_uint64(0)
    check(lib().mlora_capture_id(stream, ctypes.byref(cid)), "mlora_capture_id")
    return int(cid.value)


def check(rc: int, what: str) -> None:
    if rc != OK:
        raise HipError(f"{what}: {ERRORS.get(rc, f'status {rc}')}")
