"""ctypes binding of libstepquant_hip.so (the C ABI in include/stepquant_hip.h).

The library is built in-tree by ``__graft_entry__.build()`` (hipcc, gfx950).
There is no fallback: if the library is missing every pool operation raises.
"""
from __future__ import annotations

import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("STEPQUANT_HIP_LIB", os.path.join(_HERE, "libstepquant_hip.so"))
ABI_VERSION = 2

F32, BF16, F16, I32, I64 = 0, 1, 2, 3, 4
# sq_pool.flags bits (SQ_POOL_FAST_*)
POOL_FAST_GDN128, POOL_FAST_KDA128 = 1, 2
_DTYPES = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16, torch.int32: I32, torch.int64: I64}

_P = ctypes.c_void_p


class Pool(ctypes.Structure):
    _fields_ = [("data", _P), ("page_bytes", ctypes.c_int64), ("num_slots", ctypes.c_int64),
                ("bits", _P), ("offsets", _P), ("rows", _P), ("columns", _P), ("impact", _P),
                ("head_meta", _P), ("heads", ctypes.c_int32), ("keys", ctypes.c_int32),
                ("values", ctypes.c_int32), ("group", ctypes.c_int32), ("kda", ctypes.c_int32),
                ("storage", ctypes.c_int32), ("max_code_bytes", ctypes.c_int32),
                ("max_row_bytes", ctypes.c_int32), ("flags", ctypes.c_int32), ("reserved", ctypes.c_int32)]


class StepArgs(ctypes.Structure):
    _fields_ = [("q", _P), ("k", _P), ("v", _P), ("g", _P), ("beta", _P), ("a_log", _P),
                ("dt_bias", _P), ("out", _P), ("slots", _P), ("batch", ctypes.c_int64),
                ("q_stride", ctypes.c_int64), ("k_stride", ctypes.c_int64),
                ("v_stride", ctypes.c_int64), ("key_heads", ctypes.c_int32),
                ("qkv_dtype", ctypes.c_int32), ("gate_dtype", ctypes.c_int32),
                ("out_dtype", ctypes.c_int32), ("slots_dtype", ctypes.c_int32),
                ("normalize", ctypes.c_int32), ("scale", ctypes.c_float), ("reserved", ctypes.c_int32)]


class Scratch(ctypes.Structure):
    _fields_ = [("key", _P), ("decay", _P), ("delta", _P), ("stable_slots", _P),
                ("capacity", ctypes.c_int64)]


class PrefillArgs(ctypes.Structure):
    _fields_ = [("q", _P), ("k", _P), ("v", _P), ("g", _P), ("beta", _P), ("a_log", _P), ("dt_bias", _P),
                ("out", _P), ("cu_seqlens", _P), ("checkpoints", _P), ("init_slots", _P), ("slots", _P),
                ("init_state", _P), ("checkpoint_state", _P), ("batch", ctypes.c_int64),
                ("q_stride", ctypes.c_int64), ("k_stride", ctypes.c_int64), ("v_stride", ctypes.c_int64),
                ("key_heads", ctypes.c_int32), ("n_checkpoints", ctypes.c_int32), ("qkv_dtype", ctypes.c_int32),
                ("gate_dtype", ctypes.c_int32), ("out_dtype", ctypes.c_int32), ("slots_dtype", ctypes.c_int32),
                ("normalize", ctypes.c_int32), ("scale", ctypes.c_float), ("events", _P),
                ("beta_logits", ctypes.c_int32), ("reserved", ctypes.c_int32)]


class FormatPool(ctypes.Structure):
    _fields_ = [("data", _P), ("page_bytes", ctypes.c_int64), ("num_slots", ctypes.c_int64),
                ("offsets", _P), ("rows", _P), ("columns", _P), ("heads", ctypes.c_int32),
                ("keys", ctypes.c_int32), ("values", ctypes.c_int32), ("kind", ctypes.c_int32),
                ("bits", ctypes.c_int32), ("group", ctypes.c_int32), ("kda", ctypes.c_int32),
                ("flags", ctypes.c_int32)]


FMT_FP32, FMT_SYMMETRIC, FMT_DSQ = 0, 1, 2
FMT_ROWS_CONTIGUOUS = 1

EXPORTS = ("sq_abi_version", "sq_last_error", "sq_encode", "sq_decode_dense", "sq_decode_step",
           "sq_decode_readout", "sq_writeback", "sq_clear_slots", "sq_copy_slots",
           "sq_stream_capture_id", "sq_create_cu_stream", "sq_pool_flags", "sq_prefill",
           "sq_format_encode", "sq_format_decode", "sq_format_step", "sq_copy_slots_static",
           "sq_event_create", "sq_event_destroy", "sq_event_record", "sq_event_wait", "sq_event_query",
           "sq_event_synchronize")
COPY_STATIC_BYTES = 16 << 20

_lib = None


def library_path() -> str:
    return LIB_PATH


def lib():
    """Load the HIP library; raises RuntimeError when it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                           "(hipcc --offload-arch=gfx950); there is no CPU fallback")
    L = ctypes.CDLL(LIB_PATH)
    PP = ctypes.POINTER
    L.sq_abi_version.restype = ctypes.c_int
    L.sq_last_error.restype = ctypes.c_char_p
    L.sq_encode.argtypes = [PP(Pool), _P, _P, ctypes.c_int32, ctypes.c_int64, _P]
    L.sq_decode_dense.argtypes = [PP(Pool), _P, ctypes.c_int32, ctypes.c_int64, _P, _P]
    L.sq_decode_step.argtypes = [PP(Pool), PP(StepArgs), _P]
    L.sq_decode_readout.argtypes = [PP(Pool), PP(StepArgs), PP(Scratch), _P]
    L.sq_writeback.argtypes = [PP(Pool), PP(Scratch), ctypes.c_int64, _P]
    L.sq_prefill.argtypes = [PP(Pool), PP(PrefillArgs), _P]
    L.sq_format_encode.argtypes = [PP(FormatPool), _P, _P, ctypes.c_int32, ctypes.c_int64, _P]
    L.sq_format_decode.argtypes = [PP(FormatPool), _P, ctypes.c_int32, ctypes.c_int64, _P, _P]
    L.sq_format_step.argtypes = [PP(FormatPool), PP(StepArgs), _P]
    L.sq_clear_slots.argtypes = [PP(Pool), _P, ctypes.c_int32, ctypes.c_int64, _P]
    L.sq_copy_slots.argtypes = [PP(Pool), _P, _P, ctypes.c_int32, ctypes.c_int64, _P, _P]
    L.sq_copy_slots_static.argtypes = [PP(Pool), _P, _P, ctypes.c_int32, ctypes.c_int64, _P]
    L.sq_event_create.argtypes = [PP(_P)]
    L.sq_event_destroy.argtypes = [_P]
    L.sq_event_record.argtypes = [_P, _P]
    L.sq_event_wait.argtypes = [_P, _P]
    L.sq_event_query.argtypes = [_P]
    L.sq_event_synchronize.argtypes = [_P]
    L.sq_pool_flags.argtypes = [_P, _P, _P, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                ctypes.c_int32, ctypes.c_int32, ctypes.c_int64]
    L.sq_stream_capture_id.argtypes = [_P, PP(ctypes.c_int32), PP(ctypes.c_uint64)]
    L.sq_create_cu_stream.argtypes = [ctypes.c_int32, ctypes.c_int32, PP(_P), PP(ctypes.c_int32),
                                      PP(ctypes.c_int32)]
    for name in EXPORTS:
        if name not in ("sq_last_error",):
            getattr(L, name).restype = ctypes.c_int
    if L.sq_abi_version() != ABI_VERSION:
        raise RuntimeError(f"libstepquant_hip ABI {L.sq_abi_version()} != {ABI_VERSION}; rebuild it")
    _lib = L
    return L


def check(rc: int, what: str):
    if rc != 0:
        msg = lib().sq_last_error().decode(errors="replace")
        if rc < 0:
            raise ValueError(f"{what}: {msg} (code {rc})")
        raise RuntimeError(f"{what}: {msg} (hip error {rc})")


def dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {t.dtype}") from None


def ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_handle(stream=None) -> ctypes.c_void_p:
    s = torch.cuda.current_stream() if stream is None else stream
    return ctypes.c_void_p(s.cuda_stream)


def pool_flags(bits, head_meta, columns, H, K, V, group, kda, storage, page_bytes) -> int:
    """sq_pool_flags on host int32 lists."""
    arr = lambda xs: (ctypes.c_int32 * len(xs))(*xs)
    rc = lib().sq_pool_flags(arr(bits), arr(head_meta), arr(columns), H, K, V, group, kda, storage, page_bytes)
    if rc < 0:
        check(rc, "pool flags")
    return rc


def capture_id(stream) -> int | None:
    """Capture identifier of a capturing stream, else None."""
    capturing = ctypes.c_int32(0)
    ident = ctypes.c_uint64(0)
    check(lib().sq_stream_capture_id(ctypes.c_void_p(stream.cuda_stream), ctypes.byref(capturing),
                                     ctypes.byref(ident)), "stream capture info")
    return int(ident.value) if capturing.value == 1 else None


def create_cu_stream(device: int, cus: int):
    """(raw stream handle, actual CUs, total CUs) of a CU-restricted stream."""
    raw = ctypes.c_void_p(0)
    actual = ctypes.c_int32(0)
    total = ctypes.c_int32(0)
    check(lib().sq_create_cu_stream(int(device), int(cus), ctypes.byref(raw), ctypes.byref(actual),
                                    ctypes.byref(total)), "CU-masked writeback stream")
    return raw.value, actual.value, total.value
