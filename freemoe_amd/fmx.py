"""ctypes binding of libfmx.so (include/fmx.h) for tests and bench.

The library is the product; this module only loads it and turns status codes
into exceptions. Loading fails loudly when libfmx.so has not been built: there
is no fallback path.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char, c_char_p, c_double, c_int, c_int32, c_uint16, c_uint32, c_uint64, c_void_p
from pathlib import Path

# FMX_LIBRARY: another build of the same library (the host-sanitizer build of
# the CPU tests); by default the in-tree libfmx.so.
LIB_PATH = Path(os.environ.get("FMX_LIBRARY") or Path(__file__).resolve().parent / "libfmx.so")

FMX_TYPE_F32, FMX_TYPE_Q4_0, FMX_TYPE_Q8_0, FMX_TYPE_Q4_K, FMX_TYPE_Q6_K = 0, 2, 8, 12, 14
BLOCK_GEOMETRY = {FMX_TYPE_F32: (1, 4), FMX_TYPE_Q4_0: (32, 18), FMX_TYPE_Q8_0: (32, 34),
                  FMX_TYPE_Q4_K: (256, 144), FMX_TYPE_Q6_K: (256, 210)}
FAULT_NONE, FAULT_TRANSFER, FAULT_FENCE_DEFERRED, FAULT_FENCE_TIMEOUT, FAULT_DEVICE_LOSS = range(5)

STATUS_NAMES = {0: "OK", 1: "INVALID_ARGUMENT", 2: "UNSUPPORTED_QUANTISATION", 3: "SHAPE_MISMATCH",
                4: "INTERNAL_ERROR", 5: "ALLOCATION_FAILED", 6: "TRANSFER_FAILED", 7: "FENCE_TIMEOUT",
                8: "DEVICE_LOSS", 9: "NO_DEVICE", 10: "LAUNCH_FAILED"}


class FmxError(RuntimeError):
    def __init__(self, status: int, where: str):
        self.status = status
        super().__init__(f"{where}: {STATUS_NAMES.get(status, status)} ({status})")


class DeviceInfo(ctypes.Structure):
    _fields_ = [("name", c_char * 64), ("arch", c_char * 32), ("total_memory_bytes", c_uint64),
                ("free_memory_bytes", c_uint64), ("compute_units", c_uint32), ("wavefront_size", c_uint32),
                ("lds_bytes_per_cu", c_uint32), ("clock_khz", c_uint32), ("memory_clock_khz", c_uint32),
                ("memory_bus_bits", c_uint32)]


class MoELayer(ctypes.Structure):
    """fmx_moe_layer (all pointers are device addresses)."""
    _fields_ = [("hidden", c_uint32), ("ffn", c_uint32), ("experts", c_uint32), ("top_k", c_uint32),
                ("norm_weight", c_void_p), ("rms_eps", c_double), ("norm_bias", c_double),
                ("router_type", c_uint32), ("router", c_void_p), ("router_bias", c_void_p),
                ("weights_norm", c_int32), ("epsilon_additive", c_int32), ("weights_epsilon", c_double),
                ("weights_scale", c_double), ("gate_type", c_uint32), ("up_type", c_uint32),
                ("down_type", c_uint32), ("gate", c_void_p), ("up", c_void_p), ("down", c_void_p)]


_SIGNATURES = {
    "fmx_abi_version": (c_int, []),
    "fmx_status_name": (c_char_p, [c_int]),
    "fmx_device_info_get": (c_int, [c_int, POINTER(DeviceInfo)]),
    "fmx_alloc": (c_int, [c_uint64, POINTER(c_void_p)]),
    "fmx_free": (c_int, [c_void_p]),
    "fmx_host_alloc": (c_int, [c_uint64, POINTER(c_void_p)]),
    "fmx_host_free": (c_int, [c_void_p]),
    "fmx_upload": (c_int, [c_void_p, c_void_p, c_uint64, c_void_p, POINTER(c_void_p)]),
    "fmx_download": (c_int, [c_void_p, c_void_p, c_uint64, c_void_p]),
    "fmx_fence_query": (c_int, [c_void_p, POINTER(c_int)]),
    "fmx_fence_wait": (c_int, [c_void_p, c_uint32]),
    "fmx_fence_release": (c_int, [c_void_p]),
    "fmx_stream_sync": (c_int, [c_void_p]),
    "fmx_inject_fault": (c_int, [c_int]),
    "fmx_clear_faults": (c_int, []),
    "fmx_quant_geometry": (c_int, [c_uint32, POINTER(c_uint32), POINTER(c_uint32)]),
    "fmx_dequantize": (c_int, [c_uint32, c_void_p, c_void_p, c_uint64, c_void_p]),
    "fmx_packed_bytes": (c_uint64, [c_uint32, c_uint32, c_uint32]),
    "fmx_pack": (c_int, [c_uint32, c_void_p, c_void_p, c_uint32, c_uint32, c_void_p]),
    "fmx_matvec": (c_int, [c_uint32, c_void_p, c_void_p, c_void_p, c_uint32, c_uint32, c_void_p]),
    "fmx_gemm_quant": (c_int, [c_uint32, c_void_p, c_void_p, c_void_p, c_uint32, c_uint32, c_uint32, c_void_p]),
    "fmx_moe_workspace_bytes": (c_uint64, [POINTER(MoELayer), c_uint32]),
    "fmx_moe_route": (c_int, [POINTER(MoELayer), c_void_p, c_uint32, c_void_p, c_void_p, c_void_p, c_void_p,
                              c_void_p, c_uint64, c_void_p]),
    "fmx_moe_decode": (c_int, [POINTER(MoELayer), c_void_p, c_void_p, c_uint32, c_void_p, c_void_p, c_void_p,
                               c_uint64, c_void_p]),
    "fmx_moe_decode_static": (c_int, [POINTER(MoELayer), c_void_p, c_void_p, c_uint32, c_void_p, c_void_p,
                                      c_void_p, c_void_p]),
    "fmx_moe_decode_timed": (c_int, [POINTER(MoELayer), c_void_p, c_void_p, c_uint32, c_void_p, c_void_p,
                                     c_void_p, c_uint64, c_void_p, POINTER(c_double)]),
    "fmx_moe_prefill_workspace_bytes": (c_uint64, [POINTER(MoELayer), c_uint32]),
    "fmx_moe_prefill": (c_int, [POINTER(MoELayer), c_void_p, c_void_p, c_uint32, c_void_p, c_void_p, c_void_p,
                                c_uint64, c_void_p]),
    "fmx_moe_prefill_timed": (c_int, [POINTER(MoELayer), c_void_p, c_void_p, c_uint32, c_void_p, c_void_p,
                                      c_void_p, c_uint64, c_void_p, POINTER(c_double)]),
    "fmx_moe_status": (c_int, [c_void_p, c_void_p]),
    "fmx_moe_status_copy": (c_int, [c_void_p, c_void_p, c_void_p]),
    "fmx_moe_status_of": (c_int, [c_uint32]),
    "fmx_attention_decode": (c_int, [c_void_p, c_void_p, c_uint64, c_uint32, c_uint32, c_uint32, c_uint32, c_uint32,
                                     c_double, c_void_p, c_void_p, c_uint64, c_void_p]),
    "fmx_moe_bucket": (c_int, [c_void_p, c_uint32, c_uint32, c_uint32, c_void_p, c_void_p, c_void_p, c_void_p,
                               c_uint64, c_void_p]),
}

_lib = None


def lib() -> ctypes.CDLL:
    """The loaded libfmx.so with argument types set. Raises if it is missing."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built; run __graft_entry__.build() "
                               "(python -m freemoe_amd.build). There is no CPU fallback.")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(handle, name, None)
            if fn is None:
                continue
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def check(status: int, where: str) -> None:
    if status != 0:
        raise FmxError(status, where)


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args), name)


def ptr(t) -> int:
    """Device address of a torch tensor (0 for None)."""
    return 0 if t is None else t.data_ptr()


def stream_handle(stream=None) -> int:
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


def packed_bytes(type_id: int, rows: int, cols: int) -> int:
    n = lib().fmx_packed_bytes(type_id, rows, cols)
    if n == 0:
        raise FmxError(3, f"fmx_packed_bytes(type={type_id}, {rows}x{cols})")
    return n


def raw_row_bytes(type_id: int, cols: int) -> int:
    bs, bb = BLOCK_GEOMETRY[type_id]
    return cols // bs * bb
