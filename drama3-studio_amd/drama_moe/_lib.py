"""ctypes binding of ``libdrama_moe.so`` (the C ABI of include/drama_moe.h).

The library is independent of the PyTorch binary ABI, like the reference's
native module (src/drama_low_vram/native_backend.py:1): tensors are passed as
raw device pointers, streams as ``hipStream_t`` handles.  There is no fallback:
if the library is missing or was built for another ABI, loading raises.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import torch

LIBRARY_PATH = Path(__file__).resolve().parent / "libdrama_moe.so"
ABI_VERSION = 1

F32, BF16, F16, I32, I64 = 0, 1, 2, 3, 4
_DTYPES = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16,
           torch.int32: I32, torch.int64: I64}

STATUS_BAD_EXPERT_ID = 1
STATUS_NON_FINITE = 2
STATUS_TOO_MANY_ROWS = 4
STATUS_SYNC_TIMEOUT = 8


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPES[dtype]
    except KeyError:
        raise ValueError(f"Unsupported element type {dtype}") from None


class Fp8Proj(ctypes.Structure):
    _fields_ = [("weight", ctypes.c_void_p), ("scale", ctypes.c_void_p),
                ("weight_stride_e", ctypes.c_int64), ("weight_stride_n", ctypes.c_int64),
                ("scale_stride_e", ctypes.c_int64), ("scale_stride_n", ctypes.c_int64),
                ("scale_stride_k", ctypes.c_int64),
                ("scale_rows", ctypes.c_int32), ("scale_cols", ctypes.c_int32),
                ("n", ctypes.c_int32), ("k", ctypes.c_int32)]


class Fp8Bank(ctypes.Structure):
    _fields_ = [("w13", Fp8Proj), ("w2", Fp8Proj), ("experts", ctypes.c_int32)]


_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64

_SIGNATURES = {
    "dmoe_abi_version": ([], _I),
    "dmoe_set_fused_decode": ([_I], _I),
    "dmoe_set_sync_spin_limit": ([ctypes.c_uint64], ctypes.c_uint64),
    "dmoe_debug_force_sync_timeout": ([_I], _I),
    "dmoe_last_error": ([], ctypes.c_char_p),
    "dmoe_decode_fp8": ([_P, _P, _L, _P], _I),
    "dmoe_fp8_quantize": ([_P, _I, _L, _I, _I, _I, _P, _P, _P, _P], _I),
    "dmoe_silu_mul_quant": ([_P, _I, _L, _I, _I, _P, _P, _P, _P], _I),
    "dmoe_route_topk": ([_P, _L, _I, _I, _I, _I, _P, _P, _I, _P], _I),
    "dmoe_permute_workspace_bytes": ([_I, _I], ctypes.c_size_t),
    "dmoe_permute": ([_P, _I, _I, _I, _P, _P, _P, _P, ctypes.c_size_t, _P, _P], _I),
    "dmoe_moe_align_workspace_bytes": ([_I, _I, _I], ctypes.c_size_t),
    "dmoe_moe_align": ([_P, _I, _I, _I, _I, _P, _P, _P, _I, _P, ctypes.c_size_t, _P, _P], _I),
    "dmoe_fp8_workspace_bytes": ([ctypes.POINTER(Fp8Bank), _I], ctypes.c_size_t),
    "dmoe_fp8_moe_forward": ([ctypes.POINTER(Fp8Bank), _P, _I, _L, _I, _P, _I, _P, _I, _I, _I, _I,
                              _P, _I, _L, _P, ctypes.c_size_t, _P, _P], _I),
    "dmoe_fp8_moe_pairs": ([ctypes.POINTER(Fp8Bank), _P, _I, _L, _I, _I, _P, _I, _P, _I, _I, _I,
                            _I, _P, _P, ctypes.c_size_t, _P, _P], _I),
    "dmoe_fp8_prepare": ([ctypes.POINTER(Fp8Bank), _P, _I, _L, _I, _I, _P, _I, _I, _I, _P,
                          ctypes.c_size_t, _P, _P], _I),
    "dmoe_fp8_gate_up": ([ctypes.POINTER(Fp8Bank), _I, _I, _I, _I, _P, _P, _P, ctypes.c_size_t, _P, _P], _I),
    "dmoe_fp8_down": ([ctypes.POINTER(Fp8Bank), _P, _P, _P, _I, _I, _I, _P, _I, _L, _P, _P,
                       ctypes.c_size_t, _P, _P], _I),
    "dmoe_fp8_moe_layer": ([ctypes.POINTER(Fp8Bank), _P, _I, _L, _I, _P, _L, _I, _I, _P, _P, _I, _I, _I,
                            _P, _I, _L, _P, ctypes.c_size_t, _P, _P], _I),
    "dmoe_fp8_moe_layer_noalloc": ([ctypes.POINTER(Fp8Bank), _P, _I, _L, _I, _P, _L, _I, _I, _P, _P, _I, _I,
                                    _I, _P, _I, _L, _P, _P], _I),
    "dmoe_rotate_quantize": ([_P, _I, _L, _I, _I, _P, _P, _P], _I),
    "dmoe_quant_workspace_bytes": ([_P, _I, _I], ctypes.c_size_t),
    "dmoe_quant_projection_workspace_bytes": ([_I, _I, _I, _I], ctypes.c_size_t),
    "dmoe_quant_projection": ([_P, _I, _I, _P, _I, _L, _I, _I, _P, _I, _P, _I, _I, _I, _P, _L, _P,
                               ctypes.c_size_t, _P, _P], _I),
    "dmoe_quant_moe_forward": ([_P, _P, _I, _L, _I, _I, _P, _I, _P, _I, _I, _I, _P, _I, _L, _P, _P,
                                ctypes.c_size_t, _P, _P], _I),
    "dmoe_quant_moe_layer": ([_P, _P, _I, _L, _I, _P, _L, _I, _I, _P, _P, _I, _P, _I, _L, _P, ctypes.c_size_t,
                              _P, _P], _I),
    "dmoe_w4a16_linear": ([_P, _I, _L, _I, _P, _L, _P, _L, _I, _I, _P, _L, _P], _I),
    "dmoe_moe_block_pre": ([_P, _L, _I, _I, _P, _L, _I, _P, _P, _L, _P, _L, _I, _P, _L, _P, _P, _L, _P], _I),
    "dmoe_moe_block_post": ([_P, _L, _I, _I, _P, _L, _I, _P, _P, _L, _P, _L, _P, _L, _P], _I),
    "dmoe_fp8_quantized_pairs": ([ctypes.POINTER(Fp8Bank), _P, _P, _L, _L, _I, _I, _I, _P, _I, _P,
                                  _I, _I, _I, _P, _P, ctypes.c_size_t, _P, _P], _I),
    "dmoe_combine_slots": ([_P, _L, _P, _I, _I, _I, _I, _I, _P, _I, _L, _P], _I),
    "dmoe_silu_table": ([_P, _P], _I),
    "dmoe_stream_read": ([_P, _L, _P, _P], _I),
    "dmoe_debug_set_phase_buffer": ([_P, _L], _I),
    "dmoe_cpu_executor_create": ([_I, _I, _I, _I, _I], _P),
    "dmoe_cpu_executor_destroy": ([_P], None),
    "dmoe_cpu_executor_isa": ([_P], _I),
    "dmoe_cpu_executor_threads": ([_P], _I),
    "dmoe_cpu_executor_set_guard": ([_P, _I], _I),
    "dmoe_cpu_executor_set_silu_table": ([_P, _P], _I),
    "dmoe_cpu_expert_pairs": ([_P, ctypes.POINTER(Fp8Bank), _P, _P, _I, _P, _P, _I, _P], _I),
    "dmoe_cpu_partition_routes": ([_P, _I, _P, _I, _I, _I, _P, _P], _I),
}

_lib = None


def library():
    """Load and check the HIP library once; raise if it is absent or stale."""
    global _lib
    if _lib is None:
        if not LIBRARY_PATH.is_file():
            raise RuntimeError(
                f"HIP expert library missing: {LIBRARY_PATH}. Build it with "
                "`python -c 'import __graft_entry__ as g; g.build()'` (hipcc, gfx950).")
        lib = ctypes.CDLL(str(LIBRARY_PATH))
        for name, (args, res) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        if lib.dmoe_abi_version() != ABI_VERSION:
            raise RuntimeError("libdrama_moe.so ABI version mismatch; rebuild the library")
        _lib = lib
    return _lib


def exported_symbols():
    return sorted(_SIGNATURES)


def check(status: int) -> None:
    """Map a failed C call to an exception carrying the native message."""
    if status:
        message = library().dmoe_last_error()
        text = message.decode("utf-8", errors="replace") if message else "native error"
        raise ValueError(text)


def ptr(tensor: torch.Tensor | None):
    return None if tensor is None else ctypes.c_void_p(tensor.data_ptr())


def stream_handle(device: torch.device):
    """hipStream_t of torch's current stream on `device` (kernels run there)."""
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)
