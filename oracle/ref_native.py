"""ctypes binding of the reference's own CPU expert executor -- TEST
INFRASTRUCTURE ONLY.

The library is compiled by ``make -C oracle ref`` from the reference's
``native/src/*.cpp`` into ``oracle/_ref/libdrama_native.so``; it is never
committed.  The binding follows the C declarations of
``native/include/drama_native.h:15-66`` (ABI v1): status-returning calls, a
thread-local error string, borrowed contiguous CPU buffers.  It is used to pin
the C oracle against the reference, and as the timed CPU baseline.
"""
from __future__ import annotations

import ctypes

import numpy as np

from .oracle import REF_LIB_PATH

IMPLEMENTATIONS = {"auto": 0, "scalar": 1, "avx2": 2, "avx512": 3}


def available() -> bool:
    return REF_LIB_PATH.is_file()


class RefLibrary:
    def __init__(self, path=REF_LIB_PATH):
        self.dll = ctypes.CDLL(str(path))
        d = self.dll
        d.drama_native_abi.restype = ctypes.c_int
        d.drama_native_features.restype = ctypes.c_int
        d.drama_native_error.restype = ctypes.c_char_p
        d.drama_decode_fp8.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int]
        d.drama_quantize_bf16.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int]
        d.drama_executor_create.argtypes = [ctypes.c_int] * 5
        d.drama_executor_create.restype = ctypes.c_void_p
        d.drama_executor_destroy.argtypes = [ctypes.c_void_p]
        d.drama_executor_destroy.restype = None
        d.drama_executor_implementation.argtypes = [ctypes.c_void_p]
        d.drama_executor_forward.argtypes = (
            [ctypes.c_void_p] * 5 + [ctypes.c_int] + [ctypes.c_void_p] * 3
            + [ctypes.c_int, ctypes.c_void_p])
        d.drama_executor_forward_quantized.argtypes = (
            [ctypes.c_void_p] * 5 + [ctypes.c_int] + [ctypes.c_void_p] * 4
            + [ctypes.c_int, ctypes.c_void_p])
        if d.drama_native_abi() != 1:
            raise RuntimeError("unexpected reference native ABI")
        self.features = d.drama_native_features()

    def check(self, status):
        if status:
            raise RuntimeError(self.dll.drama_native_error().decode())

    def decode(self, raw: np.ndarray) -> np.ndarray:
        raw = np.ascontiguousarray(raw, np.uint8)
        out = np.empty(raw.shape, np.float32)
        self.check(self.dll.drama_decode_fp8(raw.ctypes.data, out.ctypes.data, raw.size))
        return out

    def quantize_bf16(self, bits: np.ndarray):
        """bits: uint16 bf16 patterns, whole 128-value groups."""
        bits = np.ascontiguousarray(bits, np.uint16)
        q = np.empty(bits.shape, np.uint8)
        s = np.empty(bits.size // 128, np.float32)
        self.check(self.dll.drama_quantize_bf16(bits.ctypes.data, q.ctypes.data, s.ctypes.data,
                                                bits.size))
        return q, s


class RefExecutor:
    """One reference executor: [E,2I,H]/[E,2I/128,H/128]/[E,H,I]/[E,H/128,I/128]
    block-FP8 banks, one bf16 row in, ordered fp32 partials out."""

    def __init__(self, lib: RefLibrary, hidden, intermediate, capacity=8, threads=1,
                 implementation="auto"):
        self.lib = lib
        self.handle = lib.dll.drama_executor_create(hidden, intermediate, capacity, threads,
                                                    IMPLEMENTATIONS[implementation])
        if not self.handle:
            lib.check(-1)
        self.hidden = hidden

    def forward(self, w13, s13, w2, s2, x_bits, ids, weights, out=None):
        ids = np.ascontiguousarray(ids, np.int64)
        weights = np.ascontiguousarray(weights, np.float32)
        if out is None:
            out = np.empty((ids.size, self.hidden), np.float32)
        self.lib.check(self.lib.dll.drama_executor_forward(
            self.handle, w13.ctypes.data, s13.ctypes.data, w2.ctypes.data, s2.ctypes.data,
            w13.shape[0], x_bits.ctypes.data, ids.ctypes.data, weights.ctypes.data, ids.size,
            out.ctypes.data))
        return out

    def close(self):
        if self.handle:
            self.lib.dll.drama_executor_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
