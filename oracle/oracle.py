"""ctypes wrapper of the C oracle (``liboracle.so``) -- TEST INFRASTRUCTURE ONLY.

Every function takes and returns numpy arrays on the host.  Floating inputs
that stand for bf16/fp16 tensors are passed as fp32 arrays holding the exact
bf16/fp16 values.  Each wrapper names the reference code it restates; see the
C source for the arithmetic.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"
REF_LIB_PATH = HERE / "_ref" / "libdrama_native.so"

DTYPE_CODES = {"fp32": 0, "bf16": 1, "fp16": 2}


def build(reference: bool = False) -> None:
    """Compile the oracle (and the reference executor when asked)."""
    subprocess.run(["make", "-s", "-C", str(HERE), "all"], check=True)
    if reference:
        subprocess.run(["make", "-s", "-C", str(HERE), "ref"], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.is_file():
            build()
        _lib = ctypes.CDLL(str(LIB_PATH))
        _lib.orc_fp8_decode.restype = ctypes.c_float
        _lib.orc_fp8_decode.argtypes = [ctypes.c_uint8]
        _lib.orc_fp8_encode.restype = ctypes.c_uint8
        _lib.orc_fp8_encode.argtypes = [ctypes.c_float]
        _lib.orc_bf16_from_f32.restype = ctypes.c_uint16
        _lib.orc_bf16_from_f32.argtypes = [ctypes.c_float]
        _lib.orc_f16_from_f32.restype = ctypes.c_uint16
        _lib.orc_f16_from_f32.argtypes = [ctypes.c_float]
        _lib.orc_f32_from_f16.restype = ctypes.c_float
        _lib.orc_f32_from_f16.argtypes = [ctypes.c_uint16]
        for name in ("orc_quantize_fp8", "orc_fp8_expert_pairs", "orc_fp8_moe_forward",
                     "orc_route_topk", "orc_permute", "orc_moe_align", "orc_rotate_quantize",
                     "orc_quant_projection", "orc_quant_dequantize"):
            getattr(_lib, name).restype = ctypes.c_int
    return _lib


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _check(status, what):
    if status != 0:
        raise ValueError(f"oracle {what} rejected its input (status {status})")


class _Fp8Proj(ctypes.Structure):
    _fields_ = [("w", ctypes.c_void_p), ("s", ctypes.c_void_p),
                ("N", ctypes.c_int64), ("K", ctypes.c_int64),
                ("se", ctypes.c_int64), ("sn", ctypes.c_int64), ("sk", ctypes.c_int64),
                ("n_div", ctypes.c_int64), ("kb_div", ctypes.c_int64), ("wfmt", ctypes.c_int64)]


class _QuantProj(ctypes.Structure):
    _fields_ = [("w", ctypes.c_void_p), ("s", ctypes.c_void_p), ("z", ctypes.c_void_p),
                ("N", ctypes.c_int64), ("K", ctypes.c_int64), ("mode", ctypes.c_int)]


# ------------------------------------------------------------------ codecs

def fp8_decode(raw: np.ndarray) -> np.ndarray:
    """All-E4M3 decode (fp8_reference.cpp:10-17)."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    out = np.empty(raw.shape, np.float32)
    lib().orc_fp8_decode_many(_ptr(raw), _ptr(out), ctypes.c_int64(raw.size))
    return out


def fp8_encode(values: np.ndarray) -> np.ndarray:
    """RNE E4M3 encode with +-448 saturation (fp8_reference.cpp:19-36)."""
    f = lib().orc_fp8_encode
    flat = np.ascontiguousarray(values, dtype=np.float32).reshape(-1)
    return np.array([f(float(v)) for v in flat], np.uint8).reshape(np.shape(values))


def bf16_round(values: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 (RNE) -> fp32, vectorised form of fp8_reference.cpp:45-50."""
    u = np.ascontiguousarray(values, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    r = np.where(nan, (u >> 16) | 0x40, r).astype(np.uint32) << 16
    return r.view(np.float32).reshape(np.shape(values))


# -------------------------------------------------------------- quantization

def quantize_fp8(x: np.ndarray, group: int = 128):
    """Dynamic FP8 activation quant of rows (fp8_reference.cpp:52-93,
    fp8_cpu_reference.py:14-20).  Returns (uint8 bytes, fp32 scales)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, cols = x.reshape(-1, x.shape[-1]).shape
    q = np.empty((rows, cols), np.uint8)
    s = np.empty((rows, cols // group), np.float32)
    _check(lib().orc_quantize_fp8(_ptr(x), ctypes.c_int64(rows), ctypes.c_int64(cols),
                                  ctypes.c_int64(group), _ptr(q), _ptr(s)), "quantize")
    return q.reshape(x.shape), s


class Fp8Bank:
    """Host copy of one FP8 projection bank: bytes [E, N, K], scales [E, a, b]
    where a in {N/128, N} and b in {K/128, 1} (block or per-channel)."""

    def __init__(self, weight_bytes: np.ndarray, scales: np.ndarray):
        self.w = np.ascontiguousarray(weight_bytes, dtype=np.uint8)
        self.s = np.ascontiguousarray(scales, dtype=np.float32)
        E, N, K = self.w.shape
        se, sa, sb = self.s.shape
        if se != E or N % sa or (K // 128) % sb:
            raise ValueError("scale shape does not tile the weight bank")
        self.struct = _Fp8Proj(self.w.ctypes.data, self.s.ctypes.data, N, K,
                               sa * sb, sb, 1 if sb > 1 else 0, N // sa, (K // 128) // sb)


class G128Bank:
    """Host copy of one projection bank of the group-128 integer formats
    (W4A8-g128: mode 4, 4-bit codes [E, N, K/2], level = code - 8; W6A8-g128:
    mode 5, the 6-bit planes [E, N, 3K/4], level = code - 32) with fp16
    scales [E, N, K/128].  Usable wherever an Fp8Bank is: the FP8 W8A8
    contract with these weights (integer level x group scale)."""

    def __init__(self, mode, weight, scales):
        if mode not in (4, 5):
            raise ValueError("group-128 integer banks are modes 4 and 5")
        self.w = np.ascontiguousarray(weight).view(np.uint8)
        self.s = np.ascontiguousarray(scales, dtype=np.float16)
        E, N, cols = self.w.shape
        K = cols * 2 if mode == 4 else cols * 4 // 3
        if self.s.shape != (E, N, K // 128):
            raise ValueError("scales must be [E, N, K/128] fp16")
        self.struct = _Fp8Proj(self.w.ctypes.data, self.s.ctypes.data, N, K, N * (K // 128), K // 128, 1,
                               1, 1, 1 if mode == 4 else 2)


def fp8_expert_pairs(w13: Fp8Bank, w2: Fp8Bank, x, ids, weights, *, x_group=128, gu_dtype="bf16"):
    """Ordered weighted fp32 partials for one row (runtime.cpp:173-237)."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    ids = np.ascontiguousarray(ids, np.int64).reshape(-1)
    weights = np.ascontiguousarray(weights, np.float32).reshape(-1)
    out = np.empty((ids.size, x.size), np.float32)
    _check(lib().orc_fp8_expert_pairs(
        ctypes.byref(w13.struct), ctypes.byref(w2.struct), ctypes.c_int64(w13.w.shape[0]),
        _ptr(x), ctypes.c_int64(x_group), _ptr(ids), _ptr(weights), ctypes.c_int64(ids.size),
        ctypes.c_int(DTYPE_CODES[gu_dtype]), _ptr(out)), "expert_pairs")
    return out


def fp8_moe_forward(w13: Fp8Bank, w2: Fp8Bank, x, ids, weights, *, x_group=128,
                    gu_dtype="bf16", out_dtype="bf16"):
    """T-token layer with slot-order fp32 combine (offload.py:1242-1244)."""
    x = np.ascontiguousarray(x, np.float32)
    ids = np.ascontiguousarray(ids, np.int64)
    weights = np.ascontiguousarray(weights, np.float32)
    tokens, top_k = ids.shape
    out = np.empty((tokens, x.shape[1]), np.float32)
    _check(lib().orc_fp8_moe_forward(
        ctypes.byref(w13.struct), ctypes.byref(w2.struct), ctypes.c_int64(w13.w.shape[0]),
        _ptr(x), ctypes.c_int64(tokens), ctypes.c_int64(x_group), _ptr(ids), _ptr(weights),
        ctypes.c_int64(top_k), ctypes.c_int(DTYPE_CODES[gu_dtype]),
        ctypes.c_int(DTYPE_CODES[out_dtype]), _ptr(out)), "moe_forward")
    return out


# ------------------------------------------- O2: dequantize, then matmul

def _round_to(values, dtype):
    values = np.asarray(values, np.float32)
    if dtype == "fp32":
        return values
    if dtype == "bf16":
        return bf16_round(values)
    return values.astype(np.float16).astype(np.float32)  # IEEE round-to-nearest-even


def dequantize_fp8_blocks(weight_bytes, scale_inv, dtype="bf16"):
    """W = fp32(E4M3 value * 128x128 block scale) rounded to the compute
    dtype (offload.py:44-56)."""
    w = fp8_decode(np.asarray(weight_bytes, np.uint8))
    n, k = w.shape
    rb, cb = scale_inv.shape
    if n != rb * 128 or k != cb * 128:
        raise ValueError("FP8 weight shape does not match its 128x128 block scales")
    scaled = (w.reshape(rb, 128, cb, 128) * np.asarray(scale_inv, np.float32)[:, None, :, None]).astype(np.float32)
    return _round_to(scaled.reshape(n, k), dtype)


def o2_expert_pairs(w13: "Fp8Bank", w2: "Fp8Bank", x, ids, weights, dtype="bf16"):
    """TorchExpertBackend.forward_pairs (offload.py:214-244): per expert the
    dequantized W13 / W2 in the compute dtype; gate, up = x @ W13^T and
    values = (silu(gate) * up) @ W2^T, each product accumulated exactly
    (float64) and rounded once to the compute dtype, silu and the product
    rounded to it too; the weighted value in fp32.  x [pairs, H] (compute
    dtype values as fp32), ids / weights [pairs]; returns fp32 [pairs, H]."""
    x = np.asarray(x, np.float32)
    ids = np.asarray(ids, np.int64).reshape(-1)
    weights = np.asarray(weights, np.float32).reshape(-1)
    out = np.empty((ids.size, w2.w.shape[1]), np.float32)
    inter = w13.w.shape[1] // 2
    for e in np.unique(ids):
        rows = np.flatnonzero(ids == e)
        m13 = dequantize_fp8_blocks(w13.w[e], w13.s[e], dtype).astype(np.float64)
        m2 = dequantize_fp8_blocks(w2.w[e], w2.s[e], dtype).astype(np.float64)
        gu = _round_to(x[rows].astype(np.float64) @ m13.T, dtype)
        gate, up = gu[:, :inter], gu[:, inter:]
        act = _round_to(_round_to(silu(gate), dtype) * up, dtype)
        values = _round_to(act.astype(np.float64) @ m2.T, dtype)
        out[rows] = values * weights[rows, None]
    return out


def o2_moe_forward(w13: "Fp8Bank", w2: "Fp8Bank", x, ids, weights, dtype="bf16"):
    """TorchExpertBackend.forward (offload.py:202-212): the pairs of each
    token summed over the top-k slots in fp32, rounded to the compute dtype."""
    ids = np.asarray(ids, np.int64)
    tokens, top_k = ids.shape
    rows = np.repeat(np.asarray(x, np.float32), top_k, axis=0)
    pairs = o2_expert_pairs(w13, w2, rows, ids.reshape(-1), np.asarray(weights).reshape(-1), dtype)
    part = pairs.reshape(tokens, top_k, -1)
    acc = part[:, 0].copy()
    for j in range(1, top_k):
        acc = (acc + part[:, j]).astype(np.float32)
    return _round_to(acc, dtype)


# ------------------------------------------------------------------ routing

def route_topk(logits, top_k, renormalize=True):
    """softmax -> top-k -> renorm (backbone_graph.py:317-323); ids int64,
    weights fp32 (the caller casts to its compute dtype)."""
    logits = np.ascontiguousarray(logits, np.float32)
    tokens, experts = logits.shape
    ids = np.empty((tokens, top_k), np.int64)
    weights = np.empty((tokens, top_k), np.float32)
    _check(lib().orc_route_topk(_ptr(logits), ctypes.c_int64(tokens), ctypes.c_int64(experts),
                                ctypes.c_int64(top_k), ctypes.c_int(int(renormalize)),
                                _ptr(ids), _ptr(weights)), "route_topk")
    return ids, weights


def permute(ids, experts):
    """Stable expert-major order, counts, offsets (offload.py:1206-1210)."""
    flat = np.ascontiguousarray(ids, np.int64).reshape(-1)
    order = np.empty(flat.size, np.int32)
    counts = np.empty(experts, np.int32)
    offsets = np.empty(experts + 1, np.int32)
    _check(lib().orc_permute(_ptr(flat), ctypes.c_int64(flat.size), ctypes.c_int64(experts),
                             _ptr(order), _ptr(counts), _ptr(offsets)), "permute")
    return order, counts, offsets


def moe_align(ids, experts, block_m):
    """Block-padded expert-sorted pair indices (the moe_align layout of
    offload.py:299-306): (sorted_ids int32 [cap * block_m], expert_ids int32
    [cap], padded) with cap = ceil(pairs / block_m) + experts blocks; sentinel
    = pairs, expert -1 past the last block; invalid ids left out."""
    flat = np.ascontiguousarray(ids, np.int64).reshape(-1)
    cap = (flat.size + block_m - 1) // block_m + experts
    sorted_ids = np.empty(cap * block_m, np.int32)
    expert_ids = np.empty(cap, np.int32)
    padded = np.zeros(1, np.int32)
    _check(lib().orc_moe_align(_ptr(flat), ctypes.c_int64(flat.size), ctypes.c_int64(experts),
                               ctypes.c_int64(block_m), ctypes.c_int64(cap), _ptr(sorted_ids),
                               _ptr(expert_ids), _ptr(padded)), "moe_align")
    return sorted_ids, expert_ids, int(padded[0])


# -------------------------------------------------- packed quantized modes

def rotate_quantize(x, rot_dtype="bf16"):
    """H256 rotation + row INT8 quant (quantized_kernels.py:15-45)."""
    x = np.ascontiguousarray(x, np.float32)
    rows, K = x.shape
    q = np.empty((rows, K), np.int8)
    s = np.empty(rows, np.float32)
    rot = np.empty((rows, K), np.float32)
    _check(lib().orc_rotate_quantize(_ptr(x), ctypes.c_int64(rows), ctypes.c_int64(K),
                                     ctypes.c_int(DTYPE_CODES[rot_dtype]), _ptr(q), _ptr(s),
                                     _ptr(rot)), "rotate_quantize")
    return q, s, rot


class QuantBank:
    """Host copy of one packed projection bank of mode 0-3 (layouts in the C
    source); ``zeros`` is the optional asymmetric W4A16 zero-point bank."""

    def __init__(self, mode, weight, scales, n, k, zeros=None):
        self.mode = mode
        self.w = np.ascontiguousarray(weight)
        self.s = np.ascontiguousarray(scales)
        self.z = None if zeros is None else np.ascontiguousarray(zeros, np.int32)
        self.experts = self.w.shape[0]
        self.struct = _QuantProj(self.w.ctypes.data, self.s.ctypes.data,
                                 None if self.z is None else self.z.ctypes.data, n, k, mode)


def quant_projection(bank: QuantBank, x, ids, weights, *, shared=False, weighted=False,
                     rot_dtype="bf16"):
    """Route-pair projection (quantized_kernels.py:115-214)."""
    x = np.ascontiguousarray(x, np.float32)
    ids = np.ascontiguousarray(ids, np.int64).reshape(-1)
    weights = np.ascontiguousarray(weights, np.float32).reshape(-1)
    out = np.empty((ids.size, bank.struct.N), np.float32)
    _check(lib().orc_quant_projection(
        ctypes.byref(bank.struct), ctypes.c_int64(bank.experts), _ptr(x),
        ctypes.c_int64(x.shape[0]), ctypes.c_int(DTYPE_CODES[rot_dtype]), _ptr(ids),
        _ptr(weights), ctypes.c_int64(ids.size), ctypes.c_int(int(shared)),
        ctypes.c_int(int(weighted)), _ptr(out)), "quant_projection")
    return out


def quant_dequantize(bank: QuantBank, expert: int):
    out = np.empty((bank.struct.N, bank.struct.K), np.float32)
    _check(lib().orc_quant_dequantize(ctypes.byref(bank.struct), ctypes.c_int64(expert),
                                      _ptr(out)), "quant_dequantize")
    return out


def silu(x):
    x = np.asarray(x, np.float32)
    return x / (np.float32(1) + np.exp(-x))


def block_pre(x, router_w, shared_gate_w, gate_w, up_w):
    """MoE block head (backbone_graph.py:317-330): bf16-rounded router logits
    [T, E], the sigmoid shared gate [T] and the shared expert's activation
    [T, I], every input a bf16 value in float32 arrays."""
    x = np.ascontiguousarray(x, np.float32)
    T, H = x.shape
    E, I = router_w.shape[0], gate_w.shape[0]
    logits = np.empty((T, E), np.float32)
    sgate = np.empty(T, np.float32)
    act = np.empty((T, I), np.float32)
    _check(lib().orc_block_pre(_ptr(x), ctypes.c_int64(T), ctypes.c_int64(H),
                               _ptr(np.ascontiguousarray(router_w, np.float32)), ctypes.c_int64(E),
                               _ptr(np.ascontiguousarray(shared_gate_w, np.float32).reshape(-1)),
                               _ptr(np.ascontiguousarray(gate_w, np.float32)),
                               _ptr(np.ascontiguousarray(up_w, np.float32)), ctypes.c_int64(I),
                               _ptr(logits), _ptr(sgate), _ptr(act)), "block_pre")
    return logits, sgate, act


def block_post(act, down_w, sgate, experts, residual):
    """MoE block tail (backbone_graph.py:329-337): residual + (experts +
    sgate * shared down projection), bf16 at every boundary."""
    act = np.ascontiguousarray(act, np.float32)
    T, I = act.shape
    H = down_w.shape[0]
    out = np.empty((T, H), np.float32)
    _check(lib().orc_block_post(_ptr(act), ctypes.c_int64(T), ctypes.c_int64(I),
                                _ptr(np.ascontiguousarray(down_w, np.float32)), ctypes.c_int64(H),
                                _ptr(np.ascontiguousarray(sgate, np.float32)),
                                _ptr(np.ascontiguousarray(experts, np.float32)),
                                _ptr(np.ascontiguousarray(residual, np.float32)), _ptr(out)), "block_post")
    return out
