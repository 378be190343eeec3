"""Batch-one FP8 decode entry points with the reference's signatures
(src/drama_low_vram/fp8_decode.py:114-147), on the gfx950 kernels.

``forward(kernel, x, ids, weights, staged)`` -> [1, H] in x.dtype;
``quantized_pairs(kernel, q, scales, ids, weights, staged, dtype=)`` -> ordered
fp32 partials from an activation the caller already quantized (a single
shared row, or one row per pair).
"""
from __future__ import annotations

import torch

from . import _lib
from .formats import StagedExperts, fp8_bank_struct
from .offload import DECODE_PAIRS, HipExpertBackend, device_state


def forward(kernel, x, ids, weights, staged: StagedExperts):
    """One input row, up to eight route slots, reference slot-order reduction."""
    return HipExpertBackend().forward(x, ids.reshape(1, -1), weights.reshape(1, -1), staged)


def quantized_pairs(kernel, q, scales, ids, weights, staged: StagedExperts, *, dtype=torch.bfloat16):
    """Ordered fp32 partials of route pairs from FP8 rows q [R, H] + scales
    [R, H/128]; R == 1 shares the row across all pairs."""
    ids = ids.reshape(-1).contiguous()
    weights = weights.reshape(-1).contiguous()
    count, hidden = ids.numel(), q.shape[1]
    if count > DECODE_PAIRS:
        raise ValueError(f"quantized_pairs takes at most {DECODE_PAIRS} pairs per call")
    if q.shape[0] not in (1, count):
        raise ValueError("quantized rows must be one shared row or one per pair")
    out = torch.empty((count, hidden), dtype=torch.float32, device=q.device)
    bank = fp8_bank_struct(staged)
    state = device_state(q.device)
    lib = _lib.library()
    ws = state.workspace_for(lib.dmoe_fp8_workspace_bytes(bank, count))
    qb = q.view(torch.uint8)
    row_div = count if q.shape[0] == 1 else 1
    gu = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16, torch.float16: _lib.F16}[dtype]
    _lib.check(lib.dmoe_fp8_quantized_pairs(
        bank, _lib.ptr(qb), _lib.ptr(scales), qb.stride(0), scales.stride(0), q.shape[0], row_div,
        128 if scales.shape[1] == hidden // 128 else hidden, _lib.ptr(ids), _lib.dtype_code(ids.dtype),
        _lib.ptr(weights), _lib.dtype_code(weights.dtype), count, gu, _lib.ptr(out), _lib.ptr(ws),
        ws.numel(), _lib.ptr(state.status), _lib.stream_handle(q.device)))
    return out
