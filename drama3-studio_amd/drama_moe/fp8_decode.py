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
from .offload import DECODE_PAIRS, MAX_PAIRS, HipExpertBackend, device_state


def forward(kernel, x, ids, weights, staged: StagedExperts):
    """One input row, up to eight route slots, reference slot-order reduction."""
    return HipExpertBackend().forward(x, ids.reshape(1, -1), weights.reshape(1, -1), staged)


def quantized_pairs(kernel, q, scales, ids, weights, staged: StagedExperts, *, dtype=torch.bfloat16):
    """Ordered fp32 partials of route pairs from FP8 rows q [R, H] + scales
    [R, H/128]; R == 1 shares the row across all pairs."""
    ids = ids.reshape(-1).contiguous()
    weights = weights.reshape(-1).contiguous()
    count, hidden = ids.numel(), q.shape[1]
    if count > MAX_PAIRS:
        raise ValueError(f"quantized_pairs takes at most {MAX_PAIRS} pairs per call")
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


def staged_forward(x, ids, weights, staged: StagedExperts, *, pairs_out: bool = False,
                   gu_dtype: torch.dtype | None = None, hidden=None):
    """The decode layer as its three single-launch stages (prepare, gate/up,
    down) -- the reference's launch sequence of fp8_decode.py:114-147.

    x [T, H] float, ids / weights [T, k]; returns the slot-order combine
    [T, H] in x.dtype, or with ``pairs_out`` the ordered fp32 partials
    [T * k, H].  ``hidden`` = (hidden_q, hidden_scales) receives the FP8 hidden
    activation of stage 1 when given.
    """
    ids = ids.contiguous()
    weights = weights.contiguous()
    tokens, top_k = ids.shape
    pairs = tokens * top_k
    if pairs > DECODE_PAIRS:
        raise ValueError(f"staged_forward takes at most {DECODE_PAIRS} route pairs per call")
    if x.dim() != 2 or x.shape[0] != tokens or x.stride(1) != 1:
        raise ValueError("x must be [tokens, H] with contiguous rows")
    device = x.device
    bank = fp8_bank_struct(staged)
    inter, hsize = staged.w2_weight.shape[2], x.shape[1]
    state = device_state(device)
    lib = _lib.library()
    ws = state.workspace_for(lib.dmoe_fp8_workspace_bytes(bank, pairs))
    hq, hs = hidden if hidden is not None else (
        torch.empty(pairs, inter, dtype=torch.uint8, device=device),
        torch.empty(pairs, inter // 128, dtype=torch.float32, device=device))
    gu = _lib.dtype_code(gu_dtype or x.dtype)
    stream = _lib.stream_handle(device)
    common = (_lib.ptr(ws), ws.numel(), _lib.ptr(state.status), stream)
    _lib.check(lib.dmoe_fp8_prepare(bank, _lib.ptr(x), _lib.dtype_code(x.dtype), x.stride(0), tokens, top_k,
                                    _lib.ptr(ids), _lib.dtype_code(ids.dtype), pairs, 128, *common))
    _lib.check(lib.dmoe_fp8_gate_up(bank, top_k, pairs, 128, gu, _lib.ptr(hq), _lib.ptr(hs), *common))
    if pairs_out:
        out = torch.empty(pairs, hsize, dtype=torch.float32, device=device)
        _lib.check(lib.dmoe_fp8_down(bank, _lib.ptr(hq), _lib.ptr(hs), _lib.ptr(weights),
                                     _lib.dtype_code(weights.dtype), pairs, 1, None, _lib.F32, 0,
                                     _lib.ptr(out), *common))
    else:
        out = torch.empty(tokens, hsize, dtype=x.dtype, device=device)
        _lib.check(lib.dmoe_fp8_down(bank, _lib.ptr(hq), _lib.ptr(hs), _lib.ptr(weights),
                                     _lib.dtype_code(weights.dtype), pairs, top_k, _lib.ptr(out),
                                     _lib.dtype_code(out.dtype), out.stride(0), None, *common))
    return out
