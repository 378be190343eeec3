"""Router top-k and stable route permutation on the device.

``route_topk`` restates the router of BackboneDecodeGraph._route_impl
(src/drama_low_vram/backbone_graph.py:317-323): softmax of fp32 logits, top-k
(logit descending, lower index first on exact ties), optional renormalisation,
weights cast to the compute dtype.  ``permute`` is the stable expert-major
order of ExpertOffloadManager._forward_partitioned (offload.py:1206-1210).
"""
from __future__ import annotations

import torch

from . import _lib


def route_topk(logits: torch.Tensor, top_k: int, *, renormalize: bool = True,
               dtype: torch.dtype = torch.bfloat16):
    if logits.device.type != "cuda":
        raise RuntimeError("route_topk requires a ROCm GPU tensor")
    logits = logits.float()
    if logits.ndim != 2 or logits.stride(-1) != 1:
        logits = logits.reshape(-1, logits.shape[-1]).contiguous()
    tokens, experts = logits.shape
    ids = torch.empty((tokens, top_k), dtype=torch.int64, device=logits.device)
    weights = torch.empty((tokens, top_k), dtype=dtype, device=logits.device)
    _lib.check(_lib.library().dmoe_route_topk(
        _lib.ptr(logits), logits.stride(0), tokens, experts, top_k, int(renormalize),
        _lib.ptr(ids), _lib.ptr(weights), _lib.dtype_code(dtype), _lib.stream_handle(logits.device)))
    return weights, ids


def permute(ids: torch.Tensor, num_experts: int):
    """(order int32 [pairs], counts int32 [E], offsets int32 [E+1]) of the
    flattened ids; invalid ids are left out and flagged in the status word."""
    from .offload import device_state

    flat = ids.reshape(-1).contiguous()
    pairs = flat.numel()
    order = torch.empty(pairs, dtype=torch.int32, device=ids.device)
    counts = torch.empty(num_experts, dtype=torch.int32, device=ids.device)
    offsets = torch.empty(num_experts + 1, dtype=torch.int32, device=ids.device)
    lib = _lib.library()
    scratch = torch.empty(max(1, lib.dmoe_permute_workspace_bytes(pairs, num_experts)), dtype=torch.uint8,
                          device=ids.device)
    _lib.check(lib.dmoe_permute(
        _lib.ptr(flat), _lib.dtype_code(flat.dtype), pairs, num_experts, _lib.ptr(order),
        _lib.ptr(counts), _lib.ptr(offsets), _lib.ptr(scratch), scratch.numel(),
        _lib.ptr(device_state(ids.device).status), _lib.stream_handle(ids.device)))
    return order, counts, offsets


def decode_fp8(raw: torch.Tensor) -> torch.Tensor:
    """Device E4M3 decode of bytes (validation helper)."""
    raw = raw.contiguous().view(torch.uint8)
    out = torch.empty(raw.shape, dtype=torch.float32, device=raw.device)
    _lib.check(_lib.library().dmoe_decode_fp8(_lib.ptr(raw), _lib.ptr(out), raw.numel(),
                                              _lib.stream_handle(raw.device)))
    return out
