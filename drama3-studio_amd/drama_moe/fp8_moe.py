"""gfx950 counterpart of the fish-speech ``fp8_moe`` kernel module the
reference calls (fishaudio/fish-speech@541566932abbaebcb0a40e562a1f846738383f38,
not vendored in the reference).  Same call-site API as used at
src/drama_low_vram/offload.py:251-356, fp8_decode.py:114-147 and
hybrid_decode.py:182-183:

* ``quantize_groups(kernel, x, columns)`` with ``kernel`` = ``quant_kernel``
  (FP8 128-groups of x) or ``silu_mul_quant_kernel`` (SiLU(gate) * up of a
  gate|up row, then FP8 128-groups), returning ``(q e4m3, fp32 scales)``;
* ``moe_align(ids, num_experts, block_m)`` -> ``(sorted_ids, expert_ids,
  padded)``, the block-padded expert-sorted pair layout
  (offload.py:299-306, hybrid_layer.py:39);
* ``fp8_moe_forward(x, ids, weights, w13, s13, w2, s2)``;
* ``fp8_gemm_supported(devices)``.
"""
from __future__ import annotations

import torch

from . import _lib
from .formats import FP8_DTYPE, StagedExperts

quant_kernel = "quant_kernel"
silu_mul_quant_kernel = "silu_mul_quant_kernel"


def fp8_gemm_supported(devices) -> bool:
    """True when every device is a ROCm GPU of the gfx950 family."""
    if not torch.cuda.is_available():
        return False
    for device in devices:
        device = torch.device(device)
        if device.type != "cuda":
            return False
        arch = getattr(torch.cuda.get_device_properties(device), "gcnArchName", "")
        if not arch.startswith("gfx950"):
            return False
    return True


def quantize_groups(kernel, x: torch.Tensor, columns: int):
    """FP8 E4M3 quantization in 128-column groups on the current stream."""
    if x.device.type != "cuda":
        raise RuntimeError("quantize_groups requires a ROCm GPU tensor")
    if x.ndim != 2 or x.stride(-1) != 1:
        raise ValueError("quantize_groups expects row-contiguous [rows, cols] input")
    rows = x.shape[0]
    q = torch.empty((rows, columns), dtype=FP8_DTYPE, device=x.device)
    scales = torch.empty((rows, columns // 128), dtype=torch.float32, device=x.device)
    lib = _lib.library()
    from .offload import device_state
    status = device_state(x.device).status
    stream = _lib.stream_handle(x.device)
    if kernel == quant_kernel:
        if x.shape[1] != columns:
            raise ValueError("quant_kernel quantizes whole rows")
        _lib.check(lib.dmoe_fp8_quantize(_lib.ptr(x), _lib.dtype_code(x.dtype), x.stride(0), rows,
                                         columns, 128, _lib.ptr(q), _lib.ptr(scales),
                                         _lib.ptr(status), stream))
    elif kernel == silu_mul_quant_kernel:
        if x.shape[1] != 2 * columns:
            raise ValueError("silu_mul_quant_kernel expects [rows, 2 * columns] gate|up")
        _lib.check(lib.dmoe_silu_mul_quant(_lib.ptr(x), _lib.dtype_code(x.dtype), x.stride(0), rows,
                                           columns, _lib.ptr(q), _lib.ptr(scales),
                                           _lib.ptr(status), stream))
    else:
        raise ValueError(f"Unknown quantization kernel {kernel!r}")
    return q, scales


def moe_align(ids: torch.Tensor, num_experts: int, block_m: int):
    """Route pairs sorted by expert and padded per expert to whole blocks of
    ``block_m`` rows, on the current stream: ``sorted_ids`` int32
    [blocks * block_m] (pair indices, the sentinel ``pairs`` in padding rows),
    ``expert_ids`` int32 [blocks] (-1 past the last block) and ``padded``, a
    device int32 [1] holding the padded row count; blocks = ceil(pairs /
    block_m) + num_experts is the capacity."""
    if ids.device.type != "cuda":
        raise RuntimeError("moe_align requires a ROCm GPU tensor")
    from .offload import device_state

    flat = ids.reshape(-1).contiguous()
    pairs = flat.numel()
    blocks = -(-pairs // block_m) + num_experts
    sorted_ids = torch.empty(blocks * block_m, dtype=torch.int32, device=ids.device)
    expert_ids = torch.empty(blocks, dtype=torch.int32, device=ids.device)
    padded = torch.zeros(1, dtype=torch.int32, device=ids.device)
    if pairs == 0:
        return sorted_ids.fill_(0), expert_ids.fill_(-1), padded
    lib = _lib.library()
    state = device_state(ids.device)
    ws = state.workspace_for(lib.dmoe_moe_align_workspace_bytes(pairs, num_experts, block_m))
    _lib.check(lib.dmoe_moe_align(_lib.ptr(flat), _lib.dtype_code(flat.dtype), pairs, num_experts, block_m,
                                  _lib.ptr(sorted_ids), _lib.ptr(expert_ids), _lib.ptr(padded), blocks,
                                  _lib.ptr(ws), ws.numel(), _lib.ptr(state.status),
                                  _lib.stream_handle(ids.device)))
    return sorted_ids, expert_ids, padded


def fp8_moe_forward(x, ids, weights, w13, s13, w2, s2):
    """Whole routed-expert layer (the official FP8 MoE entry point)."""
    from .offload import HipExpertBackend

    return HipExpertBackend().forward(x, ids, weights, StagedExperts(w13, s13, w2, s2))
