"""gfx950 counterpart of the fish-speech ``fp8_moe`` kernel module the
reference calls (fishaudio/fish-speech@541566932abbaebcb0a40e562a1f846738383f38,
not vendored in the reference).  Same call-site API as used at
src/drama_low_vram/offload.py:251-356, fp8_decode.py:114-147 and
hybrid_decode.py:182-183:

* ``quantize_groups(kernel, x, columns)`` with ``kernel`` = ``quant_kernel``
  (FP8 128-groups of x) or ``silu_mul_quant_kernel`` (SiLU(gate) * up of a
  gate|up row, then FP8 128-groups), returning ``(q e4m3, fp32 scales)``;
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


def fp8_moe_forward(x, ids, weights, w13, s13, w2, s2):
    """Whole routed-expert layer (the official FP8 MoE entry point)."""
    from .offload import HipExpertBackend

    return HipExpertBackend().forward(x, ids, weights, StagedExperts(w13, s13, w2, s2))
