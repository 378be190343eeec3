"""MI355X (gfx950) quantized MoE expert path.

Host-side mirror of the reference's expert interface (src/drama_low_vram:
offload.py ExpertBackend / install_expert_offload, fp8_decode.py,
quantized_kernels.py) over hand-written HIP kernels behind the C ABI of
include/drama_moe.h (libdrama_moe.so, loaded with ctypes).
"""
from .formats import (EXPERT_BUFFER_NAMES, FP8_DTYPE, ExpertStore, QuantizedStore,  # noqa: F401
                      StagedExperts)

__all__ = ["EXPERT_BUFFER_NAMES", "FP8_DTYPE", "ExpertStore", "QuantizedStore", "StagedExperts"]
