"""Expert bank formats of the quantized MoE path, resident in HBM.

Mirrors the reference's bank types -- ``ExpertStore`` / ``StagedExperts``
(src/drama_low_vram/offload.py:101-184) for FP8 and ``QuantizedStore``
(src/drama_low_vram/quantized_model.py:26-68) for W4A16 / INT8 / W6A8 / W4A8 --
without the CPU-residency requirement: with 288 GB of HBM every expert stays on
the device, so ``staged`` is simply the whole bank and local ids are global ids.

Also holds the packers used to build synthetic banks (the reference's test
helpers tests/test_quantized_kernels.py:10-24 define the packed layouts).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Callable

import torch

from . import _lib

FP8_DTYPE = torch.float8_e4m3fn
FP8_BLOCK_SIZE = 128
FP8_MAX = 448.0
EXPERT_BUFFER_NAMES = ("w13_weight", "w13_scale_inv", "w2_weight", "w2_scale_inv")


def select_fp8(weight: torch.Tensor, index) -> torch.Tensor:
    """Select FP8 entries through their bytes (offload.py:39-41)."""
    return weight.view(torch.uint8)[index].view(weight.dtype)


# ------------------------------------------------------------- bank geometry

@dataclass(frozen=True)
class ProjectionFormat:
    """How one projection [E, N, K] of a bank format is stored: the weight
    element type and its packed column count (a function of K), the scale
    element type and the trailing scale shapes allowed for (N, K)."""

    weight_dtype: torch.dtype
    weight_columns: Callable[[int], int]
    scale_dtype: torch.dtype
    scale_shapes: Callable[[int, int], tuple]


# FP8 (the reference's StagedExperts, offload.py:175-184) and the packed
# modes 0-3 of QuantizedStore (quantized_model.py:26-68): 128x128 block or
# per-channel scales; GPTQ int32 words with fp16 group scales; INT8 rows with
# a channel scale; 6-bit (nibble + 2-bit planes) and 4-bit codebook codes
# with E4M3 group-16 scale bytes followed by the fp32 channel scale (and, in
# mode 3, the codebook).  Modes 4 and 5 have no reference counterpart: 4-bit
# (level = code - 8) and 6-bit (level = code - 32, the mode-2 planes) codes
# with one fp16 scale per (row, 128-group), computed on FP8 per-token
# activations (W4A8-g128 / W6A8-g128).
BANK_FORMATS: dict = {
    "fp8": ProjectionFormat(FP8_DTYPE, lambda k: k, torch.float32,
                            lambda n, k: ((n // FP8_BLOCK_SIZE, k // FP8_BLOCK_SIZE), (n, 1))),
    0: ProjectionFormat(torch.int32, lambda k: k // 8, torch.float16, lambda n, k: ((n, k // 128),)),
    1: ProjectionFormat(torch.int8, lambda k: k, torch.float32, lambda n, k: ((n, 1),)),
    2: ProjectionFormat(torch.int8, lambda k: 3 * k // 4, torch.uint8, lambda n, k: ((n, k // 16 + 4),)),
    3: ProjectionFormat(torch.int8, lambda k: k // 2, torch.uint8, lambda n, k: ((n, k // 16 + 8),)),
    4: ProjectionFormat(torch.int8, lambda k: k // 2, torch.float16, lambda n, k: ((n, k // 128),)),
    5: ProjectionFormat(torch.int8, lambda k: 3 * k // 4, torch.float16, lambda n, k: ((n, k // 128),)),
}
G128_MODES = (4, 5)


def check_bank_buffers(fmt, buffers: dict, experts: int, hidden: int, inter: int) -> None:
    """Check the four buffers of a bank of format ``fmt`` against the
    geometry (E, H, I): w13 holds [E, 2I, H] and w2 [E, H, I] in that
    format's storage.  Raises ValueError naming the first buffer whose element
    type or shape differs, or when the buffers span several devices."""
    spec = BANK_FORMATS[fmt]
    for prefix, n, k in (("w13", 2 * inter, hidden), ("w2", hidden, inter)):
        wanted = ((f"{prefix}_weight", spec.weight_dtype, ((experts, n, spec.weight_columns(k)),)),
                  (f"{prefix}_scale_inv", spec.scale_dtype,
                   tuple((experts, *shape) for shape in spec.scale_shapes(n, k))))
        for name, dtype, shapes in wanted:
            tensor = buffers[name]
            if tensor.dtype != dtype:
                raise ValueError(f"{name} must be {dtype}; got {tensor.dtype}")
            if tuple(tensor.shape) not in shapes:
                raise ValueError(f"{name} has shape {tuple(tensor.shape)}; expected "
                                 + " or ".join(str(s) for s in shapes))
    if len({t.device for t in buffers.values()}) != 1:
        raise ValueError("Expert bank tensors must share one device")


@dataclass(frozen=True)
class StagedExperts:
    """FP8 expert bank as handed to a backend (offload.py:175-184).

    w13_weight [S, 2I, H] e4m3, w13_scale_inv [S, 2I/128, H/128] fp32 (the
    reference's 128x128 block scales) or [S, 2I, 1] (one scale per output
    channel); w2_weight [S, H, I], w2_scale_inv [S, H/128, I/128] or [S, H, 1].
    Tensors may be strided; rows with a non-unit K stride are materialised
    contiguously once per bank object.
    """

    w13_weight: torch.Tensor
    w13_scale_inv: torch.Tensor
    w2_weight: torch.Tensor
    w2_scale_inv: torch.Tensor

    @property
    def count(self) -> int:
        return self.w13_weight.shape[0]

    @property
    def hidden(self) -> int:
        return self.w13_weight.shape[2]

    @property
    def intermediate(self) -> int:
        return self.w13_weight.shape[1] // 2

    @property
    def nbytes(self) -> int:
        return sum(getattr(self, n).numel() * getattr(self, n).element_size()
                   for n in EXPERT_BUFFER_NAMES)

    def buffers(self) -> dict:
        return {name: getattr(self, name) for name in EXPERT_BUFFER_NAMES}

    def validate(self) -> None:
        w13 = self.w13_weight
        if w13.ndim != 3:
            raise ValueError("w13_weight must be a stacked [experts, 2 * intermediate, hidden] tensor")
        experts, gate_up, hidden = w13.shape
        if experts < 1 or gate_up % 2 or hidden % FP8_BLOCK_SIZE or (gate_up // 2) % FP8_BLOCK_SIZE:
            raise ValueError("FP8 banks need at least one expert, and hidden and intermediate sizes "
                             "that are multiples of the FP8 block size")
        check_bank_buffers("fp8", self.buffers(), experts, hidden, gate_up // 2)

    @property
    def device(self) -> torch.device:
        return self.w13_weight.device


# The reference's host-resident store has the same four buffers; here it may
# live on the device too (all experts resident in HBM).
ExpertStore = StagedExperts


def _proj_struct(weight: torch.Tensor, scale: torch.Tensor, keep: list) -> _lib.Fp8Proj:
    w = weight.view(torch.uint8)
    if (w.stride(2) != 1 or w.stride(1) % 16 or w.stride(0) % 16 or w.data_ptr() % 16):
        w = w.contiguous()
    keep.append(w)
    e, n, k = w.shape
    return _lib.Fp8Proj(w.data_ptr(), scale.data_ptr(), w.stride(0), w.stride(1),
                        scale.stride(0), scale.stride(1), scale.stride(2),
                        scale.shape[1], scale.shape[2], n, k)


def fp8_bank_struct(staged: StagedExperts) -> _lib.Fp8Bank:
    """C descriptor of a bank, cached on the bank object (which keeps any
    contiguous copy alive)."""
    cached = getattr(staged, "_dmoe_struct", None)
    if cached is not None:
        return cached
    staged.validate()
    keep: list = []
    bank = _lib.Fp8Bank(_proj_struct(staged.w13_weight, staged.w13_scale_inv, keep),
                        _proj_struct(staged.w2_weight, staged.w2_scale_inv, keep), staged.count)
    object.__setattr__(staged, "_dmoe_keep", keep)
    object.__setattr__(staged, "_dmoe_struct", bank)
    return bank


# ------------------------------------------------------- synthetic FP8 banks

def quantize_fp8_weights(weight: torch.Tensor, layout: str = "block"):
    """Quantize fp32 weights [E, N, K] to E4M3 with 128x128 block scales
    (the reference layout, offload.py:44-56) or one scale per output channel.
    Returns (e4m3 weights, fp32 scales) with scale = amax / 448."""
    e, n, k = weight.shape
    w = weight.float()
    if layout == "block":
        blocks = w.view(e, n // 128, 128, k // 128, 128)
        scale = blocks.abs().amax(dim=(2, 4)).clamp_min(1e-12) / FP8_MAX
        q = (blocks / scale[:, :, None, :, None]).clamp(-FP8_MAX, FP8_MAX).to(FP8_DTYPE)
        return q.view(e, n, k), scale.contiguous()
    if layout == "channel":
        scale = w.abs().amax(dim=2, keepdim=True).clamp_min(1e-12) / FP8_MAX
        return (w / scale).clamp(-FP8_MAX, FP8_MAX).to(FP8_DTYPE), scale.contiguous()
    raise ValueError("layout must be 'block' or 'channel'")


def random_fp8_bank(experts: int, hidden: int, inter: int, *, layout: str = "block",
                    std: float = 0.02, generator: torch.Generator | None = None,
                    device="cpu") -> StagedExperts:
    """Seeded synthetic bank: weights ~ N(0, std) quantized to E4M3.  Drawn
    per expert to bound temporary memory."""
    parts = {name: [] for name in EXPERT_BUFFER_NAMES}
    for _ in range(experts):
        for prefix, rows, cols in (("w13", 2 * inter, hidden), ("w2", hidden, inter)):
            w = torch.randn(1, rows, cols, generator=generator, device=device) * std
            q, s = quantize_fp8_weights(w, layout)
            parts[prefix + "_weight"].append(q)
            parts[prefix + "_scale_inv"].append(s)
    return StagedExperts(**{k: torch.cat(v) for k, v in parts.items()})


# ------------------------------------------------------- packed quantized banks

def gptq_pack(codes: torch.Tensor) -> torch.Tensor:
    """[.., N, K] 4-bit codes -> [.., N, K/8] int32, nibble i of word w <-> k = 8w+i
    (tests/test_quantized_kernels.py:10-15)."""
    *lead, n, k = codes.shape
    c = codes.long().reshape(*lead, n, k // 8, 8)
    words = torch.zeros(*lead, n, k // 8, dtype=torch.int64, device=codes.device)
    for shift in range(8):
        words |= (c[..., shift] & 15) << (4 * shift)
    return (words - ((words >> 31) & 1) * (1 << 32)).to(torch.int32)


def zeros_pack(zeros: torch.Tensor) -> torch.Tensor:
    """Per-group 4-bit zero points [.., K/128, N] -> GPTQ qzeros [.., K/128, N/8]
    int32 (nibble i of word w <-> column n = 8w+i)."""
    return gptq_pack(zeros)


def six_pack(codes: torch.Tensor) -> torch.Tensor:
    """[.., N, K] 6-bit codes -> [.., N, 3K/4] int8: K/2 bytes of low nibbles
    (even k low) then K/4 bytes of 2-bit high parts, LSB first
    (tests/test_quantized_kernels.py:18-24)."""
    c = codes.long()
    low = (c[..., 0::2] & 15) | ((c[..., 1::2] & 15) << 4)
    high = torch.zeros(*c.shape[:-1], c.shape[-1] // 4, dtype=torch.int64, device=c.device)
    for shift in range(4):
        high |= (c[..., shift::4] >> 4) << (2 * shift)
    return torch.cat((low.to(torch.uint8), high.to(torch.uint8)), dim=-1).view(torch.int8)


def nibble_pack(codes: torch.Tensor) -> torch.Tensor:
    """[.., N, K] 4-bit codes -> [.., N, K/2] int8, even k in the low nibble
    (tests/test_quantized_kernels.py:53-54)."""
    c = codes.long()
    return ((c[..., 0::2] & 15) | ((c[..., 1::2] & 15) << 4)).to(torch.uint8).view(torch.int8)


@dataclass(frozen=True)
class QuantizedStore:
    """Packed expert bank of one mode (quantized_model.py:26-68):
    mode 0 W4A16 GPTQ, 1 INT8 ConvRot, 2 W6A8, 3 W4A8 codebook; ``w13_zeros`` /
    ``w2_zeros`` (GPTQ qzeros [E, K/128, N/8] int32) make mode 0 asymmetric.
    Modes 4 (W4A8-g128) and 5 (W6A8-g128) hold 4- / 6-bit codes with fp16
    scales per (row, 128-group) and run on FP8 per-token activations."""

    w13_weight: torch.Tensor
    w13_scale_inv: torch.Tensor
    w2_weight: torch.Tensor
    w2_scale_inv: torch.Tensor
    hidden: int
    intermediate: int
    mode: int
    w13_zeros: torch.Tensor | None = None
    w2_zeros: torch.Tensor | None = None

    @property
    def num_experts(self) -> int:
        return self.w13_weight.shape[0]

    count = num_experts

    @property
    def nbytes(self) -> int:
        total = sum(getattr(self, n).numel() * getattr(self, n).element_size()
                    for n in EXPERT_BUFFER_NAMES)
        for z in (self.w13_zeros, self.w2_zeros):
            if z is not None:
                total += z.numel() * z.element_size()
        return total

    def buffers(self) -> dict:
        return {name: getattr(self, name) for name in EXPERT_BUFFER_NAMES}

    def validate(self) -> None:
        if self.mode not in (0, 1, 2, 3, 4, 5):
            raise ValueError("Unknown quantized bank format")
        if self.w13_weight.ndim != 3:
            raise ValueError("Quantized banks are stacked [experts, rows, columns] tensors")
        check_bank_buffers(self.mode, self.buffers(), self.num_experts, self.hidden, self.intermediate)
        zero_points = {"w13_zeros": (self.w13_zeros, 2 * self.intermediate, self.hidden),
                       "w2_zeros": (self.w2_zeros, self.hidden, self.intermediate)}
        for name, (zeros, n, k) in zero_points.items():
            if zeros is None:
                continue
            if self.mode != 0:
                raise ValueError("Zero points apply to W4A16 banks only")
            if zeros.dtype != torch.int32 or tuple(zeros.shape) != (self.num_experts, k // 128, n // 8):
                raise ValueError(f"{name} must be GPTQ qzeros [E, K/128, N/8] int32")


def random_quantized_bank(mode: int, experts: int, hidden: int, inter: int, *,
                          asymmetric: bool = False, generator=None, device="cpu") -> QuantizedStore:
    """Seeded synthetic packed bank of one mode with random codes and scales of
    realistic magnitude (outputs stay O(1) for N(0, 1) activations)."""
    def rand(*shape):
        return torch.rand(*shape, generator=generator, device=device)

    def randint(high, *shape):
        return torch.randint(0, high, shape, generator=generator, device=device)

    tensors = {}
    for prefix, n, k in (("w13", 2 * inter, hidden), ("w2", hidden, inter)):
        if mode in G128_MODES:
            codes = randint(16 if mode == 4 else 64, experts, n, k)
            tensors[prefix + "_weight"] = nibble_pack(codes) if mode == 4 else six_pack(codes)
            levels = 7.5 if mode == 4 else 31.5  # largest |level| of the format
            tensors[prefix + "_scale_inv"] = ((rand(experts, n, k // 128) * 0.5 + 0.75)
                                              * (0.02 * 2.5 / levels)).half()
        elif mode == 0:
            codes = randint(16, experts, n, k)
            tensors[prefix + "_weight"] = gptq_pack(codes)
            tensors[prefix + "_scale_inv"] = ((rand(experts, n, k // 128) * 0.5 + 0.75)
                                              * (0.02 * 2.5 / 8)).half()
            if asymmetric:
                tensors[prefix + "_zeros"] = zeros_pack(randint(16, experts, k // 128, n))
        elif mode == 1:
            tensors[prefix + "_weight"] = (randint(255, experts, n, k) - 127).to(torch.int8)
            tensors[prefix + "_scale_inv"] = (rand(experts, n, 1) * 0.5 + 0.75) * (0.02 * 2.5 / 127)
        else:
            codes = randint(64 if mode == 2 else 16, experts, n, k)
            bank = six_pack(codes) if mode == 2 else nibble_pack(codes)
            relative = (rand(experts, n, k // 16) + 1).to(FP8_DTYPE)
            channel = (rand(experts, n, 1) * 0.5 + 0.75) * (0.02 * 2.5 / 64)
            if mode == 3:
                table = torch.linspace(-60, 60, 16, device=device)
                aux = torch.zeros(experts, n, k // 16 + 8, dtype=torch.uint8, device=device)
                aux[..., :k // 16] = relative.view(torch.uint8)
                aux[..., k // 16:k // 16 + 4] = channel.contiguous().view(torch.uint8)
                aux[:, :16, k // 16 + 4:] = table.repeat(experts, 1).contiguous().view(torch.uint8).reshape(experts, 16, 4)
            else:
                aux = torch.cat((relative.view(torch.uint8), channel.contiguous().view(torch.uint8)), dim=-1)
            tensors[prefix + "_weight"] = bank
            tensors[prefix + "_scale_inv"] = aux
    return QuantizedStore(**tensors, hidden=hidden, intermediate=inter, mode=mode)


def as_ctypes_bank(bank: _lib.Fp8Bank):
    return ctypes.byref(bank)
