"""Packed-integer expert banks (W4A16 GPTQ, INT8 ConvRot, W6A8, W4A8 codebook)
on the gfx950 kernels, with the reference's interface
(src/drama_low_vram/quantized_kernels.py:30-45, 192-260):
``rotate_quantize(x)``, ``projection(x, ids, weights, bank, scales, *, mode,
shared=False, weighted=False)`` and ``QuantizedExpertBackend(mode)`` with
``forward`` / ``forward_pairs``.  Banks are ``formats.QuantizedStore``.
There is no CPU path: a missing library or a non-ROCm device raises.
"""
from __future__ import annotations

import ctypes

import torch
from torch import Tensor

from . import _lib
from .formats import QuantizedStore
from .offload import MAX_PAIRS, _device_of, device_state

MODE_NAMES = ("W4A16-GPTQ", "INT8-ConvRot/BF16", "W6A8/BF16", "W4A8-Codebook/BF16", "W4A8-G128/FP8",
              "W6A8-G128/FP8")


class QuantProj(ctypes.Structure):
    _fields_ = [("weight", ctypes.c_void_p), ("scale", ctypes.c_void_p), ("zeros", ctypes.c_void_p),
                ("weight_stride_e", ctypes.c_int64), ("weight_stride_n", ctypes.c_int64),
                ("scale_stride_e", ctypes.c_int64), ("scale_stride_n", ctypes.c_int64),
                ("zeros_stride_e", ctypes.c_int64), ("n", ctypes.c_int32), ("k", ctypes.c_int32)]


class QuantBank(ctypes.Structure):
    _fields_ = [("w13", QuantProj), ("w2", QuantProj), ("experts", ctypes.c_int32), ("mode", ctypes.c_int32)]


def _k_of(bank: Tensor, mode: int) -> int:
    cols = bank.shape[-1]
    return cols * 8 if mode == 0 else cols if mode == 1 else cols * 4 // 3 if mode in (2, 5) else cols * 2


def _bytes_stride(t: Tensor, dim: int) -> int:
    return t.stride(dim) * t.element_size()


def proj_struct(bank: Tensor, scales: Tensor, mode: int, zeros: Tensor | None = None) -> QuantProj:
    """Descriptor of one packed projection bank [E, N, cols] (+ scales, zeros)."""
    if bank.ndim != 3 or scales.ndim != 3 or bank.stride(-1) != 1 or scales.stride(-1) != 1:
        raise ValueError("Packed bank and scales must be [E, N, columns] with contiguous rows")
    if zeros is not None and (not zeros.is_contiguous() or zeros.dtype != torch.int32):
        raise ValueError("W4A16 zero points must be contiguous int32 [E, K/128, N/8]")
    return QuantProj(bank.data_ptr(), scales.data_ptr(), zeros.data_ptr() if zeros is not None else None,
                     _bytes_stride(bank, 0), _bytes_stride(bank, 1), _bytes_stride(scales, 0),
                     _bytes_stride(scales, 1), zeros.stride(0) if zeros is not None else 0,
                     bank.shape[1], _k_of(bank, mode))


def bank_struct(store: QuantizedStore) -> QuantBank:
    return QuantBank(proj_struct(store.w13_weight, store.w13_scale_inv, store.mode, store.w13_zeros),
                     proj_struct(store.w2_weight, store.w2_scale_inv, store.mode, store.w2_zeros),
                     store.num_experts, store.mode)


def rotate_quantize(x: Tensor):
    """(q int8 [rows, K], scale fp32 [rows]) of the ConvRot rotation of x rows
    (quantized_kernels.py:30-45)."""
    if x.ndim != 2 or x.stride(-1) != 1:
        raise ValueError("rotate_quantize expects [rows, K] rows with contiguous columns")
    _device_of(x)
    q = torch.empty(x.shape, dtype=torch.int8, device=x.device)
    scale = torch.empty(x.shape[0], dtype=torch.float32, device=x.device)
    _lib.check(_lib.library().dmoe_rotate_quantize(
        _lib.ptr(x), _lib.dtype_code(x.dtype), x.stride(0), x.shape[0], x.shape[1], _lib.ptr(q), _lib.ptr(scale),
        _lib.stream_handle(x.device)))
    return q, scale


def projection(x: Tensor, ids: Tensor, weights: Tensor, bank: Tensor, scales: Tensor, *, mode: int,
               shared: bool = False, weighted: bool = False, tile=None, zeros: Tensor | None = None) -> Tensor:
    """[pairs, N] = bf16(x_p . W[ids_p]^T) (bf16), or fp32 * weights_p when
    ``weighted`` (quantized_kernels.py:192-214).  ``shared`` reads row 0 for
    every pair; ``tile`` is accepted for interface parity and ignored."""
    device = _device_of(x)
    ids = ids.reshape(-1).contiguous()
    weights = weights.reshape(-1).contiguous()
    pairs = ids.numel()
    desc = proj_struct(bank, scales, mode, zeros)
    out = torch.empty((pairs, desc.n), dtype=torch.float32 if weighted else torch.bfloat16, device=device)
    if pairs == 0:
        return out
    if x.stride(-1) != 1:
        x = x.contiguous()
    rows = x.shape[0]
    if not shared and rows != pairs:
        raise ValueError("projection expects one activation row per pair unless shared")
    row_div = pairs if shared else 1
    lib = _lib.library()
    state = device_state(device)
    ws = state.workspace_for(lib.dmoe_quant_projection_workspace_bytes(bank.shape[0], desc.k, rows, pairs))
    _lib.check(lib.dmoe_quant_projection(
        ctypes.byref(desc), bank.shape[0], mode, _lib.ptr(x), _lib.dtype_code(x.dtype), x.stride(0), rows,
        row_div, _lib.ptr(ids), _lib.dtype_code(ids.dtype), _lib.ptr(weights), _lib.dtype_code(weights.dtype),
        pairs, int(weighted), _lib.ptr(out), out.stride(0), _lib.ptr(ws), ws.numel(),
        _lib.ptr(state.status), _lib.stream_handle(device)))
    return out


class QuantizedExpertBackend:
    """Routed experts of a packed bank (quantized_kernels.py:217-260): gate/up
    projection, bf16 silu(gate) * up, down projection * route weight, slot-order
    combine.  Never synchronizes the host."""

    def __init__(self, mode: int) -> None:
        if mode not in (0, 1, 2, 3, 4, 5):
            raise ValueError("Unknown quantized bank format")
        self.mode = mode
        self.quantized_mode = MODE_NAMES[mode]
        self.tuned_tiles = True

    @staticmethod
    def status(device=None, clear: bool = True) -> int:
        """Read (and clear) the device status bits; synchronizes the stream."""
        state = device_state(torch.device(device) if device is not None else
                             torch.device("cuda", torch.cuda.current_device()))
        value = int(state.status.item())
        if clear:
            state.status.zero_()
        return value

    def _call(self, x: Tensor, ids: Tensor, weights: Tensor, staged: QuantizedStore, *, rows: int,
              row_div: int, top_k: int, out: Tensor | None, out_pairs: Tensor | None) -> None:
        if staged.mode != self.mode:
            raise ValueError(f"Bank is mode {staged.mode}, backend is mode {self.mode}")
        if x.shape[-1] != staged.hidden or x.stride(-1) != 1:
            raise ValueError(f"Expected hidden rows [N, {staged.hidden}] with contiguous columns")
        device = _device_of(x)
        bank = bank_struct(staged)
        lib = _lib.library()
        state = device_state(device)
        pairs = ids.numel()
        ws = state.workspace_for(lib.dmoe_quant_workspace_bytes(ctypes.byref(bank), rows, pairs))
        _lib.check(lib.dmoe_quant_moe_forward(
            ctypes.byref(bank), _lib.ptr(x), _lib.dtype_code(x.dtype), x.stride(0), rows, row_div,
            _lib.ptr(ids), _lib.dtype_code(ids.dtype), _lib.ptr(weights), _lib.dtype_code(weights.dtype), pairs,
            top_k, _lib.ptr(out), _lib.dtype_code(out.dtype) if out is not None else _lib.F32,
            out.stride(0) if out is not None else 0, _lib.ptr(out_pairs), _lib.ptr(ws), ws.numel(),
            _lib.ptr(state.status), _lib.stream_handle(device)))

    def forward(self, x: Tensor, ids: Tensor, weights: Tensor, staged: QuantizedStore, *,
                out: Tensor | None = None) -> Tensor:
        if x.ndim != 2 or ids.ndim != 2 or ids.shape[0] != x.shape[0] or weights.shape != ids.shape:
            raise ValueError("Expected x [T, H], ids and weights [T, top_k]")
        tokens, top_k = ids.shape
        if out is None:
            out = torch.empty_like(x)
        if tokens == 0:
            return out
        ids, weights = ids.contiguous(), weights.contiguous()
        chunk = max(1, MAX_PAIRS // top_k)
        for start in range(0, tokens, chunk):
            stop = min(tokens, start + chunk)
            self._call(x[start:stop], ids[start:stop], weights[start:stop], staged, rows=stop - start,
                       row_div=top_k, top_k=top_k, out=out[start:stop], out_pairs=None)
        return out

    def forward_pairs(self, x: Tensor, ids: Tensor, weights: Tensor, staged: QuantizedStore) -> Tensor:
        """Weighted [pairs, hidden] fp32 contributions before summing."""
        if ids.shape != (x.shape[0], 1) or weights.shape != ids.shape:
            raise ValueError("Pair backend expects one expert and weight per input row")
        pairs = ids.shape[0]
        out = torch.empty((pairs, staged.hidden), dtype=torch.float32, device=x.device)
        ids, weights = ids.reshape(-1).contiguous(), weights.reshape(-1).contiguous()
        for start in range(0, pairs, MAX_PAIRS):
            stop = min(pairs, start + MAX_PAIRS)
            self._call(x[start:stop], ids[start:stop], weights[start:stop], staged, rows=stop - start, row_div=1,
                       top_k=1, out=None, out_pairs=out[start:stop])
        return out

    forward_decode_pairs = forward_pairs

    def forward_routed(self, x: Tensor, logits: Tensor, top_k: int, staged: QuantizedStore, *,
                       renormalize: bool = True, weights_dtype: torch.dtype | None = None,
                       out: Tensor | None = None):
        """Router + routed experts in one call with no host sync (graph
        capturable): returns (out [T, H], weights [T, top_k], ids [T, top_k])."""
        if x.ndim != 2 or logits.ndim != 2 or logits.shape[0] != x.shape[0]:
            raise ValueError("Expected x [T, H] and router logits [T, E]")
        if staged.mode != self.mode:
            raise ValueError(f"Bank is mode {staged.mode}, backend is mode {self.mode}")
        if x.shape[-1] != staged.hidden or x.stride(-1) != 1:
            raise ValueError(f"Expected hidden rows [N, {staged.hidden}] with contiguous columns")
        if logits.dtype != torch.float32 or logits.stride(-1) != 1:
            logits = logits.float().contiguous()
        device = _device_of(x)
        tokens = x.shape[0]
        out = torch.empty_like(x) if out is None else out
        ids = torch.empty((tokens, top_k), dtype=torch.int64, device=device)
        weights = torch.empty((tokens, top_k), dtype=weights_dtype or x.dtype, device=device)
        if tokens == 0:
            return out, weights, ids
        bank = bank_struct(staged)
        lib = _lib.library()
        state = device_state(device)
        ws = state.workspace_for(lib.dmoe_quant_workspace_bytes(ctypes.byref(bank), tokens, tokens * top_k))
        _lib.check(lib.dmoe_quant_moe_layer(
            ctypes.byref(bank), _lib.ptr(x), _lib.dtype_code(x.dtype), x.stride(0), tokens, _lib.ptr(logits),
            logits.stride(0), top_k, int(renormalize), _lib.ptr(ids), _lib.ptr(weights),
            _lib.dtype_code(weights.dtype), _lib.ptr(out), _lib.dtype_code(out.dtype), out.stride(0), _lib.ptr(ws),
            ws.numel(), _lib.ptr(state.status), _lib.stream_handle(device)))
        return out, weights, ids


class GPTQLinear(torch.nn.Module):
    """Dense W4A16 linear kept compressed on the GPU, the reference's
    GPTQLinear (src/drama_low_vram/quantized_model.py:71-91): GPTQ ``weight``
    [K/8, N] int32 and ``scales`` [K/128, N] fp16 are stored transposed
    (``qweight`` [N, K/8], ``scales`` [N, K/128]); ``forward`` multiplies rows
    of x (bf16 or fp16, any leading shape) by the dequantized matrix with the
    tiled W4A16 kernel (dmoe_w4a16_linear) and returns bf16 [..., N], as the
    reference's projection(mode=0) over one expert does."""

    def __init__(self, weight: Tensor, scales: Tensor, *, device, dtype=torch.bfloat16):
        super().__init__()
        if weight.dtype != torch.int32 or weight.ndim != 2:
            raise ValueError("GPTQ qweight must be int32 [K/8, N]")
        if scales.dtype != torch.float16 or scales.shape != (weight.shape[0] * 8 // 128, weight.shape[1]):
            raise ValueError("GPTQ scales must be fp16 [K/128, N]")
        self.in_features, self.out_features = weight.shape[0] * 8, weight.shape[1]
        self.register_buffer("qweight", weight.T.contiguous().to(device))
        self.register_buffer("scales", scales.T.contiguous().to(device))
        self.register_buffer("_anchor", torch.empty(0, device=device, dtype=dtype))

    @property
    def weight(self):
        return self._anchor

    def forward(self, x: Tensor) -> Tensor:
        if x.dtype not in (torch.bfloat16, torch.float16):
            raise ValueError("GPTQLinear inputs must be bf16 or fp16")
        shape = x.shape
        flat = x.reshape(-1, shape[-1])
        if flat.stride(-1) != 1 or (flat.stride(0) * 2) % 16 or flat.data_ptr() % 16:
            flat = flat.contiguous()
        out = torch.empty((flat.shape[0], self.out_features), dtype=torch.bfloat16, device=x.device)
        if flat.shape[0]:
            _lib.check(_lib.library().dmoe_w4a16_linear(
                _lib.ptr(flat), _lib.dtype_code(flat.dtype), flat.stride(0), flat.shape[0], _lib.ptr(self.qweight),
                self.qweight.stride(0), _lib.ptr(self.scales), self.scales.stride(0), self.out_features,
                self.in_features, _lib.ptr(out), out.stride(0), _lib.stream_handle(x.device)))
        return out.reshape(*shape[:-1], self.out_features)
