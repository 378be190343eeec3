"""Torch-CPU restatement of the reference's dequantize-then-matmul expert paths
-- TEST INFRASTRUCTURE / CPU BASELINE ONLY (never on the product path).

* ``projection`` follows projection_torch (src/drama_low_vram/quantized_kernels.py:
  48-112): modes 1-3 rotate the activation rows by H4^{x4}/16 and quantize
  them to INT8 per row in fp32, mode 0 keeps them; each used expert's weight
  matrix is reconstructed in fp32 (mode 0 rounded through the activation
  dtype), multiplied with F.linear in fp32, rounded to bf16 at the
  projection boundary and optionally scaled by the route weight.
* ``layer`` is QuantizedExpertBackend.forward (quantized_kernels.py:217-229):
  gate/up projection, bf16(bf16(silu(gate)) * up), weighted down
  projection, fp32 sum over the route slots.
* ``fp8_layer`` is TorchExpertBackend.forward (offload.py:199-244) on
  dequantize_fp8_blocks (offload.py:44-56).
* Modes 4 / 5 (the group-128 integer formats, no reference counterpart)
  reconstruct level * fp16 group scale and multiply unquantized activations.

bench.py times these with torch's CPU threads as the reference's CPU lane for
the packed formats; tests/test_oracle.py pins them against the C oracle.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

_H256 = {}


def _h256(dtype):
    if dtype not in _H256:
        h4 = torch.tensor([[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]], dtype=dtype)
        m = h4
        for _ in range(3):
            m = torch.kron(m, h4)
        _H256[dtype] = m / 16.0
    return _H256[dtype]


def _e4m3_values():
    return torch.arange(256, dtype=torch.int64).to(torch.uint8).view(torch.float8_e4m3fn).float()


def dequantize(mode: int, weight: torch.Tensor, scale: torch.Tensor, k: int, dtype=torch.bfloat16,
               zeros: torch.Tensor | None = None) -> torch.Tensor:
    """fp32 weight matrix [N, K] of one expert of a packed bank."""
    n = weight.shape[0]
    if mode == 0:
        words = weight.long() & 0xFFFFFFFF
        code = ((words[..., None] >> (torch.arange(8) * 4)) & 15).reshape(n, k).float()
        if zeros is None:
            zp = torch.full((k // 128, n), 8.0)
        else:
            zw = zeros.long() & 0xFFFFFFFF
            zp = ((zw[..., None] >> (torch.arange(8) * 4)) & 15).reshape(k // 128, n).float()
        zp = zp.t().repeat_interleave(128, -1)
        return ((code - zp) * scale.float().repeat_interleave(128, -1)).to(dtype).float()
    if mode == 1:
        return weight.float() * scale.float()
    raw = weight.view(torch.uint8)
    low = raw[:, :k // 2]
    code = torch.stack((low & 15, low >> 4), -1).reshape(n, k).long()
    if mode in (2, 5):
        high = raw[:, k // 2:].long()
        high = ((high[..., None] >> (torch.arange(4) * 2)) & 3).reshape(n, k)
        code = code | (high << 4)
    if mode in (4, 5):
        level = code.float() - (8 if mode == 4 else 32)
        return level * scale.float().repeat_interleave(128, -1)
    if mode == 3:
        level = scale[:16, k // 16 + 4:].contiguous().view(torch.float32).reshape(16)[code]
    else:
        level = code.float() - 32
    relative = _e4m3_values()[scale[:, :k // 16].long()]
    channel = scale[:, k // 16:k // 16 + 4].contiguous().view(torch.float32)
    return (level * relative.repeat_interleave(16, -1)).round().clamp(-127, 127) * channel


def projection(x, ids, weights, weight, scale, *, mode, k, shared=False, weighted=False, zeros=None):
    """[pairs, N]: bf16 projection boundary, fp32 * route weight when weighted."""
    ids = ids.reshape(-1)
    if mode in (1, 2, 3):
        rotated = torch.matmul(x.reshape(-1, 256), _h256(x.dtype)).reshape(x.shape).float()
        act_scale = rotated.abs().amax(1).clamp_min(1e-12) / 127
        inputs = (rotated / act_scale[:, None]).round().clamp(-127, 127)
    else:
        inputs = x.float()
    out = torch.empty((ids.numel(), weight.shape[1]), dtype=torch.float32)
    for expert in torch.unique(ids).tolist():
        rows = torch.nonzero(ids == expert).reshape(-1)
        matrix = dequantize(mode, weight[expert], scale[expert], k, x.dtype,
                            None if zeros is None else zeros[expert])
        src = torch.zeros_like(rows) if shared else rows
        values = F.linear(inputs.index_select(0, src), matrix)
        if mode in (1, 2, 3):
            values *= act_scale.index_select(0, src)[:, None]
        values = values.to(torch.bfloat16).float()
        if weighted:
            values *= weights.reshape(-1).index_select(0, rows).float()[:, None]
        out.index_copy_(0, rows, values)
    return out


def layer(store, x, ids, weights):
    """Routed experts of a packed bank for x [T, H] (one row per token)."""
    tokens, top_k = ids.shape
    inter, hidden = store.intermediate, store.hidden
    rows = x.repeat_interleave(top_k, dim=0)
    up = projection(rows, ids, None, store.w13_weight, store.w13_scale_inv, mode=store.mode, k=hidden,
                    zeros=store.w13_zeros)
    act = (F.silu(up[:, :inter].to(torch.bfloat16)) * up[:, inter:].to(torch.bfloat16)).to(torch.bfloat16)
    part = projection(act, ids, weights, store.w2_weight, store.w2_scale_inv, mode=store.mode, k=inter,
                      weighted=True, zeros=store.w2_zeros)
    return part.view(tokens, top_k, hidden).sum(1).to(x.dtype)


def fp8_layer(staged, x, ids, weights):
    """TorchExpertBackend.forward: per used expert the 128x128-block
    dequantized weights in x.dtype, F.linear, silu(gate) * up, weighted fp32."""
    tokens, top_k = ids.shape
    rows = x.repeat_interleave(top_k, dim=0)
    flat = ids.reshape(-1)
    out = torch.empty((flat.numel(), x.shape[1]), dtype=torch.float32)

    def deq(w, s):
        v = w.view(torch.uint8).to(torch.int64)
        n, k = v.shape
        vals = _e4m3_values()[v].view(n // 128, 128, k // 128, 128) * s[:, None, :, None]
        return vals.reshape(n, k).to(x.dtype)

    for expert in torch.unique(flat).tolist():
        sel = torch.nonzero(flat == expert).reshape(-1)
        gate, up = F.linear(rows.index_select(0, sel), deq(staged.w13_weight[expert],
                                                           staged.w13_scale_inv[expert])).chunk(2, dim=-1)
        values = F.linear(F.silu(gate) * up, deq(staged.w2_weight[expert], staged.w2_scale_inv[expert]))
        out.index_copy_(0, sel, values.float() * weights.reshape(-1).index_select(0, sel).float()[:, None])
    return out.view(tokens, top_k, -1).sum(1).to(x.dtype)
