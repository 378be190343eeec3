"""The MoE block of a Drama 3 decoder layer around the routed experts.

BackboneDecodeGraph splits a decoder layer's MoE half into _route_impl (router
softmax / top-k on ``moe.gate(flat)``), _shared_impl (the sigmoid-gated shared
expert) and _post_impl (``after_mixer + (experts + shared)``)
(src/drama_low_vram/backbone_graph.py:300-337).  ``MoeBlock`` runs the same
three steps on the GPU with no host sync (so a decode step is hipGraph
capturable): one launch for the router logits, shared gate and shared
gate/up (``dmoe_moe_block_pre``), the routed experts through the FP8 or packed
backend (``forward_routed``), and one launch for the shared down projection,
gating and residual adds (``dmoe_moe_block_post``).  Weights and rows are
bf16, the reference's compute dtype for these modules.
"""
from __future__ import annotations

import torch
from torch import Tensor

from . import _lib
from .formats import QuantizedStore, StagedExperts


def _bf16_rows(t: Tensor, name: str, cols: int, rows: int | None = None) -> Tensor:
    if t.dtype != torch.bfloat16 or t.ndim != 2 or t.shape[1] != cols or (rows is not None and t.shape[0] != rows):
        raise ValueError(f"{name} must be bf16 [{rows if rows is not None else 'rows'}, {cols}]")
    if t.stride(1) != 1 or (t.stride(0) * 2) % 16 or t.data_ptr() % 16:
        t = t.contiguous()
    return t


class MoeBlock:
    """Router GEMV + top-k, routed experts, sigmoid-gated shared expert and
    residual adds of one decoder layer (``SparseMoeBlock`` with a shared
    expert, as backbone_graph.py:317-337 drives it).

    ``router_weight`` [E, H] is ``moe.gate.weight``; ``shared_gate_weight``
    [1, H] ``moe.shared_expert_gate.weight``; ``gate_proj`` / ``up_proj``
    [I_s, H] and ``down_proj`` [H, I_s] the shared expert's weights;
    ``experts`` the routed bank (``StagedExperts`` for FP8, ``QuantizedStore``
    for the packed formats) and ``backend`` the matching expert backend.
    """

    def __init__(self, router_weight: Tensor, shared_gate_weight: Tensor, gate_proj: Tensor, up_proj: Tensor,
                 down_proj: Tensor, experts: StagedExperts | QuantizedStore, backend, *, top_k: int,
                 norm_topk_prob: bool = True):
        hidden = router_weight.shape[-1]
        inter = gate_proj.shape[0]
        self.router_weight = _bf16_rows(router_weight, "router weight", hidden)
        self.shared_gate_weight = _bf16_rows(shared_gate_weight.reshape(1, -1), "shared gate weight", hidden, 1)
        self.gate_proj = _bf16_rows(gate_proj, "shared gate_proj", hidden, inter)
        self.up_proj = _bf16_rows(up_proj, "shared up_proj", hidden, inter)
        self.down_proj = _bf16_rows(down_proj, "shared down_proj", inter, hidden)
        self.experts = experts
        self.backend = backend
        self.top_k = int(top_k)
        self.norm_topk_prob = bool(norm_topk_prob)
        self.hidden, self.shared_inter = hidden, inter
        self.num_experts = self.router_weight.shape[0]

    def pre(self, mlp_input: Tensor):
        """(router logits [T, E] fp32, shared gate [T] bf16, shared act [T, I_s] bf16)."""
        x = _bf16_rows(mlp_input, "MoE input", self.hidden)
        tokens = x.shape[0]
        logits = torch.empty((tokens, self.num_experts), dtype=torch.float32, device=x.device)
        sgate = torch.empty(tokens, dtype=torch.bfloat16, device=x.device)
        act = torch.empty((tokens, self.shared_inter), dtype=torch.bfloat16, device=x.device)
        if tokens == 0:
            return logits, sgate, act
        lib = _lib.library()
        _lib.check(lib.dmoe_moe_block_pre(
            _lib.ptr(x), x.stride(0), tokens, self.hidden, _lib.ptr(self.router_weight), self.router_weight.stride(0),
            self.num_experts, _lib.ptr(self.shared_gate_weight), _lib.ptr(self.gate_proj), self.gate_proj.stride(0),
            _lib.ptr(self.up_proj), self.up_proj.stride(0), self.shared_inter, _lib.ptr(logits), logits.stride(0),
            _lib.ptr(sgate), _lib.ptr(act), act.stride(0), _lib.stream_handle(x.device)))
        return logits, sgate, act

    def post(self, act: Tensor, sgate: Tensor, experts_out: Tensor, after_mixer: Tensor,
             out: Tensor | None = None) -> Tensor:
        """after_mixer + (experts_out + sgate * shared down projection), bf16."""
        residual = _bf16_rows(after_mixer, "after_mixer", self.hidden)
        experts_out = _bf16_rows(experts_out, "experts output", self.hidden, residual.shape[0])
        if out is None:
            out = torch.empty_like(residual)
        elif (out.dtype != torch.bfloat16 or tuple(out.shape) != tuple(residual.shape) or out.stride(1) != 1
              or (out.stride(0) * 2) % 16 or out.data_ptr() % 16 or out.device != residual.device):
            # the kernel writes the caller's buffer itself: a substitute copy
            # would leave it unwritten (and allocate inside a graph capture)
            raise ValueError(f"out must be bf16 [{residual.shape[0]}, {self.hidden}] on the input's device with "
                             "contiguous, 16-byte aligned rows")
        if residual.shape[0] == 0:
            return out
        lib = _lib.library()
        _lib.check(lib.dmoe_moe_block_post(
            _lib.ptr(act), act.stride(0), residual.shape[0], self.shared_inter, _lib.ptr(self.down_proj),
            self.down_proj.stride(0), self.hidden, _lib.ptr(sgate), _lib.ptr(experts_out), experts_out.stride(0),
            _lib.ptr(residual), residual.stride(0), _lib.ptr(out), out.stride(0), _lib.stream_handle(residual.device)))
        return out

    def forward(self, mlp_input: Tensor, after_mixer: Tensor, out: Tensor | None = None):
        """The layer's output after its MoE half, plus the routing:
        (out [T, H] bf16, topk_weights [T, k], topk_ids [T, k])."""
        if mlp_input.shape != after_mixer.shape:
            raise ValueError("mlp_input and after_mixer must have the same shape")
        logits, sgate, act = self.pre(mlp_input)
        if mlp_input.shape[0] == 0:
            empty = torch.empty((0, self.top_k), device=mlp_input.device)
            out = self.post(act, sgate, torch.empty_like(after_mixer), after_mixer, out=out)
            return out, empty.to(mlp_input.dtype), empty.long()
        experts_out, weights, ids = self.backend.forward_routed(mlp_input, logits, self.top_k, self.experts,
                                                                renormalize=self.norm_topk_prob)
        return self.post(act, sgate, experts_out, after_mixer, out=out), weights, ids

    __call__ = forward
