"""Host residency on the GPU: banks kept in pinned host memory, routed
experts staged into device slots per call, through the real FP8 and W4A16
kernels.  Calls that fit one set of slots give bit-for-bit the resident
output; grouped calls give bit-for-bit the resident per-pair contributions
added in slot order, and match the resident output within the FP8 bar."""
from __future__ import annotations

import pytest
import torch
from torch import nn

from conftest import print_case
from drama_moe import offload, staging
from drama_moe.formats import random_fp8_bank, random_quantized_bank
from drama_moe.offload import HipExpertBackend
from drama_moe.quantized import QuantizedExpertBackend

pytestmark = pytest.mark.gpu

HIDDEN, INTER, EXPERTS = 512, 256, 32


def route(tokens, top_k, g, device):
    ids = torch.stack([torch.randperm(EXPERTS, generator=g)[:top_k] for _ in range(tokens)]).to(torch.int32)
    weights = torch.softmax(torch.randn(tokens, top_k, generator=g), -1)
    x = torch.randn(tokens, HIDDEN, generator=g).bfloat16()
    return x.to(device), ids.to(device), weights.to(device)


def slot_order_sum(pairs, tokens, top_k):
    view = pairs.view(tokens, top_k, -1)
    total = view[:, 0].clone()
    for s in range(1, top_k):
        total += view[:, s]
    return total


@pytest.mark.parametrize("mode", ["fp8", 0, 1, 2, 3, 4])
def test_host_resident_calls_match_the_resident_bank(cuda, mode):
    print_case("host residency", mode)
    g = torch.Generator().manual_seed(501)
    if mode == "fp8":
        bank, backend = random_fp8_bank(EXPERTS, HIDDEN, INTER, layout="channel", generator=g), HipExpertBackend()
    else:
        bank = random_quantized_bank(mode, EXPERTS, HIDDEN, INTER, asymmetric=mode == 0, generator=g)
        backend = QuantizedExpertBackend(mode)
    resident = staging.device_copy(bank, cuda)
    tier = staging.HostResidency(max_staged_experts=8, max_pair_rows=64, cache_experts=6)
    # decode tokens through the hot cache (and the pool for the overflow), then
    # a short prompt that fits the pool, then one that needs grouped calls
    for step, (tokens, top_k) in enumerate([(1, 4), (1, 4), (1, 8), (3, 2), (12, 4), (40, 8)]):
        x, ids, weights = route(tokens, top_k, g, cuda)
        before = tier.grouped_calls
        got = tier.forward("layer", bank, backend, x, ids, weights)
        torch.cuda.synchronize()
        want = backend.forward(x, ids, weights, resident)
        pairs = backend.forward_pairs(x.repeat_interleave(top_k, 0), ids.reshape(-1, 1), weights.reshape(-1, 1),
                                      resident)
        grouped = slot_order_sum(pairs, tokens, top_k).to(x.dtype)
        torch.cuda.synchronize()
        assert torch.equal(got, grouped if tier.grouped_calls > before else want), step
        err = (got.float() - want.float()).abs().max() / want.float().abs().max()
        assert err < 2e-2, step
    stats = tier.stats()
    assert stats["grouped_calls"] >= 1 and stats["cache_hits"] >= 0 and stats["pool_loads"] > 0


class FP8Experts(nn.Module):
    def __init__(self, bank):
        super().__init__()
        for name, t in staging.bank_buffers(bank).items():
            self.register_buffer(name, t)
        self.fp8 = True


def test_manager_residency_modes_agree(cuda):
    print_case("manager residency modes")
    g = torch.Generator().manual_seed(502)
    bank = random_fp8_bank(EXPERTS, HIDDEN, INTER, layout="channel", generator=g)
    outputs = {}
    for residency in ("hbm", "host"):
        model = nn.ModuleDict({"experts": FP8Experts(bank)})  # banks left in host memory
        manager = offload.install_expert_offload(model, residency=residency, max_staged_experts=8)
        gg = torch.Generator().manual_seed(9)
        outputs[residency] = [model["experts"](*route(t, 4, gg, cuda)) for t in (1, 2)]
        manager.close()
    torch.cuda.synchronize()
    for a, b in zip(outputs["hbm"], outputs["host"]):
        assert torch.equal(a, b)


def test_profiled_transfers_report_event_time(cuda):
    """profile_transfers times the host tier's copies with HIP events
    (test_offload.py:903-947: h2d_seconds > 0 after staged calls); without it
    the event time stays 0 and the byte counts are the same."""
    print_case("host tier transfer profiling")
    g = torch.Generator().manual_seed(503)
    bank = random_fp8_bank(EXPERTS, HIDDEN, INTER, layout="channel", generator=g)
    per_expert = sum(t[0].numel() * t.element_size() for t in staging.bank_buffers(bank).values())
    seen = {}
    for profile in (False, True):
        model = nn.ModuleDict({"experts": FP8Experts(bank)})
        manager = offload.install_expert_offload(model, residency="host", max_staged_experts=8, cache_experts=4,
                                                 profile_transfers=profile)
        gg = torch.Generator().manual_seed(10)
        for tokens in (1, 1, 3):
            model["experts"](*route(tokens, 4, gg, cuda))
        torch.cuda.synchronize()
        st = manager.stats
        seen[profile] = st.h2d_bytes
        assert st.h2d_bytes == (st.expert_loads + st.hot_cache_loads) * per_expert
        assert st.pinned_bytes == bank.nbytes
        assert (st.h2d_seconds > 0) == profile
        manager.close()
    assert seen[False] == seen[True]
