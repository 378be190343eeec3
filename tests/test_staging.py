"""Host-residency staging logic on the CPU: slot placement, hot-cache
policy, grouped calls and their slot-order sum, with a stand-in backend whose
per-pair value depends on every byte of the routed expert, so a wrong slot, a
stale slot or a dropped pair changes the output."""
from __future__ import annotations

import pytest
import torch
from torch import nn

from drama_moe import offload, staging
from drama_moe.formats import random_fp8_bank, random_quantized_bank


class SignatureBackend:
    """forward / forward_pairs over a bank: pair (row, expert e, weight w)
    contributes w * x_row * sig(e), sig(e) a function of all of e's bytes;
    forward adds a token's pairs in slot order in fp32."""

    def __init__(self):
        self.calls = []

    @staticmethod
    def signature(bank, e):
        total = torch.zeros((), dtype=torch.float64)
        for i, t in enumerate(staging.bank_buffers(bank).values()):
            b = t[e].contiguous().view(torch.uint8).double()
            total += (b * torch.arange(1, b.numel() + 1, dtype=torch.float64).reshape(b.shape)).sum() * (i + 1)
        return (total % 9973).float() / 9973 + 0.5

    def forward_pairs(self, x, ids, weights, bank):
        self.calls.append(("pairs", ids.shape[0]))
        sig = torch.stack([self.signature(bank, int(e)) for e in ids.reshape(-1)])
        return weights.reshape(-1, 1).float() * x.float() * sig.reshape(-1, 1)

    def forward(self, x, ids, weights, bank, out=None):
        self.calls.append(("forward", ids.numel()))
        tokens, top_k = ids.shape
        pairs = self.forward_pairs(x.repeat_interleave(top_k, 0), ids.reshape(-1, 1), weights.reshape(-1, 1), bank)
        pairs = pairs.view(tokens, top_k, -1)
        total = pairs[:, 0].clone()
        for s in range(1, top_k):
            total += pairs[:, s]
        result = total.to(x.dtype)
        if out is not None:
            out.copy_(result)
            return out
        return result


def route(tokens, top_k, experts, g):
    ids = torch.stack([torch.randperm(experts, generator=g)[:top_k] for _ in range(tokens)])
    return ids, torch.rand(tokens, top_k, generator=g)


@pytest.fixture
def bank():
    return random_fp8_bank(16, 128, 128, layout="channel", generator=torch.Generator().manual_seed(4))


def host(**kw):
    kw.setdefault("pin_memory", False)
    return staging.HostResidency(**kw)


def test_pool_call_matches_the_whole_bank(bank):
    g = torch.Generator().manual_seed(1)
    backend = SignatureBackend()
    tier = host(max_staged_experts=8)
    for tokens in (1, 2, 3):
        ids, w = route(tokens, 2, 16, g)
        x = torch.randn(tokens, 128, generator=g).bfloat16()
        assert len(set(ids.reshape(-1).tolist())) <= 8
        got = tier.forward("layer0", bank, backend, x, ids, w)
        assert torch.equal(got, backend.forward(x, ids, w, bank))
    assert tier.grouped_calls == 0 and tier.pool.loads > 0


def test_grouped_call_when_experts_exceed_the_pool(bank):
    g = torch.Generator().manual_seed(2)
    backend = SignatureBackend()
    tier = host(max_staged_experts=3, max_pair_rows=5)
    ids, w = route(6, 4, 16, g)
    x = torch.randn(6, 128, generator=g).bfloat16()
    got = tier.forward("layer0", bank, backend, x, ids, w)
    assert tier.grouped_calls == 1
    assert all(n <= 5 for kind, n in backend.calls if kind == "pairs")
    assert torch.equal(got, SignatureBackend().forward(x, ids, w, bank))


def test_pair_row_limit_chunks_whole_calls(bank):
    g = torch.Generator().manual_seed(3)
    backend = SignatureBackend()
    tier = host(max_staged_experts=16, max_pair_rows=4)
    ids, w = route(5, 2, 16, g)
    x = torch.randn(5, 128, generator=g).bfloat16()
    got = tier.forward("layer0", bank, backend, x, ids, w)
    assert [n for kind, n in backend.calls if kind == "forward"] == [4, 4, 2]
    assert torch.equal(got, SignatureBackend().forward(x, ids, w, bank))


def test_hot_cache_keeps_a_decode_tokens_experts_per_layer(bank):
    g = torch.Generator().manual_seed(5)
    other = random_fp8_bank(16, 128, 128, layout="channel", generator=g)
    backend = SignatureBackend()
    tier = host(max_staged_experts=2, cache_experts=4)
    x = torch.randn(1, 128, generator=g).bfloat16()
    w = torch.rand(1, 3, generator=g)
    for layer, b in (("a", bank), ("b", other)):
        ids = torch.tensor([[3, 7, 9]])
        assert torch.equal(tier.forward(layer, b, backend, x, ids, w), backend.forward(x, ids, w, b))
    assert tier.stats()["cache_loads"] == 6 and tier.stats()["cache_hits"] == 0
    ids = torch.tensor([[9, 3, 12]])  # two hits, one load into the free slot
    assert torch.equal(tier.forward("a", bank, backend, x, ids, w), backend.forward(x, ids, w, bank))
    cache = tier.caches["a"]
    assert cache.hits == 2 and cache.loads == 4 and set(cache.slot_of) == {3, 7, 9, 12}
    ids = torch.tensor([[1, 9, 5]])  # 7 is least recently used: evicted first, then 3
    assert torch.equal(tier.forward("a", bank, backend, x, ids, w), backend.forward(x, ids, w, bank))
    assert set(cache.slot_of) == {1, 9, 5, 12}
    # a token routed to more experts than the cache holds: the cache takes the
    # first four in router order, the rest go through the pool as a group
    w6 = torch.rand(1, 6, generator=g)
    ids = torch.tensor([[0, 2, 4, 6, 8, 10]])
    assert torch.equal(tier.forward("b", other, backend, x, ids, w6), backend.forward(x, ids, w6, other))
    assert set(tier.caches["b"].slot_of) == {0, 2, 4, 6}


def test_prompt_reads_the_cache_without_filling_it(bank):
    g = torch.Generator().manual_seed(6)
    backend = SignatureBackend()
    tier = host(max_staged_experts=4, cache_experts=2)
    x1 = torch.randn(1, 128, generator=g).bfloat16()
    tier.forward("a", bank, backend, x1, torch.tensor([[5, 6]]), torch.rand(1, 2, generator=g))
    ids, w = route(4, 2, 16, g)
    x = torch.randn(4, 128, generator=g).bfloat16()
    loads = tier.caches["a"].loads
    assert torch.equal(tier.forward("a", bank, backend, x, ids, w), backend.forward(x, ids, w, bank))
    assert tier.caches["a"].loads == loads and set(tier.caches["a"].slot_of) == {5, 6}


def test_packed_bank_with_zero_points_stages_every_buffer():
    g = torch.Generator().manual_seed(7)
    bank = random_quantized_bank(0, 8, 256, 128, asymmetric=True, generator=g)
    assert set(staging.bank_buffers(bank)) >= {"w13_zeros", "w2_zeros"}
    backend = SignatureBackend()
    tier = host(max_staged_experts=3)
    ids = torch.tensor([[1, 6], [6, 2]])
    x = torch.randn(2, 256, generator=g).bfloat16()
    w = torch.rand(2, 2, generator=g)
    assert torch.equal(tier.forward("q", bank, backend, x, ids, w), backend.forward(x, ids, w, bank))
    staged = tier.pool.bank(bank)
    assert staged.mode == 0 and staged.w13_zeros.shape[0] == 3


def test_slot_and_keyword_validation(bank):
    with pytest.raises(ValueError, match="positive"):
        host(max_staged_experts=0)
    with pytest.raises(ValueError, match="must match"):
        host(cache_experts=2, hot_cache_experts=3)
    assert host(hot_cache_experts=3).cache_experts == 3
    tier = host()
    with pytest.raises(ValueError, match=r"Expert IDs must be in \[0, 16\)"):
        tier.forward("a", bank, SignatureBackend(), torch.zeros(1, 128), torch.tensor([[16]]), torch.ones(1, 1))
    slots = staging.ExpertSlots(2)
    slots.bind(bank, "cpu")
    slots.place(bank, [1, 2], keep={1, 2})
    with pytest.raises(RuntimeError, match="needs"):
        slots.place(bank, [3], keep={1, 2, 3})
    with pytest.raises(ValueError, match="residency"):
        offload.ResidentExpertManager(residency="disk")
    with pytest.raises(TypeError, match="boolean"):
        offload.ResidentExpertManager(pin_memory="yes")


class FP8Experts(nn.Module):
    def __init__(self, bank):
        super().__init__()
        for name, t in staging.bank_buffers(bank).items():
            self.register_buffer(name, t)
        self.fp8 = True


def test_manager_host_mode_routes_through_the_tier(bank):
    backend = SignatureBackend()
    model = nn.ModuleDict({"experts": FP8Experts(bank)})
    manager = offload.install_expert_offload(model, backend=backend, residency="host", max_staged_experts=4,
                                             pin_memory=False)
    g = torch.Generator().manual_seed(8)
    ids, w = route(2, 2, 16, g)
    x = torch.randn(2, 128, generator=g).bfloat16()
    got = model["experts"](x, ids, w)
    assert torch.equal(got, backend.forward(x, ids, w, bank))
    assert manager.host.calls == 1
    manager.close()


def test_statistics_count_the_host_traffic(bank):
    """OffloadStatistics (offload.py:59-98): hot-cache and pool loads and hits,
    the bytes and tensor copies they moved, forward calls, host timings; no
    event time without profile_transfers, and none for copies off the GPU
    (test_offload.py:521-531)."""
    per_expert = sum(t[0].numel() * t.element_size() for t in staging.bank_buffers(bank).values())
    tensors = len(staging.bank_buffers(bank))
    backend = SignatureBackend()
    model = nn.ModuleDict({"experts": FP8Experts(bank)})
    manager = offload.install_expert_offload(model, backend=backend, residency="host", max_staged_experts=4,
                                             cache_experts=3, pin_memory=False)
    g = torch.Generator().manual_seed(12)
    x1 = torch.randn(1, 128, generator=g).bfloat16()
    w2 = torch.rand(1, 2, generator=g)
    model["experts"](x1, torch.tensor([[3, 7]]), w2)   # two hot-cache loads
    model["experts"](x1, torch.tensor([[7, 3]]), w2)   # two hot-cache hits
    x2 = torch.randn(2, 128, generator=g).bfloat16()
    ids = torch.tensor([[3, 5], [11, 7]])              # a prompt: 3, 7 from the cache, 5, 11 staged
    got = model["experts"](x2, ids, torch.rand(2, 2, generator=g))
    assert got.shape == (2, 128)
    st = manager.stats
    assert (st.forward_calls, st.hot_cache_loads, st.hot_cache_hits) == (3, 2, 4)
    assert (st.expert_loads, st.staging_calls, st.peak_staged_experts, st.grouped_calls) == (2, 1, 2, 1)
    assert st.staged_bytes == 2 * per_expert and st.h2d_bytes == 4 * per_expert
    assert st.h2d_copy_calls == 4 * tensors
    assert st.hot_cache_capacity_experts == 3 and st.hot_cache_bytes == 3 * per_expert
    assert st.device_buffer_bytes == st.hot_cache_bytes + 4 * per_expert
    assert st.routing_host_seconds > 0 and st.host_staging_seconds > 0 and st.h2d_seconds == 0
    assert st.as_dict()["expert_loads"] == 2
    manager.close()


def test_empty_call_returns_empty_rows(bank):
    tier = host()
    out = tier.forward("a", bank, SignatureBackend(), torch.zeros(0, 128), torch.zeros(0, 2, dtype=torch.long),
                       torch.zeros(0, 2))
    assert out.shape == (0, 128) and tier.calls == 0
