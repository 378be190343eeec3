"""Router + packed experts in one call (QuantizedExpertBackend.forward_routed,
dmoe_quant_moe_layer) for modes 0-3: the routes it returns are the router
kernel's bits (dmoe_route_topk), and its output is bit-for-bit the expert
call on those routes -- whether the small-call gate/up kernel routes the call
itself (decode sizes, up to 128 experts and top-8) or the router kernel runs
first (larger calls, more experts, the separate launches).  At decode sizes
that give one workgroup per CU (modes 0-2, bf16 rows) the routed call is one
persistent launch, checked against the two small-call launches."""
from __future__ import annotations

import pytest
import torch

from conftest import print_case
from drama_moe import _lib, router
from drama_moe.formats import random_quantized_bank
from drama_moe.quantized import QuantizedExpertBackend

pytestmark = pytest.mark.gpu


def to_device(store, device):
    import dataclasses
    fields = {f.name: getattr(store, f.name) for f in dataclasses.fields(store)}
    return type(store)(**{k: (v.to(device) if isinstance(v, torch.Tensor) else v) for k, v in fields.items()})


@pytest.fixture
def launches(cuda):
    lib = _lib.library()
    QuantizedExpertBackend.status(cuda)  # start from a clear status word (earlier tests raise bits on purpose)
    yield lambda small: lib.dmoe_set_fused_decode(1 if small else 0)
    lib.dmoe_set_fused_decode(1)


@pytest.mark.parametrize("mode", [0, 1, 2, 3])
@pytest.mark.parametrize("tokens,experts,top_k", [(1, 128, 8), (4, 128, 8), (3, 32, 4), (1, 160, 8), (12, 128, 8)])
@pytest.mark.parametrize("small", [True, False])
def test_routed_layer_matches_router_then_experts(cuda, launches, mode, tokens, experts, top_k, small):
    print_case("packed routed layer", mode, tokens, experts, top_k, small)
    launches(small)
    g = torch.Generator().manual_seed(7000 + 100 * mode + tokens + experts + top_k)
    bank = to_device(random_quantized_bank(mode, experts, 512, 256, asymmetric=mode == 0, generator=g), cuda)
    x = torch.randn(tokens, 512, generator=g).bfloat16().to(cuda)
    logits = torch.randn(tokens, experts, generator=g).to(cuda)
    logits[0, 3] = logits[0, 7]  # a tie
    backend = QuantizedExpertBackend(mode)
    out, weights, ids = backend.forward_routed(x, logits, top_k, bank)
    want_w, want_ids = router.route_topk(logits, top_k)
    torch.cuda.synchronize()
    assert torch.equal(ids, want_ids) and torch.equal(weights, want_w)
    want = backend.forward(x, want_ids, want_w, bank)
    torch.cuda.synchronize()
    assert torch.equal(out, want)
    assert backend.status(cuda) == 0


def test_routed_layer_in_hipgraph(cuda):
    print_case("packed routed layer hipgraph")
    g = torch.Generator().manual_seed(7700)
    bank = to_device(random_quantized_bank(0, 128, 512, 256, asymmetric=True, generator=g), cuda)
    backend = QuantizedExpertBackend(0)
    x = torch.randn(2, 512, generator=g).bfloat16().to(cuda)
    logits = torch.randn(2, 128, generator=g).to(cuda)
    out = torch.empty_like(x)
    stream = torch.cuda.Stream(cuda)
    stream.wait_stream(torch.cuda.current_stream(cuda))
    with torch.cuda.stream(stream):
        backend.forward_routed(x, logits, 8, bank, out=out)
    torch.cuda.current_stream(cuda).wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        _, w_g, i_g = backend.forward_routed(x, logits, 8, bank, out=out)
    for step in range(3):
        x.copy_(torch.randn(2, 512, device=cuda).bfloat16())
        logits.copy_(torch.randn(2, 128, device=cuda))
        expected, w_e, i_e = backend.forward_routed(x, logits, 8, bank)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(i_g, i_e) and torch.equal(w_g, w_e), step
        assert torch.equal(out, expected), step


_BANKS = {}


def model_bank(mode, hidden, inter, device):
    key = (mode, hidden, inter)
    if key not in _BANKS:
        g = torch.Generator().manual_seed(7900 + 10 * mode + inter)
        _BANKS[key] = to_device(random_quantized_bank(mode, 128, hidden, inter, asymmetric=mode == 0, generator=g),
                                device)
    return _BANKS[key]


@pytest.mark.parametrize("mode", [0, 1, 2])
@pytest.mark.parametrize("hidden,inter", [(2048, 768), (2048, 512)])
def test_routed_decode_at_model_sizes(cuda, launches, mode, hidden, inter):
    """One token over 128 experts at top-8, at the 30B-A3B expert shape and
    a narrower one: the routed small call runs as one persistent launch there
    (its gate/up workgroups publish the hidden rows as hand-off words, its
    down workgroups poll them), and it equals the expert call on the same
    routes (the two small-call launches) bit for bit, over several calls in a
    row (the hand-off buffers alternate between calls)."""
    print_case("packed routed decode, model sizes", mode, hidden, inter)
    launches(True)
    bank = model_bank(mode, hidden, inter, cuda)
    backend = QuantizedExpertBackend(mode)
    g = torch.Generator().manual_seed(7950 + mode + inter)
    for call in range(3):
        x = torch.randn(1, hidden, generator=g).bfloat16().to(cuda)
        logits = torch.randn(1, 128, generator=g).to(cuda)
        out, weights, ids = backend.forward_routed(x, logits, 8, bank)
        want = backend.forward(x, ids, weights, bank)
        torch.cuda.synchronize()
        assert torch.equal(out, want), call
    assert backend.status(cuda) == 0


def test_routed_decode_sync_timeout_is_reported(cuda, launches):
    """The host forces the persistent packed decode's bounded hand-off wait
    to give up (its readers wait for a tag no producer writes, up to a 100 us
    bound): the status word carries DMOE_STATUS_SYNC_TIMEOUT, every launch
    completes, and with the switch off the next call is exact again."""
    print_case("packed routed decode, forced sync timeout")
    launches(True)
    lib = _lib.library()
    bank = model_bank(0, 2048, 768, cuda)
    backend = QuantizedExpertBackend(0)
    g = torch.Generator().manual_seed(7990)
    x = torch.randn(1, 2048, generator=g).bfloat16().to(cuda)
    logits = torch.randn(1, 128, generator=g).to(cuda)
    expected, _, _ = backend.forward_routed(x, logits, 8, bank)
    torch.cuda.synchronize()
    assert backend.status(cuda) == 0
    previous = lib.dmoe_set_sync_spin_limit(10_000)  # 100 us of the 100 MHz counter
    forced = lib.dmoe_debug_force_sync_timeout(1)
    try:
        for _ in range(2):
            backend.forward_routed(x, logits, 8, bank)
        torch.cuda.synchronize()
    finally:
        lib.dmoe_debug_force_sync_timeout(forced)
        lib.dmoe_set_sync_spin_limit(previous)
    assert backend.status(cuda) & _lib.STATUS_SYNC_TIMEOUT
    again, _, _ = backend.forward_routed(x, logits, 8, bank)
    torch.cuda.synchronize()
    assert backend.status(cuda) == 0
    assert torch.equal(again, expected)
