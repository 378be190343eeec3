"""Router + packed experts in one call (QuantizedExpertBackend.forward_routed,
dmoe_quant_moe_layer) for modes 0-3: the routes it returns are the router
kernel's bits (dmoe_route_topk), and its output is bit-for-bit the expert
call on those routes -- whether the small-call gate/up kernel routes the call
itself (decode sizes, up to 128 experts and top-8) or the router kernel runs
first (larger calls, more experts, the separate launches)."""
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
def launches():
    lib = _lib.library()
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
