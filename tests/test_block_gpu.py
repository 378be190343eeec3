"""GPU parity of the MoE block around the routed experts (router GEMV,
sigmoid-gated shared expert, residual adds; backbone_graph.py:317-337)
against the oracle's restatement, through the C ABI."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import print_case
from drama_moe import block
from drama_moe.formats import StagedExperts, random_fp8_bank
from drama_moe.offload import HipExpertBackend
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

TOL = 2e-2
BF16_STEP = 2.0 ** -7


def rel_inf(actual, expected):
    return float(np.max(np.abs(actual - expected)) / max(np.max(np.abs(expected)), 1e-30))


def weights(hidden, experts, inter, g, std=0.03):
    def mk(*shape):
        return (torch.randn(*shape, generator=g) * std).bfloat16()
    return mk(experts, hidden), mk(1, hidden), mk(inter, hidden), mk(inter, hidden), mk(hidden, inter)


def as_np(t):
    return t.float().cpu().numpy()


@pytest.mark.parametrize("tokens", [1, 5, 9, 16])
def test_block_pre_and_post_match_oracle(cuda, tokens):
    print_case("moe block pre/post", tokens)
    g = torch.Generator().manual_seed(400 + tokens)
    hidden, experts, inter = 256, 16, 64
    rw, sw, gw, uw, dw = weights(hidden, experts, inter, g)
    x = torch.randn(tokens, hidden, generator=g).bfloat16()
    after = torch.randn(tokens, hidden, generator=g).bfloat16()
    experts_out = torch.randn(tokens, hidden, generator=g).bfloat16()
    blk = block.MoeBlock(rw.to(cuda), sw.to(cuda), gw.to(cuda), uw.to(cuda), dw.to(cuda), None, None, top_k=4)
    logits, sgate, act = blk.pre(x.to(cuda))
    want_logits, want_sgate, want_act = orc.block_pre(as_np(x), as_np(rw), as_np(sw), as_np(gw), as_np(uw))
    assert logits.dtype == torch.float32 and sgate.dtype == torch.bfloat16 and act.dtype == torch.bfloat16
    got = as_np(logits)
    assert np.array_equal(got, as_np(torch.from_numpy(got).bfloat16()))  # bf16-rounded logits
    assert np.max(np.abs(got - want_logits)) <= 2 * BF16_STEP * np.max(np.abs(want_logits))
    assert np.max(np.abs(as_np(sgate) - want_sgate)) <= 2 * BF16_STEP
    assert np.max(np.abs(as_np(act) - want_act)) <= 2 * BF16_STEP * np.max(np.abs(want_act))
    out = blk.post(act, sgate, experts_out.to(cuda), after.to(cuda))
    want = orc.block_post(as_np(act), as_np(dw), as_np(sgate), as_np(experts_out), as_np(after))
    assert rel_inf(as_np(out), want) < 1e-2
    # in place over the residual, as a decoder layer updates its hidden state
    res = after.to(cuda)
    blk.post(act, sgate, experts_out.to(cuda), res, out=res)
    assert torch.equal(res, out)


@pytest.mark.parametrize("tokens", [1, 4])
def test_moe_block_full_shape_fp8(cuda, tokens):
    """Hidden 2048, 128 FP8 experts of 768 (per-channel scales), top-8, a
    768-wide shared expert: the block output against the oracle's pre, routing
    of the kernel's logits (bit-exact ids and order), FP8 experts and post."""
    print_case("moe block full", tokens)
    g = torch.Generator().manual_seed(20261206 + tokens)
    hidden, experts, inter, top_k = 2048, 128, 768, 8
    bank = random_fp8_bank(experts, hidden, inter, layout="channel", generator=g)
    rw, sw, gw, uw, dw = weights(hidden, experts, 768, g)
    dev = StagedExperts(*(getattr(bank, n).to(cuda) for n in ("w13_weight", "w13_scale_inv", "w2_weight",
                                                               "w2_scale_inv")))
    blk = block.MoeBlock(rw.to(cuda), sw.to(cuda), gw.to(cuda), uw.to(cuda), dw.to(cuda), dev, HipExpertBackend(),
                         top_k=top_k)
    x = torch.randn(tokens, hidden, generator=g).bfloat16()
    after = torch.randn(tokens, hidden, generator=g).bfloat16()
    out, w, ids = blk(x.to(cuda), after.to(cuda))
    logits, sgate, act = blk.pre(x.to(cuda))
    want_logits, want_sgate, want_act = orc.block_pre(as_np(x), as_np(rw), as_np(sw), as_np(gw), as_np(uw))
    assert np.max(np.abs(as_np(logits) - want_logits)) <= 2 * BF16_STEP * np.max(np.abs(want_logits))
    eids, ew = orc.route_topk(as_np(logits), top_k)
    assert np.array_equal(ids.cpu().numpy(), eids)
    b13 = orc.Fp8Bank(bank.w13_weight.view(torch.uint8).numpy(), bank.w13_scale_inv.numpy())
    b2 = orc.Fp8Bank(bank.w2_weight.view(torch.uint8).numpy(), bank.w2_scale_inv.numpy())
    experts_out = orc.bf16_round(orc.fp8_moe_forward(b13, b2, as_np(x), eids, as_np(w)))
    want = orc.block_post(want_act, as_np(dw), want_sgate, experts_out, as_np(after))
    assert out.dtype == torch.bfloat16 and out.shape == (tokens, hidden)
    assert rel_inf(as_np(out) - as_np(after), want - as_np(after)) < TOL


def test_moe_block_in_hipgraph(cuda):
    print_case("moe block hipgraph")
    g = torch.Generator().manual_seed(77)
    hidden, experts, inter, top_k = 512, 32, 128, 4
    bank = random_fp8_bank(experts, hidden, 256, layout="channel", generator=g)
    rw, sw, gw, uw, dw = weights(hidden, experts, inter, g)
    dev = StagedExperts(*(getattr(bank, n).to(cuda) for n in ("w13_weight", "w13_scale_inv", "w2_weight",
                                                               "w2_scale_inv")))
    blk = block.MoeBlock(rw.to(cuda), sw.to(cuda), gw.to(cuda), uw.to(cuda), dw.to(cuda), dev, HipExpertBackend(),
                         top_k=top_k)
    x = torch.randn(2, hidden, device=cuda).bfloat16()
    after = torch.randn(2, hidden, device=cuda).bfloat16()
    out = torch.empty_like(after)
    stream = torch.cuda.Stream(cuda)
    stream.wait_stream(torch.cuda.current_stream(cuda))
    with torch.cuda.stream(stream):
        blk(x, after, out=out)
    torch.cuda.current_stream(cuda).wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        blk(x, after, out=out)
    for step in range(3):
        x.copy_(torch.randn(2, hidden, device=cuda).bfloat16())
        after.copy_(torch.randn(2, hidden, device=cuda).bfloat16())
        expected, _, _ = blk(x, after)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, expected), step


def test_moe_block_empty_call(cuda):
    g = torch.Generator().manual_seed(5)
    rw, sw, gw, uw, dw = weights(256, 16, 64, g)
    bank = random_fp8_bank(16, 256, 128, layout="channel", generator=g)
    dev = StagedExperts(*(getattr(bank, n).to(cuda) for n in ("w13_weight", "w13_scale_inv", "w2_weight",
                                                               "w2_scale_inv")))
    blk = block.MoeBlock(rw.to(cuda), sw.to(cuda), gw.to(cuda), uw.to(cuda), dw.to(cuda), dev, HipExpertBackend(),
                         top_k=4)
    x = torch.zeros(0, 256, dtype=torch.bfloat16, device=cuda)
    out, w, ids = blk(x, x.clone())
    assert out.shape == (0, 256) and w.shape == (0, 4) and ids.shape == (0, 4)
