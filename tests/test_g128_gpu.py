"""GPU parity of the group-128 integer banks -- W4A8-g128 (mode 4) and
W6A8-g128 (mode 5): 4- / 6-bit codes with one fp16 scale per (row,
128-group), FP8 per-token activations -- against the oracle.

They run on the FP8 decode kernels with the integer levels expanded into
E4M3 MFMA operands in registers.  Bars: routing ids bit-exact; outputs within
||y - r||_inf / ||r||_inf <= 2e-2 of the oracle; the single-launch and the
three-launch decode bit-identical; hipGraph replays identical to eager calls.
"""
import numpy as np
import pytest
import torch

from conftest import print_case
from drama_moe import _lib
from drama_moe.formats import QuantizedStore, random_quantized_bank
from drama_moe.quantized import QuantizedExpertBackend
from oracle import oracle as orc

pytestmark = pytest.mark.gpu
TOL = 2e-2


def rel_inf(actual, expected):
    actual = np.asarray(actual, np.float64)
    expected = np.asarray(expected, np.float64)
    return float(np.max(np.abs(actual - expected)) / max(np.max(np.abs(expected)), 1e-30))


def oracle_banks(store: QuantizedStore):
    return (orc.G128Bank(store.mode, store.w13_weight.cpu().numpy(), store.w13_scale_inv.cpu().numpy()),
            orc.G128Bank(store.mode, store.w2_weight.cpu().numpy(), store.w2_scale_inv.cpu().numpy()))


def oracle_layer(store, x, ids, weights):
    b13, b2 = oracle_banks(store)
    return orc.fp8_moe_forward(b13, b2, x, ids, weights, x_group=store.hidden)


@pytest.fixture(scope="module", autouse=True)
def built():
    orc.build()


@pytest.fixture
def decode_mode():
    lib = _lib.library()

    def set_mode(fused: bool) -> None:
        lib.dmoe_set_fused_decode(2 if fused else 0)

    yield set_mode
    lib.dmoe_set_fused_decode(1)


def bank_on(cuda, mode, experts, hidden, inter, seed):
    return random_quantized_bank(mode, experts, hidden, inter, device=cuda,
                                 generator=torch.Generator(device=cuda).manual_seed(seed))


@pytest.mark.parametrize("mode", [4, 5])
@pytest.mark.parametrize("experts,hidden,inter,tokens,top_k", [
    (128, 2048, 768, 1, 8),    # the 24-layer decode step's layer shape
    (32, 2048, 768, 4, 8),     # 32 pairs: single launch
    (64, 2048, 768, 16, 8),    # 128 pairs: three launches
    (16, 1024, 512, 3, 4),
    (8, 4096, 512, 1, 4),      # H 4096: three launches in both modes
    (4, 256, 1024, 2, 2),      # I 1024
])
def test_g128_layer_matches_oracle_and_both_decodes_agree(cuda, decode_mode, mode, experts, hidden, inter, tokens,
                                                          top_k):
    print_case("g128 layer", mode, experts, hidden, inter, tokens, top_k)
    store = bank_on(cuda, mode, experts, hidden, inter, 20261206 + mode + tokens)
    g = torch.Generator().manual_seed(mode * 100 + tokens)
    x = torch.randn(tokens, hidden, generator=g).bfloat16()
    ids, w = orc.route_topk(torch.randn(tokens, experts, generator=g).numpy(), top_k)
    weights = torch.from_numpy(w).bfloat16()
    backend = QuantizedExpertBackend(mode)
    backend.status(cuda)
    args = (x.to(cuda), torch.from_numpy(ids).to(cuda), weights.to(cuda), store)
    decode_mode(True)
    fused = backend.forward(*args)
    torch.cuda.synchronize()
    decode_mode(False)
    staged = backend.forward(*args)
    torch.cuda.synchronize()
    decode_mode(True)
    assert backend.status(cuda) == 0
    assert torch.equal(fused, staged)
    expected = oracle_layer(store, x.float().numpy(), ids, weights.float().numpy())
    assert rel_inf(fused.float().cpu().numpy(), expected) < TOL


@pytest.mark.parametrize("mode", [4, 5])
def test_g128_pairs_beyond_one_decode_call_and_invalid_ids(cuda, mode):
    """600 single-pair rows run as three consecutive decode calls; rows with
    ids outside [0, E) are zero and flag the status word."""
    print_case("g128 pairs", mode)
    store = bank_on(cuda, mode, 16, 512, 256, 77 + mode)
    g = torch.Generator().manual_seed(5 + mode)
    rows = 600
    x = torch.randn(rows, 512, generator=g).bfloat16()
    ids = torch.randint(0, 16, (rows, 1), generator=g)
    ids[7, 0] = 16
    ids[300, 0] = -2
    w = torch.rand(rows, 1, generator=g) + 0.1
    backend = QuantizedExpertBackend(mode)
    backend.status(cuda)
    out = backend.forward_pairs(x.to(cuda), ids.to(cuda), w.to(cuda), store)
    assert backend.status(cuda) & _lib.STATUS_BAD_EXPERT_ID
    assert torch.count_nonzero(out[7]) == 0 and torch.count_nonzero(out[300]) == 0
    keep = [r for r in range(rows) if r not in (7, 300)]
    b13, b2 = oracle_banks(store)
    expected = np.concatenate([orc.fp8_expert_pairs(b13, b2, x[r].float().numpy(), ids[r].numpy(), w[r].numpy(),
                                                    x_group=512) for r in keep])
    assert rel_inf(out.cpu().numpy()[keep], expected) < TOL


@pytest.mark.parametrize("mode", [4, 5])
def test_g128_prefill_tokens_as_consecutive_decode_calls(cuda, mode):
    """A 100-token layer call (800 pairs) against the oracle on spread tokens."""
    print_case("g128 prefill", mode)
    store = bank_on(cuda, mode, 32, 1024, 256, 31 + mode)
    g = torch.Generator().manual_seed(99)
    x = torch.randn(100, 1024, generator=g).bfloat16()
    ids, w = orc.route_topk(torch.randn(100, 32, generator=g).numpy(), 8)
    weights = torch.from_numpy(w).bfloat16()
    out = QuantizedExpertBackend(mode).forward(x.to(cuda), torch.from_numpy(ids).to(cuda), weights.to(cuda), store)
    pick = [0, 31, 32, 63, 64, 99]  # both sides of every 32-token chunk boundary
    expected = oracle_layer(store, x.float().numpy()[pick], ids[pick], weights.float().numpy()[pick])
    assert rel_inf(out.float().cpu().numpy()[pick], expected) < TOL


@pytest.mark.parametrize("mode", [4, 5])
def test_g128_24_layer_decode_step_in_hipgraph(cuda, mode):
    """The 24-layer decode step: E 128, H 2048, I 768, top-8 router inside
    every layer call, all layers captured in one hipGraph.  Replays equal the
    eager step; the routing of every layer is bit-exact, and two layers'
    outputs match the oracle."""
    print_case("g128 24-layer graph", mode)
    layers = 24
    banks = [bank_on(cuda, mode, 128, 2048, 768, 1000 * mode + l) for l in range(layers)]
    g = torch.Generator(device=cuda).manual_seed(4242 + mode)
    xs = torch.randn(layers, 1, 2048, device=cuda, generator=g).bfloat16()
    logits = torch.randn(layers, 1, 128, device=cuda, generator=g)
    backend = QuantizedExpertBackend(mode)
    backend.status(cuda)
    eager = [backend.forward_routed(xs[l], logits[l], 8, banks[l]) for l in range(layers)]
    torch.cuda.synchronize()
    outs = torch.empty_like(xs)
    stream = torch.cuda.Stream(cuda)
    stream.wait_stream(torch.cuda.current_stream(cuda))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        routed = [backend.forward_routed(xs[l], logits[l], 8, banks[l], out=outs[l]) for l in range(layers)]
    for replay in range(3):
        outs.zero_()
        graph.replay()
        torch.cuda.synchronize()
        for l in range(layers):
            assert torch.equal(outs[l], eager[l][0]), (replay, l)
            assert torch.equal(routed[l][2], eager[l][2]) and torch.equal(routed[l][1], eager[l][1])
    assert backend.status(cuda) == 0
    for l in (0, layers - 1):
        eids, _ = orc.route_topk(logits[l].cpu().numpy(), 8)
        np.testing.assert_array_equal(eager[l][2].cpu().numpy(), eids)
        expected = oracle_layer(banks[l], xs[l].float().cpu().numpy(), eids, eager[l][1].float().cpu().numpy())
        assert rel_inf(eager[l][0].float().cpu().numpy(), expected) < TOL


@pytest.mark.parametrize("mode", [4, 5])
def test_g128_routed_layer_above_one_decode_call(cuda, mode):
    """Router + experts of a 100-token call (800 pairs): the router kernel
    writes the routing, the experts run as consecutive decode calls over it.
    Routing bit-exact with the oracle on every token, outputs within 2e-2 of
    the oracle on tokens at both sides of every decode-call boundary."""
    print_case("g128 routed 100 tokens", mode)
    store = bank_on(cuda, mode, 32, 1024, 256, 51 + mode)
    g = torch.Generator().manual_seed(700 + mode)
    tokens = 100
    x = torch.randn(tokens, 1024, generator=g).bfloat16()
    logits = torch.randn(tokens, 32, generator=g)
    backend = QuantizedExpertBackend(mode)
    backend.status(cuda)
    out, w, ids = backend.forward_routed(x.to(cuda), logits.to(cuda), 8, store)
    torch.cuda.synchronize()
    assert backend.status(cuda) == 0
    eids, ew = orc.route_topk(logits.numpy(), 8)
    np.testing.assert_array_equal(ids.cpu().numpy(), eids)
    np.testing.assert_array_equal(w.float().cpu().numpy(), torch.from_numpy(ew).bfloat16().float().numpy())
    pick = [0, 31, 32, 63, 64, 95, 96, 99]
    expected = oracle_layer(store, x.float().numpy()[pick], eids[pick], w.float().cpu().numpy()[pick])
    assert rel_inf(out.float().cpu().numpy()[pick], expected) < TOL
    # the same routes through forward() give the same bytes
    again = backend.forward(x.to(cuda), ids, w, store)
    assert torch.equal(again, out)


@pytest.mark.parametrize("mode", [4, 5])
def test_g128_moe_block_prefill_size(cuda, mode):
    """MoeBlock over a group-128 bank at 100 tokens: the routed leg takes the
    large-call path and the block output matches the oracle's composition."""
    from drama_moe import block

    print_case("g128 moe block 100 tokens", mode)
    g = torch.Generator().manual_seed(880 + mode)
    hidden, experts, inter, top_k, tokens = 512, 32, 256, 8, 100
    store = bank_on(cuda, mode, experts, hidden, inter, 60 + mode)

    def mk(*shape):
        return (torch.randn(*shape, generator=g) * 0.03).bfloat16()

    rw, sw, gw, uw, dw = mk(experts, hidden), mk(1, hidden), mk(128, hidden), mk(128, hidden), mk(hidden, 128)
    blk = block.MoeBlock(rw.to(cuda), sw.to(cuda), gw.to(cuda), uw.to(cuda), dw.to(cuda), store,
                         QuantizedExpertBackend(mode), top_k=top_k)
    x = torch.randn(tokens, hidden, generator=g).bfloat16()
    # a small residual, so the bf16 rounding of the residual sum stays far
    # below the MoE contribution the comparison measures
    after = (torch.randn(tokens, hidden, generator=g) / 64).bfloat16()
    out, w, ids = blk(x.to(cuda), after.to(cuda))
    logits, _, _ = blk.pre(x.to(cuda))
    eids, _ = orc.route_topk(logits.cpu().numpy(), top_k)
    np.testing.assert_array_equal(ids.cpu().numpy(), eids)
    f = lambda t: t.float().cpu().numpy()  # noqa: E731
    _, want_sgate, want_act = orc.block_pre(f(x), f(rw), f(sw), f(gw), f(uw))
    experts_out = orc.bf16_round(oracle_layer(store, f(x), eids, f(w)))
    want = orc.block_post(want_act, f(dw), want_sgate, experts_out, f(after))
    assert rel_inf(f(out) - f(after), want - f(after)) < TOL
    # a supplied output the kernel cannot write in place is refused, not copied
    with pytest.raises(ValueError, match="out must be bf16"):
        blk(x.to(cuda), after.to(cuda), out=torch.empty(hidden, tokens, dtype=torch.bfloat16, device=cuda).t())


@pytest.mark.parametrize("mode", [4, 5])
def test_g128_layer_combine_with_pairs_per_row_not_top_k(cuda, mode):
    """A direct C-ABI layer call whose rows hold 2 pairs each while tokens
    hold 3 (row_div 2, top_k 3, 600 pairs): decode calls cut at whole tokens
    and rows, so every token equals the oracle's sum of its three pairs."""
    import ctypes

    from drama_moe.offload import device_state
    from drama_moe.quantized import bank_struct

    print_case("g128 row_div 2 top_k 3", mode)
    store = bank_on(cuda, mode, 16, 512, 256, 90 + mode)
    g = torch.Generator().manual_seed(31 + mode)
    pairs, row_div, top_k = 600, 2, 3
    rows, tokens = pairs // row_div, pairs // top_k
    x = torch.randn(rows, 512, generator=g).bfloat16()
    ids = torch.randint(0, 16, (pairs,), generator=g)
    w = (torch.rand(pairs, generator=g) + 0.1).float()
    out = torch.empty(tokens, 512, dtype=torch.float32, device=cuda)
    xd, idd, wd = x.to(cuda), ids.to(cuda), w.to(cuda)
    lib = _lib.library()
    bank = bank_struct(store)
    state = device_state(cuda)
    ws = state.workspace_for(lib.dmoe_quant_workspace_bytes(ctypes.byref(bank), rows, pairs))
    _lib.check(lib.dmoe_quant_moe_forward(
        ctypes.byref(bank), _lib.ptr(xd), _lib.dtype_code(xd.dtype), xd.stride(0), rows, row_div, _lib.ptr(idd),
        _lib.dtype_code(idd.dtype), _lib.ptr(wd), _lib.dtype_code(wd.dtype), pairs, top_k, _lib.ptr(out),
        _lib.F32, out.stride(0), None, _lib.ptr(ws), ws.numel(), _lib.ptr(state.status),
        _lib.stream_handle(cuda)))
    torch.cuda.synchronize()
    b13, b2 = oracle_banks(store)
    xs = x.float().numpy()
    parts = np.concatenate([orc.fp8_expert_pairs(b13, b2, xs[p // row_div], ids[p:p + 1].numpy(),
                                                 w[p:p + 1].numpy(), x_group=512) for p in range(pairs)])
    expected = parts.reshape(tokens, top_k, 512).sum(1)
    assert rel_inf(out.cpu().numpy(), expected) < TOL
