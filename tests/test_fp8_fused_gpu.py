"""The single-launch decode (one persistent kernel per call) against the
three-launch decode and the oracle.

The two decodes share the arithmetic of the contract step by step (FP8
activation groups, per-128-block fma chains, cross-wave sums in wave order,
gate/up rounding, SiLU, FP8 hidden groups, the down K chain in one wave, the
slot-order combine), so their outputs must be bit-identical; both must also be
within the 2e-2 bar of the oracle.
"""
import numpy as np
import pytest
import torch

from conftest import print_case
from drama_moe import _lib, fp8_decode, fp8_moe, router
from drama_moe.formats import random_fp8_bank
from drama_moe.offload import HipExpertBackend
from oracle import oracle as orc
from test_fp8_gpu import TOL, _layer_case, oracle_banks, rel_inf, to_device

pytestmark = pytest.mark.gpu


@pytest.fixture
def decode_mode():
    lib = _lib.library()

    def set_mode(fused: bool) -> None:
        lib.dmoe_set_fused_decode(2 if fused else 0)

    yield set_mode
    lib.dmoe_set_fused_decode(1)


def both(decode_mode, fn):
    decode_mode(True)
    fused = fn()
    torch.cuda.synchronize()
    decode_mode(False)
    staged = fn()
    torch.cuda.synchronize()
    decode_mode(True)
    return fused, staged


@pytest.mark.parametrize("experts,hidden,inter,tokens,top_k,layout,dtype,x_group", [
    (128, 2048, 768, 1, 8, "channel", torch.bfloat16, 128),   # the decode benchmark layer
    (128, 2048, 768, 1, 8, "block", torch.bfloat16, 128),
    (32, 2048, 768, 4, 8, "block", torch.bfloat16, 128),
    (64, 2048, 768, 8, 8, "channel", torch.bfloat16, 128),     # 64 pairs: the fused limit
    (32, 2048, 768, 4, 8, "channel", torch.bfloat16, "token"),
    (16, 1024, 512, 3, 4, "block", torch.float16, 128),
    (8, 256, 256, 2, 8, "block", torch.float32, 128),
    (1, 2048, 1024, 1, 1, "channel", torch.bfloat16, 128),     # single expert, I 1024
    (8, 4096, 512, 1, 4, "block", torch.bfloat16, 128),        # H 4096: three-launch in both modes
    (512, 1024, 256, 2, 8, "channel", torch.bfloat16, 128),    # 512 experts
    (16, 256, 512, 64, 1, "block", torch.bfloat16, 128),       # 64 tokens, top-1
])
def test_fused_equals_three_launch_and_oracle(cuda, decode_mode, experts, hidden, inter, tokens, top_k, layout,
                                              dtype, x_group):
    print_case("fused vs staged", experts, hidden, inter, tokens, top_k, layout, dtype, x_group)
    group = 128 if x_group == 128 else hidden
    staged, x, ids, weights, expected = _layer_case(cuda, experts, hidden, inter, tokens, top_k, layout, dtype,
                                                    31337 + tokens * 7 + experts, x_group=group,
                                                    bank_on_device=experts * hidden * inter > (1 << 26))
    backend = HipExpertBackend(x_group=x_group)
    fused, three = both(decode_mode, lambda: backend.forward(x, ids, weights, staged))
    assert torch.equal(fused, three)
    assert rel_inf(fused.float().cpu().numpy(), expected) < TOL


@pytest.mark.parametrize("tokens", [1, 4, 8])
def test_fused_router_layer_equals_three_launch(cuda, decode_mode, tokens):
    print_case("fused routed layer", tokens)
    g = torch.Generator().manual_seed(777 + tokens)
    bank = random_fp8_bank(128, 2048, 768, layout="channel", generator=g)
    staged = to_device(bank, cuda)
    x = torch.randn(tokens, 2048, generator=g).bfloat16().to(cuda)
    logits = torch.randn(tokens, 128, generator=g).to(cuda)
    backend = HipExpertBackend()
    (fo, fw, fi), (so, sw, si) = both(decode_mode, lambda: backend.forward_routed(x, logits, 8, staged))
    assert torch.equal(fi, si) and torch.equal(fw, sw)
    assert torch.equal(fo, so)
    eids, ew = orc.route_topk(logits.cpu().numpy(), 8)
    np.testing.assert_array_equal(fi.cpu().numpy(), eids)
    # the full decode layer (E 128, H 2048, I 768) against the oracle on every token
    np.testing.assert_array_equal(fw.float().cpu().numpy(), torch.from_numpy(ew).bfloat16().float().numpy())
    b13, b2 = oracle_banks(bank)
    expected = orc.fp8_moe_forward(b13, b2, x.float().cpu().numpy(), eids, fw.float().cpu().numpy())
    assert rel_inf(fo.float().cpu().numpy(), expected) < TOL


@pytest.mark.parametrize("experts,tokens,top_k", [(128, 1, 8), (100, 3, 8), (8, 2, 8), (128, 1, 5), (64, 2, 12)])
def test_fused_router_ties_and_partial_lanes(cuda, decode_mode, experts, tokens, top_k):
    """Heavily tied logits (8 distinct values) and a -inf logit, with expert
    counts that leave the second logit of some or all lanes empty, top_k up to
    8 (the sorting network) and above (serial rounds): the single-launch
    router's ids and weights equal the router kernel's, its ids the oracle's
    (ties to the lower expert)."""
    print_case("fused router ties", experts, tokens, top_k)
    g = torch.Generator().manual_seed(99 + experts + tokens)
    staged = to_device(random_fp8_bank(experts, 1024, 256, layout="channel", generator=g), cuda)
    x = torch.randn(tokens, 1024, generator=g).bfloat16().to(cuda)
    logits = torch.randint(0, 8, (tokens, experts), generator=g).float() / 4.0
    logits[0, experts // 2] = float("-inf")
    logits = logits.to(cuda)
    backend = HipExpertBackend()
    (fo, fw, fi), (so, sw, si) = both(decode_mode, lambda: backend.forward_routed(x, logits, top_k, staged))
    assert torch.equal(fi, si) and torch.equal(fw, sw)
    assert torch.equal(fo, so)
    eids, _ = orc.route_topk(logits.cpu().numpy(), top_k)
    np.testing.assert_array_equal(fi.cpu().numpy(), eids)


@pytest.mark.parametrize("experts,tokens,top_k,tied", [(128, 16, 8, False), (128, 32, 8, True), (100, 12, 8, True),
                                                        (64, 20, 12, False)])
def test_three_launch_routed_layer_matches_router_kernel(cuda, experts, tokens, top_k, tied):
    """Routed calls past the single-launch limit (65-256 pairs) route in the
    prep kernel, one wave per token: ids and weights equal the router
    kernel's, the output equals the expert call on those routes, and no
    status bit is raised (every token's slots are in place before they are
    validated)."""
    print_case("three-launch routed layer", experts, tokens, top_k, tied)
    g = torch.Generator().manual_seed(4242 + experts + tokens)
    staged = to_device(random_fp8_bank(experts, 1024, 256, layout="channel", generator=g), cuda)
    x = torch.randn(tokens, 1024, generator=g).bfloat16().to(cuda)
    logits = (torch.randint(0, 8, (tokens, experts), generator=g).float() / 4.0 if tied
              else torch.randn(tokens, experts, generator=g)).to(cuda)
    backend = HipExpertBackend()
    backend.status(cuda)
    out, w, ids = backend.forward_routed(x, logits, top_k, staged)
    rw, rids = router.route_topk(logits, top_k)
    torch.cuda.synchronize()
    assert backend.status(cuda) == 0
    assert torch.equal(ids, rids) and torch.equal(w, rw)
    assert torch.equal(out, backend.forward(x, rids, rw, staged))


def test_fused_pairs_shared_row_and_quantized_handoff(cuda, decode_mode):
    print_case("fused pairs")
    g = torch.Generator().manual_seed(4040)
    staged = to_device(random_fp8_bank(16, 2048, 768, generator=g), cuda)
    x = torch.randn(1, 2048, generator=g).bfloat16().to(cuda)
    ids = torch.tensor([3, 9, 3, 0, 15, 2], device=cuda)
    weights = torch.softmax(torch.randn(6, generator=g), -1).to(cuda)
    backend = HipExpertBackend()
    fused, three = both(decode_mode, lambda: backend.forward_pairs(x.expand(6, -1), ids[:, None], weights[:, None],
                                                                   staged))
    assert torch.equal(fused, three)
    b13, b2 = oracle_banks(staged)
    ref = orc.fp8_expert_pairs(b13, b2, x[0].float().cpu().numpy(), ids.cpu().numpy(), weights.cpu().numpy())
    assert rel_inf(fused.cpu().numpy(), ref) < TOL
    q, s = fp8_moe.quantize_groups(fp8_moe.quant_kernel, x, 2048)
    hf, hs = both(decode_mode, lambda: fp8_decode.quantized_pairs(fp8_moe, q, s, ids, weights, staged))
    assert torch.equal(hf, hs) and torch.equal(hf, fused)


def test_fused_invalid_ids_contribute_zero_and_raise_status(cuda, decode_mode):
    print_case("fused invalid ids")
    staged = to_device(random_fp8_bank(4, 256, 256, generator=torch.Generator().manual_seed(3)), cuda)
    backend = HipExpertBackend()
    backend.status(cuda)
    x = torch.randn(1, 256, device=cuda).bfloat16()
    good = backend.forward(x, torch.tensor([[2, 1]], device=cuda), torch.tensor([[0.5, 0.5]], device=cuda), staged)
    assert backend.status(cuda) == 0
    bad = backend.forward(x, torch.tensor([[2, 1, 7]], device=cuda), torch.tensor([[0.5, 0.5, 0.5]], device=cuda),
                          staged)
    assert backend.status(cuda) & _lib.STATUS_BAD_EXPERT_ID
    torch.testing.assert_close(bad, good, rtol=0, atol=0)


def test_fused_repeated_calls_rearm_the_grid_counters(cuda):
    """Hundreds of back-to-back single-launch calls (eager and graph-replayed)
    stay identical: each call derives its own epoch from the call counters,
    never accepts an older call's hand-off words, and no wait times out."""
    print_case("fused repeated calls")
    g = torch.Generator().manual_seed(99)
    staged = to_device(random_fp8_bank(128, 2048, 768, layout="channel", generator=g), cuda)
    backend = HipExpertBackend()
    backend.status(cuda)
    x = torch.randn(1, 2048, generator=g).bfloat16().to(cuda)
    logits = torch.randn(1, 128, generator=g).to(cuda)
    first, _, _ = backend.forward_routed(x, logits, 8, staged)
    out = torch.empty_like(x)
    for _ in range(200):
        backend.forward_routed(x, logits, 8, staged, out=out)
    torch.cuda.synchronize()
    assert torch.equal(out, first)
    stream = torch.cuda.Stream(cuda)
    stream.wait_stream(torch.cuda.current_stream(cuda))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for _ in range(16):
            backend.forward_routed(x, logits, 8, staged, out=out)
    for _ in range(8):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, first)
    assert backend.status(cuda) == 0


def test_sync_timeout_is_reported_and_every_kernel_exits(cuda):
    """The host forces the single-launch decode's bounded hand-off wait to
    give up: with the diagnostic switch on, readers wait for a tag no producer
    writes, so each wait runs to a 100 us bound.  The status word then carries
    DMOE_STATUS_SYNC_TIMEOUT and every launch still completes; with the switch
    off and the default bound restored the next call is exact again."""
    print_case("forced sync timeout")
    lib = _lib.library()
    g = torch.Generator().manual_seed(123)
    staged = to_device(random_fp8_bank(128, 2048, 768, layout="channel", generator=g), cuda)
    backend = HipExpertBackend()
    x = torch.randn(1, 2048, generator=g).bfloat16().to(cuda)
    logits = torch.randn(1, 128, generator=g).to(cuda)
    expected, _, _ = backend.forward_routed(x, logits, 8, staged)
    torch.cuda.synchronize()
    assert backend.status(cuda) == 0
    previous = lib.dmoe_set_sync_spin_limit(10_000)  # 100 us of the 100 MHz counter
    forced = lib.dmoe_debug_force_sync_timeout(1)
    try:
        for _ in range(2):
            backend.forward_routed(x, logits, 8, staged)
        torch.cuda.synchronize()
    finally:
        lib.dmoe_debug_force_sync_timeout(forced)
        lib.dmoe_set_sync_spin_limit(previous)
    assert backend.status(cuda) & _lib.STATUS_SYNC_TIMEOUT
    again, _, _ = backend.forward_routed(x, logits, 8, staged)
    torch.cuda.synchronize()
    assert backend.status(cuda) == 0
    assert torch.equal(again, expected)


def test_decode_after_prefill_on_one_workspace(cuda, decode_mode):
    """A 2048-token grouped call and then a 1-token single-launch call on the
    same per-device workspace: the grouped call's permutation and tile map
    never reach the decode's hand-off words, so the decode equals the
    three-launch decode bit for bit."""
    print_case("decode after prefill, shared workspace")
    g = torch.Generator().manual_seed(321)
    staged = to_device(random_fp8_bank(128, 2048, 768, layout="channel", generator=g), cuda)
    backend = HipExpertBackend()
    xs = torch.randn(2048, 2048, generator=g).bfloat16().to(cuda)
    big_logits = torch.randn(2048, 128, generator=g).to(cuda)
    x = torch.randn(1, 2048, generator=g).bfloat16().to(cuda)
    logits = torch.randn(1, 128, generator=g).to(cuda)

    def run():
        backend.forward_routed(xs, big_logits, 8, staged)
        out, _, _ = backend.forward_routed(x, logits, 8, staged)
        return out

    fused, staged_out = both(decode_mode, run)
    assert torch.equal(fused, staged_out)
    assert backend.status(cuda) == 0


def test_single_launch_decodes_on_two_streams_with_own_workspaces(cuda):
    """Direct C-ABI callers with a workspace each issue single-launch decodes
    on two streams back to back, without ordering them: the library orders
    the persistent launches itself (each waits for the previous one on
    another stream), so none waits for workgroups the other keeps out --
    every call is exact and no status bit is raised, where two concurrent
    launches could only end in the hand-off bound."""
    import ctypes

    from drama_moe.formats import fp8_bank_struct

    print_case("fused decodes on two streams")
    lib = _lib.library()
    g = torch.Generator().manual_seed(404)
    staged = to_device(random_fp8_bank(128, 2048, 768, layout="channel", generator=g), cuda)
    bank = fp8_bank_struct(staged)
    size = lib.dmoe_fp8_workspace_bytes(ctypes.byref(bank), 8)
    workspaces = [torch.zeros(size, dtype=torch.uint8, device=cuda) for _ in range(2)]
    status = torch.zeros(1, dtype=torch.int32, device=cuda)
    calls = 12
    xs = torch.randn(calls, 1, 2048, generator=g).bfloat16().to(cuda)
    logits = torch.randn(calls, 1, 128, generator=g).to(cuda)
    outs = torch.empty_like(xs)
    ids = torch.empty(calls, 1, 8, dtype=torch.int64, device=cuda)
    weights = torch.empty(calls, 1, 8, dtype=torch.bfloat16, device=cuda)

    def layer(i, stream, ws):
        _lib.check(lib.dmoe_fp8_moe_layer(
            ctypes.byref(bank), _lib.ptr(xs[i]), _lib.BF16, 2048, 1, _lib.ptr(logits[i]), 128, 8, 1,
            _lib.ptr(ids[i]), _lib.ptr(weights[i]), _lib.BF16, 128, _lib.BF16, _lib.ptr(outs[i]), _lib.BF16, 2048,
            _lib.ptr(ws), ws.numel(), _lib.ptr(status), ctypes.c_void_p(stream.cuda_stream)))

    streams = [torch.cuda.Stream(cuda), torch.cuda.Stream(cuda)]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream(cuda))
    for i in range(calls):
        layer(i, streams[i % 2], workspaces[i % 2])
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    backend = HipExpertBackend()
    for i in range(calls):
        want, _, _ = backend.forward_routed(xs[i], logits[i], 8, staged)
        assert torch.equal(outs[i], want), i


def test_manager_reports_a_given_up_hand_off_at_its_sync(cuda):
    """ResidentExpertManager(validate_ids=True) reads the device status word
    at the host sync it already has: after a call whose hand-off wait gave
    up (forced from the host with a 100 us bound), the next call raises
    instead of returning with the earlier output silently invalid."""
    from drama_moe.offload import ResidentExpertManager

    print_case("manager status surfacing")

    class Experts(torch.nn.Module):
        fp8 = True

        def __init__(self, bank):
            super().__init__()
            for name, tensor in bank.buffers().items():
                self.register_buffer(name, tensor)

    lib = _lib.library()
    g = torch.Generator().manual_seed(505)
    module = Experts(to_device(random_fp8_bank(16, 512, 256, layout="channel", generator=g), cuda))
    manager = ResidentExpertManager(backend=HipExpertBackend())
    manager.attach("0", module)
    x = torch.randn(1, 512, generator=g).bfloat16().to(cuda)
    ids = torch.tensor([[3, 1, 7, 2, 6, 0, 4, 5]], device=cuda)
    w = torch.full((1, 8), 0.125, dtype=torch.bfloat16, device=cuda)
    try:
        good = module(x, ids, w)
        previous = lib.dmoe_set_sync_spin_limit(10_000)
        forced = lib.dmoe_debug_force_sync_timeout(1)
        try:
            module(x, ids, w)
        finally:
            lib.dmoe_debug_force_sync_timeout(forced)
            lib.dmoe_set_sync_spin_limit(previous)
        with pytest.raises(RuntimeError, match="gave up its hand-off wait"):
            module(x, ids, w)
        assert torch.equal(module(x, ids, w), good)  # the status was cleared; the next call is exact
    finally:
        manager.close()


def test_phase_timing_instance_gives_the_same_bits_and_ordered_stamps(cuda):
    """dmoe_debug_set_phase_buffer swaps in the kernel's timing instance: its
    outputs equal the ordinary kernel's bit for bit, every workgroup stamps
    its seven phases in order, and clearing the buffer restores the ordinary
    kernel (the buffer is no longer written)."""
    print_case("fused phase timing instance")
    lib = _lib.library()
    g = torch.Generator().manual_seed(606)
    staged = to_device(random_fp8_bank(128, 2048, 768, layout="channel", generator=g), cuda)
    x = torch.randn(1, 2048, generator=g).bfloat16().to(cuda)
    logits = torch.randn(1, 128, generator=g).to(cuda)
    backend = HipExpertBackend()
    plain, _, _ = backend.forward_routed(x, logits, 8, staged)
    cus = torch.cuda.get_device_properties(cuda).multi_processor_count
    buf = torch.zeros(cus * 7, dtype=torch.int64, device=cuda)
    _lib.check(lib.dmoe_debug_set_phase_buffer(_lib.ptr(buf), buf.numel()))
    try:
        timed, _, _ = backend.forward_routed(x, logits, 8, staged)
        torch.cuda.synchronize()
    finally:
        _lib.check(lib.dmoe_debug_set_phase_buffer(None, 0))
    assert torch.equal(timed, plain)
    stamps = buf.view(cus, 7).cpu()
    assert bool((stamps > 0).all())
    assert bool((stamps[:, 1:] >= stamps[:, :-1]).all())
    buf.zero_()
    again, _, _ = backend.forward_routed(x, logits, 8, staged)
    torch.cuda.synchronize()
    assert torch.equal(again, plain) and int(buf.abs().sum()) == 0
    assert int(backend.status(cuda)) == 0
