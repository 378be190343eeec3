"""GPU tests of the cooperative decode (host cores take the lowest-ranked route
slots of a one-token FP8 layer call; the reference's HybridDecodeRuntime,
src/drama_low_vram/hybrid_decode.py:33-416, and its tests
tests/test_hybrid_decode.py).

Bars: the GPU slots are the resident path's own partials, bit for bit; the
host slots follow the decode kernels' arithmetic with fp32 block products
in a fixed lane order (the device's FP8 MFMA truncates inside groups of 8 products), so
they and the layer output are within 2e-2 of the all-GPU resident call and
of the oracle.  A call is deterministic: repeats, other streams and
asynchronous returns give the same bits.  The boundary guard's GPU
recompute, scratch reuse across streams, eligibility and close are checked
as the reference's tests do.
"""
from concurrent.futures import ThreadPoolExecutor
from threading import Event
from unittest.mock import patch

import numpy as np
import pytest
import torch

from conftest import print_case
from drama_moe.formats import random_fp8_bank
from drama_moe.hybrid import CpuQuantizationBoundary
from drama_moe.offload import HipExpertBackend, ResidentExpertManager
from oracle import oracle as orc

pytestmark = pytest.mark.gpu
TOL = 2e-2


class Experts(torch.nn.Module):
    """An expert module holding its FP8 bank in host memory."""
    fp8 = True

    def __init__(self, bank):
        super().__init__()
        for name, tensor in bank.buffers().items():
            self.register_buffer(name, tensor)

    def forward(self, *_args):
        raise AssertionError("the manager runs the experts")


def make_manager(layers, *, experts=128, hidden=2048, inter=768, layout="channel", seed=20261210):
    manager = ResidentExpertManager(backend=HipExpertBackend())
    banks = []
    for i in range(layers):
        bank = random_fp8_bank(experts, hidden, inter, layout=layout,
                               generator=torch.Generator().manual_seed(seed + i))
        banks.append(bank)
        manager.attach(str(i), Experts(bank))
    return manager, banks


def inputs(cuda, hidden=2048, experts=128, top_k=8, seed=219):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(1, hidden, generator=g).bfloat16().to(cuda)
    ids, w = orc.route_topk(torch.randn(1, experts, generator=g).numpy(), top_k)
    return x, torch.from_numpy(ids).to(cuda), torch.from_numpy(w).bfloat16().to(cuda)


def rel_inf(actual, expected):
    actual = np.asarray(actual, np.float64)
    expected = np.asarray(expected, np.float64)
    return float(np.max(np.abs(actual - expected)) / max(np.max(np.abs(expected)), 1e-30))


def device_pairs(manager, module, bank, x, ids, w, cuda):
    count = ids.numel()
    return HipExpertBackend().forward_pairs(x.expand(count, -1), ids.reshape(count, 1),
                                            w.reshape(count, 1).float(), manager._on_device(module, bank, cuda))


@pytest.mark.parametrize("layout,jobs,top_k", [("channel", 4, 8), ("channel", 8, 8), ("block", 1, 8),
                                               ("block", 3, 4)])
def test_hybrid_layer_matches_resident_call_and_oracle(cuda, layout, jobs, top_k):
    print_case("hybrid layer", layout, jobs, top_k)
    manager, banks = make_manager(2, layout=layout)
    try:
        modules = list(manager.modules.values())
        x, ids, w = inputs(cuda, top_k=top_k)
        expected = [m(x, ids, w) for m in modules]
        torch.cuda.synchronize()
        hybrid = manager.configure_hybrid_decode(jobs, threads=8)
        first = None
        for repeat in range(2):
            with hybrid.decode():
                actual = [m(x, ids, w) for m in modules]
            torch.cuda.synchronize()
            if first is None:
                first = actual
            for a, f, e in zip(actual, first, expected):
                assert torch.equal(a, f), repeat  # deterministic
                assert rel_inf(a.float().cpu().numpy(), e.float().cpu().numpy()) < TOL
        # the last call's ordered partials: GPU slots bit-exact with the resident pairs
        cpu_slots = set(range(top_k - min(jobs, top_k), top_k))
        ordered = hybrid._buffers["ordered"][:top_k]
        want = device_pairs(manager, modules[1], banks[1], x, ids, w, cuda)
        for slot in range(top_k):
            if slot in cpu_slots:
                assert rel_inf(ordered[slot].cpu().numpy(), want[slot].cpu().numpy()) < TOL, slot
            else:
                assert torch.equal(ordered[slot], want[slot]), slot
        assert hybrid.stats.calls == 4 and hybrid.stats.cpu_pairs == 4 * min(jobs, top_k)
        b13 = orc.Fp8Bank(banks[0].w13_weight.view(torch.uint8).numpy(), banks[0].w13_scale_inv.numpy())
        b2 = orc.Fp8Bank(banks[0].w2_weight.view(torch.uint8).numpy(), banks[0].w2_scale_inv.numpy())
        want0 = orc.fp8_moe_forward(b13, b2, x.float().cpu().numpy(), ids.cpu().numpy(), w.float().cpu().numpy())
        assert rel_inf(actual[0].float().cpu().numpy(), want0) < TOL
        report = hybrid.report()
        assert report["device_workspace_bytes"] == 2 * 8 * 2048 * 4 and report["pinned_workspace_bytes"] < 80000
    finally:
        manager.close()


def test_host_slots_match_device_pairs(cuda):
    """The executor's partials against the decode kernels' own pair rows for
    the same FP8 row, every route slot on the host."""
    print_case("hybrid host slots vs device pairs")
    manager, banks = make_manager(1, layout="block")
    try:
        hybrid = manager.configure_hybrid_decode(8, threads=8, guard_fp8_boundaries=False)
        from drama_moe import fp8_moe

        x, ids, w = inputs(cuda, seed=5)
        q, s = fp8_moe.quantize_groups(fp8_moe.quant_kernel, x, x.shape[1])
        dev = device_pairs(manager, list(manager.modules.values())[0], banks[0], x, ids, w, cuda)
        host = hybrid.executor.forward_quantized_pairs(q.view(torch.uint8).cpu().reshape(-1).contiguous(),
                                                       s.cpu().reshape(-1).contiguous(), ids.cpu().reshape(-1),
                                                       w.float().cpu().reshape(-1), store=banks[0])
        for slot in range(8):
            err = rel_inf(host[slot].numpy(), dev[slot].cpu().numpy())
            print(f"slot {slot}: rel err {err:.2e}, equal values {float((host[slot] == dev[slot].cpu()).float().mean()):.3f}")
            assert err < TOL
    finally:
        manager.close()


@pytest.mark.parametrize("jobs", [4, 8])
def test_guard_recomputes_host_slots_on_the_gpu(cuda, jobs):
    print_case("hybrid guard", jobs)
    manager, _ = make_manager(1, experts=16, hidden=512, inter=256)
    try:
        module = list(manager.modules.values())[0]
        x, ids, w = inputs(cuda, hidden=512, experts=16)
        expected = module(x, ids, w)
        hybrid = manager.configure_hybrid_decode(jobs, threads=2)
        with hybrid.decode():
            with patch.object(hybrid.executor, "forward_quantized_pairs",
                              side_effect=CpuQuantizationBoundary("forced midpoint")):
                actual = module(x, ids, w)
            assert torch.equal(actual, expected)
            assert hybrid.stats.boundary_fallback_calls == 1
            assert hybrid.stats.boundary_recomputed_pairs == jobs
            assert hybrid.stats.gpu_pairs == 8 and hybrid.stats.partial_h2d_bytes == 0
            # the next call runs its host slots again
            again = module(x, ids, w)
            assert rel_inf(again.float().cpu().numpy(), expected.float().cpu().numpy()) < TOL
            assert hybrid.stats.cpu_pairs == 2 * jobs
    finally:
        manager.close()


@pytest.mark.parametrize("synchronize_return", [False, True])
def test_shared_scratch_across_streams_and_release(cuda, synchronize_return):
    """No host waits between calls with an asynchronous return: the shared
    buffers are fenced by stream dependencies (test_hybrid_decode.py:151-180)."""
    print_case("hybrid streams", synchronize_return)
    manager, _ = make_manager(3, experts=16, hidden=512, inter=256)
    try:
        modules = list(manager.modules.values())
        x, ids, w = inputs(cuda, hidden=512, experts=16)
        reference = manager.configure_hybrid_decode(2, threads=2)
        with reference.decode():
            expected = [m(x, ids, w).clone() for m in modules]
        torch.cuda.synchronize()
        hybrid = manager.configure_hybrid_decode(2, threads=2, synchronize_return=synchronize_return)
        streams = [torch.cuda.Stream(cuda), torch.cuda.Stream(cuda)]
        actual = []
        for repeat in range(4):
            for index, module in enumerate(modules):
                with torch.cuda.stream(streams[(repeat + index) % 2]), hybrid.decode():
                    torch.cuda._sleep(100000)
                    actual.append((index, module(x, ids, w)))
        hybrid.release_runtime_buffers()
        assert not hybrid._pending and not hybrid._buffers
        torch.cuda.synchronize()
        for index, out in actual:
            assert torch.equal(out, expected[index])
        assert hybrid.stats.completion_host_waits == (12 if synchronize_return else 0)
        assert hybrid.stats.completion_stream_waits == (0 if synchronize_return else 11)
        with hybrid.decode():
            assert torch.equal(modules[0](x, ids, w), expected[0])
        assert hybrid.stats.workspace_allocations == 2
    finally:
        manager.close()


def test_only_decode_scoped_one_token_calls_are_eligible(cuda):
    print_case("hybrid eligibility")
    manager, _ = make_manager(2, experts=16, hidden=512, inter=256)
    try:
        modules = list(manager.modules.values())
        x, ids, w = inputs(cuda, hidden=512, experts=16)
        hybrid = manager.configure_hybrid_decode(4, threads=2)
        modules[0](x, ids, w)  # outside decode(): the GPU path
        assert hybrid.stats.calls == 0
        two = torch.cat([x, x])
        with hybrid.decode():
            modules[0](two, torch.cat([ids, ids]), torch.cat([w, w]))  # two tokens: not eligible
            modules[0](x.float(), ids, w)                              # fp32 rows: not eligible
        assert hybrid.stats.calls == 0 and hybrid.stats.fallbacks == 2
        with hybrid.decode(layers=[1]):
            modules[0](x, ids, w)
            modules[1](x, ids, w)
        assert hybrid.stats.calls == 1
        with hybrid.suspend(), hybrid.decode():
            assert not hybrid.eligible(modules[0], x, ids)
        with hybrid.decode():
            with ThreadPoolExecutor(max_workers=1) as worker:  # scopes are per thread
                assert not worker.submit(hybrid.eligible, modules[0], x, ids).result()
            bad = ids.clone()
            bad[0, 0] = 99
            with pytest.raises(ValueError, match="outside bank"):
                modules[0](x, bad, w)
        manager.configure_hybrid_decode(0)
        assert manager.hybrid_decode is None and hybrid._closed
    finally:
        manager.close()


def test_close_waits_for_inflight_host_work(cuda):
    print_case("hybrid close")
    manager, _ = make_manager(1, experts=16, hidden=512, inter=256)
    try:
        module = list(manager.modules.values())[0]
        x, ids, w = inputs(cuda, hidden=512, experts=16)
        hybrid = manager.configure_hybrid_decode(4, threads=2)
        with hybrid.decode():
            expected = module(x, ids, w).clone()
        entered, release = Event(), Event()
        original = hybrid.executor.forward_quantized_pairs

        def delayed(*args, **kwargs):
            entered.set()
            if not release.wait(timeout=10):
                raise RuntimeError("test worker was not released")
            return original(*args, **kwargs)

        def forward():
            with hybrid.decode():
                return module(x, ids, w)

        with patch.object(hybrid.executor, "forward_quantized_pairs", delayed), \
                ThreadPoolExecutor(max_workers=2) as workers:
            pending = workers.submit(forward)
            try:
                assert entered.wait(timeout=10)
                closing = workers.submit(hybrid.close)
                assert not closing.done()
            finally:
                release.set()
            assert torch.equal(pending.result(timeout=30), expected)
            closing.result(timeout=30)
        assert hybrid._closed and not hybrid._buffers
    finally:
        manager.close()
