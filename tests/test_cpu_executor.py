"""The cooperative decode's host side on the CPU (no GPU): the C++ expert
executor behind dmoe_cpu_expert_pairs and the route planner.

The executor follows the FP8 decode kernels' arithmetic step for step, so it
is checked three ways here: its scalar, AVX2 and AVX-512 block products give
the same bits; it equals, bit for bit, an independent numpy statement of that
arithmetic (fp32 block products in the fixed lane order, glibc's correctly
rounded fmaf for the block chains, the 8-wave K split of gate/up, bf16 gate/up, SiLU
by table, E4M3 hidden groups through torch's float8 conversion); and it is
within the path's 2e-2 bar of the oracle (the reference contract, which
chains gate/up blocks in one sequence).  The guard's known answer: a hidden
value landing exactly on the E4M3 midpoint 42.0 is reported for GPU
recompute.  Route planning follows hybrid_layer.py:17-28 and the reference's
own cases (tests/test_hybrid_layer.py:12-32).
"""
import ctypes
import ctypes.util

import numpy as np
import pytest
import torch

from drama_moe import _lib
from drama_moe.formats import StagedExperts, random_fp8_bank
from drama_moe.hybrid import (CpuExpertExecutor, CpuQuantizationBoundary, native_partition_routes,
                              partition_routes)
from oracle import oracle as orc

TOL = 2e-2
_libm = ctypes.CDLL(ctypes.util.find_library("m"))
_libm.fmaf.argtypes = [ctypes.c_float, ctypes.c_float, ctypes.c_float]
_libm.fmaf.restype = ctypes.c_float


def host_silu_table():
    g = (torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)).float().numpy()
    with np.errstate(over="ignore", invalid="ignore"):
        return torch.from_numpy((g / (np.float32(1) + np.exp(-g))).astype(np.float32))


def available_isas():
    names = ["scalar"]
    for name in ("avx2", "avx512"):
        try:
            CpuExpertExecutor(random_fp8_bank(1, 128, 128), silu_table=host_silu_table(), implementation=name).close()
            names.append(name)
        except ValueError:
            pass
    return names


def quantized_row(hidden, seed, group=128):
    x = torch.randn(1, hidden, generator=torch.Generator().manual_seed(seed)).bfloat16().float().numpy()
    q, s = orc.quantize_fp8(x, group)
    return torch.from_numpy(q.reshape(-1).copy()), torch.from_numpy(s.reshape(-1).copy()), x


def e4m3(v):
    return torch.from_numpy(np.clip(np.asarray(v, np.float32), -448, 448)).to(torch.float8_e4m3fn).float().numpy()


def scales_of(t: torch.Tensor, e: int, n: int, kb: int, rows: int, cols: int) -> np.float32:
    s = t[e]
    return np.float32(s[n // (rows // s.shape[0]), kb // ((cols // 128) // s.shape[1])])


def emulate(store: StagedExperts, xq: np.ndarray, xs: np.ndarray, ids, weights, table: np.ndarray):
    """The decode kernels' arithmetic for one FP8 row, in numpy."""
    H, I = store.hidden, store.intermediate
    w13 = store.w13_weight.float().numpy()
    w2 = store.w2_weight.float().numpy()
    xdec = orc.fp8_decode(xq).astype(np.float64)
    KB, KBd = H // 128, I // 128
    out = np.empty((len(ids), H), np.float32)

    def dot(w, x):  # fp32 lane l sums the (exact) products k = l, l + 16, ...; the lanes fold in halves
        products = (w.astype(np.float32) * x.astype(np.float32)).reshape(8, 16)
        lanes = np.zeros(16, np.float32)
        for step in products:
            lanes = (lanes + step).astype(np.float32)
        for width in (8, 4, 2, 1):
            lanes[:width] = lanes[:width] + lanes[width:2 * width]
        return np.float32(lanes[0])

    for j, (e, wt) in enumerate(zip(ids, weights)):
        h = np.empty(I, np.float32)
        for n in range(I):
            gu = []
            for row in (n, I + n):
                total = np.float32(0)
                for w in range(8):
                    acc = np.float32(0)
                    for kb in range(w, KB, 8):
                        d = dot(w13[e, row, kb * 128:(kb + 1) * 128], xdec[kb * 128:(kb + 1) * 128])
                        sx = np.float32(xs[kb if xs.size > 1 else 0])
                        acc = np.float32(_libm.fmaf(float(np.float32(d * sx)),
                                                    float(scales_of(store.w13_scale_inv, e, row, kb, 2 * I, H)),
                                                    float(acc)))
                    total = acc if w == 0 else np.float32(total + acc)
                gu.append(torch.tensor([float(total)]).bfloat16())
            g, u = gu
            h[n] = np.float32(table[int(g.view(torch.int16).item()) & 0xFFFF] * np.float32(u.float().item()))
        hq = np.empty(I, np.float32)
        hs = np.empty(KBd, np.float32)
        for g in range(KBd):
            grp = h[g * 128:(g + 1) * 128]
            scale = np.float32(max(np.float32(np.max(np.abs(grp))), np.float32(1e-10)) * np.float32(1.0 / 448.0))
            hs[g] = scale
            hq[g * 128:(g + 1) * 128] = e4m3((grp / scale).astype(np.float32))
        for m in range(H):
            acc = np.float32(0)
            for kb in range(KBd):
                d = dot(w2[e, m, kb * 128:(kb + 1) * 128], hq[kb * 128:(kb + 1) * 128].astype(np.float64))
                acc = np.float32(_libm.fmaf(float(np.float32(d * hs[kb])),
                                            float(scales_of(store.w2_scale_inv, e, m, kb, H, I)), float(acc)))
            out[j, m] = np.float32(acc * np.float32(wt))
    return out


@pytest.mark.parametrize("layout", ["block", "channel"])
def test_every_isa_gives_the_same_bits(layout):
    store = random_fp8_bank(6, 512, 256, layout=layout, generator=torch.Generator().manual_seed(3))
    q, s, _ = quantized_row(512, 4)
    ids = torch.tensor([5, 0, 3, 3, 1], dtype=torch.int64)
    w = torch.rand(5, generator=torch.Generator().manual_seed(5)).float()
    table = host_silu_table()
    results = {}
    for isa in available_isas():
        ex = CpuExpertExecutor(store, silu_table=table, implementation=isa, threads=3)
        assert ex.implementation == isa
        results[isa] = ex.forward_quantized_pairs(q, s, ids, w)
        ex.close()
    first = next(iter(results.values()))
    for isa, out in results.items():
        assert torch.equal(out, first), isa


@pytest.mark.parametrize("layout,hidden,inter,group", [("block", 1024, 256, 128), ("channel", 256, 384, 128),
                                                       ("channel", 512, 128, "row")])
def test_executor_equals_numpy_statement_of_the_decode_arithmetic(layout, hidden, inter, group):
    store = random_fp8_bank(4, hidden, inter, layout=layout, generator=torch.Generator().manual_seed(hidden))
    q, s, _ = quantized_row(hidden, 7, 128 if group == 128 else hidden)
    ids = [2, 0, 3]
    w = np.float32([0.5, 0.25, 0.125])
    table = host_silu_table()
    ex = CpuExpertExecutor(store, silu_table=table, threads=4)
    got = ex.forward_quantized_pairs(q, s, torch.tensor(ids), torch.from_numpy(w)).numpy()
    ex.close()
    want = emulate(store, q.numpy(), s.numpy(), ids, w, table.numpy())
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("threads", [1, 8])
def test_executor_within_bar_of_the_oracle_at_layer_shape(threads):
    g = torch.Generator().manual_seed(20261201)
    store = random_fp8_bank(8, 2048, 768, layout="block", generator=g)
    q, s, x = quantized_row(2048, 11)
    ids = torch.tensor([7, 2, 5, 0], dtype=torch.int64)
    w = torch.tensor([0.4, 0.3, 0.2, 0.1])
    ex = CpuExpertExecutor(store, silu_table=host_silu_table(), threads=threads)
    got = ex.forward_quantized_pairs(q, s, ids, w).numpy()
    ex.close()
    b13 = orc.Fp8Bank(store.w13_weight.view(torch.uint8).numpy(), store.w13_scale_inv.numpy())
    b2 = orc.Fp8Bank(store.w2_weight.view(torch.uint8).numpy(), store.w2_scale_inv.numpy())
    want = orc.fp8_expert_pairs(b13, b2, x, ids.numpy(), w.numpy())
    err = float(np.max(np.abs(got - want)) / np.max(np.abs(want)))
    assert err < TOL


def _tie_bank():
    """One expert, H = I = 128, unit per-channel scales.  With activation
    bytes of 1.0, gate row n sums its weights (all zero: silu table forced to
    1 below) and up row n carries 448 (n = 0), 42 = 32 + 8 + 2 (n = 1) or 0,
    so h = [448, 42, 0, ...]: scale 448 * fl(1/448) = 1 and h[1] / scale lands
    exactly on the E4M3 midpoint between 40 and 44."""
    H = I = 128
    w13 = torch.zeros(1, 2 * I, H)
    w13[0, I + 0, 0] = 448.0
    w13[0, I + 1, :3] = torch.tensor([32.0, 8.0, 2.0])
    w2 = torch.zeros(1, H, I)
    w2[0, :, 1] = 1.0  # every output row reads h[1]
    return StagedExperts(w13.to(torch.float8_e4m3fn), torch.ones(1, 2 * I, 1), w2.to(torch.float8_e4m3fn),
                         torch.ones(1, H, 1))


def test_guard_reports_the_e4m3_midpoint_and_rounds_it_to_even_without_guard():
    store = _tie_bank()
    q = torch.full((128,), 0x38, dtype=torch.uint8)  # E4M3 1.0
    s = torch.ones(1, dtype=torch.float32)
    s = torch.ones(1)
    ones = torch.ones(65536)
    ids, w = torch.tensor([0]), torch.tensor([1.0])
    guarded = CpuExpertExecutor(store, silu_table=ones, guard_fp8_boundaries=True)
    with pytest.raises(CpuQuantizationBoundary):
        guarded.forward_quantized_pairs(q, s, ids, w)
    guarded.close()
    plain = CpuExpertExecutor(store, silu_table=ones)
    out = plain.forward_quantized_pairs(q, s, ids, w)
    plain.close()
    # h[1] = 42 -> E4M3 40 (ties to the even mantissa), times scale 1, times w2 = 1
    assert torch.equal(out, torch.full((1, 128), 40.0))


def test_executor_validates_before_any_work():
    store = random_fp8_bank(2, 256, 128)
    q, s, _ = quantized_row(256, 1)
    ex = CpuExpertExecutor(store, silu_table=host_silu_table(), capacity=2)
    with pytest.raises(ValueError, match="outside the bank"):
        ex.forward_quantized_pairs(q, s, torch.tensor([0, 2]), torch.tensor([1.0, 1.0]))
    with pytest.raises(ValueError, match="Invalid host route"):
        ex.forward_quantized_pairs(q, s, torch.tensor([0, 1, 1]), torch.tensor([1.0, 1.0, 1.0]))
    with pytest.raises(ValueError, match="non-finite route weight"):
        ex.forward_quantized_pairs(q, s, torch.tensor([0]), torch.tensor([float("nan")]))
    other = random_fp8_bank(2, 512, 128)
    with pytest.raises(ValueError, match="geometry"):
        ex.forward_quantized_pairs(q, s, torch.tensor([0]), torch.tensor([1.0]), store=other)
    ex.close()
    with pytest.raises(RuntimeError, match="closed"):
        ex.forward_quantized_pairs(q, s, torch.tensor([0]), torch.tensor([1.0]))
    with pytest.raises(ValueError, match="unavailable|Unknown"):
        CpuExpertExecutor(store, silu_table=host_silu_table(), implementation="neon")
    assert _lib.library().dmoe_cpu_executor_create(100, 128, 8, 4, 0) is None
    assert b"geometry" in _lib.library().dmoe_last_error()


@pytest.mark.parametrize("count", [0, 1, 2, 4, 8])
def test_partition_keeps_every_slot_once(count):
    # tests/test_hybrid_layer.py:12-20
    ids = [6, 3, 6, 2, 1, 3, 7, 0]
    for planner in (lambda: partition_routes(ids, {3: 0, 0: 1}, count),
                    lambda: native_partition_routes(ids, {3, 0}, 8, count)):
        cpu, gpu = planner()
        assert len(cpu) == count
        assert cpu == sorted(cpu) and gpu == sorted(gpu)
        assert sorted(cpu + gpu) == list(range(8))
        if count <= 6:
            assert all(ids[slot] not in (3, 0) for slot in cpu)


def test_partition_prefers_cold_routes_then_hot_and_checks_bounds():
    # tests/test_hybrid_layer.py:23-28
    assert partition_routes([1, 2, 3, 4], {4: 0}, 2) == ([1, 2], [0, 3])
    assert partition_routes([1, 2, 3, 4], {4: 0}, 4) == ([0, 1, 2, 3], [])
    assert native_partition_routes([1, 2, 3, 4], {4}, 8, 2) == ([1, 2], [0, 3])
    assert native_partition_routes([1, 2, 3, 4], {4}, 8, 4) == ([0, 1, 2, 3], [])
    with pytest.raises(ValueError, match="route count"):
        partition_routes([1], {}, 2)
    with pytest.raises(ValueError, match="bad counts"):
        native_partition_routes([1], set(), 8, 2)
    with pytest.raises(ValueError, match="outside the bank"):
        native_partition_routes([9], set(), 8, 1)
