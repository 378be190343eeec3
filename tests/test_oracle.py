"""Pin the CPU oracle before trusting it (CPU only).

Every oracle function is checked against something it does not share code
with: torch's own float8/bfloat16/float16 conversions, the reference's own CPU
executor compiled from its sources (oracle/_ref, when present), committed
golden vectors written by that executor, closed forms (orthogonality of the
H256 rotation, exact integer dots, monotone softmax) and brute force in
float64.  Scenario seeds and shapes follow the reference's tests
(tests/test_native_backend.py, tests/test_quantized_kernels.py,
tests/test_offload.py, tests/test_hybrid_layer.py).
"""
from pathlib import Path

import numpy as np
import pytest
import torch

from drama_moe.formats import random_fp8_bank
from oracle import oracle as orc
from oracle import ref_native

GOLDEN = Path(__file__).resolve().parent / "golden"


@pytest.fixture(scope="module", autouse=True)
def built():
    orc.build()


def bf16_values(t: torch.Tensor) -> np.ndarray:
    return t.to(torch.bfloat16).float().numpy()


# ------------------------------------------------------------------ codecs

def test_fp8_decode_all_bytes_match_torch_including_signed_zero_and_nan():
    # test_native_backend.py:33-37
    raw = np.arange(256, dtype=np.uint8)
    actual = orc.fp8_decode(raw)
    expected = torch.from_numpy(raw).view(torch.float8_e4m3fn).float().numpy()
    np.testing.assert_array_equal(actual, expected)
    assert np.signbit(actual[128]) and np.isnan(actual[127]) and np.isnan(actual[255])


def _fp8_grid():
    values = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float()
    return np.sort(values[torch.isfinite(values)].numpy())


def test_fp8_encode_matches_torch_on_values_midpoints_and_neighbours():
    grid = np.unique(_fp8_grid())
    mids = (grid[:-1].astype(np.float64) + grid[1:]) / 2
    mids = mids.astype(np.float32)
    up = np.nextafter(mids, np.float32(np.inf))
    down = np.nextafter(mids, np.float32(-np.inf))
    rng = np.random.default_rng(5)
    randoms = np.concatenate([rng.uniform(-448, 448, 4000), rng.uniform(-0.02, 0.02, 4000)]).astype(np.float32)
    values = np.concatenate([grid, mids, up, down, randoms, np.float32([0.0, -0.0])]).astype(np.float32)
    actual = orc.fp8_encode(values)
    expected = torch.from_numpy(values).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(actual, expected)


def test_fp8_encode_saturates_instead_of_overflowing():
    values = np.float32([448.0, 449.0, 464.0, 1e6, -1e30])
    assert list(orc.fp8_encode(values)) == [0x7E, 0x7E, 0x7E, 0x7E, 0xFE]


def test_bf16_and_fp16_rounding_match_torch():
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.standard_normal(20000) * 10.0 ** rng.integers(-8, 8, 20000),
                        [0.0, -0.0, 65504.0, 65519.0, 65520.0, 6e-8, 3e-8, 1e-40]]).astype(np.float32)
    np.testing.assert_array_equal(orc.bf16_round(x), torch.from_numpy(x).bfloat16().float().numpy())
    lib = orc.lib()
    halves = np.array([lib.orc_f16_from_f32(float(v)) for v in x], np.uint16)
    np.testing.assert_array_equal(halves, torch.from_numpy(x).half().view(torch.int16).numpy().view(np.uint16))


# -------------------------------------------------------------- activation quant

def _quant_case(kind):
    x = torch.randn(16, 128, generator=torch.Generator().manual_seed(22))
    if kind == "zero":
        x.zero_()
        x[0, :4] = torch.tensor([0.0, -0.0, 0.0, -0.0])
    elif kind == "tiny":
        x *= 1e-20
    elif kind == "saturated":
        x *= 1e20
    return x.to(torch.bfloat16)


def _torch_contract_quant(x):
    # the closed form of fp8_cpu_reference.py:14-20, evaluated by torch
    blocks = x.float().reshape(-1, 128)
    scales = blocks.abs().amax(-1).clamp_min(1e-10) * (1.0 / 448.0)
    raw = (blocks / scales[:, None]).clamp(-448, 448).to(torch.float8_e4m3fn)
    return raw.view(torch.uint8).reshape(x.shape).numpy(), scales.numpy()


@pytest.mark.parametrize("kind", ["random", "zero", "tiny", "saturated"])
def test_activation_quantization_exact_bytes_and_scales(kind):
    # test_native_backend.py:41-55
    x = _quant_case(kind)
    q, s = orc.quantize_fp8(x.float().numpy())
    eq, es = _torch_contract_quant(x)
    np.testing.assert_array_equal(q, eq)
    np.testing.assert_array_equal(s.reshape(-1), es)


@pytest.mark.parametrize("kind", ["random", "zero", "tiny", "saturated"])
def test_activation_quantization_matches_golden_reference_executor(kind):
    data = np.load(GOLDEN / "fp8_quant.npz")
    x = _quant_case(kind)
    q, s = orc.quantize_fp8(x.float().numpy())
    np.testing.assert_array_equal(q.reshape(-1), data[f"{kind}_q"])
    np.testing.assert_array_equal(s.reshape(-1), data[f"{kind}_s"])


def test_per_token_quantization_uses_one_scale_per_row():
    rng = np.random.default_rng(9)
    x = bf16_values(torch.from_numpy(rng.standard_normal((3, 512)).astype(np.float32)))
    q, s = orc.quantize_fp8(x, group=512)
    assert s.shape == (3, 1)
    amax = np.abs(x).max(axis=1)
    np.testing.assert_array_equal(s[:, 0], (amax * np.float32(1 / 448)).astype(np.float32))
    decoded = orc.fp8_decode(q) * s
    assert np.max(np.abs(decoded - x) / amax[:, None]) < 2 ** -4


# ---------------------------------------------------------- FP8 expert pairs

def _store(seed, experts, inter2, hidden, random_scales):
    g = torch.Generator().manual_seed(seed)
    w13 = torch.randint(-3, 4, (experts, inter2, hidden), generator=g).to(torch.float8_e4m3fn)
    if random_scales:
        s13 = torch.rand(experts, inter2 // 128, hidden // 128, generator=g) * 0.02 + 0.01
    else:
        s13 = torch.full((experts, inter2 // 128, hidden // 128), 0.03125)
    w2 = torch.randint(-3, 4, (experts, hidden, inter2 // 2), generator=g).to(torch.float8_e4m3fn)
    if random_scales:
        s2 = torch.rand(experts, hidden // 128, inter2 // 2 // 128, generator=g) * 0.02 + 0.01
    else:
        s2 = torch.full((experts, hidden // 128, inter2 // 2 // 128), 0.03125)
    return g, w13, s13, w2, s2


def _banks(w13, s13, w2, s2):
    return (orc.Fp8Bank(w13.view(torch.uint8).numpy(), s13.numpy()),
            orc.Fp8Bank(w2.view(torch.uint8).numpy(), s2.numpy()))


def _fp64_contract(w13, s13, w2, s2, x, ids, weights, x_group=128):
    """Brute-force float64 evaluation of the same contract: exact FP8 products,
    fp64 block sums and scaling, activation quantization emulated."""
    def dequant(w, s):
        wf = w.float().double()
        e, n, k = wf.shape
        rs = s.double().repeat_interleave(n // s.shape[1], 1).repeat_interleave(k // s.shape[2], 2)
        return wf * rs

    W13, W2 = dequant(w13, s13), dequant(w2, s2)
    q, sx = orc.quantize_fp8(x.reshape(1, -1), x_group)
    xq = (orc.fp8_decode(q).astype(np.float64) * np.repeat(sx, x_group, axis=1))[0]
    out = []
    inter = W2.shape[2]
    for e, wr in zip(ids, weights):
        gu = W13[e].numpy() @ xq
        gu = orc.bf16_round(gu.astype(np.float32)).astype(np.float64)
        gate, up = gu[:inter], gu[inter:]
        h = (gate / (1 + np.exp(-gate)) * up).astype(np.float32)
        hq, hs = orc.quantize_fp8(h.reshape(1, -1))
        hd = (orc.fp8_decode(hq).astype(np.float64) * np.repeat(hs, 128, axis=1))[0]
        out.append((W2[e].numpy() @ hd) * wr)
    return np.stack(out)


def test_duplicate_route_partials_stay_separate_and_ordered():
    # test_native_backend.py:58-77 (store seed 194, ids [3,1,3,0])
    _, w13, s13, w2, s2 = _store(194, 4, 256, 128, random_scales=False)
    b13, b2 = _banks(w13, s13, w2, s2)
    x = bf16_values(torch.linspace(-1, 1, 128))
    ids, weights = [3, 1, 3, 0], np.float32([0.4, 0.2, 0.3, 0.1])
    actual = orc.fp8_expert_pairs(b13, b2, x, ids, weights)
    np.testing.assert_allclose(actual[0] / np.float32(0.4), actual[2] / np.float32(0.3), rtol=1e-6, atol=1e-6)
    expected = _fp64_contract(w13, s13, w2, s2, x, ids, weights)
    np.testing.assert_allclose(actual, expected, rtol=1e-5, atol=2e-6)


def test_multiple_weight_scale_blocks_against_float64_brute_force():
    # test_native_backend.py:234-254 (seed 882, E=3, [512,256]/[256,256])
    g, w13, s13, w2, s2 = _store(882, 3, 512, 256, random_scales=True)
    x = bf16_values(torch.randn(256, generator=g))
    ids, weights = [2, 0, 1, 2], np.float32([0.4, 0.3, 0.2, 0.1])
    actual = orc.fp8_expert_pairs(*_banks(w13, s13, w2, s2), x, ids, weights)
    expected = _fp64_contract(w13, s13, w2, s2, x, ids, weights)
    np.testing.assert_allclose(actual, expected, rtol=2e-5, atol=2e-6)


def test_a_transposed_scale_index_would_be_caught():
    # plant a plausible mistake in the oracle's input (scales transposed per
    # expert) and check the float64 contract notices it
    g, w13, s13, w2, s2 = _store(882, 3, 512, 256, random_scales=True)
    x = bf16_values(torch.randn(256, generator=g))
    ids, weights = [2, 0], np.float32([0.6, 0.4])
    wrong = s13.clone()
    wrong[:, 0, 1], wrong[:, 1, 0] = s13[:, 1, 0], s13[:, 0, 1]
    actual = orc.fp8_expert_pairs(*_banks(w13, wrong, w2, s2), x, ids, weights)
    expected = _fp64_contract(w13, s13, w2, s2, x, ids, weights)
    assert not np.allclose(actual, expected, rtol=2e-5, atol=2e-6)


def test_per_channel_scales_against_float64_brute_force():
    g = torch.Generator().manual_seed(31)
    w13 = torch.randint(-40, 41, (2, 256, 256), generator=g).to(torch.float8_e4m3fn)
    w2 = torch.randint(-40, 41, (2, 256, 128), generator=g).to(torch.float8_e4m3fn)
    s13 = torch.rand(2, 256, 1, generator=g) * 0.001 + 0.0005
    s2 = torch.rand(2, 256, 1, generator=g) * 0.001 + 0.0005
    x = bf16_values(torch.randn(256, generator=g))
    ids, weights = [1, 0, 1], np.float32([0.5, 0.3, 0.2])
    for x_group in (128, 256):
        actual = orc.fp8_expert_pairs(*_banks(w13, s13, w2, s2), x, ids, weights, x_group=x_group)
        expected = _fp64_contract(w13, s13, w2, s2, x, ids, weights, x_group=x_group)
        np.testing.assert_allclose(actual, expected, rtol=3e-5, atol=1e-6)


@pytest.mark.skipif(not ref_native.available(), reason="reference executor not built (make -C oracle ref)")
@pytest.mark.parametrize("seed,experts,inter2,hidden,random_scales", [
    (194, 4, 256, 128, False), (882, 3, 512, 256, True)])
def test_oracle_equals_reference_scalar_executor_bitwise(seed, experts, inter2, hidden, random_scales):
    g, w13, s13, w2, s2 = _store(seed, experts, inter2, hidden, random_scales)
    xb = torch.randn(hidden, generator=g).bfloat16()
    ids = np.array([experts - 1, 0, experts - 1, 1][:4], np.int64) % experts
    weights = np.float32([0.4, 0.3, 0.2, 0.1])
    lib = ref_native.RefLibrary()
    with ref_native.RefExecutor(lib, hidden, inter2 // 2, capacity=8, threads=1,
                                implementation="scalar") as ex:
        ref = ex.forward(w13.view(torch.uint8).numpy(), s13.numpy(), w2.view(torch.uint8).numpy(),
                         s2.numpy(), xb.view(torch.int16).numpy().view(np.uint16), ids, weights)
    actual = orc.fp8_expert_pairs(*_banks(w13, s13, w2, s2), xb.float().numpy(), ids, weights)
    np.testing.assert_array_equal(actual, ref)


def test_oracle_matches_golden_reference_executor_partials():
    data = np.load(GOLDEN / "fp8_pairs.npz")
    for case in ("s194", "s882"):
        w13 = torch.from_numpy(data[f"{case}_w13"]).view(torch.float8_e4m3fn)
        w2 = torch.from_numpy(data[f"{case}_w2"]).view(torch.float8_e4m3fn)
        s13 = torch.from_numpy(data[f"{case}_s13"])
        s2 = torch.from_numpy(data[f"{case}_s2"])
        x = torch.from_numpy(data[f"{case}_x"].view(np.int16)).view(torch.bfloat16).float().numpy()
        actual = orc.fp8_expert_pairs(*_banks(w13, s13, w2, s2), x, data[f"{case}_ids"], data[f"{case}_weights"])
        np.testing.assert_array_equal(actual, data[f"{case}_out"])


def test_layer_reduction_follows_router_slot_order():
    # test_offload.py:394-409: with +-1e20 partials only a slot-order sum
    # gives 3 * p
    _, w13, s13, w2, s2 = _store(194, 4, 256, 128, random_scales=False)
    b13, b2 = _banks(w13, s13, w2, s2)
    x = bf16_values(torch.linspace(-1, 1, 128))
    weights = np.float32([[1e20, 1.0, -1e20, 3.0]])
    ids = np.array([[1, 1, 1, 1]])
    single = orc.fp8_expert_pairs(b13, b2, x, [1], np.float32([1.0]))[0]
    out = orc.fp8_moe_forward(b13, b2, x.reshape(1, -1), ids, weights, out_dtype="fp32")
    np.testing.assert_array_equal(out[0], (single * np.float32(3.0)))


# ------------------------------------------------------------------ routing

def test_route_topk_matches_torch_softmax_topk_on_tie_free_logits():
    g = torch.Generator().manual_seed(20261202)
    logits = torch.randn(512, 128, generator=g)
    probs = torch.softmax(logits, -1)
    tw, ti = probs.topk(8, -1)
    tw = tw / tw.sum(-1, keepdim=True)
    ids, weights = orc.route_topk(logits.numpy(), 8)
    np.testing.assert_array_equal(ids, ti.numpy())
    np.testing.assert_allclose(weights, tw.numpy(), rtol=2e-6, atol=0)
    np.testing.assert_array_equal(orc.bf16_round(weights), tw.bfloat16().float().numpy())


def test_route_topk_ties_resolve_to_the_lower_index():
    logits = np.full((2, 16), -1.0, np.float32)
    logits[0, [3, 1]] = 2.0
    logits[1, [15, 0]] = 2.0
    ids, weights = orc.route_topk(logits, 4)
    np.testing.assert_array_equal(ids, [[1, 3, 0, 2], [0, 15, 1, 2]])
    assert weights[0, 0] == weights[0, 1]
    # the set torch picks for the strict winners is the same
    t = torch.softmax(torch.from_numpy(logits), -1).topk(2, -1).indices.sort(-1).values
    np.testing.assert_array_equal(np.sort(ids[:, :2], -1), t.numpy())


def _equal_probability_logits():
    """Rows where two DISTINCT logits give the SAME fp32 softmax probability
    (exp(-2^-30) rounds to 1.0): the larger logit is the larger probability
    in exact arithmetic, but fp32 ties them."""
    logits = np.full((3, 8), -4.0, np.float32)
    logits[0, [1, 5]] = [np.float32(-2.0 ** -30), 0.0]      # higher index has the larger logit
    logits[1, [2, 6]] = [0.0, np.float32(-2.0 ** -30)]      # lower index has the larger logit
    logits[2, [0, 3, 7]] = [np.float32(-2.0 ** -28), np.float32(-2.0 ** -29), 0.0]
    return logits


def test_route_topk_orders_equal_probabilities_by_logit():
    """The router's rule is (logit desc, index asc): on distinct logits whose
    fp32 probabilities tie, the larger logit goes first -- the exact-arithmetic
    order of the probabilities.  The reference calls probabilities.topk
    (backbone_graph.py:319-320), whose order among equal values torch leaves
    unspecified; both rules pick the same set."""
    logits = _equal_probability_logits()
    probs = torch.softmax(torch.from_numpy(logits), -1)
    assert probs[0, 1] == probs[0, 5] and probs[1, 2] == probs[1, 6]
    assert probs[2, 0] == probs[2, 3] == probs[2, 7]
    ids, weights = orc.route_topk(logits, 3)
    np.testing.assert_array_equal(ids[:, :2], [[5, 1], [2, 6], [7, 3]])
    assert ids[2, 2] == 0
    assert weights[0, 0] == weights[0, 1]
    t = probs.topk(2, -1).indices.sort(-1).values.numpy()
    np.testing.assert_array_equal(np.sort(ids[:2, :2], -1), t[:2])


def test_route_without_renormalisation_returns_probabilities():
    logits = torch.randn(4, 32, generator=torch.Generator().manual_seed(1))
    ids, weights = orc.route_topk(logits.numpy(), 4, renormalize=False)
    np.testing.assert_allclose(weights, torch.softmax(logits, -1).topk(4, -1).values.numpy(), rtol=2e-6)


def test_permute_is_torch_stable_argsort_and_bincount():
    g = torch.Generator().manual_seed(4)
    ids = torch.randint(0, 12, (37, 8), generator=g)
    order, counts, offsets = orc.permute(ids.numpy(), 12)
    flat = ids.reshape(-1)
    np.testing.assert_array_equal(order, torch.argsort(flat, stable=True).numpy())
    np.testing.assert_array_equal(counts, torch.bincount(flat, minlength=12).numpy())
    np.testing.assert_array_equal(offsets[:-1], (torch.cumsum(torch.bincount(flat, minlength=12), 0)
                                                 - torch.bincount(flat, minlength=12)).numpy())


def test_permute_rejects_out_of_range_ids():
    with pytest.raises(ValueError):
        orc.permute(np.array([[0, 12]]), 12)


# --------------------------------------------------- packed quantized modes

def _h256():
    h = torch.tensor([[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]], dtype=torch.float64)
    r = h
    for _ in range(3):
        r = torch.kron(r, h)
    return r / 16


def test_rotation_is_the_published_orthogonal_h256():
    x = torch.randn(3, 512, generator=torch.Generator().manual_seed(8), dtype=torch.float64)
    xb = x.to(torch.bfloat16).double()
    _, _, rot = orc.rotate_quantize(xb.float().numpy(), rot_dtype="fp32")
    H = _h256()
    assert torch.allclose(H @ H.T, torch.eye(256, dtype=torch.float64))
    expected = (xb.reshape(-1, 256) @ H).reshape(3, 512)
    np.testing.assert_allclose(rot, expected.numpy(), rtol=0, atol=1e-5)
    # inverse rotation recovers the input
    back = (torch.from_numpy(rot).double().reshape(-1, 256) @ H.T).reshape(3, 512)
    np.testing.assert_allclose(back.numpy(), xb.numpy(), atol=1e-5)


def test_rotate_quantize_row_int8_against_torch_closed_form():
    x = torch.randn(4, 256, generator=torch.Generator().manual_seed(71)).bfloat16()
    q, s, rot = orc.rotate_quantize(x.float().numpy())
    rotated = torch.from_numpy(rot)
    assert torch.equal(rotated.bfloat16().float(), rotated)  # stored through bf16
    scale = rotated.abs().amax(1).clamp_min(1e-12) / 127
    np.testing.assert_array_equal(s, scale.numpy())
    np.testing.assert_array_equal(q, (rotated / scale[:, None]).round().clamp(-127, 127).to(torch.int8).numpy())
    # torch's own bf16 rotation agrees to one bf16 rounding
    torch_rot = (x.reshape(-1, 256) @ _h256().to(torch.bfloat16)).reshape(4, 256).float()
    np.testing.assert_allclose(rot, torch_rot.numpy(), rtol=2 ** -7, atol=1e-6)


def _explicit_projection(mode, bank, x, ids, weights, weighted, n, k):
    """test_quantized_kernels.py:27-83 explicit reconstruction oracle."""
    if mode == 0:
        inputs = x.float()
    else:
        q, s, _ = orc.rotate_quantize(x.float().numpy())
        inputs = torch.from_numpy(q).float() * torch.from_numpy(s)[:, None]
    mats = [torch.from_numpy(orc.quant_dequantize(bank, e)) for e in range(bank.experts)]
    out = torch.stack([inputs[i] @ mats[e].T for i, e in enumerate(ids)]).bfloat16()
    if weighted:
        out = out.float() * torch.from_numpy(weights)[:, None]
    return out.float().numpy()


@pytest.mark.parametrize("mode", [0, 1, 2, 3])
@pytest.mark.parametrize("weighted", [False, True])
def test_quant_projection_matches_explicit_reconstruction(mode, weighted):
    from drama_moe.formats import gptq_pack, nibble_pack, six_pack

    torch.manual_seed(71)
    n, k = 128, 256
    x = torch.randn(3, k, dtype=torch.bfloat16)
    weights = np.float32([0.2, 0.6, 0.3])
    ids = [1, 0, 1]
    if mode == 0:
        codes = torch.randint(0, 16, (2, n, k))
        scales = (torch.rand(2, n, k // 128) * 0.03).half()
        bank = orc.QuantBank(0, gptq_pack(codes).numpy(), scales.view(torch.int16).numpy(), n, k)
        explicit = ((codes.float() - 8) * scales.float().repeat_interleave(128, -1)).bfloat16().float()
    elif mode == 1:
        w8 = torch.randint(-127, 128, (2, n, k), dtype=torch.int8)
        sc = torch.rand(2, n, 1) * 0.02
        bank = orc.QuantBank(1, w8.numpy(), sc.numpy(), n, k)
        explicit = w8.float() * sc
    else:
        codes = torch.randint(0, 16 if mode == 3 else 64, (2, n, k))
        packed = six_pack(codes) if mode == 2 else nibble_pack(codes)
        relative = (torch.rand(2, n, k // 16) + 1).to(torch.float8_e4m3fn)
        channel = torch.rand(2, n, 1) * 0.02
        if mode == 3:
            tables = torch.linspace(-12, 13, 16).repeat(2, 1).contiguous()
            aux = torch.zeros(2, n, k // 16 + 8, dtype=torch.uint8)
            aux[..., :k // 16] = relative.view(torch.uint8)
            aux[..., k // 16:k // 16 + 4] = channel.view(torch.uint8)
            aux[:, :16, k // 16 + 4:] = tables.view(torch.uint8).reshape(2, 16, 4)
            levels = torch.stack([tables[i][codes[i]] for i in range(2)])
        else:
            aux = torch.cat((relative.view(torch.uint8), channel.view(torch.uint8)), dim=-1)
            levels = codes.float() - 32
        bank = orc.QuantBank(mode, packed.numpy(), aux.numpy(), n, k)
        explicit = (levels * relative.float().repeat_interleave(16, -1)).round().clamp(-127, 127) * channel
    # the oracle's own dequantization equals the independent reconstruction
    for e in range(2):
        np.testing.assert_allclose(orc.quant_dequantize(bank, e), explicit[e].numpy(), rtol=1e-6, atol=1e-9)
    actual = orc.quant_projection(bank, x.float().numpy(), ids, weights, weighted=weighted)
    expected = _explicit_projection(mode, bank, x, ids, weights, weighted, n, k)
    np.testing.assert_allclose(actual, expected, rtol=0.01, atol=0.02)


def test_asymmetric_w4a16_zero_points():
    from drama_moe.formats import gptq_pack, zeros_pack

    g = torch.Generator().manual_seed(12)
    n, k = 64, 256
    codes = torch.randint(0, 16, (1, n, k), generator=g)
    zeros = torch.randint(0, 16, (1, k // 128, n), generator=g)
    scales = (torch.rand(1, n, k // 128, generator=g) * 0.03).half()
    bank = orc.QuantBank(0, gptq_pack(codes).numpy(), scales.view(torch.int16).numpy(), n, k,
                         zeros=zeros_pack(zeros).numpy())
    zp = zeros.permute(0, 2, 1).repeat_interleave(128, -1).float()  # [1, n, k]
    explicit = ((codes.float() - zp) * scales.float().repeat_interleave(128, -1)).bfloat16().float()
    np.testing.assert_array_equal(orc.quant_dequantize(bank, 0), explicit[0].numpy())


# --------------------------------------------------------------- moe_align

def test_moe_align_known_answer():
    # ids flattened [2, 0, 2, 1, 0, 5] over 4 experts (5 is invalid), blocks of 2:
    # expert 0 -> pairs 1, 4; expert 1 -> pair 3 + sentinel; expert 2 -> pairs 0, 2
    sorted_ids, expert_ids, padded = orc.moe_align(np.array([[2, 0], [2, 1], [0, 5]]), 4, 2)
    assert padded == 6
    assert sorted_ids[:6].tolist() == [1, 4, 3, 6, 0, 2]
    assert expert_ids.tolist()[:4] == [0, 1, 2, -1]
    assert np.all(sorted_ids[6:] == 6)


@pytest.mark.parametrize("pairs,experts,block_m", [(1, 1, 16), (37, 8, 4), (1000, 128, 16),
                                                   (4096, 128, 64), (513, 7, 1), (300, 512, 32)])
def test_moe_align_properties(pairs, experts, block_m):
    from moe_align_props import check_moe_align

    rng = np.random.default_rng(pairs + experts)
    ids = rng.integers(0, experts, pairs)
    if pairs > 10:
        ids[rng.integers(0, pairs, 3)] = [-1, experts, experts + 9]
    sorted_ids, expert_ids, padded = orc.moe_align(ids, experts, block_m)
    check_moe_align(sorted_ids, expert_ids, padded, ids, experts, block_m)
    # agrees with the stable permutation of the valid pairs
    valid = ids[(ids >= 0) & (ids < experts)]
    order, counts, _ = orc.permute(valid, experts)
    index = np.flatnonzero((ids >= 0) & (ids < experts))
    assert np.array_equal(sorted_ids[sorted_ids != pairs], index[order])


def test_moe_align_checker_catches_planted_mistakes():
    from moe_align_props import check_moe_align

    rng = np.random.default_rng(3)
    ids = rng.integers(0, 8, 200)
    sorted_ids, expert_ids, padded = orc.moe_align(ids, 8, 16)
    swapped = sorted_ids.copy()
    swapped[[0, 1]] = swapped[[1, 0]]  # two pairs of expert 0 out of order
    with pytest.raises(AssertionError):
        check_moe_align(swapped, expert_ids, padded, ids, 8, 16)
    shifted = expert_ids.copy()
    shifted[0] = 1
    with pytest.raises(AssertionError):
        check_moe_align(sorted_ids, shifted, padded, ids, 8, 16)
    with pytest.raises(AssertionError):
        check_moe_align(sorted_ids, expert_ids, padded + 16, ids, 8, 16)


# ------------------------------------------------- O2 dequantize-then-matmul

def _torch_o2_pairs(b13_w, b13_s, b2_w, b2_s, x, ids, weights, dtype):
    """The same pipeline on torch's CPU kernels: dequantize in fp32, cast to
    the compute dtype, F.linear in that dtype, silu, product, weighted in fp32."""
    import torch.nn.functional as F

    out = []
    for r in range(x.shape[0]):
        e = int(ids[r])
        def deq(w, s):
            v = torch.from_numpy(w[e]).view(torch.float8_e4m3fn).float()
            n, k = v.shape
            blocks = v.view(n // 128, 128, k // 128, 128) * torch.from_numpy(s[e])[:, None, :, None]
            return blocks.reshape(n, k).to(dtype)
        gate, up = F.linear(x[r:r + 1].to(dtype), deq(b13_w, b13_s)).chunk(2, dim=-1)
        values = F.linear(F.silu(gate) * up, deq(b2_w, b2_s))
        out.append(values.float() * float(weights[r]))
    return torch.cat(out).numpy()


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
def test_o2_pairs_match_torch_cpu_linear(dtype):
    """O2 (TorchExpertBackend semantics) against torch's own CPU bf16 / fp16
    kernels: the only freedom is the accumulation order inside F.linear
    before its single rounding, so nearly every value is bit-identical and
    the rest differ by a last-place rounding."""
    torch_dtype = torch.bfloat16 if dtype == "bf16" else torch.float16
    g = torch.Generator().manual_seed(77)
    bank = random_fp8_bank(4, 256, 256, generator=g)
    b13 = orc.Fp8Bank(bank.w13_weight.view(torch.uint8).numpy(), bank.w13_scale_inv.numpy())
    b2 = orc.Fp8Bank(bank.w2_weight.view(torch.uint8).numpy(), bank.w2_scale_inv.numpy())
    x = torch.randn(6, 256, generator=g).to(torch_dtype)
    ids = np.array([0, 3, 1, 3, 2, 0])
    weights = np.array([0.5, 0.25, 1.0, 0.125, 0.75, 2.0], np.float32)
    got = orc.o2_expert_pairs(b13, b2, x.float().numpy(), ids, weights, dtype)
    want = _torch_o2_pairs(b13.w, b13.s, b2.w, b2.s, x, ids, weights, torch_dtype)
    assert np.mean(got == want) > 0.95
    assert np.max(np.abs(got - want)) / np.max(np.abs(want)) < 1e-2
    # a planted mistake -- each row block scaled by another block's scale -- is far off
    bad = orc.Fp8Bank(b13.w, np.ascontiguousarray(b13.s[:, ::-1, :]))  # block scales of the wrong rows
    wrong = orc.o2_expert_pairs(bad, b2, x.float().numpy(), ids, weights, dtype)
    assert np.max(np.abs(wrong - want)) / np.max(np.abs(want)) > 5e-2


def test_o2_layer_sums_slots_in_order():
    g = torch.Generator().manual_seed(5)
    bank = random_fp8_bank(4, 128, 128, generator=g)
    b13 = orc.Fp8Bank(bank.w13_weight.view(torch.uint8).numpy(), bank.w13_scale_inv.numpy())
    b2 = orc.Fp8Bank(bank.w2_weight.view(torch.uint8).numpy(), bank.w2_scale_inv.numpy())
    x = torch.randn(2, 128, generator=g).bfloat16().float().numpy()
    ids = np.array([[1, 2, 3], [0, 0, 2]])
    w = np.array([[0.5, 0.3, 0.2], [0.6, 0.3, 0.1]], np.float32)
    out = orc.o2_moe_forward(b13, b2, x, ids, w)
    pairs = orc.o2_expert_pairs(b13, b2, np.repeat(x, 3, 0), ids.reshape(-1), w.reshape(-1)).reshape(2, 3, -1)
    expect = orc.bf16_round(((pairs[:, 0] + pairs[:, 1]).astype(np.float32) + pairs[:, 2]).astype(np.float32))
    np.testing.assert_array_equal(out, expect)


# ------------------------------------ W4A8 / W6A8 with group-128 scales

def _g128_case(mode, E=3, H=256, I=128, seed=0):
    from drama_moe.formats import nibble_pack, six_pack

    rng = np.random.default_rng(seed + mode)
    top = 16 if mode == 4 else 64
    bias = 8 if mode == 4 else 32
    codes = {"w13": rng.integers(0, top, (E, 2 * I, H)), "w2": rng.integers(0, top, (E, H, I))}
    scales = {"w13": rng.uniform(0.002, 0.006, (E, 2 * I, H // 128)).astype(np.float16),
              "w2": rng.uniform(0.002, 0.006, (E, H, I // 128)).astype(np.float16)}
    pack = nibble_pack if mode == 4 else six_pack
    banks = {k: orc.G128Bank(mode, pack(torch.from_numpy(codes[k])).numpy(), scales[k]) for k in codes}
    dense = {k: (codes[k] - bias).astype(np.float64) * np.repeat(scales[k].astype(np.float64), 128, axis=-1)
             for k in codes}
    return banks, dense, codes, scales


def _g128_brute(dense, x, e, weight, H, I):
    """fp64 W8A8 arithmetic: per-token FP8 activation, gate/up rounded to bf16,
    silu(gate) * up, FP8 128-group hidden, down, route weight."""
    q, s = orc.quantize_fp8(x[None], H)
    xq = orc.fp8_decode(q[0]).astype(np.float64) * np.float64(s[0, 0])
    gu = orc.bf16_round((dense["w13"][e] @ xq).astype(np.float32))
    h = (gu[:I] / (1 + np.exp(-gu[:I].astype(np.float64))) * gu[I:]).astype(np.float32)
    hq, hs = orc.quantize_fp8(h[None], 128)
    hv = orc.fp8_decode(hq[0]).astype(np.float64) * np.repeat(hs[0].astype(np.float64), 128)
    return dense["w2"][e] @ hv * weight


@pytest.mark.parametrize("mode", [4, 5])
def test_g128_pairs_match_fp64_brute_force(mode):
    """The oracle's group-128 integer formats against an fp64 evaluation from
    the raw codes (not the packed bytes), so packing, level offset, scale
    indexing and the per-token activation scale are all pinned."""
    H, I = 256, 128
    banks, dense, _, _ = _g128_case(mode, H=H, I=I)
    rng = np.random.default_rng(9)
    x = orc.bf16_round(rng.standard_normal(H).astype(np.float32))
    ids = np.array([2, 0, 2, 1])
    w = np.array([0.4, 0.3, 0.2, 0.1], np.float32)
    got = orc.fp8_expert_pairs(banks["w13"], banks["w2"], x, ids, w, x_group=H)
    want = np.stack([_g128_brute(dense, x, e, wt, H, I) for e, wt in zip(ids, w)])
    assert np.max(np.abs(got - want)) / np.max(np.abs(want)) < 5e-3
    # plausible mistakes are far outside that: swapped nibbles, a level
    # offset off by one, the other projection's scales
    swapped = dict(dense)
    c = _g128_case(mode, H=H, I=I)[2]
    bias = 8 if mode == 4 else 32
    perm = np.arange(H).reshape(-1, 2)[:, ::-1].reshape(-1)
    swapped["w13"] = (c["w13"][..., perm] - bias) * np.repeat(_g128_case(mode, H=H, I=I)[3]["w13"].astype(np.float64),
                                                               128, axis=-1)
    off = {k: v + np.repeat(_g128_case(mode, H=H, I=I)[3][k].astype(np.float64), 128, axis=-1)
           for k, v in dense.items()}
    for bad in (swapped, off):  # each would fail the 5e-3 check above by a wide margin
        wrong = np.stack([_g128_brute(bad, x, e, wt, H, I) for e, wt in zip(ids, w)])
        assert np.max(np.abs(got - wrong)) / np.max(np.abs(wrong)) > 2e-2


def test_g128_layer_combines_in_slot_order():
    H, I = 256, 128
    banks, dense, _, _ = _g128_case(4, H=H, I=I, seed=4)
    rng = np.random.default_rng(1)
    x = orc.bf16_round(rng.standard_normal((2, H)).astype(np.float32))
    ids = np.array([[0, 1], [2, 2]])
    w = np.array([[0.7, 0.3], [0.5, 0.5]], np.float32)
    out = orc.fp8_moe_forward(banks["w13"], banks["w2"], x, ids, w, x_group=H)
    for t in range(2):
        pairs = orc.fp8_expert_pairs(banks["w13"], banks["w2"], x[t], ids[t], w[t], x_group=H)
        np.testing.assert_array_equal(out[t], orc.bf16_round((pairs[0] + pairs[1]).astype(np.float32)))


# ------------------------------------------- torch-CPU baseline restatements

@pytest.mark.parametrize("mode", [0, 1, 2, 3, 4, 5])
def test_torch_cpu_layer_matches_the_oracle(mode):
    """The torch-CPU dequantize-then-matmul lane that bench.py times as the
    reference's CPU path for the packed formats agrees with the C oracle:
    modes 0-3 with quant_projection (projection_torch semantics), modes 4-5
    with the O2 reading of the group-128 formats."""
    from drama_moe.formats import random_quantized_bank
    from oracle import torch_cpu

    g = torch.Generator().manual_seed(40 + mode)
    store = random_quantized_bank(mode, 6, 512, 256, asymmetric=mode == 0, generator=g)
    x = torch.randn(3, 512, generator=g).bfloat16()
    ids, w = orc.route_topk(torch.randn(3, 6, generator=g).numpy(), 4)
    weights = torch.from_numpy(w).bfloat16()
    got = torch_cpu.layer(store, x, torch.from_numpy(ids), weights).float().numpy()
    if mode < 4:
        def bank(prefix, n, k):
            zeros = getattr(store, prefix + "_zeros")
            return orc.QuantBank(mode, getattr(store, prefix + "_weight").numpy(),
                                 getattr(store, prefix + "_scale_inv").numpy(), n, k,
                                 None if zeros is None else zeros.numpy())
        b13, b2 = bank("w13", 512, 512), bank("w2", 512, 256)
        flat = ids.reshape(-1)
        up = orc.quant_projection(b13, np.repeat(x.float().numpy(), 4, 0), flat, np.ones(flat.size, np.float32))
        act = orc.bf16_round(orc.bf16_round(orc.silu(up[:, :256])) * up[:, 256:])
        part = orc.quant_projection(b2, act, flat, weights.float().numpy().reshape(-1), weighted=True)
        want = orc.bf16_round(part.reshape(3, 4, -1).sum(1, dtype=np.float32))
    else:
        # group-128 formats: level * fp16 scale, unquantized activations
        def dense(prefix, k):
            from oracle import torch_cpu as tc
            wt, sc = getattr(store, prefix + "_weight"), getattr(store, prefix + "_scale_inv")
            return np.stack([tc.dequantize(mode, wt[e], sc[e], k).numpy() for e in range(6)])
        m13, m2 = dense("w13", 512), dense("w2", 256)
        want = np.zeros((3, 512), np.float64)
        for t in range(3):
            for j in range(4):
                e = ids[t, j]
                gu = orc.bf16_round((m13[e].astype(np.float64) @ x[t].float().numpy()).astype(np.float32))
                act = orc.bf16_round(orc.bf16_round(orc.silu(gu[:256])) * gu[256:])
                want[t] += orc.bf16_round((m2[e].astype(np.float64) @ act).astype(np.float32)) * w[t, j]
        want = orc.bf16_round(want.astype(np.float32))
        # and the level decode itself against the packing helpers' codes
        from drama_moe.formats import nibble_pack, six_pack
        codes = torch.randint(0, 16 if mode == 4 else 64, (32, 256), generator=g)
        packed = (nibble_pack if mode == 4 else six_pack)(codes)
        ones = torch.ones(32, 2, dtype=torch.float16)
        level = torch_cpu.dequantize(mode, packed, ones, 256)
        assert torch.equal(level, codes.float() - (8 if mode == 4 else 32))
    assert np.max(np.abs(got - want)) / np.max(np.abs(want)) < 2e-2


def test_torch_cpu_fp8_layer_is_o2():
    from oracle import torch_cpu

    g = torch.Generator().manual_seed(12)
    bank = random_fp8_bank(4, 256, 128, generator=g)
    x = torch.randn(2, 256, generator=g).bfloat16()
    ids = np.array([[0, 3], [2, 2]])
    w = np.array([[0.6, 0.4], [0.5, 0.5]], np.float32)
    got = torch_cpu.fp8_layer(bank, x, torch.from_numpy(ids), torch.from_numpy(w)).float().numpy()
    b13 = orc.Fp8Bank(bank.w13_weight.view(torch.uint8).numpy(), bank.w13_scale_inv.numpy())
    b2 = orc.Fp8Bank(bank.w2_weight.view(torch.uint8).numpy(), bank.w2_scale_inv.numpy())
    want = orc.o2_moe_forward(b13, b2, x.float().numpy(), ids, w)
    assert np.mean(got == want) > 0.95
    assert np.max(np.abs(got - want)) / np.max(np.abs(want)) < 1e-2


def _reference_moe_block_modules(hidden, experts, inter, g):
    """The torch modules BackboneDecodeGraph drives (backbone_graph.py:317-337),
    bf16, random weights: moe.gate, shared_expert_gate and a shared SwiGLU MLP."""
    nn = torch.nn
    gate = nn.Linear(hidden, experts, bias=False).bfloat16()
    sgate = nn.Linear(hidden, 1, bias=False).bfloat16()
    gp = nn.Linear(hidden, inter, bias=False).bfloat16()
    up = nn.Linear(hidden, inter, bias=False).bfloat16()
    down = nn.Linear(inter, hidden, bias=False).bfloat16()
    with torch.no_grad():
        for m, std in ((gate, 0.05), (sgate, 0.05), (gp, 0.05), (up, 0.05), (down, 0.05)):
            m.weight.copy_(torch.randn(m.weight.shape, generator=g) * std)
    return gate, sgate, gp, up, down


def test_moe_block_oracle_matches_torch_modules():
    """orc_block_pre / orc_block_post against the reference's own expressions on
    torch's CPU bf16 modules: softmax input moe.gate(flat).float(),
    torch.sigmoid(shared_expert_gate(flat)), down(silu(gate(x)) * up(x)),
    after_mixer + (experts + shared).  Accumulation order differs (torch's
    blocked bf16 GEMM vs a sequential fp32 sum), so values agree to about one
    bf16 rounding step; a planted mistake (the sigmoid gate dropped) must fail."""
    g = torch.Generator().manual_seed(31)
    hidden, experts, inter, tokens = 256, 16, 64, 5
    gate, sgate, gp, up, down = _reference_moe_block_modules(hidden, experts, inter, g)
    flat = torch.randn(tokens, hidden, generator=g).bfloat16()
    after = torch.randn(tokens, hidden, generator=g).bfloat16()
    experts_out = torch.randn(tokens, hidden, generator=g).bfloat16()
    with torch.no_grad():
        want_logits = gate(flat).float()
        want_sgate = torch.sigmoid(sgate(flat))
        want_act = torch.nn.functional.silu(gp(flat)) * up(flat)
        shared = want_sgate * down(want_act)
        want_out = after + (experts_out + shared)
    w = {name: m.weight.detach().float().numpy() for name, m in
         (("gate", gate), ("sgate", sgate), ("gp", gp), ("up", up), ("down", down))}
    logits, sg, act = orc.block_pre(flat.float().numpy(), w["gate"], w["sgate"], w["gp"], w["up"])
    bf16_step = 2.0 ** -7  # one bf16 rounding step, relative
    assert np.max(np.abs(logits - want_logits.numpy())) <= 2 * bf16_step * np.max(np.abs(want_logits.numpy()))
    assert np.max(np.abs(sg - want_sgate.float().numpy().reshape(-1))) <= 2 * bf16_step
    assert np.max(np.abs(act - want_act.float().numpy())) <= 2 * bf16_step * np.max(np.abs(want_act.float().numpy()))
    out = orc.block_post(act, w["down"], sg, experts_out.float().numpy(), after.float().numpy())
    ref = want_out.float().numpy()
    assert np.max(np.abs(out - ref)) / np.max(np.abs(ref)) < 1e-2
    # planted mistake: the sigmoid gate dropped from the shared expert
    wrong = orc.block_post(act, w["down"], np.ones_like(sg), experts_out.float().numpy(), after.float().numpy())
    assert np.max(np.abs(wrong - ref)) / np.max(np.abs(ref)) > 1e-2
