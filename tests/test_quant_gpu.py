"""GPU parity of the packed-integer expert banks against the oracle.

Modes: 0 W4A16 GPTQ (bf16 MFMA), 1 INT8 ConvRot, 2 W6A8, 3 W4A8 codebook (int8
MFMA on rotated, row-quantized activations).  Bars:
  * rotation + INT8 quantization: bytes and scales bit-exact (same summation
    order as the oracle, exact sign flips and 1/16);
  * projections of modes 1-3: bit-exact (exact int32 accumulation, the same
    fp32 epilogue and bf16 rounding);
  * mode 0 projections and every layer output: ||y - r||_inf / ||r||_inf <= 2e-2
    (the INT4/INT8 bar), mode 0 projections also >= 95% bit-identical.
"""
import dataclasses

import numpy as np
import pytest
import torch

from conftest import print_case
from drama_moe import _lib, quantized
from drama_moe.formats import QuantizedStore, random_quantized_bank
from oracle import oracle as orc

pytestmark = pytest.mark.gpu
TOL = 2e-2
MODES = [0, 1, 2, 3]


def rel_inf(actual, expected):
    actual = np.asarray(actual, np.float64)
    expected = np.asarray(expected, np.float64)
    return float(np.max(np.abs(actual - expected)) / max(np.max(np.abs(expected)), 1e-30))


def to_device(store: QuantizedStore, device) -> QuantizedStore:
    fields = {f.name: getattr(store, f.name) for f in dataclasses.fields(store)}
    return QuantizedStore(**{k: (v.to(device) if isinstance(v, torch.Tensor) else v) for k, v in fields.items()})


def oracle_banks(store: QuantizedStore):
    def host(t):
        return None if t is None else t.cpu().numpy()
    H, I = store.hidden, store.intermediate
    return (orc.QuantBank(store.mode, host(store.w13_weight), host(store.w13_scale_inv), 2 * I, H,
                          host(store.w13_zeros)),
            orc.QuantBank(store.mode, host(store.w2_weight), host(store.w2_scale_inv), H, I, host(store.w2_zeros)))


def oracle_layer(store, x, ids, weights, x_dtype="bf16"):
    """QuantizedExpertBackend.forward of quantized_kernels.py:217-260 on the
    oracle: up projection, bf16(bf16(silu(g)) * u), weighted down projection,
    slot-order fp32 sum, output type."""
    b13, b2 = oracle_banks(store)
    tokens, top_k = ids.shape
    I = store.intermediate
    flat = ids.reshape(-1)
    rows = x if tokens == 1 else np.repeat(x, top_k, axis=0)
    up = orc.quant_projection(b13, rows, flat, np.ones(flat.size, np.float32), shared=tokens == 1,
                              rot_dtype=x_dtype)
    act = orc.bf16_round(orc.bf16_round(orc.silu(up[:, :I])) * up[:, I:])
    part = orc.quant_projection(b2, act, flat, weights.reshape(-1), weighted=True, rot_dtype="bf16")
    part = part.reshape(tokens, top_k, -1)
    out = part[:, 0].copy()
    for j in range(1, top_k):
        out = (out + part[:, j]).astype(np.float32)
    return out


@pytest.fixture(scope="module", autouse=True)
def built():
    orc.build()


@pytest.mark.parametrize("k", [256, 768, 2048])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_rotate_quantize_bit_exact(cuda, k, dtype):
    print_case("rotate_quantize", k, dtype)
    x = (torch.randn(37, k, generator=torch.Generator().manual_seed(k)) * 2).to(dtype)
    x[3] = 0.0  # all-zero row: the 1e-12 floor
    q, s = quantized.rotate_quantize(x.to(cuda))
    eq, es, _ = orc.rotate_quantize(x.float().numpy(), "bf16" if dtype == torch.bfloat16 else "fp32")
    np.testing.assert_array_equal(q.cpu().numpy(), eq)
    np.testing.assert_array_equal(s.cpu().numpy(), es)


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("shared,weighted", [(True, False), (False, False), (False, True)])
def test_projection_matches_oracle(cuda, mode, shared, weighted):
    print_case("projection", mode, shared, weighted)
    g = torch.Generator().manual_seed(100 + mode)
    store = random_quantized_bank(mode, 8, 512, 256, generator=g)
    pairs = 24
    rows = 1 if shared else pairs
    x = torch.randn(rows, 512, generator=g).bfloat16()
    ids = torch.randint(0, 8, (pairs,), generator=g)
    ids[1] = ids[0]
    w = torch.rand(pairs, generator=g) + 0.5
    dev = to_device(store, cuda)
    out = quantized.projection(x.to(cuda), ids.to(cuda), w.to(cuda), dev.w13_weight, dev.w13_scale_inv,
                               mode=mode, shared=shared, weighted=weighted)
    assert out.dtype == (torch.float32 if weighted else torch.bfloat16) and out.shape == (pairs, 512)
    b13, _ = oracle_banks(store)
    expected = orc.quant_projection(b13, x.float().numpy(), ids.numpy(), w.numpy(), shared=shared,
                                    weighted=weighted)
    actual = out.float().cpu().numpy()
    if mode:
        np.testing.assert_array_equal(actual, expected)
    else:
        assert rel_inf(actual, expected) < TOL
        assert np.mean(actual == expected) > 0.95


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("tokens", [1, 4, 16])
def test_layer_decode_matches_oracle(cuda, mode, tokens):
    print_case("quant layer", mode, tokens)
    g = torch.Generator().manual_seed(7 * tokens + mode)
    store = random_quantized_bank(mode, 32, 512, 256, generator=g)
    x = torch.randn(tokens, 512, generator=g).bfloat16()
    ids, w = orc.route_topk(torch.randn(tokens, 32, generator=g).numpy(), 8)
    weights = torch.from_numpy(w).bfloat16()
    out = quantized.QuantizedExpertBackend(mode).forward(x.to(cuda), torch.from_numpy(ids).to(cuda),
                                                         weights.to(cuda), to_device(store, cuda))
    assert out.dtype == torch.bfloat16 and out.shape == x.shape
    expected = oracle_layer(store, x.float().numpy(), ids, weights.float().numpy())
    assert rel_inf(out.float().cpu().numpy(), expected) < TOL


@pytest.fixture
def small_launches():
    """Selects the two small-call launches of packed calls (True) or the
    separate permutation, rotation, projection and combine launches (False)."""
    lib = _lib.library()
    yield lambda single: lib.dmoe_set_fused_decode(1 if single else 0)
    lib.dmoe_set_fused_decode(1)


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("tokens,top_k", [(1, 4), (1, 8), (2, 8), (3, 5), (8, 8)])
def test_small_call_launches_match_separate_launches(cuda, small_launches, mode, tokens, top_k):
    """The small-call launches (pairs grouped inside each workgroup,
    activation and hidden rotation + INT8 in LDS, slot-order combine in the
    down launch) against the separate launches: bit-identical for modes 1-3
    (exact int32 dots, the same epilogues and combine order), within the bar
    for mode 0 (fp32 dot order differs); both paths against the oracle.
    Invalid ids (-1, E) raise the status bit, are skipped by the combine and
    give zero pair rows.  The gate/up launch takes at most 4 activation rows
    (forward: tokens; forward_pairs: pairs), the down launch at most 16 pairs
    in modes 1-3 (64 in mode 0 at this size); larger calls take the separate
    launches on both sides."""
    print_case("quant down launch", mode, tokens, top_k)
    g = torch.Generator().manual_seed(900 + 16 * mode + tokens)
    store = random_quantized_bank(mode, 32, 512, 256, generator=g)
    dev = to_device(store, cuda)
    x = torch.randn(tokens, 512, generator=g).bfloat16()
    ids, w = orc.route_topk(torch.randn(tokens, 32, generator=g).numpy(), top_k)
    ids = ids.copy()
    ids[0, 1] = -1
    ids[-1, -1] = 32
    weights = torch.from_numpy(w).bfloat16()
    backend = quantized.QuantizedExpertBackend(mode)
    args = (x.to(cuda), torch.from_numpy(ids).to(cuda), weights.to(cuda), dev)
    results = {}
    for single in (True, False):
        small_launches(single)
        backend.status(cuda)
        results[single] = (backend.forward(*args), backend.forward_pairs(
            x.to(cuda).repeat_interleave(top_k, 0), torch.from_numpy(ids).reshape(-1, 1).to(cuda),
            weights.reshape(-1, 1).to(cuda), dev))
        assert backend.status(cuda) & 1, single
    (out1, pairs1), (out0, pairs0) = results[True], results[False]
    if mode:
        assert torch.equal(out1, out0) and torch.equal(pairs1, pairs0)
    else:
        assert rel_inf(out1.float().cpu().numpy(), out0.float().cpu().numpy()) < TOL
        assert rel_inf(pairs1.cpu().numpy(), pairs0.cpu().numpy()) < TOL
    flat = ids.reshape(-1)
    bad = np.flatnonzero((flat < 0) | (flat >= 32))
    assert torch.count_nonzero(pairs1[torch.from_numpy(bad).to(cuda)]) == 0
    valid = np.where((ids >= 0) & (ids < 32), ids, 0)
    wv = np.where((ids >= 0) & (ids < 32), weights.float().numpy(), 0.0).astype(np.float32)
    expected = oracle_layer(store, x.float().numpy(), valid, wv)
    assert rel_inf(out1.float().cpu().numpy(), expected) < TOL


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("inter,tokens,top_k,x_dtype", [(768, 1, 8, torch.bfloat16), (768, 2, 8, torch.bfloat16),
                                                        (768, 1, 8, torch.float16)])
def test_small_call_wide_gateup_workgroups(cuda, small_launches, mode, inter, tokens, top_k, x_dtype):
    """Expert widths divisible by 24 whose 16-column gate/up workgroups would
    outnumber the CUs take 24-column workgroups (a third MFMA tile holding
    gate and up columns 16-23): bit-identical to the separate launches for
    modes 1-3, within the bar for mode 0, and against the oracle; bf16 and
    fp16 activations."""
    print_case("quant wide gate/up", mode, inter, tokens, top_k, x_dtype)
    g = torch.Generator().manual_seed(1700 + 16 * mode + tokens)
    store = random_quantized_bank(mode, 32, 512, inter, generator=g)
    dev = to_device(store, cuda)
    x = torch.randn(tokens, 512, generator=g).to(x_dtype)
    ids, w = orc.route_topk(torch.randn(tokens, 32, generator=g).numpy(), top_k)
    weights = torch.from_numpy(w).bfloat16()
    backend = quantized.QuantizedExpertBackend(mode)
    args = (x.to(cuda), torch.from_numpy(ids).to(cuda), weights.to(cuda), dev)
    outs = {}
    for single in (True, False):
        small_launches(single)
        outs[single] = backend.forward(*args)
    if mode:
        assert torch.equal(outs[True], outs[False])
    else:
        assert rel_inf(outs[True].float().cpu().numpy(), outs[False].float().cpu().numpy()) < TOL
    expected = oracle_layer(store, x.float().numpy(), ids, weights.float().numpy(),
                            "fp16" if x_dtype == torch.float16 else "bf16")
    assert rel_inf(outs[True].float().cpu().numpy(), expected) < TOL


def test_w4a16_asymmetric_zero_points(cuda):
    print_case("w4a16 asym")
    g = torch.Generator().manual_seed(404)
    store = random_quantized_bank(0, 16, 512, 256, asymmetric=True, generator=g)
    assert store.w13_zeros is not None
    x = torch.randn(4, 512, generator=g).bfloat16()
    ids, w = orc.route_topk(torch.randn(4, 16, generator=g).numpy(), 8)
    weights = torch.from_numpy(w).bfloat16()
    out = quantized.QuantizedExpertBackend(0).forward(x.to(cuda), torch.from_numpy(ids).to(cuda),
                                                      weights.to(cuda), to_device(store, cuda))
    expected = oracle_layer(store, x.float().numpy(), ids, weights.float().numpy())
    assert rel_inf(out.float().cpu().numpy(), expected) < TOL
    # the zero points matter: the symmetric reading of the same codes differs
    sym = dataclasses.replace(store, w13_zeros=None, w2_zeros=None)
    other = oracle_layer(sym, x.float().numpy(), ids, weights.float().numpy())
    assert rel_inf(other, expected) > 10 * TOL


def test_w4a16_fp16_activations_dequantize_to_fp16(cuda):
    """Mode 0 with fp16 activations rounds the dequantized weights to fp16
    (quantized_kernels.py:145-147), checked against a torch reconstruction."""
    print_case("w4a16 fp16")
    g = torch.Generator().manual_seed(16)
    store = random_quantized_bank(0, 4, 256, 128, generator=g)
    x = torch.randn(6, 256, generator=g).half()
    ids = torch.tensor([0, 1, 2, 3, 1, 0])
    out = quantized.projection(x.to(cuda), ids.to(cuda), torch.ones(6).to(cuda), store.w13_weight.to(cuda),
                               store.w13_scale_inv.to(cuda), mode=0)
    words = store.w13_weight.long() & 0xFFFFFFFF
    codes = ((words[..., None] >> (torch.arange(8) * 4)) & 15).reshape(4, 256, 256)
    scale = store.w13_scale_inv.float().repeat_interleave(128, -1)
    matrix = ((codes.float() - 8) * scale).half().float()
    expected = torch.stack([x[r].float() @ matrix[ids[r]].T for r in range(6)]).bfloat16().float()
    assert rel_inf(out.float().cpu().numpy(), expected.numpy()) < TOL


@pytest.mark.parametrize("mode,rows,asymmetric", [(0, 40, False), (2, 40, False), (0, 200, True),
                                                   (0, 40, True), (2, 200, False)])
def test_forward_pairs_and_invalid_ids(cuda, mode, rows, asymmetric):
    """Ordered partials of single-pair rows; 40 rows take the small-call
    kernels, 200 rows the grouped projection kernel (with qzeros for the
    asymmetric W4A16 bank)."""
    print_case("quant pairs invalid", mode, rows, asymmetric)
    g = torch.Generator().manual_seed(55 + mode + rows)
    store = random_quantized_bank(mode, 8, 512, 256, asymmetric=asymmetric, generator=g)
    x = torch.randn(rows, 512, generator=g).bfloat16()
    ids = torch.randint(0, 8, (rows, 1), generator=g)
    ids[5, 0] = 8
    ids[9, 0] = -1
    w = torch.rand(rows, 1, generator=g) + 0.1
    backend = quantized.QuantizedExpertBackend(mode)
    backend.status(cuda)
    out = backend.forward_pairs(x.to(cuda), ids.to(cuda), w.to(cuda), to_device(store, cuda))
    assert backend.status(cuda) & 1
    assert out.dtype == torch.float32 and out.shape == (rows, 512)
    assert torch.count_nonzero(out[5]) == 0 and torch.count_nonzero(out[9]) == 0
    keep = [r for r in range(rows) if r not in (5, 9)]
    b13, b2 = oracle_banks(store)
    xf = x.float().numpy()[keep]
    up = orc.quant_projection(b13, xf, ids.numpy()[keep, 0], np.ones(len(keep), np.float32))
    act = orc.bf16_round(orc.bf16_round(orc.silu(up[:, :256])) * up[:, 256:])
    expected = orc.quant_projection(b2, act, ids.numpy()[keep, 0], w.numpy()[keep, 0], weighted=True)
    assert rel_inf(out.cpu().numpy()[keep], expected) < TOL


def test_quant_layer_in_hipgraph(cuda):
    print_case("quant hipgraph")
    g = torch.Generator().manual_seed(8)
    store = to_device(random_quantized_bank(3, 16, 512, 256, generator=g), cuda)
    backend = quantized.QuantizedExpertBackend(3)
    x = torch.randn(2, 512, device=cuda).bfloat16()
    ids = torch.randint(0, 16, (2, 8), device=cuda)
    w = torch.rand(2, 8, device=cuda).bfloat16()
    out = torch.empty_like(x)
    stream = torch.cuda.Stream(cuda)
    stream.wait_stream(torch.cuda.current_stream(cuda))
    with torch.cuda.stream(stream):
        backend.forward(x, ids, w, store, out=out)
    torch.cuda.current_stream(cuda).wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        backend.forward(x, ids, w, store, out=out)
    for step in range(3):
        x.copy_(torch.randn(2, 512, device=cuda).bfloat16())
        ids.copy_(torch.randint(0, 16, (2, 8), device=cuda))
        expected = backend.forward(x, ids, w, store)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, expected), step


@pytest.mark.parametrize("mode", MODES)
def test_full_size_decode_and_prefill(cuda, mode):
    """Layer shape E=128, H=2048, I=768, top-8: decode T=1 in full, and a
    512-token prefill (4096 pairs: the grouped projection kernel) checked on
    64 spread tokens (every eighth).  W4A16 uses asymmetric banks (GPTQ
    qzeros), the format of the 512-token W4A16 benchmark."""
    print_case("quant full size", mode)
    g = torch.Generator().manual_seed(20261204 + mode)
    dev = random_quantized_bank(mode, 128, 2048, 768, device=cuda, asymmetric=mode == 0,
                                generator=torch.Generator(device=cuda).manual_seed(20261204 + mode))
    assert (dev.w13_zeros is not None) == (mode == 0)
    store = dev  # the oracle copies it to the host
    backend = quantized.QuantizedExpertBackend(mode)
    for tokens, pick in ((1, [0]), (512, list(range(3, 512, 8)))):
        x = torch.randn(tokens, 2048, generator=g).bfloat16()
        ids, w = orc.route_topk(torch.randn(tokens, 128, generator=g).numpy(), 8)
        weights = torch.from_numpy(w).bfloat16()
        out = backend.forward(x.to(cuda), torch.from_numpy(ids).to(cuda), weights.to(cuda), dev)
        expected = oracle_layer(store, x.float().numpy()[pick], ids[pick], weights.float().numpy()[pick])
        assert rel_inf(out.float().cpu().numpy()[pick], expected) < TOL, tokens


@pytest.mark.parametrize("x_dtype", [torch.bfloat16, torch.float16])
def test_w4a16_tiled_prefill_every_token(cuda, x_dtype):
    """The tiled W4A16 GEMM at the layer shape (E=128, H=2048, I=768, top-8,
    asymmetric GPTQ banks): every token of a 512-token call against the
    torch-CPU dequantize-then-matmul restatement of projection_torch /
    QuantizedExpertBackend.forward (quantized_kernels.py:48-112, 217-229),
    with bf16 and fp16 activations (fp16 rounds the gate/up weights to fp16)."""
    from oracle import torch_cpu

    print_case("w4a16 tiled prefill", x_dtype)
    g = torch.Generator().manual_seed(20261205)
    store = random_quantized_bank(0, 128, 2048, 768, asymmetric=True, generator=g)
    x = torch.randn(512, 2048, generator=g).to(x_dtype)
    ids, w = orc.route_topk(torch.randn(512, 128, generator=g).numpy(), 8)
    ids = torch.from_numpy(ids)
    weights = torch.from_numpy(w).bfloat16()
    out = quantized.QuantizedExpertBackend(0).forward(x.to(cuda), ids.to(cuda), weights.to(cuda),
                                                      to_device(store, cuda))
    expected = torch_cpu.layer(store, x, ids, weights)
    assert out.dtype == x_dtype
    assert rel_inf(out.float().cpu().numpy(), expected.float().numpy()) < TOL


@pytest.mark.parametrize("rows,n,k,x_dtype", [(1, 2048, 2048, torch.bfloat16), (7, 256, 512, torch.bfloat16),
                                              (300, 1024, 768, torch.float16), (2048, 512, 2048, torch.bfloat16)])
def test_gptq_linear_matches_dequantize_then_matmul(cuda, rows, n, k, x_dtype):
    """Dense GPTQLinear (quantized_model.py:71-91) on the tiled W4A16 kernel
    against the torch-CPU reconstruction of projection_torch (one expert,
    zero point 8), including leading shapes and M in many 64-row chunks."""
    from oracle import torch_cpu

    print_case("gptq linear", rows, n, k, x_dtype)
    g = torch.Generator().manual_seed(rows + n + k)
    words = torch.randint(-2 ** 31, 2 ** 31 - 1, (k // 8, n), generator=g, dtype=torch.int64).to(torch.int32)
    scales = (torch.rand(k // 128, n, generator=g) * 0.02 + 0.002).half()
    lin = quantized.GPTQLinear(words, scales, device=cuda)
    x = torch.randn(rows, k, generator=g).to(x_dtype)
    out = lin(x.to(cuda).reshape(1, rows, k))
    assert out.shape == (1, rows, n) and out.dtype == torch.bfloat16
    matrix = torch_cpu.dequantize(0, words.T.contiguous(), scales.T.contiguous(), k, x_dtype)
    expected = (x.float() @ matrix.T).bfloat16().float()
    assert rel_inf(out.reshape(rows, n).float().cpu().numpy(), expected.numpy()) < 5e-3
