"""GPU parity of the grouped (prefill) FP8 W8A8 expert path against the oracle.

Calls above 256 route pairs run the moe_align permutation, the grouped
gate/up and down GEMMs and the slot-order combine.  Routing ids are bit-exact;
outputs within ||y - r||_inf / ||r||_inf <= 2e-2 of the contract oracle
(activation quantization emulated, compute-dtype gate/up boundary).  Expert
popularity follows Zipf(1.1) over a seeded rank permutation (top-k by
log p + Gumbel noise), so some experts span many 64-row tiles and some get few
or no pairs.
"""
import numpy as np
import pytest
import torch

from conftest import print_case
from drama_moe import fp8_moe, router
from moe_align_props import check_moe_align
from drama_moe.formats import StagedExperts, random_fp8_bank
from drama_moe.offload import HipExpertBackend
from oracle import oracle as orc

pytestmark = pytest.mark.gpu
TOL = 2e-2


def rel_inf(actual, expected):
    actual = np.asarray(actual, np.float64)
    expected = np.asarray(expected, np.float64)
    return float(np.max(np.abs(actual - expected)) / max(np.max(np.abs(expected)), 1e-30))


def zipf_logits(tokens, experts, seed, exponent=1.1):
    """log p_e + Gumbel(0, 1) with p_e ~ rank_e^-exponent over a seeded rank
    permutation: top-k of these logits samples experts without replacement."""
    g = torch.Generator().manual_seed(seed)
    ranks = torch.randperm(experts, generator=g).double() + 1
    logp = -exponent * torch.log(ranks)
    logp -= torch.logsumexp(logp, 0)
    u = torch.rand(tokens, experts, generator=g, dtype=torch.float64).clamp_(1e-12, 1 - 1e-12)
    return (logp - torch.log(-torch.log(u))).float()


def oracle_banks(staged: StagedExperts):
    return (orc.Fp8Bank(staged.w13_weight.view(torch.uint8).cpu().numpy(), staged.w13_scale_inv.cpu().numpy()),
            orc.Fp8Bank(staged.w2_weight.view(torch.uint8).cpu().numpy(), staged.w2_scale_inv.cpu().numpy()))


def to_device(staged: StagedExperts, device) -> StagedExperts:
    return StagedExperts(*(getattr(staged, n).to(device) for n in
                           ("w13_weight", "w13_scale_inv", "w2_weight", "w2_scale_inv")))


@pytest.fixture(scope="module", autouse=True)
def built():
    orc.build()


def _case(cuda, experts, hidden, inter, tokens, top_k, layout, seed, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    staged = random_fp8_bank(experts, hidden, inter, layout=layout, generator=g)
    x = torch.randn(tokens, hidden, generator=g).to(dtype)
    ids, w = orc.route_topk(zipf_logits(tokens, experts, seed).numpy(), top_k)
    weights = torch.from_numpy(w).to(dtype)
    return staged, x, ids, weights


@pytest.mark.parametrize("layout", ["block", "channel"])
@pytest.mark.parametrize("x_group", [128, "token"])
def test_grouped_layer_matches_oracle(cuda, layout, x_group):
    print_case("grouped layer", layout, x_group)
    staged, x, ids, weights = _case(cuda, 32, 1024, 512, 96, 8, layout, 31337)
    counts = np.bincount(ids.reshape(-1), minlength=32)
    assert counts.max() > 64 and (counts < 64).any()  # multi-tile and partial-tile experts
    b13, b2 = oracle_banks(staged)
    expected = orc.fp8_moe_forward(b13, b2, x.float().numpy(), ids, weights.float().numpy(),
                                   x_group=128 if x_group == 128 else 1024)
    out = HipExpertBackend(x_group=x_group).forward(x.to(cuda), torch.from_numpy(ids).to(cuda),
                                                    weights.to(cuda), to_device(staged, cuda))
    assert out.dtype == torch.bfloat16 and out.shape == x.shape
    assert rel_inf(out.float().cpu().numpy(), expected) < TOL


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_grouped_layer_other_compute_dtypes(cuda, dtype):
    print_case("grouped dtype", dtype)
    staged, x, ids, weights = _case(cuda, 16, 512, 256, 40, 8, "block", 4040, dtype)
    gu = {torch.float16: "fp16", torch.float32: "fp32"}[dtype]
    b13, b2 = oracle_banks(staged)
    expected = orc.fp8_moe_forward(b13, b2, x.float().numpy(), ids, weights.float().numpy(),
                                   gu_dtype=gu, out_dtype=gu)
    out = HipExpertBackend().forward(x.to(cuda), torch.from_numpy(ids).to(cuda), weights.to(cuda),
                                     to_device(staged, cuda))
    assert out.dtype == dtype
    assert rel_inf(out.float().cpu().numpy(), expected) < TOL


def test_grouped_pairs_with_duplicates_match_oracle(cuda):
    """forward_pairs above 256 rows: ordered fp32 partials, duplicates kept apart."""
    print_case("grouped pairs")
    g = torch.Generator().manual_seed(77)
    staged = random_fp8_bank(8, 512, 256, generator=g)
    rows = 300
    x = torch.randn(rows, 512, generator=g).bfloat16()
    ids = torch.randint(0, 8, (rows, 1), generator=g)
    ids[1] = ids[0]
    x[1] = x[0]
    weights = torch.rand(rows, 1, generator=g) + 0.1
    out = HipExpertBackend().forward_pairs(x.to(cuda), ids.to(cuda), weights.to(cuda), to_device(staged, cuda))
    assert out.dtype == torch.float32 and out.shape == (rows, 512)
    b13, b2 = oracle_banks(staged)
    xf = x.float().numpy()
    expected = np.concatenate([orc.fp8_expert_pairs(b13, b2, xf[r], ids[r].numpy(), weights[r].numpy())
                               for r in range(rows)])
    assert rel_inf(out.cpu().numpy(), expected) < TOL
    torch.testing.assert_close(out[0] / weights[0].to(cuda), out[1] / weights[1].to(cuda), rtol=1e-6, atol=1e-6)


def test_grouped_invalid_ids_contribute_zero_and_raise_status(cuda):
    print_case("grouped invalid ids")
    staged, x, ids, weights = _case(cuda, 16, 512, 256, 48, 8, "block", 99)
    bad = ids.copy()
    bad[3, 2] = -1
    bad[10, 0] = 16
    backend = HipExpertBackend()
    backend.status(cuda)
    out = backend.forward(x.to(cuda), torch.from_numpy(bad).to(cuda), weights.to(cuda), to_device(staged, cuda))
    assert backend.status(cuda) & 1
    clean_ids, clean_w = ids.copy(), weights.float().numpy().copy()
    clean_ids[3, 2] = clean_ids[10, 0] = 0
    clean_w[3, 2] = clean_w[10, 0] = 0.0
    b13, b2 = oracle_banks(staged)
    expected = orc.fp8_moe_forward(b13, b2, x.float().numpy(), clean_ids, clean_w)
    assert rel_inf(out.float().cpu().numpy(), expected) < TOL
    pairs = backend.forward_pairs(x.to(cuda).repeat_interleave(8, 0), torch.from_numpy(bad).reshape(-1, 1).to(cuda),
                                  weights.reshape(-1, 1).to(cuda), to_device(staged, cuda))
    assert backend.status(cuda) & 1
    assert torch.count_nonzero(pairs[3 * 8 + 2]) == 0 and torch.count_nonzero(pairs[10 * 8]) == 0


def test_grouped_layer_in_hipgraph(cuda):
    print_case("grouped hipgraph")
    g = torch.Generator().manual_seed(5)
    staged = to_device(random_fp8_bank(16, 512, 256, generator=g), cuda)
    backend = HipExpertBackend()
    x = torch.randn(64, 512, device=cuda).bfloat16()
    logits = zipf_logits(64, 16, 5).to(cuda)
    out = torch.empty_like(x)
    stream = torch.cuda.Stream(cuda)
    stream.wait_stream(torch.cuda.current_stream(cuda))
    with torch.cuda.stream(stream):
        backend.forward_routed(x, logits, 8, staged, out=out)
    torch.cuda.current_stream(cuda).wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        _, w_g, i_g = backend.forward_routed(x, logits, 8, staged, out=out)
    for step in range(3):
        logits.copy_(zipf_logits(64, 16, 100 + step).to(cuda))
        x.copy_(torch.randn(64, 512, device=cuda).bfloat16())
        expected, w_e, i_e = backend.forward_routed(x, logits, 8, staged)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(i_g, i_e) and torch.equal(w_g, w_e), step
        assert torch.equal(out, expected), step


@pytest.mark.parametrize("x_group", ["token", 128])
def test_prefill_2048_tokens_full_shape(cuda, x_group):
    """The prefill workload: 2048 tokens, top-8 of 128 Zipf(1.1) experts,
    H 2048, I 768, per-channel FP8 weights.  ids bit-exact for every token;
    every token's output within the bar of the decode kernels (pinned to the
    oracle by the decode tests) run on the same routes in 32-token calls, so
    every tile of every expert is covered; and 64 spread tokens against the
    oracle directly."""
    print_case("prefill 2048", x_group)
    experts, hidden, inter, tokens = 128, 2048, 768, 2048
    staged = random_fp8_bank(experts, hidden, inter, layout="channel", device=cuda,
                             generator=torch.Generator(device=cuda).manual_seed(20261203))
    g = torch.Generator().manual_seed(20261203)
    x = torch.randn(tokens, hidden, generator=g).bfloat16()
    logits = zipf_logits(tokens, experts, 20261203)
    out, weights, ids = HipExpertBackend(x_group=x_group).forward_routed(x.to(cuda), logits.to(cuda), 8, staged)
    eids, _ = orc.route_topk(logits.numpy(), 8)
    np.testing.assert_array_equal(ids.cpu().numpy(), eids)
    counts = np.bincount(eids.reshape(-1), minlength=experts)
    assert counts.max() > 1000
    backend = HipExpertBackend(x_group=x_group)
    xd = x.to(cuda)
    decode = torch.cat([backend.forward(xd[t:t + 32], ids[t:t + 32], weights[t:t + 32], staged)
                        for t in range(0, tokens, 32)])
    got, ref = out.float(), decode.float()
    per_token = ((got - ref).abs().amax(1) / ref.abs().amax(1).clamp_min(1e-30)).cpu().numpy()
    assert per_token.max() < TOL, (int(per_token.argmax()), float(per_token.max()))
    pick = np.linspace(0, tokens - 1, 64).astype(int)
    b13, b2 = oracle_banks(staged)
    expected = orc.fp8_moe_forward(b13, b2, x.float().numpy()[pick], eids[pick],
                                   weights.float().cpu().numpy()[pick],
                                   x_group=128 if x_group == 128 else hidden)
    assert rel_inf(out.float().cpu().numpy()[pick], expected) < TOL
    assert torch.isfinite(out.float()).all()


@pytest.mark.parametrize("x_group", ["token", 128])
def test_grouped_work_lists_longer_than_one_chunk(cuda, x_group):
    """8192 tokens x top-8 over 64 experts at H 1280, I 768: both grouped GEMMs
    have more (column tile, row tile) work items than the persistent grid
    holds in one chunk of tile metadata per workgroup (gate/up 6 x ~1100,
    down 5 x ~1100 items over 256 workgroups of 16-item chunks), so the
    expert-major work order runs across chunk boundaries.  Every token within
    the bar of the decode kernels on the same routes (32-token calls), and 32
    spread tokens against the oracle."""
    print_case("grouped multi-chunk", x_group)
    experts, hidden, inter, tokens = 64, 1280, 768, 8192
    staged = random_fp8_bank(experts, hidden, inter, layout="channel", device=cuda,
                             generator=torch.Generator(device=cuda).manual_seed(20261204))
    g = torch.Generator().manual_seed(20261204)
    x = torch.randn(tokens, hidden, generator=g).bfloat16()
    logits = zipf_logits(tokens, experts, 20261204)
    backend = HipExpertBackend(x_group=x_group)
    xd = x.to(cuda)
    out, weights, ids = backend.forward_routed(xd, logits.to(cuda), 8, staged)
    counts = np.bincount(ids.cpu().numpy().reshape(-1), minlength=experts)
    row_tiles = int(((counts + 63) // 64).sum())
    cus = torch.cuda.get_device_properties(cuda).multi_processor_count
    assert min(inter // 128, (hidden + 255) // 256) * row_tiles > 16 * (cus // 8 * 8)  # > one chunk each
    decode = torch.cat([backend.forward(xd[t:t + 32], ids[t:t + 32], weights[t:t + 32], staged)
                        for t in range(0, tokens, 32)])
    torch.cuda.synchronize()
    assert backend.status(cuda) == 0
    got, ref = out.float(), decode.float()
    per_token = ((got - ref).abs().amax(1) / ref.abs().amax(1).clamp_min(1e-30)).cpu().numpy()
    assert per_token.max() < TOL, (int(per_token.argmax()), float(per_token.max()))
    pick = np.linspace(0, tokens - 1, 32).astype(int)
    b13, b2 = oracle_banks(staged)
    expected = orc.fp8_moe_forward(b13, b2, x.float().numpy()[pick], ids.cpu().numpy()[pick],
                                   weights.float().cpu().numpy()[pick],
                                   x_group=128 if x_group == 128 else hidden)
    assert rel_inf(out.float().cpu().numpy()[pick], expected) < TOL


@pytest.mark.parametrize("pairs,experts,block_m,zipf", [
    (16384, 128, 64, True),    # the prefill workload's tile map (one-launch placement)
    (16384, 128, 16, True),
    (16384, 128, 32, True),
    (600, 32, 16, False),      # single-workgroup permutation
    (100000, 128, 64, False),  # scan + scatter permutation
    (5000, 512, 128, False),
])
def test_moe_align_tile_map(cuda, pairs, experts, block_m, zipf):
    """dmoe_moe_align (the permutation kernels' tile map expanded to the
    moe_align layout) bit-exact against the oracle, and the properties that
    fix the layout: every valid pair in exactly one block of its expert,
    ascending within the expert, sentinels only at each expert's tail."""
    print_case("moe_align", pairs, experts, block_m)
    if zipf:
        ids, _ = orc.route_topk(zipf_logits(pairs // 8, experts, 20261203).numpy(), 8)
    else:
        rng = np.random.default_rng(pairs + block_m)
        ids = rng.integers(0, experts, pairs)
        ids[rng.integers(0, pairs, 4)] = [-3, experts, experts + 1, -1]
    for dtype in (torch.int64, torch.int32):
        sorted_ids, expert_ids, padded = fp8_moe.moe_align(torch.from_numpy(ids).to(dtype).to(cuda), experts,
                                                           block_m)
        esorted, eexperts, epadded = orc.moe_align(ids, experts, block_m)
        assert int(padded.item()) == epadded
        np.testing.assert_array_equal(expert_ids.cpu().numpy(), eexperts)
        np.testing.assert_array_equal(sorted_ids.cpu().numpy(), esorted)
        check_moe_align(sorted_ids.cpu().numpy(), expert_ids.cpu().numpy(), epadded, ids, experts, block_m)
