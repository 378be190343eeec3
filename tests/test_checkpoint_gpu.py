"""Banks loaded from each checkpoint layout straight onto the GPU run through
the expert kernels and give bit-for-bit the output of the same bank built in
memory (whose parity with the oracle the other GPU tests hold), and the FP8
one matches the oracle directly."""
from __future__ import annotations

import dataclasses

import numpy as np
import pytest
import torch

from checkpoint_fixtures import (comfy_tensors, gptq_expert_tensors, official_fp8_tensors, packed_fp8_tensors,
                                 write_config, write_sharded, write_shared)
from conftest import print_case
from drama_moe import checkpoint as ckpt
from drama_moe.formats import QuantizedStore, StagedExperts, random_fp8_bank, random_quantized_bank
from drama_moe.offload import HipExpertBackend
from drama_moe.quantized import QuantizedExpertBackend
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

HIDDEN, INTER, EXPERTS, TOP_K = 512, 256, 8, 4


def routing(tokens, g, device):
    ids = torch.stack([torch.randperm(EXPERTS, generator=g)[:TOP_K] for _ in range(tokens)]).to(torch.int32)
    weights = torch.softmax(torch.randn(tokens, TOP_K, generator=g), -1)
    x = torch.randn(tokens, HIDDEN, generator=g).bfloat16()
    return x.to(device), ids.to(device), weights.to(device)


def on_device(bank, device):
    fields = {f.name: getattr(bank, f.name) for f in dataclasses.fields(bank)}
    return type(bank)(**{k: (v.to(device) if isinstance(v, torch.Tensor) else v) for k, v in fields.items()})


@pytest.mark.parametrize("layout", ["fp8", "fp8-shared"])
@pytest.mark.parametrize("tokens", [1, 6])
def test_fp8_checkpoint_bank_runs_like_the_in_memory_bank(cuda, tmp_path, layout, tokens):
    print_case("checkpoint fp8", layout, tokens)
    g = torch.Generator().manual_seed(61 + tokens)
    bank = random_fp8_bank(EXPERTS, HIDDEN, INTER, layout="block", generator=g)
    write_config(tmp_path, 1, EXPERTS, HIDDEN, INTER)
    if layout == "fp8":
        write_sharded(tmp_path, official_fp8_tensors([bank]))
    else:
        write_shared(tmp_path, packed_fp8_tensors([bank]))
    loaded = ckpt.load_expert_banks(tmp_path, device=cuda)[0]
    assert isinstance(loaded, StagedExperts) and loaded.w13_weight.device.type == "cuda"
    x, ids, weights = routing(tokens, g, cuda)
    backend = HipExpertBackend()
    got = backend.forward(x, ids, weights, loaded)
    want = backend.forward(x, ids, weights, on_device(bank, cuda))
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    b13 = orc.Fp8Bank(bank.w13_weight.view(torch.uint8).numpy(), bank.w13_scale_inv.numpy())
    b2 = orc.Fp8Bank(bank.w2_weight.view(torch.uint8).numpy(), bank.w2_scale_inv.numpy())
    expected = orc.fp8_moe_forward(b13, b2, x.float().cpu().numpy(), ids.cpu().numpy(), weights.cpu().numpy())
    actual = got.float().cpu().numpy()
    assert np.max(np.abs(actual - expected)) / max(np.max(np.abs(expected)), 1e-30) < 2e-2


@pytest.mark.parametrize("mode", [0, 1, 2, 3])
@pytest.mark.parametrize("tokens", [1, 6])
def test_packed_checkpoint_bank_runs_like_the_in_memory_bank(cuda, tmp_path, mode, tokens):
    print_case("checkpoint packed", mode, tokens)
    g = torch.Generator().manual_seed(90 + 10 * mode + tokens)
    bank = random_quantized_bank(mode, EXPERTS, HIDDEN, INTER, asymmetric=mode == 0, generator=g)
    if mode == 0:
        write_config(tmp_path, 1, EXPERTS, HIDDEN, INTER, quantization_config={"quant_method": "drama3-int4"})
        write_sharded(tmp_path, gptq_expert_tensors([bank]))
    else:
        write_config(tmp_path, 1, EXPERTS, HIDDEN, INTER)
        write_shared(tmp_path, comfy_tensors([bank], mode), quantization={1: "int8_convrot", 2: "w6a8",
                                                                         3: "w4a8"}[mode])
    loaded = ckpt.load_expert_banks(tmp_path, device=cuda)[0]
    assert isinstance(loaded, QuantizedStore) and loaded.mode == mode
    x, ids, weights = routing(tokens, g, cuda)
    backend = QuantizedExpertBackend(mode)
    got = backend.forward(x, ids, weights, loaded)
    want = backend.forward(x, ids, weights, on_device(bank, cuda))
    torch.cuda.synchronize()
    assert torch.equal(got, want)
