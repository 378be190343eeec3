"""Checkpoint bank loaders on the CPU: each layout written from a bank in
memory (tests/checkpoint_fixtures.py) loads back byte for byte, the
reference's own fixture checks hold (official FP8 bytes per expert slice,
expert_cache_file tests; the W4A8 codebook staging of
tests/test_quantized_model.py), and malformed files are refused before any
bank is built."""
from __future__ import annotations

import json

import pytest
import torch
from safetensors.torch import save_file

from checkpoint_fixtures import (GPTQ_SYMMETRIC_ZEROS, comfy_tensors, gptq_expert_tensors, official_fp8_tensors,
                                 packed_fp8_tensors, same_bank, write_config, write_sharded, write_shared)
from drama_moe import checkpoint as ckpt
from drama_moe.formats import FP8_DTYPE, StagedExperts, random_fp8_bank, random_quantized_bank


def fp8_banks(layers, experts, hidden, inter, seed=5):
    g = torch.Generator().manual_seed(seed)
    return [random_fp8_bank(experts, hidden, inter, layout="block", generator=g) for _ in range(layers)]


def official_checkpoint(tmp_path, layers=2, experts=3, hidden=128, inter=128, stem="model.language_model.layers"):
    banks = fp8_banks(layers, experts, hidden, inter)
    write_config(tmp_path, layers, experts, hidden, inter)
    tensors = official_fp8_tensors(banks, stem)
    tensors["model.language_model.embed_tokens.weight"] = torch.zeros(4, hidden, dtype=torch.bfloat16)
    write_sharded(tmp_path, tensors)
    return banks, tensors


@pytest.mark.parametrize("stem", ["model.language_model.layers", "model.layers"])
def test_official_fp8_banks_round_trip(tmp_path, stem):
    banks, _ = official_checkpoint(tmp_path, stem=stem)
    assert ckpt.expert_format(tmp_path) == "fp8"
    loaded = ckpt.load_expert_banks(tmp_path, device="cpu")
    assert len(loaded) == 2 and all(isinstance(b, StagedExperts) for b in loaded)
    assert all(same_bank(a, b) for a, b in zip(banks, loaded))


def test_official_fp8_expert_slices_keep_the_checkpoint_bytes(tmp_path):
    """The reference's known answer (test_expert_cache_file.py:121-180): raw
    byte tensors as FP8 weights; the gate rows are w13[:, :I], the up rows
    w13[:, I:], scale rows split at I/128, down is w2."""
    hidden = inter = 128
    tensors = {}
    for layer in range(2):
        for expert in range(3):
            for index, (proj, shape) in enumerate((("gate_proj", (inter, hidden)), ("up_proj", (inter, hidden)),
                                                   ("down_proj", (hidden, inter)))):
                g = torch.Generator().manual_seed(100 + layer * 20 + expert * 3 + index)
                base = f"model.language_model.layers.{layer}.mlp.experts.{expert}.{proj}"
                tensors[base + ".weight"] = torch.randint(0, 255, shape, generator=g, dtype=torch.uint8).view(FP8_DTYPE)
                tensors[base + ".weight_scale_inv"] = torch.rand((shape[0] // 128, shape[1] // 128), generator=g)
    write_sharded(tmp_path, tensors)
    write_config(tmp_path, 2, 3, hidden, inter)
    loaded = ckpt.load_expert_banks(tmp_path, device="cpu")
    assert loaded[0].w13_weight.shape == (3, 256, 128) and loaded[0].w2_weight.shape == (3, 128, 128)
    for layer in range(2):
        for expert in range(3):
            for proj, target, rows in (("gate_proj", "w13", slice(0, 128)), ("up_proj", "w13", slice(128, 256)),
                                       ("down_proj", "w2", slice(0, 128))):
                base = f"model.language_model.layers.{layer}.mlp.experts.{expert}.{proj}"
                got = getattr(loaded[layer], target + "_weight")[expert, rows].view(torch.uint8)
                assert torch.equal(got, tensors[base + ".weight"].view(torch.uint8))
                srows = slice(rows.start // 128, rows.stop // 128)
                assert torch.equal(getattr(loaded[layer], target + "_scale_inv")[expert, srows],
                                   tensors[base + ".weight_scale_inv"])


def test_official_fp8_refuses_missing_unknown_and_misshaped_tensors(tmp_path):
    official_checkpoint(tmp_path)
    index_path = tmp_path / "model.safetensors.index.json"
    index = json.loads(index_path.read_text())
    popped = next(n for n in index["weight_map"] if ".mlp.experts." in n)
    shard = index["weight_map"].pop(popped)
    index_path.write_text(json.dumps(index))
    with pytest.raises(ValueError, match="Missing expert"):
        ckpt.load_expert_banks(tmp_path, device="cpu")
    index["weight_map"][popped] = shard
    index["weight_map"]["model.language_model.layers.0.mlp.experts.0.gate_proj.zeros"] = shard
    index_path.write_text(json.dumps(index))
    with pytest.raises(ValueError, match="index/header mismatch"):
        ckpt.load_expert_banks(tmp_path, device="cpu")


def test_official_fp8_refuses_unknown_expert_keys_and_wrong_dtypes(tmp_path):
    banks, tensors = official_checkpoint(tmp_path)
    for path in tmp_path.glob("*.safetensors"):
        path.unlink()
    (tmp_path / "model.safetensors.index.json").unlink()
    bad = dict(tensors)
    bad["model.language_model.layers.0.mlp.experts.0.gate_proj.zeros"] = torch.zeros(1)
    save_file({k: v.contiguous() for k, v in bad.items()}, str(tmp_path / "model.safetensors"))
    with pytest.raises(ValueError, match="Unsupported routed expert"):
        ckpt.load_expert_banks(tmp_path, device="cpu")
    bad = dict(tensors)
    name = "model.language_model.layers.1.mlp.experts.2.up_proj.weight"
    bad[name] = bad[name].float()
    save_file({k: v.contiguous() for k, v in bad.items()}, str(tmp_path / "model.safetensors"))
    with pytest.raises(ValueError, match="Wrong expert shape/dtype"):
        ckpt.load_expert_banks(tmp_path, device="cpu")
    bad = dict(tensors)
    bad["model.language_model.layers.0.mlp.experts.3.up_proj.weight"] = bad[name].clone()
    save_file({k: v.contiguous() for k, v in bad.items()}, str(tmp_path / "model.safetensors"))
    with pytest.raises(ValueError, match="outside model config"):
        ckpt.load_expert_banks(tmp_path, device="cpu")


def test_shared_packed_fp8_banks_round_trip_and_name_checks(tmp_path):
    banks = fp8_banks(2, 4, 256, 128, seed=9)
    write_config(tmp_path, 2, 4, 256, 128)
    tensors = packed_fp8_tensors(banks)
    tensors["model.norm.weight"] = torch.ones(256, dtype=torch.bfloat16)
    write_shared(tmp_path, tensors)
    assert ckpt.expert_format(tmp_path) == "fp8-shared" and ckpt.quantization_mode(tmp_path) is None
    loaded = ckpt.load_expert_banks(tmp_path, device="cpu", layers=[1])
    assert len(loaded) == 1 and same_bank(banks[1], loaded[0])
    tensors["model.layers.1.mlp.experts.extra"] = torch.zeros(1)
    write_shared(tmp_path, tensors)
    with pytest.raises(ValueError, match="Unexpected or missing packed FP8"):
        ckpt.load_expert_banks(tmp_path, device="cpu")
    del tensors["model.layers.1.mlp.experts.extra"]
    tensors["model.layers.0.mlp.experts.down_scale"] = torch.ones(4, 2, 2)
    write_shared(tmp_path, tensors)
    with pytest.raises(ValueError, match="Wrong expert shape/dtype"):
        ckpt.load_expert_banks(tmp_path, device="cpu")


def test_shared_descriptor_is_checked(tmp_path):
    banks = fp8_banks(1, 2, 128, 128)
    write_config(tmp_path, 1, 2, 128, 128)
    write_shared(tmp_path, packed_fp8_tensors(banks))
    descriptor = json.loads((tmp_path / "shared-model.json").read_text())
    for change in ({"format": "other"}, {"sha256": "xyz"}, {"size": descriptor["size"] + 1}):
        (tmp_path / "shared-model.json").write_text(json.dumps({**descriptor, **change}))
        with pytest.raises(ValueError, match="descriptor|size changed"):
            ckpt.expert_format(tmp_path)


@pytest.mark.parametrize("asymmetric", [False, True])
def test_gptq_expert_banks_round_trip(tmp_path, asymmetric):
    g = torch.Generator().manual_seed(31 + asymmetric)
    banks = [random_quantized_bank(0, 3, 256, 128, asymmetric=asymmetric, generator=g) for _ in range(2)]
    write_config(tmp_path, 2, 3, 256, 128, quantization_config={"quant_method": "drama3-int4"})
    write_sharded(tmp_path, gptq_expert_tensors(banks))
    assert ckpt.quantization_mode(tmp_path) == 0 and ckpt.expert_format(tmp_path) == 0
    loaded = ckpt.load_expert_banks(tmp_path, device="cpu")
    assert all(same_bank(a, b) for a, b in zip(banks, loaded))
    assert (loaded[0].w13_zeros is None) == (not asymmetric)


def test_gptq_expert_bank_without_qzeros_and_with_permuted_groups(tmp_path):
    g = torch.Generator().manual_seed(3)
    banks = [random_quantized_bank(0, 2, 256, 128, generator=g)]
    write_config(tmp_path, 1, 2, 256, 128, quantization_config={"quant_method": "drama3-int4"})
    tensors = gptq_expert_tensors(banks, with_zeros=False)
    write_sharded(tmp_path, tensors)
    assert same_bank(banks[0], ckpt.load_expert_banks(tmp_path, device="cpu")[0])
    name = "model.language_model.layers.0.mlp.experts.1.gate_proj.g_idx"  # K = 256: two groups
    tensors[name] = tensors[name].flip(0).contiguous()
    write_sharded(tmp_path, tensors)
    with pytest.raises(ValueError, match="permuted GPTQ"):
        ckpt.load_expert_banks(tmp_path, device="cpu")


def test_gptq_dense_linear_checks_symmetry_and_grouping(tmp_path):
    g = torch.Generator().manual_seed(8)
    k, n = 512, 256
    qweight = torch.randint(-2 ** 31, 2 ** 31 - 1, (k // 8, n), generator=g, dtype=torch.int32)
    scales = (torch.rand(k // 128, n, generator=g) * 0.01).half()
    base = "model.language_model.layers.0.self_attn.q_proj"
    tensors = {base + ".qweight": qweight, base + ".scales": scales,
               base + ".qzeros": torch.full((k // 128, n // 8), GPTQ_SYMMETRIC_ZEROS, dtype=torch.int32),
               base + ".g_idx": torch.arange(k, dtype=torch.int32) // 128,
               "model.language_model.layers.0.mlp.experts.0.gate_proj.qweight": qweight.clone()}
    save_file(tensors, str(tmp_path / "model.safetensors"))
    reader = ckpt.CheckpointTensors.from_directory(tmp_path)
    assert ckpt.gptq_dense_names(reader) == [base]
    linear = ckpt.gptq_dense_linear(reader, base, device="cpu")
    assert (linear.in_features, linear.out_features) == (k, n)
    assert torch.equal(linear.qweight, qweight.T) and torch.equal(linear.scales, scales.T)
    tensors[base + ".qzeros"] = tensors[base + ".qzeros"].clone()
    tensors[base + ".qzeros"][1, 3] = 0x77777777
    save_file(tensors, str(tmp_path / "model.safetensors"))
    with pytest.raises(ValueError, match="asymmetric or permuted"):
        ckpt.gptq_dense_linear(ckpt.CheckpointTensors.from_directory(tmp_path), base, device="cpu")


@pytest.mark.parametrize("mode,quantization", [(1, "int8_convrot"), (2, "w6a8"), (3, "w4a8")])
def test_comfy_banks_round_trip(tmp_path, mode, quantization):
    g = torch.Generator().manual_seed(40 + mode)
    banks = [random_quantized_bank(mode, 2, 256, 256, generator=g) for _ in range(2)]
    write_config(tmp_path, 2, 2, 256, 256)
    write_shared(tmp_path, comfy_tensors(banks, mode), quantization=quantization)
    assert ckpt.quantization_mode(tmp_path) == mode and ckpt.expert_format(tmp_path) == mode
    loaded = ckpt.load_expert_banks(tmp_path, device="cpu")
    assert all(same_bank(a, b) for a, b in zip(banks, loaded))


def _reference_w4a8_values(rotation=256):
    """The synthetic W4A8 bank of the reference's tests/test_quantized_model.py:
    two experts, H = I = 512, zero codes, relative scale bytes of 1, channel
    scales of 1.0 and the codebook linspace(-10, 11, 16)."""
    table = torch.linspace(-10, 11, 16)
    tensors = {}
    for name, rows in (("gate_up_proj", 1024), ("down_proj", 512)):
        base = "model.layers.0.mlp.experts." + name
        tensors[base + ".weight"] = torch.zeros(2, rows, 256, dtype=torch.int8)
        tensors[base + ".weight_s_rel"] = torch.ones(2, rows, 32, dtype=torch.uint8)
        tensors[base + ".weight_s_channel"] = torch.ones(2, rows)
        tensors[base + ".weight_codebook"] = table.clone()
        config = {"format": "asym_w4a8_int8", "group_size": 16, "convrot_groupsize": rotation, "num_experts": 2}
        tensors[base + ".comfy_quant"] = torch.tensor(list(json.dumps(config).encode()), dtype=torch.uint8)
    return tensors, table


def test_w4a8_codebook_sits_in_each_experts_first_sixteen_aux_rows(tmp_path):
    tensors, table = _reference_w4a8_values()
    write_config(tmp_path, 1, 2, 512, 512)
    write_shared(tmp_path, tensors, quantization="w4a8")
    store = ckpt.load_expert_banks(tmp_path, device="cpu")[0]
    for aux in (store.w13_scale_inv, store.w2_scale_inv):
        restored = aux[:, :16, 36:40].contiguous().view(torch.float32).squeeze(-1)
        assert torch.equal(restored, table.expand(2, 16))
        assert torch.equal(aux[..., 32:36].contiguous().view(torch.float32), torch.ones(*aux.shape[:2], 1))
        assert not aux[:, 16:, 36:40].any()


def test_w4a8_refuses_another_rotation_or_format(tmp_path):
    tensors, _ = _reference_w4a8_values(rotation=64)
    write_config(tmp_path, 1, 2, 512, 512)
    write_shared(tmp_path, tensors, quantization="w4a8")
    with pytest.raises(ValueError, match="ConvRot group"):
        ckpt.load_expert_banks(tmp_path, device="cpu")
    tensors, _ = _reference_w4a8_values()
    write_shared(tmp_path, tensors, quantization="w6a8")  # mode 2 reading a W4A8 bank
    with pytest.raises(ValueError, match="w6a8_int8"):
        ckpt.load_expert_banks(tmp_path, device="cpu")


def test_quantization_mode_and_geometry_checks(tmp_path):
    assert ckpt.quantization_mode(tmp_path) is None
    write_config(tmp_path, 1, 2, 128, 128, quantization_config={"quant_method": "drama3-int4"})
    assert ckpt.quantization_mode(tmp_path) == 0
    with pytest.raises(ValueError, match="text_config"):
        ckpt.BankGeometry.from_config({})
    with pytest.raises(ValueError, match="num_experts"):
        ckpt.BankGeometry.from_config({"text_config": {"num_hidden_layers": 1, "num_experts": 0, "hidden_size": 8,
                                                       "moe_intermediate_size": 8}})
    geometry = ckpt.BankGeometry.from_config(json.loads((tmp_path / "config.json").read_text()))
    assert geometry == ckpt.BankGeometry(1, 2, 128, 128)


def test_bound_banks_are_what_the_expert_manager_runs(tmp_path):
    """bind_expert_bank makes a module hold a loaded bank the way the
    reference's loaders do, and the expert manager resolves exactly that bank."""
    from torch import nn

    from drama_moe import offload
    g = torch.Generator().manual_seed(12)
    fp8 = fp8_banks(1, 4, 128, 128)[0]
    packed = random_quantized_bank(2, 4, 256, 256, generator=g)
    for bank in (fp8, packed):
        module = nn.Module()
        ckpt.bind_expert_bank(module, bank)
        resolved = offload.store_from_module(module)
        assert resolved is bank if bank is packed else same_bank(resolved, bank)
        assert module.w13_weight is bank.w13_weight
    module = nn.Module()
    ckpt.bind_expert_bank(module, packed)
    ckpt.bind_expert_bank(module, fp8)  # rebinding to FP8 drops the packed store
    assert isinstance(offload.store_from_module(module), StagedExperts)
