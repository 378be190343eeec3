"""Writers of small synthetic checkpoints in each layout the bank loaders
read, from a bank held in memory: each splits the bank the way the
checkpoint stores it (per-expert gate / up / down tensors, GPTQ's [K/8, N]
transposed words, ComfyUI's separate relative / channel scales), so a load
must undo exactly that to give the bank back."""
from __future__ import annotations

import json
from pathlib import Path

import torch
from safetensors.torch import save_file

from drama_moe.formats import QuantizedStore, StagedExperts

GPTQ_SYMMETRIC_ZEROS = -2004318072  # 0x88888888 as int32: eight zero points of 8


def write_config(root: Path, layers: int, experts: int, hidden: int, inter: int, **extra) -> None:
    text = {"num_hidden_layers": layers, "num_experts": experts, "hidden_size": hidden,
            "moe_intermediate_size": inter}
    (root / "config.json").write_text(json.dumps({"model_type": "fish_omni", "text_config": text, **extra}))


def write_sharded(root: Path, tensors: dict, shards: int = 2) -> None:
    """Tensors spread round-robin over ``shards`` files plus the index."""
    weight_map = {}
    for index in range(shards):
        name = f"model-{index + 1:05d}-of-{shards:05d}.safetensors"
        part = {k: v.contiguous() for i, (k, v) in enumerate(tensors.items()) if i % shards == index}
        save_file(part, str(root / name))
        weight_map.update({k: name for k in part})
    (root / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": weight_map}))


def write_shared(root: Path, tensors: dict, quantization: str | None = None) -> None:
    """One packed file plus its ``shared-model.json`` descriptor."""
    model = root / "packed.safetensors"
    save_file({k: v.contiguous() for k, v in tensors.items()}, str(model))
    document = {"format": "drama3-packed-shared-v1", "model": model.name, "size": model.stat().st_size,
                "sha256": "0" * 64}
    if quantization is not None:
        document["quantization"] = quantization
    (root / "shared-model.json").write_text(json.dumps(document))


def official_fp8_tensors(banks: list, stem: str = "model.language_model.layers") -> dict:
    """Per-expert gate / up / down weights and block scales of FP8 banks."""
    tensors = {}
    for layer, bank in enumerate(banks):
        inter = bank.w13_weight.shape[1] // 2
        for e in range(bank.w13_weight.shape[0]):
            base = f"{stem}.{layer}.mlp.experts.{e}"
            for proj, weight, scale in (
                    ("gate_proj", bank.w13_weight[e, :inter], bank.w13_scale_inv[e, :inter // 128]),
                    ("up_proj", bank.w13_weight[e, inter:], bank.w13_scale_inv[e, inter // 128:]),
                    ("down_proj", bank.w2_weight[e], bank.w2_scale_inv[e])):
                tensors[f"{base}.{proj}.weight"] = weight.clone()
                tensors[f"{base}.{proj}.weight_scale_inv"] = scale.clone()
    return tensors


def packed_fp8_tensors(banks: list) -> dict:
    names = {"w13_weight": "gate_up_weight", "w13_scale_inv": "gate_up_scale", "w2_weight": "down_weight",
             "w2_scale_inv": "down_scale"}
    return {f"model.layers.{layer}.mlp.experts.{src}": getattr(bank, dst).clone()
            for layer, bank in enumerate(banks) for dst, src in names.items()}


def gptq_expert_tensors(banks: list, *, with_zeros: bool = True) -> dict:
    """GPTQ per-expert ``qweight`` [K/8, N], ``scales`` [K/128, N],
    ``qzeros`` [K/128, N/8] (symmetric ones when the bank has none) and
    ``g_idx``."""
    tensors = {}
    for layer, bank in enumerate(banks):
        inter, hidden = bank.intermediate, bank.hidden
        for e in range(bank.num_experts):
            base = f"model.language_model.layers.{layer}.mlp.experts.{e}"
            for proj, rows, target, k in (("gate_proj", slice(0, inter), "w13", hidden),
                                          ("up_proj", slice(inter, 2 * inter), "w13", hidden),
                                          ("down_proj", slice(0, hidden), "w2", inter)):
                w = getattr(bank, target + "_weight")[e, rows]
                tensors[f"{base}.{proj}.qweight"] = w.T.clone()
                tensors[f"{base}.{proj}.scales"] = getattr(bank, target + "_scale_inv")[e, rows].T.clone()
                zeros = getattr(bank, target + "_zeros")
                words = slice(rows.start // 8, rows.stop // 8)
                if zeros is not None:
                    tensors[f"{base}.{proj}.qzeros"] = zeros[e][:, words].clone()
                elif with_zeros:
                    tensors[f"{base}.{proj}.qzeros"] = torch.full((k // 128, w.shape[0] // 8), GPTQ_SYMMETRIC_ZEROS,
                                                                  dtype=torch.int32)
                tensors[f"{base}.{proj}.g_idx"] = torch.arange(k, dtype=torch.int32) // 128
    return tensors


def comfy_tensors(banks: list, mode: int, *, rotation: int = 256) -> dict:
    """ComfyUI-style packed modes 1-3: ``weight``, ``comfy_quant`` JSON and
    ``weight_scale`` (mode 1) or ``weight_s_rel`` / ``weight_s_channel``
    (+ ``weight_codebook``, read from the first aux row of expert 0)."""
    fmt = {1: "int8_tensorwise", 2: "w6a8_int8", 3: "asym_w4a8_int8"}[mode]
    tensors = {}
    for layer, bank in enumerate(banks):
        for target, source, k in (("w13", "gate_up_proj", bank.hidden), ("w2", "down_proj", bank.intermediate)):
            base = f"model.layers.{layer}.mlp.experts.{source}"
            weight, aux = getattr(bank, target + "_weight"), getattr(bank, target + "_scale_inv")
            config = {"format": fmt, "convrot_groupsize": rotation, "num_experts": bank.num_experts}
            if mode == 1:
                config["convrot"] = True
                tensors[base + ".weight_scale"] = aux[..., 0].clone()
            else:
                config["group_size"] = 16
                tensors[base + ".weight_s_rel"] = aux[..., :k // 16].clone()
                tensors[base + ".weight_s_channel"] = aux[..., k // 16:k // 16 + 4].contiguous().view(
                    torch.float32)[..., 0].clone()
                if mode == 3:
                    tensors[base + ".weight_codebook"] = aux[0, :16, k // 16 + 4:].contiguous().view(
                        torch.float32)[:, 0].clone()
            tensors[base + ".weight"] = weight.clone()
            tensors[base + ".comfy_quant"] = torch.tensor(list(json.dumps(config).encode()), dtype=torch.uint8)
    return tensors


def same_bank(a, b) -> bool:
    """Byte equality of two banks (and of their zero points)."""
    names = ["w13_weight", "w13_scale_inv", "w2_weight", "w2_scale_inv"]
    if isinstance(a, QuantizedStore):
        if (a.mode, a.hidden, a.intermediate) != (b.mode, b.hidden, b.intermediate):
            return False
        for z in ("w13_zeros", "w2_zeros"):
            za, zb = getattr(a, z), getattr(b, z)
            if (za is None) != (zb is None) or (za is not None and not torch.equal(za.cpu(), zb.cpu())):
                return False
    else:
        assert isinstance(a, StagedExperts)
    for n in names:
        x, y = getattr(a, n).cpu(), getattr(b, n).cpu()
        if x.shape != y.shape or x.dtype != y.dtype or not torch.equal(x.contiguous().view(torch.uint8),
                                                                        y.contiguous().view(torch.uint8)):
            return False
    return True
