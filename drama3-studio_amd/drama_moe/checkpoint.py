"""Routed-expert banks read from Drama 3 safetensors checkpoints.

Every checkpoint layout the reference loads a layer's experts from, turned
into the bank types the HIP backends take (``StagedExperts`` for FP8,
``QuantizedStore`` for the packed modes):

* official FP8 (per-expert ``...mlp.experts.{e}.{gate,up,down}_proj.weight``
  e4m3 with ``weight_scale_inv`` 128x128 block scales;
  src/drama_low_vram/expert_cache_file.py:35-54, 243-266),
* the shared packed FP8 file (``model.layers.{i}.mlp.experts.gate_up_weight``
  / ``down_weight`` / ``gate_up_scale`` / ``down_scale``;
  src/drama_low_vram/shared_checkpoint.py:26-43, 108-130),
* INT4 GPTQ (``quant_method: drama3-int4``: per-expert ``qweight`` [K/8, N]
  int32 and ``scales`` [K/128, N] fp16, stored transposed with gate and up
  concatenated; src/drama_low_vram/quantized_model.py:156-168) and its dense
  GPTQ linears (quantized_model.py:186-200),
* the ComfyUI-style packed banks of modes 1-3 (INT8 ConvRot, W6A8, W4A8
  codebook: ``weight`` + ``comfy_quant`` JSON + ``weight_scale`` or
  ``weight_s_rel`` / ``weight_s_channel`` / ``weight_codebook``;
  quantized_model.py:94-153).

Files are opened with ``safetensors.safe_open`` (a header plus raw payload;
nothing in the file is executed) and checked against the config's geometry
from the headers before any payload is read.  Banks are built on the host and
moved to ``device`` whole: every expert of a layer stays resident in HBM.
"""
from __future__ import annotations

import json
import re
from dataclasses import dataclass
from pathlib import Path

import torch
from safetensors import safe_open

from .formats import FP8_BLOCK_SIZE, FP8_DTYPE, QuantizedStore, StagedExperts
from .quantized import GPTQLinear

DESCRIPTOR = "shared-model.json"
SHARED_FORMAT = "drama3-packed-shared-v1"
GPTQ_METHOD = "drama3-int4"
GPTQ_SYMMETRIC_ZEROS = 0x88888888 - (1 << 32)  # eight 4-bit zero points of 8, as int32
GPTQ_GROUP = 128

# safetensors header dtype names -> torch dtypes (the ones these layouts use)
_DTYPES = {"F8_E4M3": FP8_DTYPE, "F32": torch.float32, "F16": torch.float16, "BF16": torch.bfloat16,
           "I32": torch.int32, "I8": torch.int8, "U8": torch.uint8}

# Which source projections make up each bank projection: w13 is the gate rows
# followed by the up rows, w2 the down projection.
_PARTS = {"w13": ("gate_proj", "up_proj"), "w2": ("down_proj",)}

# packed ComfyUI banks: bank projection -> the fused source module name
_COMFY_SOURCES = {"w13": "gate_up_proj", "w2": "down_proj"}
# mode -> (comfy_quant "format", packed columns per K, group size or None)
_COMFY_MODES = {1: ("int8_tensorwise", lambda k: k, None),
                2: ("w6a8_int8", lambda k: 3 * k // 4, 16),
                3: ("asym_w4a8_int8", lambda k: k // 2, 16)}
_SHARED_QUANTIZATION = {"int8_convrot": 1, "w6a8": 2, "w4a8": 3}

_OFFICIAL_KEY = re.compile(r"(?:model\.language_model|model)\.layers\.(\d+)\.mlp\.experts\.(\d+)\."
                           r"(gate_proj|up_proj|down_proj)\.(weight|weight_scale_inv)")


@dataclass(frozen=True)
class BankGeometry:
    """The text model's MoE sizes (config.json ``text_config``)."""

    layers: int
    experts: int
    hidden: int
    intermediate: int

    @classmethod
    def from_config(cls, config: dict) -> "BankGeometry":
        text = config.get("text_config")
        if not isinstance(text, dict):
            raise ValueError("Checkpoint config has no text_config")
        values = []
        for key in ("num_hidden_layers", "num_experts", "hidden_size", "moe_intermediate_size"):
            value = text.get(key)
            if isinstance(value, bool) or not isinstance(value, int) or value < 1:
                raise ValueError(f"text_config.{key} must be an integer >= 1")
            values.append(value)
        return cls(*values)

    def shapes(self, prefix: str) -> tuple:
        """(N, K) of bank projection ``w13`` ([2I, H]) or ``w2`` ([H, I])."""
        return (2 * self.intermediate, self.hidden) if prefix == "w13" else (self.hidden, self.intermediate)

    def part_shape(self, projection: str) -> tuple:
        """(N, K) of one source projection of one expert."""
        return ((self.hidden, self.intermediate) if projection == "down_proj"
                else (self.intermediate, self.hidden))


def _read_json(path: Path) -> dict:
    try:
        value = json.loads(path.read_text(encoding="utf-8"))
    except (UnicodeDecodeError, json.JSONDecodeError) as exc:
        raise ValueError(f"Invalid JSON file: {path}") from exc
    if not isinstance(value, dict):
        raise ValueError(f"Expected a JSON object: {path}")
    return value


def shared_descriptor(directory) -> dict | None:
    """The shared packed model's descriptor (``shared-model.json``) with its
    ``model`` path resolved, or None when the directory has none
    (shared_checkpoint.py:26-39): format ``drama3-packed-shared-v1``, a file
    whose size matches ``size``, a 64-hex-digit ``sha256``."""
    path = Path(directory).resolve() / DESCRIPTOR
    if not path.is_file():
        return None
    document = _read_json(path)
    if (document.get("format") != SHARED_FORMAT or not isinstance(document.get("model"), str)
            or isinstance(document.get("size"), bool) or not isinstance(document.get("size"), int)
            or not re.fullmatch(r"[a-f0-9]{64}", str(document.get("sha256", "")))):
        raise ValueError("Invalid shared model descriptor")
    model = (path.parent / document["model"]).resolve()
    if not model.is_file() or model.stat().st_size != document["size"]:
        raise ValueError(f"Shared model missing or size changed: {model}")
    return {**document, "model": str(model)}


def quantization_mode(directory) -> int | None:
    """Packed mode of a quantized checkpoint, as quantized_model.py:94-103
    decides it: a shared descriptor's ``quantization`` (int8_convrot 1, w6a8 2,
    w4a8 3), else 0 when config.json says ``quant_method: drama3-int4``, else
    None (not a quantized checkpoint)."""
    entry = shared_descriptor(directory)
    if entry:
        return _SHARED_QUANTIZATION.get(entry.get("quantization"))
    config = Path(directory) / "config.json"
    if config.is_file() and _read_json(config).get("quantization_config", {}).get("quant_method") == GPTQ_METHOD:
        return 0
    return None


class CheckpointTensors:
    """Name -> tensor reader over the safetensors files of a checkpoint.
    Shapes and dtypes come from the headers; ``get`` reads one payload."""

    def __init__(self, files, weight_map: dict | None = None):
        """``files``: the safetensors files.  With ``weight_map`` (tensor name
        -> file, as an index names them) only those tensors are visible, and
        each must be in the file the map names."""
        self._handles, self._where = {}, {}
        for path in files:
            self._handles[str(path)] = safe_open(str(path), framework="pt", device="cpu")
        if weight_map is None:
            for handle in self._handles.values():
                for name in handle.keys():
                    if name in self._where:
                        raise ValueError(f"Tensor {name} appears in more than one checkpoint file")
                    self._where[name] = handle
            return
        keys = {path: set(handle.keys()) for path, handle in self._handles.items()}
        for name, path in weight_map.items():
            if name not in keys[str(path)]:
                raise ValueError(f"Checkpoint index/header mismatch: {name}")
            self._where[name] = self._handles[str(path)]

    @classmethod
    def from_directory(cls, directory) -> "CheckpointTensors":
        """The shared packed file when the directory has a descriptor, else the
        shards a ``model.safetensors.index.json`` names, else every
        ``*.safetensors`` file in the directory."""
        root = Path(directory).resolve()
        entry = shared_descriptor(root)
        if entry:
            return cls([entry["model"]])
        index = root / "model.safetensors.index.json"
        if index.is_file():
            weight_map = _read_json(index).get("weight_map")
            if not isinstance(weight_map, dict) or not weight_map or not all(
                    isinstance(k, str) and isinstance(v, str) for k, v in weight_map.items()):
                raise ValueError("Checkpoint index has no weight_map of tensor names to shards")
            shards = {}
            for shard_name in sorted(set(weight_map.values())):
                shard = (root / shard_name).resolve()
                if not shard.is_relative_to(root):
                    raise ValueError(f"Checkpoint shard escapes its directory: {shard_name!r}")
                shards[shard_name] = shard
            return cls(list(shards.values()), {name: shards[v] for name, v in weight_map.items()})
        files = sorted(root.glob("*.safetensors"))
        if not files:
            raise ValueError(f"No safetensors files in {root}")
        return cls(files)

    def close(self) -> None:
        """Drop the file handles (tensors already read stay valid)."""
        self._where.clear()
        self._handles.clear()

    def __enter__(self) -> "CheckpointTensors":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def names(self):
        return self._where.keys()

    def __contains__(self, name: str) -> bool:
        return name in self._where

    def meta(self, name: str) -> tuple:
        """(shape, torch dtype or the header's dtype name) from the header."""
        if name not in self._where:
            raise KeyError(f"Checkpoint tensor missing: {name}")
        piece = self._where[name].get_slice(name)
        dtype = piece.get_dtype()
        return tuple(piece.get_shape()), _DTYPES.get(dtype, dtype)

    def get(self, name: str) -> torch.Tensor:
        if name not in self._where:
            raise KeyError(f"Checkpoint tensor missing: {name}")
        return self._where[name].get_tensor(name)

    def checked(self, name: str, shape: tuple, dtype: torch.dtype) -> torch.Tensor:
        """The tensor, after its header shape and dtype are checked."""
        have_shape, have_dtype = self.meta(name)
        if have_shape != tuple(shape) or have_dtype != dtype:
            raise ValueError(f"Wrong expert shape/dtype: {name} is {have_shape} {have_dtype}; "
                             f"expected {tuple(shape)} {dtype}")
        return self.get(name)


# ------------------------------------------------------------------ FP8 banks

def official_expert_prefix(tensors: CheckpointTensors, layer: int) -> str:
    """``model.language_model.layers.{i}.mlp.experts`` or the
    ``model.layers.{i}`` form, whichever the checkpoint uses
    (expert_cache_file.py:35-39 accepts both)."""
    for stem in ("model.language_model.layers", "model.layers"):
        prefix = f"{stem}.{layer}.mlp.experts"
        if f"{prefix}.0.gate_proj.weight" in tensors:
            return prefix
    raise ValueError(f"No official FP8 experts for layer {layer}")


def official_fp8_bank(tensors: CheckpointTensors, layer: int, geometry: BankGeometry) -> StagedExperts:
    """One layer's experts from the official per-expert FP8 tensors: w13 the
    gate rows then the up rows of each expert (weights [I, H] e4m3 and block
    scales [I/128, H/128] fp32 concatenated along the rows), w2 the down
    projection ([H, I], [H/128, I/128]); the pairing of
    expert_cache_file.py:47-54 with the header checks of :255-266."""
    prefix = official_expert_prefix(tensors, layer)
    bank = {}
    for target, parts in _PARTS.items():
        weights, scales = [], []
        for expert in range(geometry.experts):
            w_parts, s_parts = [], []
            for projection in parts:
                n, k = geometry.part_shape(projection)
                base = f"{prefix}.{expert}.{projection}"
                w_parts.append(tensors.checked(base + ".weight", (n, k), FP8_DTYPE))
                s_parts.append(tensors.checked(base + ".weight_scale_inv",
                                               (n // FP8_BLOCK_SIZE, k // FP8_BLOCK_SIZE), torch.float32))
            weights.append(torch.cat(w_parts) if len(w_parts) > 1 else w_parts[0])
            scales.append(torch.cat(s_parts) if len(s_parts) > 1 else s_parts[0])
        bank[target + "_weight"] = torch.stack(weights)
        bank[target + "_scale_inv"] = torch.stack(scales)
    return StagedExperts(**bank)


def check_official_fp8_names(tensors: CheckpointTensors, geometry: BankGeometry) -> None:
    """Every ``.mlp.experts.`` tensor is one of the six per-expert FP8 tensors
    of a layer and expert inside the config, none twice, none missing
    (expert_cache_file.py:243-275)."""
    seen = set()
    for name in tensors.names():
        if ".mlp.experts." not in name:
            continue
        match = _OFFICIAL_KEY.fullmatch(name)
        if match is None:
            raise ValueError(f"Unsupported routed expert checkpoint key: {name}")
        layer, expert = int(match.group(1)), int(match.group(2))
        if layer >= geometry.layers or expert >= geometry.experts:
            raise ValueError(f"Expert index outside model config: {name}")
        key = (layer, expert, match.group(3), match.group(4))
        if key in seen:
            raise ValueError(f"Duplicate expert projection: {name}")
        seen.add(key)
    expected = geometry.layers * geometry.experts * 6
    if len(seen) != expected:
        raise ValueError(f"Missing expert tensors: {len(seen)}/{expected}")


# bank buffer -> (packed tensor suffix, shape of (E, I, H), dtype)
_PACKED_FP8 = {
    "w13_weight": ("gate_up_weight", lambda g: (g.experts, 2 * g.intermediate, g.hidden), FP8_DTYPE),
    "w13_scale_inv": ("gate_up_scale", lambda g: (g.experts, 2 * g.intermediate // FP8_BLOCK_SIZE,
                                                  g.hidden // FP8_BLOCK_SIZE), torch.float32),
    "w2_weight": ("down_weight", lambda g: (g.experts, g.hidden, g.intermediate), FP8_DTYPE),
    "w2_scale_inv": ("down_scale", lambda g: (g.experts, g.hidden // FP8_BLOCK_SIZE,
                                              g.intermediate // FP8_BLOCK_SIZE), torch.float32),
}


def packed_fp8_bank(tensors: CheckpointTensors, layer: int, geometry: BankGeometry) -> StagedExperts:
    """One layer's experts from the shared packed FP8 file: four stacked
    tensors per layer whose shapes and dtypes shared_checkpoint.py:114-125
    fixes."""
    prefix = f"model.layers.{layer}.mlp.experts."
    return StagedExperts(**{target: tensors.checked(prefix + source, shape(geometry), dtype)
                            for target, (source, shape, dtype) in _PACKED_FP8.items()})


def check_packed_fp8_names(tensors: CheckpointTensors, geometry: BankGeometry) -> None:
    """Every layer has exactly the four packed FP8 expert tensors and no other
    ``.mlp.experts.`` tensor exists (shared_checkpoint.py:119-127)."""
    wanted = {f"model.layers.{layer}.mlp.experts.{source}" for layer in range(geometry.layers)
              for source, _, _ in _PACKED_FP8.values()}
    actual = {name for name in tensors.names() if ".mlp.experts." in name}
    if actual != wanted:
        raise ValueError("Unexpected or missing packed FP8 expert tensors: "
                         f"{sorted(actual ^ wanted)[:4]}")


# -------------------------------------------------------------- GPTQ banks

def _check_gptq_groups(tensors: CheckpointTensors, base: str, k: int) -> None:
    name = base + ".g_idx"
    if name in tensors:
        groups = tensors.get(name)
        if not torch.equal(groups, torch.arange(k, dtype=groups.dtype) // GPTQ_GROUP):
            raise ValueError(f"Unsupported permuted GPTQ groups (act-order): {base}")


def gptq_expert_bank(tensors: CheckpointTensors, layer: int, geometry: BankGeometry) -> QuantizedStore:
    """One layer's INT4 GPTQ experts (mode 0): each expert's ``qweight``
    [K/8, N] int32 and ``scales`` [K/128, N] fp16 transposed to rows, the gate
    rows then the up rows for w13 (quantized_model.py:156-168).  ``qzeros``
    [K/128, N/8], when the checkpoint holds them for the experts, are kept
    unless every word is the symmetric 0x88888888 (a zero point of 8, which
    the kernels assume by default); ``g_idx`` must be the identity grouping."""
    prefix = f"model.language_model.layers.{layer}.mlp.experts"
    bank, zeros, asymmetric = {}, {}, False
    for target, parts in _PARTS.items():
        weights, scales, zero_rows = [], [], []
        for expert in range(geometry.experts):
            w_parts, s_parts, z_parts = [], [], []
            for projection in parts:
                n, k = geometry.part_shape(projection)
                if k % GPTQ_GROUP or n % 8:
                    raise ValueError("GPTQ banks need K a multiple of 128 and N a multiple of 8")
                base = f"{prefix}.{expert}.{projection}"
                w_parts.append(tensors.checked(base + ".qweight", (k // 8, n), torch.int32).T)
                s_parts.append(tensors.checked(base + ".scales", (k // GPTQ_GROUP, n), torch.float16).T)
                if base + ".qzeros" in tensors:
                    z = tensors.checked(base + ".qzeros", (k // GPTQ_GROUP, n // 8), torch.int32)
                    asymmetric |= not bool((z == GPTQ_SYMMETRIC_ZEROS).all())
                    z_parts.append(z)
                else:
                    z_parts.append(torch.full((k // GPTQ_GROUP, n // 8), GPTQ_SYMMETRIC_ZEROS, dtype=torch.int32))
                _check_gptq_groups(tensors, base, k)
            weights.append(torch.cat(w_parts))
            scales.append(torch.cat(s_parts))
            zero_rows.append(torch.cat(z_parts, dim=1))  # zero words run along N
        bank[target + "_weight"] = torch.stack(weights).contiguous()
        bank[target + "_scale_inv"] = torch.stack(scales).contiguous()
        zeros[target + "_zeros"] = torch.stack(zero_rows).contiguous()
    if not asymmetric:
        zeros = {}
    return QuantizedStore(**bank, **zeros, hidden=geometry.hidden, intermediate=geometry.intermediate, mode=0)


def gptq_dense_linear(tensors: CheckpointTensors, base: str, *, device, dtype=torch.bfloat16) -> GPTQLinear:
    """A dense INT4 projection (``{base}.qweight`` / ``.scales``) as a
    ``GPTQLinear`` on ``device``; its ``qzeros`` must all be the symmetric
    0x88888888 and its ``g_idx`` the identity grouping, the conditions
    quantized_model.py:192-196 enforces."""
    k8, n = tensors.meta(base + ".qweight")[0]
    linear = GPTQLinear(tensors.checked(base + ".qweight", (k8, n), torch.int32),
                        tensors.checked(base + ".scales", (k8 * 8 // GPTQ_GROUP, n), torch.float16),
                        device=device, dtype=dtype)
    zeros = tensors.get(base + ".qzeros")
    groups = tensors.get(base + ".g_idx")
    if not bool((zeros == GPTQ_SYMMETRIC_ZEROS).all()) or not torch.equal(
            groups, torch.arange(linear.in_features, dtype=torch.int32) // GPTQ_GROUP):
        raise ValueError(f"Unsupported asymmetric or permuted GPTQ dense weight: {base}")
    return linear


def gptq_dense_names(tensors: CheckpointTensors) -> list:
    """Bases of every dense GPTQ projection (a ``.qweight`` outside the
    routed experts), as quantized_model.py:186-189 selects them."""
    return sorted(name[:-len(".qweight")] for name in tensors.names()
                  if name.endswith(".qweight") and ".mlp.experts." not in name)


# --------------------------------------------------- ComfyUI packed banks

def comfy_expert_bank(tensors: CheckpointTensors, layer: int, geometry: BankGeometry, mode: int) -> QuantizedStore:
    """One layer's ComfyUI-style packed experts (quantized_model.py:114-153).
    Per projection: ``weight`` [E, N, packed K] int8 and a ``comfy_quant``
    JSON blob (ConvRot group 256, the config's expert count, the mode's
    format; group 16 for W6A8 / W4A8).  Mode 1 takes ``weight_scale`` [E, N]
    fp32 as the channel scale; modes 2 and 3 put ``weight_s_rel`` (E4M3
    group-16 scale bytes, [E, N, K/16]) before the 4 bytes of
    ``weight_s_channel`` (fp32 [E, N]) in each row, and mode 3 adds one float
    of the 16-level fp32 ``weight_codebook`` to the 4 trailing bytes of each
    of an expert's first 16 rows."""
    if mode not in _COMFY_MODES:
        raise ValueError(f"Not a packed ComfyUI mode: {mode}")
    fmt, columns, group = _COMFY_MODES[mode]
    experts = geometry.experts
    bank = {}
    for target, source in _COMFY_SOURCES.items():
        n, k = geometry.shapes(target)
        base = f"model.layers.{layer}.mlp.experts.{source}"
        blob = tensors.get(base + ".comfy_quant")
        try:
            config = json.loads(bytes(blob.to(torch.uint8).tolist()).decode("utf-8"))
        except (UnicodeDecodeError, json.JSONDecodeError) as exc:
            raise ValueError(f"Invalid comfy_quant JSON: {base}") from exc
        if not isinstance(config, dict) or config.get("convrot_groupsize") != 256 \
                or config.get("num_experts") != experts:
            raise ValueError("Unsupported ConvRot group size or expert count")
        if config.get("format") != fmt or (mode == 1 and not config.get("convrot")) \
                or (group is not None and config.get("group_size") != group):
            raise ValueError(f"Expected a {fmt} expert bank: {base}")
        bank[target + "_weight"] = tensors.checked(base + ".weight", (experts, n, columns(k)), torch.int8)
        if mode == 1:
            scale = tensors.checked(base + ".weight_scale", (experts, n), torch.float32)
            bank[target + "_scale_inv"] = scale.reshape(experts, n, 1)
            continue
        relative = tensors.get(base + ".weight_s_rel")
        if relative.numel() != experts * n * (k // 16) or relative.element_size() != 1:
            raise ValueError(f"weight_s_rel must hold one byte per 16 columns: {base}")
        relative = relative.view(torch.uint8).reshape(experts, n, k // 16)
        channel = tensors.checked(base + ".weight_s_channel", (experts, n), torch.float32)
        channel = channel.contiguous().view(torch.uint8).reshape(experts, n, 4)
        aux = torch.zeros((experts, n, k // 16 + (8 if mode == 3 else 4)), dtype=torch.uint8)
        aux[..., :k // 16] = relative
        aux[..., k // 16:k // 16 + 4] = channel
        if mode == 3:
            codebook = tensors.checked(base + ".weight_codebook", (16,), torch.float32)
            aux[:, :16, k // 16 + 4:] = codebook.contiguous().view(torch.uint8).reshape(16, 4)
        bank[target + "_scale_inv"] = aux
    return QuantizedStore(**bank, hidden=geometry.hidden, intermediate=geometry.intermediate, mode=mode)


# --------------------------------------------------------------- loading

def expert_format(directory) -> int | str:
    """How a checkpoint stores its routed experts: a packed mode 0-3, or
    ``"fp8-shared"`` (shared packed FP8 file) / ``"fp8"`` (official
    per-expert FP8 tensors)."""
    root = Path(directory).resolve()
    mode = quantization_mode(root)
    if mode is not None:
        return mode
    entry = shared_descriptor(root)
    if entry is not None:
        if entry.get("quantization") not in (None, "fp8"):
            raise ValueError(f"Unsupported shared model quantization: {entry.get('quantization')}")
        return "fp8-shared"
    return "fp8"


def _to_device(bank, device):
    if isinstance(bank, StagedExperts):
        staged = StagedExperts(*(getattr(bank, n).to(device) for n in ("w13_weight", "w13_scale_inv", "w2_weight",
                                                                       "w2_scale_inv")))
        staged.validate()
        return staged
    moved = QuantizedStore(bank.w13_weight.to(device), bank.w13_scale_inv.to(device), bank.w2_weight.to(device),
                           bank.w2_scale_inv.to(device), bank.hidden, bank.intermediate, bank.mode,
                           None if bank.w13_zeros is None else bank.w13_zeros.to(device),
                           None if bank.w2_zeros is None else bank.w2_zeros.to(device))
    moved.validate()
    return moved


def load_expert_bank(tensors: CheckpointTensors, layer: int, geometry: BankGeometry, fmt, *,
                     device="cpu") -> StagedExperts | QuantizedStore:
    """One layer's bank in format ``fmt`` (see ``expert_format``), validated
    and moved to ``device``."""
    if not 0 <= layer < geometry.layers:
        raise ValueError(f"Layer {layer} outside the model's {geometry.layers} layers")
    if fmt == "fp8":
        bank = official_fp8_bank(tensors, layer, geometry)
    elif fmt == "fp8-shared":
        bank = packed_fp8_bank(tensors, layer, geometry)
    elif fmt == 0:
        bank = gptq_expert_bank(tensors, layer, geometry)
    else:
        bank = comfy_expert_bank(tensors, layer, geometry, fmt)
    return _to_device(bank, device)


def bind_expert_bank(module, bank) -> None:
    """Make ``module`` (a routed-expert module) hold ``bank`` the way the
    reference's loaders bind one (quantized_model.py:106-111,
    shared_checkpoint.py:128-130): the four bank tensors as its
    w13_weight / w13_scale_inv / w2_weight / w2_scale_inv buffers, plus the
    packed store itself for the packed modes, so install_expert_offload
    finds it."""
    bank.validate()
    for name in ("w13_weight", "w13_scale_inv", "w2_weight", "w2_scale_inv"):
        module._buffers[name] = getattr(bank, name)
    if isinstance(bank, QuantizedStore):
        module._drama_quant_store = bank
    else:
        module.fp8 = True
        module.__dict__.pop("_drama_quant_store", None)


def load_expert_banks(directory, *, device, layers=None) -> list:
    """Every layer's routed-expert bank of the checkpoint in ``directory``
    (or the layers listed), resident on ``device``."""
    root = Path(directory).resolve()
    geometry = BankGeometry.from_config(_read_json(root / "config.json"))
    fmt = expert_format(root)
    with CheckpointTensors.from_directory(root) as tensors:
        if fmt == "fp8-shared":
            check_packed_fp8_names(tensors, geometry)
        elif fmt == "fp8":
            check_official_fp8_names(tensors, geometry)
        chosen = range(geometry.layers) if layers is None else layers
        return [load_expert_bank(tensors, layer, geometry, fmt, device=device) for layer in chosen]
