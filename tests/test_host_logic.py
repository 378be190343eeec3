"""Host-side logic of the expert runtime on the CPU: bank geometry checks of
every format, and the expert manager's caller contract (validation before any
expert runs, attach / detach, install keywords).  No kernel is launched: the
HIP backend is only reached by calls that pass every check, and those are
the GPU tests' business."""
import pytest
import torch
from torch import nn

from drama_moe.formats import (BANK_FORMATS, QuantizedStore, StagedExperts, random_fp8_bank,
                               random_quantized_bank)
from drama_moe.offload import (STAGING_KEYWORDS, HipExpertBackend, ResidentExpertManager,
                               install_expert_offload)


def fp8_module(bank: StagedExperts) -> nn.Module:
    module = nn.Module()
    module.fp8 = True
    for name, tensor in bank.buffers().items():
        module.register_buffer(name, tensor)
    return module


@pytest.fixture(scope="module")
def bank():
    return random_fp8_bank(4, 128, 128, generator=torch.Generator().manual_seed(5))


def test_fp8_bank_accepts_block_and_channel_scales(bank):
    bank.validate()
    channel = random_fp8_bank(2, 256, 128, layout="channel", generator=torch.Generator().manual_seed(1))
    channel.validate()
    assert channel.w13_scale_inv.shape == (2, 256, 1)


@pytest.mark.parametrize("name,make,message", [
    ("w13_weight", lambda b: b.w13_weight.float(), "w13_weight must be"),
    ("w2_weight", lambda b: b.w2_weight[:, :, :64], "w2_weight has shape"),
    ("w13_scale_inv", lambda b: b.w13_scale_inv.double(), "w13_scale_inv must be"),
    ("w2_scale_inv", lambda b: b.w2_scale_inv[:, :, :0], "w2_scale_inv has shape"),
    ("w13_weight", lambda b: b.w13_weight[:, :192], "multiples of the FP8 block"),
    ("w13_weight", lambda b: b.w13_weight[0], "stacked"),
])
def test_fp8_bank_rejects_bad_geometry(bank, name, make, message):
    parts = bank.buffers()
    parts[name] = make(bank)
    with pytest.raises(ValueError, match=message):
        StagedExperts(**parts).validate()


@pytest.mark.parametrize("mode", [0, 1, 2, 3])
def test_packed_banks_of_every_mode_validate(mode):
    store = random_quantized_bank(mode, 2, 256, 256, asymmetric=mode == 0,
                                  generator=torch.Generator().manual_seed(mode))
    store.validate()
    spec = BANK_FORMATS[mode]
    assert store.w13_weight.dtype == spec.weight_dtype
    assert store.w2_weight.shape[-1] == spec.weight_columns(store.intermediate)


def test_packed_bank_errors():
    store = random_quantized_bank(2, 2, 256, 256, generator=torch.Generator().manual_seed(9))
    parts = dict(store.buffers(), hidden=256, intermediate=256)
    with pytest.raises(ValueError, match="Unknown quantized bank format"):
        QuantizedStore(**parts, mode=7).validate()
    bad = dict(parts, w2_weight=store.w2_weight[:, :, :10])
    with pytest.raises(ValueError, match="w2_weight has shape"):
        QuantizedStore(**bad, mode=2).validate()
    zeros = torch.zeros(2, 2, 64, dtype=torch.int32)
    with pytest.raises(ValueError, match="W4A16 banks only"):
        QuantizedStore(**parts, mode=2, w13_zeros=zeros).validate()
    w4 = random_quantized_bank(0, 2, 256, 256, generator=torch.Generator().manual_seed(3))
    w4parts = dict(w4.buffers(), hidden=256, intermediate=256, mode=0)
    with pytest.raises(ValueError, match="w13_zeros must be GPTQ qzeros"):
        QuantizedStore(**w4parts, w13_zeros=torch.zeros(2, 2, 8, dtype=torch.int32)).validate()


def test_manager_validates_calls_before_any_expert_runs(bank):
    module = fp8_module(bank)
    manager = ResidentExpertManager(backend=HipExpertBackend())
    manager.attach("layers.0.experts", module)
    x = torch.randn(2, 128).bfloat16()
    ids = torch.tensor([[0, 1], [2, 3]])
    w = torch.full((2, 2), 0.5)
    cases = [
        ((torch.randn(2, 64), ids, w), "hidden rows"),
        ((x, ids[:1], w[:1]), "Expert IDs must be \\[tokens, top_k\\]"),
        ((x, ids, w[:, :1]), "shape of the expert IDs"),
        ((x, ids.float(), w), "int32 or int64"),
        ((x, ids, w.long()), "floating point"),
        ((x.to(torch.float64), ids, w), "compute dtype"),
        ((x, torch.tensor([[0, 1], [2, 9]]), w), "Expert IDs must be in \\[0, 4\\)"),
        ((x, torch.tensor([[0, -1], [2, 3]]), w), "Expert IDs must be in"),
    ]
    for args, message in cases:
        with pytest.raises(ValueError, match=message):
            module(*args)
    assert manager.forward_calls == 2  # the id-range failures passed the contract checks
    assert torch.equal(module(x[:0], ids[:0], w[:0]), torch.zeros(0, 128, dtype=torch.bfloat16))


def test_attach_detach_restores_the_module_forward(bank):
    module = fp8_module(bank)
    own = module.forward
    manager = ResidentExpertManager(backend=HipExpertBackend())
    manager.attach("experts", module)
    assert module.forward != own
    with pytest.raises(ValueError, match="already has an offload manager"):
        manager.attach("experts", module)
    with pytest.raises(ValueError, match="already has an offload manager"):
        ResidentExpertManager(backend=HipExpertBackend()).attach("again", module)
    manager.close()
    assert module.forward == own
    assert "forward" not in module.__dict__
    with pytest.raises(RuntimeError, match="closed"):
        manager.attach("experts", module)

    custom = fp8_module(bank)
    custom.forward = lambda *a: "own"
    manager = ResidentExpertManager(backend=HipExpertBackend())
    manager.attach("experts", custom)
    manager.close()
    assert custom.forward() == "own"


def test_manager_picks_the_bank_of_a_packed_module():
    store = random_quantized_bank(3, 2, 256, 256, generator=torch.Generator().manual_seed(2))
    module = nn.Module()
    for name, tensor in store.buffers().items():
        module.register_buffer(name, tensor)
    module._drama_quant_store = store
    manager = ResidentExpertManager(backend=HipExpertBackend())
    manager.attach("experts", module)
    bank = manager._bank_of(module)
    assert bank is store
    assert type(manager._backend_for(bank)).__name__ == "QuantizedExpertBackend"
    with pytest.raises(ValueError, match="Expert IDs must be in \\[0, 2\\)"):
        module(torch.randn(1, 256).bfloat16(), torch.tensor([[5]]), torch.ones(1, 1))


def test_install_checks_every_bank_and_keyword(bank):
    backbone = nn.Module()
    backbone.add_module("a", fp8_module(bank))
    backbone.add_module("b", fp8_module(bank))
    with pytest.raises(TypeError, match="unexpected keywords"):
        install_expert_offload(backbone, staging_arena=True)
    with pytest.raises(ValueError, match="provides 'hip'"):
        install_expert_offload(backbone, backend="torch")
    broken = nn.Module()
    broken.add_module("a", fp8_module(bank))
    bad = fp8_module(bank)
    bad.w2_weight = bad.w2_weight[:, :64]
    broken.add_module("b", bad)
    with pytest.raises(ValueError):
        install_expert_offload(broken)
    assert "forward" not in broken.a.__dict__  # nothing attached when any bank is bad
    flags = {"max_staged_experts": 8, "max_pair_rows": 64, "cache_experts": 4, "hot_cache_experts": None,
             "pin_memory": True, "profile_transfers": False, "combined_decode_bank": True, "packed_staging": False}
    assert set(flags) == STAGING_KEYWORDS
    with pytest.raises(ValueError, match="positive"):
        install_expert_offload(backbone, **{**flags, "max_pair_rows": 0})
    with pytest.raises(TypeError, match="boolean"):
        install_expert_offload(backbone, **{**flags, "packed_staging": 1})
    manager = install_expert_offload(backbone, backend="triton", **flags)
    assert manager.residency == "hbm" and manager.host is None
    assert sorted(manager.modules) == ["a", "b"]
    with pytest.raises(ValueError, match="already has an expert offload manager"):
        install_expert_offload(backbone)
    manager.close()
    with pytest.raises(ValueError, match="no routed expert modules"):
        install_expert_offload(nn.Linear(2, 2))
