"""dmoe_fp8_moe_layer_noalloc -- the decode layer that allocates nothing and
keeps its scratch in the library's fixed per-GPU array -- against
dmoe_fp8_moe_layer with a caller workspace, both called through the C ABI on
the same inputs.  Routing ids, routing weights and outputs must be
bit-identical, on two calls in a row with the second one smaller, through the
single-launch decode and through the three-launch decode."""
import ctypes

import pytest
import torch

from conftest import print_case
from drama_moe import _lib
from drama_moe.formats import fp8_bank_struct, random_fp8_bank

pytestmark = pytest.mark.gpu

TOP_K = 8


def layer_call(entry, bank, x, logits, workspace=None):
    tokens = x.shape[0]
    ids = torch.full((tokens, TOP_K), -7, dtype=torch.int64, device=x.device)
    weights = torch.full((tokens, TOP_K), float("nan"), dtype=torch.bfloat16, device=x.device)
    out = torch.full_like(x, float("nan"))
    status = torch.zeros(1, dtype=torch.int32, device=x.device)
    args = [ctypes.byref(bank), _lib.ptr(x), _lib.BF16, x.stride(0), tokens, _lib.ptr(logits), logits.stride(0),
            TOP_K, 1, _lib.ptr(ids), _lib.ptr(weights), _lib.BF16, 128, _lib.BF16, _lib.ptr(out), _lib.BF16,
            out.stride(0)]
    if workspace is not None:
        args += [_lib.ptr(workspace), workspace.numel()]
    args += [_lib.ptr(status), _lib.stream_handle(x.device)]
    _lib.check(entry(*args))
    torch.cuda.synchronize()
    return out, ids, weights, int(status.item())


@pytest.fixture(scope="module")
def bank(cuda):
    g = torch.Generator(device=cuda).manual_seed(20261207)
    staged = random_fp8_bank(64, 2048, 768, layout="channel", generator=g, device=cuda)
    return staged, fp8_bank_struct(staged)


@pytest.mark.parametrize("fused,token_counts", [(True, (4, 1)), (False, (16, 2))])
def test_noalloc_layer_equals_workspace_layer(cuda, bank, fused, token_counts):
    staged, desc = bank
    lib = _lib.library()
    previous = lib.dmoe_set_fused_decode(2 if fused else 0)
    try:
        g = torch.Generator(device=cuda).manual_seed(7 + token_counts[0])
        for tokens in token_counts:
            print_case("noalloc layer", "fused" if fused else "three-launch", f"tokens={tokens}")
            x = torch.randn(tokens, 2048, device=cuda, generator=g).bfloat16()
            logits = torch.randn(tokens, 64, device=cuda, generator=g)
            ws = torch.zeros(lib.dmoe_fp8_workspace_bytes(ctypes.byref(desc), tokens * TOP_K), dtype=torch.uint8,
                             device=cuda)
            want = layer_call(lib.dmoe_fp8_moe_layer, desc, x, logits, ws)
            got = layer_call(lib.dmoe_fp8_moe_layer_noalloc, desc, x, logits)
            again = layer_call(lib.dmoe_fp8_moe_layer_noalloc, desc, x, logits)
            assert want[3] == 0 and got[3] == 0 and again[3] == 0
            for a, b, c in zip(want[:3], got[:3], again[:3]):
                assert torch.equal(a, b)
                assert torch.equal(b, c)
            assert torch.isfinite(got[0].float()).all()
    finally:
        lib.dmoe_set_fused_decode(previous)


def test_noalloc_layer_rejects_calls_beyond_its_scratch(cuda, bank):
    staged, desc = bank
    lib = _lib.library()
    x = torch.zeros(40, 2048, device=cuda, dtype=torch.bfloat16)
    logits = torch.zeros(40, 64, device=cuda)
    with pytest.raises(ValueError, match="at most 256 route pairs"):
        layer_call(lib.dmoe_fp8_moe_layer_noalloc, desc, x, logits)


def _capture_on_first_call() -> None:
    """Body of the capture test, run in a fresh process: the entry point's
    FIRST call of the process (which looks up the scratch address) happens
    inside a hipGraph capture; replays, with eager work between them, must
    equal the allocating entry point on new inputs each time."""
    cuda = torch.device("cuda", 0)
    lib = _lib.library()
    g = torch.Generator(device=cuda).manual_seed(20261208)
    staged = random_fp8_bank(64, 2048, 768, layout="channel", generator=g, device=cuda)
    desc = fp8_bank_struct(staged)
    for tokens in (2, 16):  # single-launch decode, then the three launches
        print_case("noalloc capture", f"tokens={tokens}")
        x = torch.randn(tokens, 2048, device=cuda, generator=g).bfloat16()
        logits = torch.randn(tokens, 64, device=cuda, generator=g)
        ids = torch.empty((tokens, TOP_K), dtype=torch.int64, device=cuda)
        weights = torch.empty((tokens, TOP_K), dtype=torch.bfloat16, device=cuda)
        out = torch.empty_like(x)
        status = torch.zeros(1, dtype=torch.int32, device=cuda)
        ws = torch.zeros(lib.dmoe_fp8_workspace_bytes(ctypes.byref(desc), tokens * TOP_K), dtype=torch.uint8,
                         device=cuda)
        stream = torch.cuda.Stream(cuda)
        stream.wait_stream(torch.cuda.current_stream(cuda))
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            _lib.check(lib.dmoe_fp8_moe_layer_noalloc(
                ctypes.byref(desc), _lib.ptr(x), _lib.BF16, x.stride(0), tokens, _lib.ptr(logits), logits.stride(0),
                TOP_K, 1, _lib.ptr(ids), _lib.ptr(weights), _lib.BF16, 128, _lib.BF16, _lib.ptr(out), _lib.BF16,
                out.stride(0), _lib.ptr(status), _lib.stream_handle(cuda)))
        for replay in range(3):
            x.copy_(torch.randn(tokens, 2048, device=cuda, generator=g).bfloat16())
            logits.copy_(torch.randn(tokens, 64, device=cuda, generator=g))
            want = layer_call(lib.dmoe_fp8_moe_layer, desc, x, logits, ws)
            out.fill_(float("nan"))
            ids.fill_(-7)
            graph.replay()
            torch.cuda.synchronize()
            assert want[3] == 0 and int(status.item()) == 0, replay
            assert torch.equal(out, want[0]) and torch.equal(ids, want[1]) and torch.equal(weights, want[2]), replay
    print("capture on first call: ok", flush=True)


def test_noalloc_layer_captured_on_its_first_call(cuda):
    """The no-allocation entry point captured in a hipGraph on its first call
    in the process (fresh subprocess), replayed three times against the
    allocating entry point."""
    import os
    import subprocess
    import sys
    from pathlib import Path

    here = Path(__file__).resolve().parent
    env = dict(os.environ)
    env["PYTHONPATH"] = os.pathsep.join([str(here), str(here.parent), str(here.parent / "drama3-studio_amd"),
                                         env.get("PYTHONPATH", "")])
    proc = subprocess.run([sys.executable, "-u", "-c", "import test_zz_no_alloc as t; t._capture_on_first_call()"],
                          cwd=here, env=env, capture_output=True, text=True, timeout=110)
    print(proc.stdout[-4000:], proc.stderr[-4000:])
    assert proc.returncode == 0, proc.stderr[-2000:]
    assert "capture on first call: ok" in proc.stdout
