"""Write the committed golden vectors of the FP8 path from the reference's own
CPU executor (native/src/*.cpp, compiled into oracle/_ref by
``make -C oracle ref`` in a checkout that has the reference sources).

Fixtures (numpy .npz, no pickles):
  fp8_quant.npz  drama_quantize_bf16 bytes/scales of the four activation cases
                 of tests/test_native_backend.py:41-55 (seed 22, [16, 128])
  fp8_pairs.npz  drama_executor_forward partials (scalar implementation) of
                 the stores of tests/test_native_backend.py:24-31 (seed 194)
                 and :234-254 (seed 882), with their inputs

Run:  python tests/golden/make_golden.py
"""
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import oracle as orc  # noqa: E402
from oracle import ref_native  # noqa: E402

HERE = Path(__file__).resolve().parent


def quant_cases():
    out = {}
    lib = ref_native.RefLibrary()
    for kind in ("random", "zero", "tiny", "saturated"):
        x = torch.randn(16, 128, generator=torch.Generator().manual_seed(22))
        if kind == "zero":
            x.zero_()
            x[0, :4] = torch.tensor([0.0, -0.0, 0.0, -0.0])
        elif kind == "tiny":
            x *= 1e-20
        elif kind == "saturated":
            x *= 1e20
        bits = x.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16).reshape(-1)
        q, s = lib.quantize_bf16(bits)
        out[f"{kind}_q"] = q
        out[f"{kind}_s"] = s
    np.savez_compressed(HERE / "fp8_quant.npz", **out)


def pair_cases():
    out = {}
    lib = ref_native.RefLibrary()
    for case, seed, experts, inter2, hidden, random_scales, ids, weights in (
        ("s194", 194, 4, 256, 128, False, [3, 1, 3, 0], [0.4, 0.2, 0.3, 0.1]),
        ("s882", 882, 3, 512, 256, True, [2, 0, 1, 2], [0.4, 0.3, 0.2, 0.1]),
    ):
        g = torch.Generator().manual_seed(seed)
        w13 = torch.randint(-3, 4, (experts, inter2, hidden), generator=g).to(torch.float8_e4m3fn)
        s13 = (torch.rand(experts, inter2 // 128, hidden // 128, generator=g) * 0.02 + 0.01
               if random_scales else torch.full((experts, inter2 // 128, hidden // 128), 0.03125))
        w2 = torch.randint(-3, 4, (experts, hidden, inter2 // 2), generator=g).to(torch.float8_e4m3fn)
        s2 = (torch.rand(experts, hidden // 128, inter2 // 256, generator=g) * 0.02 + 0.01
              if random_scales else torch.full((experts, hidden // 128, inter2 // 256), 0.03125))
        x = torch.randn(hidden, generator=g).bfloat16().view(torch.int16).numpy().view(np.uint16)
        ids = np.array(ids, np.int64)
        weights = np.float32(weights)
        with ref_native.RefExecutor(lib, hidden, inter2 // 2, capacity=8, threads=1,
                                    implementation="scalar") as ex:
            partials = ex.forward(w13.view(torch.uint8).numpy(), s13.numpy(), w2.view(torch.uint8).numpy(),
                                  s2.numpy(), x, ids, weights)
        out.update({f"{case}_w13": w13.view(torch.uint8).numpy(), f"{case}_s13": s13.numpy(),
                    f"{case}_w2": w2.view(torch.uint8).numpy(), f"{case}_s2": s2.numpy(),
                    f"{case}_x": x, f"{case}_ids": ids, f"{case}_weights": weights,
                    f"{case}_out": partials})
    np.savez_compressed(HERE / "fp8_pairs.npz", **out)


if __name__ == "__main__":
    orc.build(reference=True)
    quant_cases()
    pair_cases()
    print("wrote", sorted(p.name for p in HERE.glob("*.npz")))
