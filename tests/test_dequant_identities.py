"""Arithmetic identities the packed-bank kernels rely on, checked exhaustively
on the CPU.

W6A8 dequantization (quant_moe.hip, decode_wrow for mode 2) turns a 6-bit code
c and the E4M3 scale byte of its 16-code group into the INT8 weight
q8(c - 32, rel) = clamp(rint((c - 32) * rel), -127, 127) (the reference's
level * relative-scale rounding, quantized_kernels.py:148-173) in packed fp16
arithmetic: x = fp16(1024 + c), v = (x - 1056) * rel, clamped to [-127, 127],
then + 1536, whose low byte is the INT8 value.  numpy's float16 operations
round exactly as the hardware's (the exact results fit float32 before the one
rounding to float16), so every (code, scale byte) pair is checked here.
"""
import numpy as np
import torch


def q8(level: np.float32, rel: np.float32) -> int:
    v = np.float32(level * rel)
    if np.isnan(v):
        return -127  # fmaxf(NaN, -127) = -127
    return int(min(max(np.rint(v), np.float32(-127)), np.float32(127)))


def packed_fp16(code: int, rel: np.float32) -> int:
    x = np.float16(1024 + code)
    v = np.float16(np.float16(x - np.float16(1056)) * np.float16(rel))
    v = np.float16(-127) if np.isnan(v) else max(v, np.float16(-127))  # maxNum
    v = min(v, np.float16(127))
    m = np.float16(v + np.float16(1536))
    return int(np.int8(np.uint8(int(m.view(np.uint16)) & 0xFF)))


def test_w6_packed_fp16_dequant_equals_q8_for_every_code_and_scale_byte():
    rels = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    for byte in range(256):
        rel = np.float32(rels[byte])
        if not np.isnan(rel):
            assert np.float32(np.float16(rel)) == rel  # E4M3 values are exact in fp16
        for code in range(64):
            assert packed_fp16(code, rel) == q8(np.float32(code - 32), rel), (byte, code)


def test_packed_fp16_check_catches_a_wrong_offset():
    # the same sequence with 1055 in place of 1056 (level off by one) must fail
    rel = np.float32(torch.tensor([0x38], dtype=torch.uint8).view(torch.float8_e4m3fn).float().item())
    x = np.float16(1024 + 40)
    wrong = np.float16(np.float16(x - np.float16(1055)) * np.float16(rel))
    assert int(np.rint(wrong)) != q8(np.float32(40 - 32), rel)
