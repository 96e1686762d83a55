#!/usr/bin/env python3
"""Writes the known-answer fixtures of tests/golden/ from closed forms, without the oracle or the library.

ggml itself is not available (the reference's ggml submodule is empty), so these vectors are built from the block
layouts of ggml-common.h and from inputs for which every quantizer's result is fixed by arithmetic alone:

  q8_0_exact.json   blocks whose largest |x| is 127 * 2^k: d = 2^k exactly and every quant is x / 2^k.
  q8_ties.json      d = 1 blocks holding x.5 values: roundf (quantize_row_q8_0_ref) goes away from zero, the x86
                    AVX2 path (_MM_ROUND_NEAREST) to even.
  q8_K_ties.json    256-blocks whose largest |x| occurs twice with opposite signs: the first one sets the scale.
  q4_K_grid.json    a super-block whose every 32-value sub-block lies on an exact grid d*sc_j*l - dmin*m_j with
                    l in 0..15 all present and max sc = max m = 63: any least-squares fit lands on the grid, so the
                    block is d = 2^-10, dmin = 2^-11, the given 6-bit scales/mins and codes l.
  q5_K_grid.json    the Q4_K construction with 5-bit codes: every 32-value sub-block holds each l in 0..31 once, on
                    d*sc_j*l - dmin*m_j; codes split into nibbles (qs) and bit 4 (bit j of qh[l]).
  q6_K_grid.json    a super-block whose 16-value sub-blocks lie on D*k_j*q with q in -32..31, q = -32 present and
                    max k = 128: the block is d = -D, scales = -k_j, codes q + 32.

Each fixture stores the input floats and the expected ggml block bytes (hex), and where it applies the exact
dequantized values. Run from the repository root: python tests/golden/make_golden.py
"""
import json
import pathlib

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent


def f16_bits(v: float) -> int:
    return int(np.array([v], dtype=np.float32).astype(np.float16).view(np.uint16)[0])


def hexs(b: bytes) -> str:
    return bytes(b).hex()


def q8_0_exact():
    rng = np.random.default_rng(20241)
    cases = []
    for k in (-14, -6, -1, 0, 3):
        q = rng.integers(-127, 128, size=32)
        q[rng.integers(0, 32)] = 127 if rng.random() < 0.5 else -127
        x = (q * 2.0 ** k).astype(np.float32)
        blk = f16_bits(2.0 ** k).to_bytes(2, "little") + q.astype(np.int8).tobytes()
        cases.append({"x": x.tolist(), "block": hexs(blk), "dequant": x.tolist()})
    return cases


def q8_ties():
    x = np.zeros(32, np.float32)
    x[0] = 127.0
    x[1], x[2], x[3], x[4], x[5], x[6] = 2.5, -2.5, 0.5, -0.5, 3.5, 126.5
    d = f16_bits(1.0).to_bytes(2, "little")
    away = np.sign(x) * np.floor(np.abs(x) + 0.5)   # half away from zero
    even = np.round(x)                               # numpy rounds half to even
    return {"x": x.tolist(), "ref_block": hexs(d + away.astype(np.int8).tobytes()),
            "x86_block": hexs(d + even.astype(np.int8).tobytes())}


def q8_K_ties():
    x = np.zeros(256, np.float32)
    x[5], x[9], x[100], x[200] = -3.0, 3.0, 1.0, -1.5
    # max = -3 (first of the two |x| = 3), iscale = -127/max = 127/3, d = 1/iscale
    iscale = np.float32(-127.0) / np.float32(-3.0)
    q = np.clip(np.rint((iscale * x).astype(np.float32)), -128, 127).astype(np.int8)
    bsums = q.astype(np.int32).reshape(16, 16).sum(axis=1).astype(np.int16)
    d = np.float32(1.0) / iscale
    blk = np.array([d], np.float32).tobytes() + q.tobytes() + bsums.tobytes()
    return {"x": x.tolist(), "block": hexs(blk)}


def pack_q4_K_scales(sc, m):
    """12 bytes from eight 6-bit scales and mins (the inverse of get_scale_min_k4)."""
    s = [0] * 12
    for j in range(4):
        s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = (m[j] & 63) | ((m[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 0xF) | ((m[j + 4] & 0xF) << 4)
    return bytes(s)


def q4_K_grid():
    d, dmin = 2.0 ** -10, 2.0 ** -11
    sc = [63, 40, 17, 5, 63, 22, 31, 50]
    m = [10, 63, 0, 7, 33, 63, 1, 20]
    rng = np.random.default_rng(4096)
    L = np.zeros(256, np.int64)
    x = np.zeros(256, np.float64)
    for j in range(8):
        l = np.concatenate([np.arange(16), rng.integers(0, 16, size=16)])
        rng.shuffle(l)
        L[32 * j:32 * j + 32] = l
        x[32 * j:32 * j + 32] = d * sc[j] * l - dmin * m[j]
    x32 = x.astype(np.float32)
    assert np.array_equal(x32.astype(np.float64), x)  # the grid is exact in fp32
    # qs: byte 32c + i holds element 64c + i (low nibble) and 64c + 32 + i (high nibble)
    qs = bytearray(128)
    for c in range(4):
        for i in range(32):
            qs[32 * c + i] = int(L[64 * c + i]) | (int(L[64 * c + 32 + i]) << 4)
    blk = (f16_bits(d).to_bytes(2, "little") + f16_bits(dmin).to_bytes(2, "little") + pack_q4_K_scales(sc, m) +
           bytes(qs))
    return {"x": x32.tolist(), "block": hexs(blk), "dequant": x32.tolist(), "sc": sc, "m": m}


def q5_K_grid():
    d, dmin = 2.0 ** -10, 2.0 ** -11
    sc = [17, 63, 40, 2, 33, 63, 9, 58]
    m = [63, 0, 12, 45, 63, 3, 28, 51]
    rng = np.random.default_rng(5005)
    L = np.zeros(256, np.int64)
    x = np.zeros(256, np.float64)
    for j in range(8):
        l = rng.permutation(32)   # every level once: the fit has no freedom left
        L[32 * j:32 * j + 32] = l
        x[32 * j:32 * j + 32] = d * sc[j] * l - dmin * m[j]
    x32 = x.astype(np.float32)
    assert np.array_equal(x32.astype(np.float64), x)
    # qs: byte 32c + i holds the low 4 bits of elements 64c + i (low nibble) and 64c + 32 + i (high nibble);
    # qh[i] bit j holds bit 4 of element 32j + i
    qs = bytearray(128)
    qh = bytearray(32)
    for c in range(4):
        for i in range(32):
            qs[32 * c + i] = (int(L[64 * c + i]) & 0xF) | ((int(L[64 * c + 32 + i]) & 0xF) << 4)
    for j in range(8):
        for i in range(32):
            qh[i] |= ((int(L[32 * j + i]) >> 4) & 1) << j
    blk = (f16_bits(d).to_bytes(2, "little") + f16_bits(dmin).to_bytes(2, "little") + pack_q4_K_scales(sc, m) +
           bytes(qh) + bytes(qs))
    return {"x": x32.tolist(), "block": hexs(blk), "dequant": x32.tolist(), "sc": sc, "m": m}


def q6_K_grid():
    D = 2.0 ** -12
    k = [128, 100, 64, 37, 1, 90, 128, 12, 77, 50, 3, 127, 64, 99, 20, 45]
    rng = np.random.default_rng(6006)
    Q = np.zeros(256, np.int64)
    x = np.zeros(256, np.float64)
    for j in range(16):
        q = rng.integers(-31, 32, size=16)
        q[rng.integers(0, 16)] = -32   # the sub-block's largest |x| is its -32 code
        Q[16 * j:16 * j + 16] = q
        x[16 * j:16 * j + 16] = D * k[j] * q
    x32 = x.astype(np.float32)
    assert np.array_equal(x32.astype(np.float64), x)
    L = Q + 32  # codes 0..63
    ql = bytearray(128)
    qh = bytearray(64)
    for h in range(2):       # two halves of 128 elements
        for l in range(32):
            e = 128 * h + l
            ql[64 * h + l] = (int(L[e]) & 0xF) | ((int(L[e + 64]) & 0xF) << 4)
            ql[64 * h + 32 + l] = (int(L[e + 32]) & 0xF) | ((int(L[e + 96]) & 0xF) << 4)
            qh[32 * h + l] = ((int(L[e]) >> 4) | ((int(L[e + 32]) >> 4) << 2) | ((int(L[e + 64]) >> 4) << 4) |
                              ((int(L[e + 96]) >> 4) << 6))
    scales = np.array([-v for v in k], np.int64).clip(-128, 127).astype(np.int8).tobytes()
    blk = bytes(ql) + bytes(qh) + scales + f16_bits(-D).to_bytes(2, "little")
    return {"x": x32.tolist(), "block": hexs(blk), "dequant": x32.tolist(), "k": k}


def main():
    fixtures = {
        "q8_0_exact.json": q8_0_exact(),
        "q8_ties.json": q8_ties(),
        "q8_K_ties.json": q8_K_ties(),
        "q4_K_grid.json": q4_K_grid(),
        "q5_K_grid.json": q5_K_grid(),
        "q6_K_grid.json": q6_K_grid(),
    }
    for name, data in fixtures.items():
        (HERE / name).write_text(json.dumps(data, indent=1) + "\n")
        print("wrote", HERE / name)


if __name__ == "__main__":
    main()
