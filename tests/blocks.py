"""Independent block encoders for known-answer tests.

Each encoder writes chosen integer fields into one GGUF block following the
published layouts (the reference decoders' field order, restated in
src/quantized_linear.cpp:53-62, 166-205, 286-358, 387-423) and returns the block with
the value every element must decode to, computed in float64 from the fields.
They share no code with the decoders under test.
"""
from __future__ import annotations

import numpy as np


def _f16(v: float) -> bytes:
    return np.array([v], dtype=np.float16).view(np.uint8).tobytes()


def pack_scale_min(block: bytearray, g: int, s: int, m: int) -> None:
    """6-bit scale/min of sub-block g into the 12-byte field at block[4:16]
    (the packing of tests/regression_test.cpp:75-84 in the reference)."""
    if g < 4:
        block[4 + g] |= s
        block[8 + g] |= m
    else:
        block[g] |= (s >> 4) << 6
        block[4 + g] |= (m >> 4) << 6
        block[8 + g] |= (s & 15) | ((m & 15) << 4)


def q4_k_block(d, dmin, scales, mins, q):
    """q: 256 ints in [0, 15]; element e = d*scales[e//32]*q[e] - dmin*mins[e//32]."""
    b = bytearray(144)
    b[0:2] = _f16(d)
    b[2:4] = _f16(dmin)
    for g in range(8):
        pack_scale_min(b, g, int(scales[g]), int(mins[g]))
    for e in range(256):
        g, lane = e // 32, e % 32
        b[16 + (g // 2) * 32 + lane] |= (int(q[e]) & 15) << (4 * (g % 2))
    exp = np.array([d * scales[e // 32] * q[e] - dmin * mins[e // 32] for e in range(256)])
    return bytes(b), exp


def q5_k_block(d, dmin, scales, mins, q):
    """q: 256 ints in [0, 31]."""
    b = bytearray(176)
    b[0:2] = _f16(d)
    b[2:4] = _f16(dmin)
    for g in range(8):
        pack_scale_min(b, g, int(scales[g]), int(mins[g]))
    for e in range(256):
        g, lane = e // 32, e % 32
        b[16 + lane] |= ((int(q[e]) >> 4) & 1) << g
        b[48 + (g // 2) * 32 + lane] |= (int(q[e]) & 15) << (4 * (g % 2))
    exp = np.array([d * scales[e // 32] * q[e] - dmin * mins[e // 32] for e in range(256)])
    return bytes(b), exp


def q6_k_block(d, scales, q):
    """q: 256 ints in [-32, 31]; scales: 16 int8; element e = d*scales[e//16]*q[e]."""
    b = bytearray(210)
    for e in range(256):
        h, r = divmod(e, 128)
        quarter, lane = divmod(r, 32)
        u = int(q[e]) + 32
        lo, hi = u & 15, u >> 4
        ql_index = 64 * h + (32 if quarter in (1, 3) else 0) + lane
        b[ql_index] |= lo << (4 if quarter >= 2 else 0)
        b[128 + 32 * h + lane] |= hi << (2 * quarter)
    for i in range(16):
        b[192 + i] = int(scales[i]) & 0xFF
    b[208:210] = _f16(d)
    exp = np.array([d * scales[e // 16] * q[e] for e in range(256)])
    return bytes(b), exp


def q8_0_block(d, q):
    """q: 32 ints in [-128, 127]."""
    b = bytearray(34)
    b[0:2] = _f16(d)
    b[2:34] = np.asarray(q, dtype=np.int8).view(np.uint8).tobytes()
    return bytes(b), np.array([d * v for v in q])


def q4_0_block(d, q):
    """q: 32 ints in [-8, 7]; element i < 16 in the low nibble of byte i,
    element 16 + i in its high nibble."""
    b = bytearray(18)
    b[0:2] = _f16(d)
    for i in range(16):
        b[2 + i] = ((int(q[i]) + 8) & 15) | (((int(q[16 + i]) + 8) & 15) << 4)
    return bytes(b), np.array([d * v for v in q])


def q4_1_block(d, m, q):
    """q: 32 ints in [0, 15]; element i = d*q[i] + m, element i < 16 in the
    low nibble of byte i, element 16 + i in its high nibble."""
    b = bytearray(20)
    b[0:2] = _f16(d)
    b[2:4] = _f16(m)
    for i in range(16):
        b[4 + i] = (int(q[i]) & 15) | ((int(q[16 + i]) & 15) << 4)
    return bytes(b), np.array([d * v + m for v in q])
