"""Independent block encoders for known-answer tests.

Each encoder writes chosen integer fields into one GGUF block following the
published layouts (the reference decoders' field order, restated in
src/quantized_linear.cpp:53-164, 166-205, 286-358, 387-423) and returns the block with
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


def q5_0_block(d, q):
    """q: 32 ints in [-16, 15]; u = q + 16: low 4 bits of element i < 16 in the
    low nibble of byte 6 + i, of element 16 + i in its high nibble; bit 4 of
    element i in bit i of the 32-bit qh at byte 2."""
    b = bytearray(22)
    b[0:2] = _f16(d)
    qh = 0
    for i in range(32):
        u = int(q[i]) + 16
        qh |= (u >> 4) << i
        b[6 + (i % 16)] |= (u & 15) << (4 * (i // 16))
    b[2:6] = qh.to_bytes(4, "little")
    return bytes(b), np.array([d * v for v in q])


def q5_1_block(d, m, q):
    """q: 32 ints in [0, 31]; element i = d*q[i] + m; qh at byte 4, nibbles
    from byte 8."""
    b = bytearray(24)
    b[0:2] = _f16(d)
    b[2:4] = _f16(m)
    qh = 0
    for i in range(32):
        u = int(q[i])
        qh |= (u >> 4) << i
        b[8 + (i % 16)] |= (u & 15) << (4 * (i // 16))
    b[4:8] = qh.to_bytes(4, "little")
    return bytes(b), np.array([d * v + m for v in q])


def q2_k_block(d, dmin, scales, mins, q):
    """q: 256 ints in [0, 3]; scales/mins: 16 ints in [0, 15] per 16-element
    group g (byte g: scale low nibble, min high nibble).  Element e of half h
    = e // 128, shift pair s = (e % 128) // 32, sub-run t = (e % 32) // 16,
    lane i = e % 16 sits in bits 2s of quant byte 16 + 32h + 16t + i; its
    group is g = 8h + 2s + t; value d*scales[g]*q - dmin*mins[g]."""
    b = bytearray(84)
    for g in range(16):
        b[g] = (int(scales[g]) & 15) | ((int(mins[g]) & 15) << 4)
    exp = np.zeros(256)
    for e in range(256):
        h, r = divmod(e, 128)
        s2, r2 = divmod(r, 32)
        t, i = divmod(r2, 16)
        g = 8 * h + 2 * s2 + t
        b[16 + 32 * h + 16 * t + i] |= (int(q[e]) & 3) << (2 * s2)
        exp[e] = d * scales[g] * q[e] - dmin * mins[g]
    b[80:82] = _f16(d)
    b[82:84] = _f16(dmin)
    return bytes(b), exp


def q3_k_block(d, scales, q):
    """q: 256 ints in [-4, 3]; scales: 16 ints in [-32, 31] (stored as 6-bit
    scale + 32).  Element e: half h, shift pair s, sub-run t, lane i as
    q2_k_block; low 2 bits of q + 4 at bits 2s of byte 32 + 32h + 16t + i, the
    high bit (set when q >= 0) at bit 4h + s of hmask byte 16t + i; group g =
    8h + 2s + t.  The 6-bit scales: low nibble of scale j < 8 in byte 96 + j,
    of scale 8 + j in its high nibble; the top 2 bits of scale j at bits
    2 * (j // 4) of byte 104 + j % 4."""
    b = bytearray(110)
    exp = np.zeros(256)
    for e in range(256):
        h, r = divmod(e, 128)
        s2, r2 = divmod(r, 32)
        t, i = divmod(r2, 16)
        g = 8 * h + 2 * s2 + t
        u = int(q[e]) + 4
        b[32 + 32 * h + 16 * t + i] |= (u & 3) << (2 * s2)
        b[16 * t + i] |= (u >> 2) << (4 * h + s2)
        exp[e] = d * scales[g] * q[e]
    for j in range(16):
        v = int(scales[j]) + 32
        b[96 + (j % 8)] |= (v & 15) << (4 * (j // 8))
        b[104 + (j % 4)] |= (v >> 4) << (2 * (j // 4))
    b[108:110] = _f16(d)
    return bytes(b), exp
