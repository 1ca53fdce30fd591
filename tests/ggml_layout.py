"""Superblock packers in the byte layout ggml writes (block_q4_K / block_q6_K
of ggml-common.h; quantize_row_q4_K_ref / quantize_row_q6_K_ref of
ggml-quants.c, ggml GIT_TAG master as fetched by the reference's
CMakeLists.txt:30-37). They state the layout from the writer's side, the
inverse of the dequantizers under test, so a wrong nibble, plane or scale
index in a dequantizer shows up as a mismatch against the values packed here.
"""
from __future__ import annotations

import numpy as np


def f16_bits(value: float) -> int:
    return int(np.array([value], dtype=np.float16).view(np.uint16)[0])


def pack_q4k(d_bits: int, dmin_bits: int, sc, mn, L) -> bytes:
    """block_q4_K {half d; half dmin; u8 scales[12]; u8 qs[128]}.
    sc, mn: 8 six-bit values; L: 256 four-bit codes."""
    sc = [int(v) for v in sc]
    mn = [int(v) for v in mn]
    L = [int(v) for v in L]
    assert len(sc) == 8 and len(mn) == 8 and len(L) == 256
    assert all(0 <= v < 64 for v in sc + mn) and all(0 <= v < 16 for v in L)
    scales = [0] * 12
    for j in range(8):
        ls, lm = sc[j], mn[j]
        if j < 4:
            scales[j] = ls
            scales[j + 4] = lm
        else:
            scales[j + 4] = (ls & 0xF) | ((lm & 0xF) << 4)
            scales[j - 4] |= (ls >> 4) << 6
            scales[j] |= (lm >> 4) << 6
    qs = []
    for j in range(0, 256, 64):
        for l in range(32):
            qs.append(L[j + l] | (L[j + l + 32] << 4))
    out = bytes([d_bits & 0xFF, d_bits >> 8, dmin_bits & 0xFF, dmin_bits >> 8])
    return out + bytes(scales) + bytes(qs)


def pack_q6k(L, scales, d_bits: int) -> bytes:
    """block_q6_K {u8 ql[128]; u8 qh[64]; i8 scales[16]; half d}.
    L: 256 six-bit codes (weight = d*scale*(L-32)); scales: 16 int8."""
    L = [int(v) for v in L]
    assert len(L) == 256 and all(0 <= v < 64 for v in L)
    ql = [0] * 128
    qh = [0] * 64
    for half, j in enumerate(range(0, 256, 128)):
        for l in range(32):
            q1, q2, q3, q4 = L[j + l], L[j + l + 32], L[j + l + 64], L[j + l + 96]
            ql[64 * half + l] = (q1 & 0xF) | ((q3 & 0xF) << 4)
            ql[64 * half + l + 32] = (q2 & 0xF) | ((q4 & 0xF) << 4)
            qh[32 * half + l] = (q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6)
    sc = bytes(np.asarray(scales, dtype=np.int8).view(np.uint8).tolist())
    assert len(sc) == 16
    return bytes(ql) + bytes(qh) + sc + bytes([d_bits & 0xFF, d_bits >> 8])
