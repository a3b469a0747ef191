"""MXFP4 codec and the low-precision expert tile layouts (test oracle only).

No reference counterpart exists: the reference plans FP8 / MXFP4 expert
GEMMs for a tensor-core fused MoE (docs/next-optimizations.md:160-184) and
names MXFP4 as "the native Blackwell 4-bit float".  MXFP4 is the OCP
Microscaling format (OCP Microscaling Formats (MX) Specification v1.0,
section 6.3, "conversion from a vector of scalars"), restated here for
blocks of 32 consecutive elements along a row:

  * shared scale X = 2^(floor(log2(max|V_i|)) - emax), emax = 2 for E2M1
    (largest normal 6 = 1.5 * 2^2), stored as E8M0 = exponent + 127,
    clamped to [-127, 127]; an all-zero block takes X = 1 (E8M0 127);
  * P_i = V_i / X rounded to E2M1 (magnitudes 0, 0.5, 1, 1.5, 2, 3, 4, 6)
    to nearest, ties to the even code, saturating at 6; the sign bit is
    the sign of V_i (negative values that round to zero keep it: code 8);
  * value = E2M1(P_i) * X.
X is a power of two, so V_i / X is exact except where it underflows, which
cannot move a value across a rounding threshold (all are >= 0.25).

Pins (tests/test_oracle_mx.py): a brute-force nearest-code search with
explicit tie handling, exact round trips of blocks that are E2M1 codes times
a power of two with a full-scale element, closed-form exponents, and
brute-force loops over the two tile layouts.
"""
from __future__ import annotations

import numpy as np

F32 = np.float32
E2M1_MAG = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], dtype=F32)
# upper bounds of each code's rounding interval (ties at a bound go to the
# even code: 0.25 -> 0, 0.75 -> 1.0, 1.25 -> 1.0, 1.75 -> 2, 2.5 -> 2,
# 3.5 -> 4, 5 -> 4)
_BOUNDS = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0], dtype=F32)
_TIE_TO_LOWER = np.array([True, False, True, False, True, False, True])
MX_BLOCK = 32


def e2m1_encode(p) -> np.ndarray:
    """fp32 (already divided by the block scale) -> E2M1 code 0..15."""
    p = np.asarray(p, dtype=F32)
    a = np.abs(p)
    code = np.zeros(a.shape, dtype=np.int64)
    for i, (b, lower) in enumerate(zip(_BOUNDS, _TIE_TO_LOWER)):
        code += (a > b) if lower else (a >= b)
    sign = np.signbit(p).astype(np.int64) << 3
    return (code | sign).astype(np.uint8)


def e2m1_decode(c) -> np.ndarray:
    c = np.asarray(c, dtype=np.uint8)
    v = E2M1_MAG[c & 7]
    return np.where(c & 8, -v, v).astype(F32)


def e8m0_exponent(amax) -> np.ndarray:
    """floor(log2(amax)) - 2 clamped to [-127, 127] (0 for amax == 0), from
    the fp32 exponent field (subnormal amax clamps to -127)."""
    amax = np.asarray(amax, dtype=F32)
    biased = (amax.view(np.uint32) >> 23).astype(np.int64) & 0xFF
    e = np.clip(biased - 127 - 2, -127, 127)
    return np.where(amax == 0, 0, e).astype(np.int64)


def pow2(e) -> np.ndarray:
    """2^e as fp32 for integer e in [-127, 127] (2^-127 is subnormal)."""
    e = np.asarray(e, dtype=np.int64)
    return np.ldexp(F32(1.0), e).astype(F32)


def quantize_mxfp4(w):
    """w (R, C) fp32, C % 32 == 0 -> (codes (R, C/2) u8, element 2i in the low
    nibble of byte i; e8 (R, C/32) u8 E8M0 scales)."""
    w = np.asarray(w, dtype=F32)
    R, C = w.shape
    assert C % MX_BLOCK == 0
    blk = w.reshape(R, C // MX_BLOCK, MX_BLOCK)
    amax = np.abs(blk).max(axis=2)
    e = e8m0_exponent(amax)
    p = blk / pow2(e)[:, :, None]
    codes = e2m1_encode(p).reshape(R, C)
    packed = (codes[:, 0::2] | (codes[:, 1::2] << 4)).astype(np.uint8)
    return np.ascontiguousarray(packed), (e + 127).astype(np.uint8)


def dequantize_mxfp4(packed, e8):
    packed = np.asarray(packed, dtype=np.uint8)
    R, half = packed.shape
    codes = np.empty((R, half * 2), dtype=np.uint8)
    codes[:, 0::2] = packed & 0xF
    codes[:, 1::2] = packed >> 4
    v = e2m1_decode(codes).reshape(R, -1, MX_BLOCK)
    s = pow2(np.asarray(e8, dtype=np.int64) - 127)
    return (v * s[:, :, None]).reshape(R, half * 2).astype(F32)


# ------------------------------------------------ fused-MoE tile layouts
# Both follow the INT4 tile layout's geometry (rows/16 row tiles x in/128
# k-blocks, lane l = c + 16 q of a 64-lane wave holding row 16 t + c); they
# differ in which k a lane holds.


def moe_tile_pack_fp8(q):
    """Row-major e4m3 codes (rows, in) -> (rows/16, in/128, 2048) u8: half
    h of block (t, kb) at 1024 h holds at 16 (c + 16 q) the 16 codes of row
    16 t + c, k = 128 kb + 32 q + 16 h + 0..15 in order (lane (c, q)'s MFMA
    step j takes codes 8 j .. 8 j + 7 of its 32, halves 0 then 1).  The
    128x128 block scales of quantize_fp8_block are used as they are."""
    q = np.asarray(q, dtype=np.uint8)
    rows, cols = q.shape
    x = q.reshape(rows // 16, 16, cols // 128, 4, 2, 16)      # t, c, kb, q, h, byte
    return np.ascontiguousarray(x.transpose(0, 2, 4, 3, 1, 5).reshape(rows // 16, cols // 128, 2048))


def moe_tile_pack_mxfp4(packed, e8):
    """Row-major MXFP4 (codes (rows, in/2), e8 (rows, in/32)) ->
    qtile (rows/16, in/128, 1024) u8 and e8w (rows/16, in/128, 16) u32.
    Lane (c, q)'s 16 bytes at 16 (c + 16 q): word j (MFMA step j) holds the
    8 codes of row 16 t + c at k = 128 kb + 32 j + 8 q + 0..7, two per byte,
    the lower k in the low nibble -- so step j covers exactly MX block
    4 kb + j.  e8w[t, kb, c] holds the E8M0 scales of row 16 t + c, blocks
    4 kb + j, in byte j."""
    packed = np.asarray(packed, dtype=np.uint8)
    rows, half = packed.shape
    cols = half * 2
    # bytes of row r for k = 128 kb + 32 j + 8 q + 2 b (+1): packed[r, 64 kb + 16 j + 4 q + b]
    x = packed.reshape(rows // 16, 16, cols // 128, 4, 4, 4)  # t, c, kb, j, q, b
    qt = x.transpose(0, 2, 4, 1, 3, 5).reshape(rows // 16, cols // 128, 1024)  # t, kb, q, c, j, b
    e = np.asarray(e8, dtype=np.uint32).reshape(rows // 16, 16, cols // 128, 4)  # t, c, kb, j
    w = e[..., 0] | (e[..., 1] << 8) | (e[..., 2] << 16) | (e[..., 3] << 24)
    return np.ascontiguousarray(qt), np.ascontiguousarray(w.transpose(0, 2, 1)).astype(np.uint32)
