"""numpy restatement of the reference packers/unpackers (test oracle only).

Pins (tests/test_oracle_quant.py):
  * e4m3 encode/decode: the reference's exact known values
    (tests/test_quantizer.py:10-16), torch.float8_e4m3fn's round-to-nearest-even
    cast outside the documented subnormal band, the band itself
    (quantizer.py:48-49 clips to code 7), and an exhaustive 256-code decode
    against the closed form sign * 2^(e-7) * (1 + m/8).
  * int4 quantizers: error <= step/2 (tests/test_quantizer.py:48-56), brute
    force per-element loops on tiny shapes, and the documented disagreement
    counts between the three RTN variants.
  * GPTQ packing and the Marlin permutation: brute-force bit loops.
  * 128x128 FP8 blocks: per-block loops on tiny shapes, padding invariance.

All arithmetic is float32 with one rounding per numpy operation, exactly as the
reference's vectorised numpy code does it.
"""
from __future__ import annotations

import numpy as np

F32 = np.float32
E4M3_MAX = F32(448.0)


# ------------------------------------------------------------------ E4M3 codec
def e4m3_encode(x) -> np.ndarray:
    """fp32 -> e4m3fn byte (fastllm_py/quantizer.py:26-51).

    Normals round to nearest even at fp32 mantissa bit 20 and are clipped to
    code 0x7E; |x| < 2^-6 encodes rint(|x|*512) clipped to 7; sign from bit 31."""
    xc = np.clip(np.asarray(x, dtype=F32), -E4M3_MAX, E4M3_MAX).astype(F32)
    bits = xc.view(np.uint32).astype(np.int64)
    sign = (bits >> 24) & 0x80
    mag = bits & 0x7FFFFFFF
    ax = np.abs(xc)
    rounded = mag + 0x7FFFF + ((mag >> 20) & 1)
    expo = ((rounded >> 23) & 0xFF) - 120
    mant = (rounded >> 20) & 0x7
    normal_code = np.clip((expo << 3) | mant, 0, 0x7E)
    sub_code = np.clip(np.rint(ax * F32(512.0)).astype(np.int64), 0, 7)
    code = np.where(ax >= F32(2.0 ** -6), normal_code, sub_code)
    return (code | sign).astype(np.uint8)


def e4m3_decode(b) -> np.ndarray:
    """e4m3fn byte -> fp32, exact (fastllm_py/quantizer.py:54-62); 0x7F -> 480."""
    b = np.asarray(b).astype(np.int64)
    e = (b >> 3) & 0xF
    m = (b & 0x7).astype(np.float64)
    mag = np.where(e > 0, np.ldexp(1.0 + m / 8.0, (e - 7).astype(np.int32)), m * 2.0 ** -9)
    return np.where(b & 0x80, -mag, mag).astype(F32)


def e4m3_encode_rne_sat(x) -> np.ndarray:
    """fp32 -> e4m3fn byte, IEEE round-to-nearest-even everywhere, saturating
    to +-448 (the satfinite E4M3 conversion of
    native/fastllm_fp8_block128.cu:93-94).  NaN -> 0x7F."""
    x = np.asarray(x, dtype=F32)
    bits = x.view(np.uint32).astype(np.int64)
    sign = (bits >> 24) & 0x80
    mag = bits & 0x7FFFFFFF
    ax = np.abs(x)
    rounded = mag + 0x7FFFF + ((mag >> 20) & 1)
    normal_code = ((((rounded >> 23) & 0xFF) - 120) << 3) | ((rounded >> 20) & 0x7)
    sub_code = np.rint(np.where(ax < F32(2.0 ** -6), ax, F32(0)) * F32(512.0)).astype(np.int64)
    code = np.where(ax >= F32(2.0 ** -6), normal_code, sub_code)
    code = np.where(ax >= E4M3_MAX, 0x7E, code)
    code = np.where(np.isnan(x), 0x7F, code)
    return (code | sign).astype(np.uint8)


# ------------------------------------------------------------ FP8 block 128x128
def quantize_fp8_block(w, bs: int = 128):
    """(q uint8 (R, C), scales fp32 (ceil(R/bs), ceil(C/bs)))
    (fastllm_py/quantizer.py:65-85): per block scale = amax/448 (1 if amax==0),
    q = encode(w / scale) with true fp32 division."""
    w = np.asarray(w, dtype=F32)
    R, C = w.shape
    Rp, Cp = -(-R // bs) * bs, -(-C // bs) * bs
    wp = np.zeros((Rp, Cp), dtype=F32)
    wp[:R, :C] = w
    blk = wp.reshape(Rp // bs, bs, Cp // bs, bs)
    amax = np.abs(blk).max(axis=(1, 3))
    scales = np.where(amax == 0, F32(1.0), amax / E4M3_MAX).astype(F32)
    q = e4m3_encode(blk / scales[:, None, :, None]).reshape(Rp, Cp)[:R, :C]
    return np.ascontiguousarray(q), scales


def dequantize_fp8_block(q, scales, bs: int = 128):
    """decode(q) * scale (fastllm_py/quantizer.py:88-94)."""
    q = np.asarray(q)
    R, C = q.shape
    s = np.repeat(np.repeat(scales, bs, axis=0), bs, axis=1)[:R, :C]
    return e4m3_decode(q) * s


# ------------------------------------------------- FP8 1x128 inline-scale rows
def fp8_inline_row_bytes(k: int) -> int:
    """k + 4*k/128 (native/fastllm_fp8_block128.cu:262-264)."""
    return k + (k // 128) * 4


def quantize_fp8_inline(w):
    """[rows, cols] fp16/bf16 (given as fp32 values) -> uint8 [rows, perRow]:
    per (row, 128-col block) scale = amax/448 (1 if not > 0), stored as fp32
    after the 128 codes; codes = rne_sat(x * (1/scale))
    (native/fastllm_fp8_block128.cu:52-97)."""
    w = np.asarray(w, dtype=F32)
    rows, cols = w.shape
    nb = cols // 128
    blk = w.reshape(rows, nb, 128)
    amax = np.abs(blk).max(axis=2)
    scale = (amax / E4M3_MAX).astype(F32)
    scale = np.where(scale > 0, scale, F32(1.0)).astype(F32)
    inv = (F32(1.0) / scale).astype(F32)
    codes = e4m3_encode_rne_sat(blk * inv[:, :, None])
    out = np.zeros((rows, nb, 132), dtype=np.uint8)
    out[:, :, :128] = codes
    out[:, :, 128:] = scale.reshape(rows, nb, 1).view(np.uint8).reshape(rows, nb, 4)
    return out.reshape(rows, nb * 132)


def dequantize_fp8_inline(packed, cols: int):
    """Inverse view of quantize_fp8_inline: fp32 [rows, cols] = decode * scale."""
    packed = np.asarray(packed, dtype=np.uint8)
    rows = packed.shape[0]
    nb = cols // 128
    blk = packed.reshape(rows, nb, 132)
    codes = blk[:, :, :128]
    scale = np.ascontiguousarray(blk[:, :, 128:]).view(np.float32).reshape(rows, nb)
    return (e4m3_decode(codes) * scale[:, :, None]).reshape(rows, cols)


# ------------------------------------------------ INT4 group format (u8 pairs)
def _groups(w, gs):
    w = np.asarray(w).astype(F32)
    rows, cols = w.shape
    assert cols % gs == 0
    g = w.reshape(rows, cols // gs, gs)
    lo, hi = g.min(axis=2), g.max(axis=2)
    s = ((hi - lo) / F32(15.0)).astype(F32)
    s = np.where(s == 0, F32(1.0), s).astype(F32)
    return g, lo, hi, s


def _pack_pairs(q):
    return (q[..., 0::2] | (q[..., 1::2] << 4)).astype(np.uint8)


def _unpack_pairs(p):
    p = np.asarray(p)
    q = np.empty(p.shape[:-1] + (p.shape[-1] * 2,), dtype=F32)
    q[..., 0::2] = p & 0xF
    q[..., 1::2] = p >> 4
    return q


def quantize_int4_group(w, gs: int = 128):
    """(packed (R, C/2) u8, scales (R, C/gs) f32, zeros = group min f32)
    (fastllm_py/quantizer.py:97-117): q = clip(rint((g - min)/s), 0, 15)."""
    g, lo, _, s = _groups(w, gs)
    q = np.clip(np.rint((g - lo[..., None]) / s[..., None]), 0, 15).astype(np.uint8)
    return _pack_pairs(q.reshape(g.shape[0], -1)), s, lo.astype(F32)


def dequantize_int4_group(packed, scales, zeros, gs: int = 128):
    """q*s + min, two roundings (fastllm_py/quantizer.py:120-129)."""
    q = _unpack_pairs(packed)
    s = np.repeat(np.asarray(scales, F32), gs, axis=1)
    z = np.repeat(np.asarray(zeros, F32), gs, axis=1)
    return (q * s + z).astype(F32)


# -------------------------------------------------- INT4 Marlin-style format
def quantize_int4_marlin(w, gs: int = 128):
    """(q (N, K) u8, scale (N, G) f32, zero (N, G) int64)
    (fastllm_py/moe.py:40-46): zero = clip(rint(-min/s)), q = clip(rint(w/s) + zero)."""
    g, lo, _, s = _groups(w, gs)
    z = np.clip(np.rint(-lo / s), 0, 15).astype(np.int64)
    q = np.clip(np.rint(g / s[..., None]) + z[..., None], 0, 15).astype(np.uint8)
    return q.reshape(g.shape[0], -1), s, z


def pack_gptq(q):
    """q (N, K) 0..15 -> u32 (K/8, N), value k at bits 4*(k%8) of word
    [k/8, n] (fastllm_py/kernels/marlin.py:113-127)."""
    q = np.asarray(q).astype(np.uint32)
    N, K = q.shape
    words = np.zeros((N, K // 8), dtype=np.uint64)
    for i in range(8):
        words += q[:, i::8].astype(np.uint64) << np.uint64(4 * i)
    return np.ascontiguousarray((words & 0xFFFFFFFF).astype(np.uint32).T)


def marlin_scale_perm_index(n_local: np.ndarray) -> np.ndarray:
    """Stored position of column n within its 64-chunk: 8*(n%8) + n//8
    (the inverse of _SCALE_PERM, fastllm_py/kernels/marlin.py:41-50)."""
    return 8 * (n_local % 8) + n_local // 8


def marlin_scales_zeros(scale, zero):
    """(scales fp16 (G, N), zeros u32 (G, N/8)) in the Marlin layout
    (fastllm_py/kernels/marlin.py:130-159)."""
    scale = np.asarray(scale).astype(F32)
    zero = np.asarray(zero).astype(np.int64)
    N, G = scale.shape
    assert N % 64 == 0
    n = np.arange(N)
    pos = (n // 64) * 64 + marlin_scale_perm_index(n % 64)
    s_out = np.empty((G, N), dtype=F32)
    s_out[:, pos] = scale.T
    z_perm = np.empty((G, N), dtype=np.int64)
    z_perm[:, pos] = zero.T
    interleave = np.array([0, 2, 4, 6, 1, 3, 5, 7])
    z8 = z_perm.reshape(G, N // 8, 8)[:, :, interleave].astype(np.uint32).astype(np.uint64)
    words = np.zeros((G, N // 8), dtype=np.uint64)
    for slot in range(8):
        words += z8[:, :, slot] << np.uint64(4 * slot)
    return s_out.astype(np.float16), (words & 0xFFFFFFFF).astype(np.uint32)


def marlin_dequant(q, scales_fp16_perm, zeros_perm, gs: int):
    """fp32 W_hat (N, K) = s[g, n] * (q[n, k] - z[g, n]) read back through the
    Marlin permutation — what the INT4 GEMM multiplies by."""
    q = np.asarray(q).astype(F32)
    N, K = q.shape
    G = K // gs
    n = np.arange(N)
    pos = (n // 64) * 64 + marlin_scale_perm_index(n % 64)
    s = np.asarray(scales_fp16_perm).astype(F32)[:, pos]  # (G, N)
    word = (n // 64) * 8 + (n % 8)
    inv_interleave = np.array([0, 4, 1, 5, 2, 6, 3, 7])
    slot = inv_interleave[(n % 64) // 8]
    z = ((np.asarray(zeros_perm)[:, word] >> (4 * slot).astype(np.uint32)) & 0xF).astype(F32)
    deq = (q.reshape(N, G, gs) - z.T[:, :, None]) * s.T[:, :, None]
    return deq.reshape(N, K).astype(F32)


# ----------------------------------------------------- INT4 row-major format
def quantize_int4_rowmajor(w, gs: int = 128):
    """(packed (.., out, in/2) u8, scales f16, zeros f16)
    (fastllm_py/kernels/moe_int4.py:24-40, batched :97-113):
    zero = clip(rint(-min/s)), q = clip(rint(w/s + zero))."""
    w = np.asarray(w)
    lead = w.shape[:-1]
    w2 = w.reshape(-1, w.shape[-1])
    g, lo, _, s = _groups(w2, gs)
    z = np.clip(np.rint(-lo / s), 0, 15).astype(F32)
    q = np.clip(np.rint((g / s[..., None]) + z[..., None]), 0, 15).astype(np.uint8)
    packed = _pack_pairs(q.reshape(g.shape[0], -1))
    return (packed.reshape(*lead, -1), s.astype(np.float16).reshape(*lead, -1),
            z.astype(np.float16).reshape(*lead, -1))


def dequantize_int4_rowmajor(packed, scales, zeros, gs: int = 128):
    """(q - zero) * scale (fastllm_py/kernels/moe_int4.py:43-54)."""
    q = _unpack_pairs(packed)
    s = np.repeat(np.asarray(scales).astype(F32), gs, axis=-1)
    z = np.repeat(np.asarray(zeros).astype(F32), gs, axis=-1)
    return ((q - z) * s).astype(F32)


# ------------------------------------------------------------------ matmuls
def nibble_interleave_u32(words):
    """u32 holding k-offsets r = 0..7 at bits 4r -> the same nibbles with
    r in slot {0,4,1,5,2,6,3,7}[r] (bits 4 slot)."""
    w = np.asarray(words, np.uint32)
    out = np.zeros_like(w)
    for r in range(8):
        slot = (r >> 1) + (4 if r & 1 else 0)
        out |= ((w >> np.uint32(4 * r)) & np.uint32(0xF)) << np.uint32(4 * slot)
    return out


def moe_tile_pack(packed, scales, zeros):
    """Row-major INT4 (rows, in/2) u8 + (rows, G) fp16 scales/zeros -> the
    fused MoE tile layout of this library (no reference counterpart: the
    reference's kernels read the row-major arrays): qtile (rows/16, in/128,
    1024) u8 whose bytes [16 (c + 16 q), + 16) hold the row-major bytes
    [64 kb + 16 q, + 16) of row 16 t + c as four little-endian u32, each with
    its 8 nibbles interleaved by nibble_interleave_u32; sz (rows/16, G, 16)
    u32 = scale bits | zero bits << 16 of row 16 t + c."""
    rows, half = packed.shape
    q = np.asarray(packed, np.uint8).reshape(rows // 16, 16, half // 64, 4, 16)
    qt = q.transpose(0, 2, 3, 1, 4).reshape(rows // 16, half // 64, 1024)
    qt = nibble_interleave_u32(np.ascontiguousarray(qt).view("<u4")).view(np.uint8)
    sb = np.asarray(scales, np.float16).view(np.uint16).astype(np.uint32)
    zb = np.asarray(zeros, np.float16).view(np.uint16).astype(np.uint32)
    G = sb.shape[1]
    sz = (sb | (zb << 16)).reshape(rows // 16, 16, G).transpose(0, 2, 1)
    return np.ascontiguousarray(qt), np.ascontiguousarray(sz)


def matmul_ref(x, w_hat):
    """fp32 x @ w_hat.T (the reference tests' dequantize-then-matmul)."""
    return np.asarray(x, dtype=F32) @ np.asarray(w_hat, dtype=F32).T


def max_abs_rel(y, ref) -> float:
    """max|y - ref| / max|ref| (tests/test_moe_int4.py:139)."""
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.abs(y - ref).max() / (np.abs(ref).max() + 1e-30))
