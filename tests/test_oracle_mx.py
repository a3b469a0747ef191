"""Pins of the MXFP4 codec and the low-precision expert tile layouts
(oracle/mx.py) against what the format's definition fixes: a brute-force
nearest-code search, the E2M1 bit-field closed form, exact round trips,
the scale exponent from frexp, and element-by-element loops over the tile
layouts."""
import math

import numpy as np

from oracle import mx
from oracle import quant as Q


def _brute_e2m1(p):
    """Nearest E2M1 magnitude by explicit distances; a tie takes the even
    code; beyond 6 the code saturates at 7."""
    out = []
    for v in np.asarray(p, np.float32).tolist():
        a = abs(v)
        d = [abs(a - float(m)) for m in mx.E2M1_MAG]
        best = min(d)
        cands = [c for c in range(8) if d[c] == best]
        c = cands[0] if len(cands) == 1 else [c for c in cands if c % 2 == 0][0]
        out.append(c | (8 if math.copysign(1.0, v) < 0 else 0))
    return np.array(out, np.uint8)


def test_e2m1_decode_closed_form():
    # bits s e1 e0 m, exponent bias 1: e = 0 -> 0.5 m, else 2^(e-1) (1 + m/2)
    for c in range(16):
        s, e, m = c >> 3, (c >> 1) & 3, c & 1
        v = 0.5 * m if e == 0 else 2.0 ** (e - 1) * (1 + m / 2)
        assert mx.e2m1_decode(np.array([c], np.uint8))[0] == (-v if s else v)


def test_e2m1_encode_matches_brute_force():
    rng = np.random.default_rng(1)
    mids = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0], np.float32)
    near = np.concatenate([mids, np.nextafter(mids, np.float32(0)), np.nextafter(mids, np.float32(9))])
    vals = np.concatenate([near, -near, mx.E2M1_MAG, -mx.E2M1_MAG, [0.0, -0.0, 6.5, 7.9, 100.0, -7.0],
                           rng.uniform(-8, 8, 20000).astype(np.float32)]).astype(np.float32)
    np.testing.assert_array_equal(mx.e2m1_encode(vals), _brute_e2m1(vals))


def test_exponent_from_frexp():
    rng = np.random.default_rng(2)
    amax = np.concatenate([rng.uniform(0, 1, 2000) * 10.0 ** rng.integers(-40, 38, 2000),
                           [2.0 ** -149, 2.0 ** -127, 1.0, 6.0, 8.0, 3.0e38]]).astype(np.float32)
    for a in amax.tolist():
        _, ex = math.frexp(a)  # a = f 2^ex, f in [0.5, 1): floor(log2 a) = ex - 1
        want = 0 if a == 0 else max(-127, min(127, ex - 1 - 2))
        got = int(mx.e8m0_exponent(np.array([a], np.float32))[0])
        if a < 2.0 ** -126:  # subnormal: the exponent field alone clamps to -127
            want = -127
        assert got == want, a


def test_round_trip_of_representable_blocks():
    rng = np.random.default_rng(3)
    R, C = 24, 256
    codes = rng.integers(0, 16, (R, C)).astype(np.uint8)
    codes[:, ::32] = 7  # a full-scale element (6) in every block fixes X = 2^s
    s = rng.integers(-20, 10, (R, C // 32))
    w = mx.e2m1_decode(codes).reshape(R, C // 32, 32) * np.ldexp(np.float32(1), s)[:, :, None]
    w = w.reshape(R, C).astype(np.float32)
    p, e8 = mx.quantize_mxfp4(w)
    np.testing.assert_array_equal(e8.astype(np.int64) - 127, s)
    np.testing.assert_array_equal(mx.dequantize_mxfp4(p, e8), w)


def test_quantization_error_bound():
    rng = np.random.default_rng(4)
    w = (rng.standard_normal((32, 512)) * 0.02).astype(np.float32)
    w[0, :32] = 0.0  # all-zero block: X = 1, codes 0
    p, e8 = mx.quantize_mxfp4(w)
    assert (e8[0, 0] == 127) and not (p[0, :16] & 0x77).any()
    d = mx.dequantize_mxfp4(p, e8)
    X = np.repeat(np.ldexp(np.float32(1), e8.astype(np.int64) - 127), 32, axis=1)
    a = np.abs(w) / X
    # unsaturated: within half the local code gap (<= 1 above 4, 0.5 above 2, 0.25 below)
    gap = np.where(a > 4, 1.0, np.where(a > 2, 0.5, 0.25))
    ok = a <= 6
    assert (np.abs(d - w)[ok] <= gap[ok] * X[ok]).all()
    assert np.allclose(np.abs(d)[~ok], 6 * X[~ok])


def test_fp8_tile_layout_brute_force():
    rng = np.random.default_rng(5)
    rows, cols = 32, 256
    q = rng.integers(0, 256, (rows, cols)).astype(np.uint8)
    t = mx.moe_tile_pack_fp8(q)
    for r in range(rows):
        for k in range(cols):
            tt, c, kb, kk = r // 16, r % 16, k // 128, k % 128
            qq, h, i = kk // 32, (kk % 32) // 16, kk % 16
            assert t[tt, kb, 1024 * h + 16 * (c + 16 * qq) + i] == q[r, k]


def test_mxfp4_tile_layout_brute_force():
    rng = np.random.default_rng(6)
    rows, cols = 32, 256
    p = rng.integers(0, 256, (rows, cols // 2)).astype(np.uint8)
    e8 = rng.integers(0, 256, (rows, cols // 32)).astype(np.uint8)
    qt, ew = mx.moe_tile_pack_mxfp4(p, e8)
    for r in range(rows):
        for k in range(cols):
            code = (p[r, k // 2] >> (4 * (k % 2))) & 0xF
            tt, c, kb, kk = r // 16, r % 16, k // 128, k % 128
            j, rest = kk // 32, kk % 32
            qq, i = rest // 8, rest % 8
            byte = qt[tt, kb, 16 * (c + 16 * qq) + 4 * j + i // 2]
            assert (byte >> (4 * (i % 2))) & 0xF == code
        for g in range(cols // 32):
            kb, j = g // 4, g % 4
            assert (int(ew[r // 16, kb, r % 16]) >> (8 * j)) & 0xFF == e8[r, g]


def test_fp8_expert_blocks_align_with_experts():
    """Stacked experts quantized as one (E*out, in) matrix with 128x128
    blocks equal each expert quantized alone when out % 128 == 0."""
    rng = np.random.default_rng(7)
    E, out_f, in_f = 3, 256, 384
    w = (rng.standard_normal((E, out_f, in_f)) * 0.02).astype(np.float32)
    q, s = Q.quantize_fp8_block(w.reshape(E * out_f, in_f))
    for e in range(E):
        qe, se = Q.quantize_fp8_block(w[e])
        np.testing.assert_array_equal(q[e * out_f:(e + 1) * out_f], qe)
        np.testing.assert_array_equal(s[e * out_f // 128:(e + 1) * out_f // 128], se)
