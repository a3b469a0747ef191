"""Pins of the numpy oracle (oracle/quant.py) — CPU only.

Each check is chosen so that a plausible restatement mistake (a dropped
term, a wrong shift/index, a swapped rounding order) fails it.
"""
import numpy as np
import pytest

from oracle import quant as Q


# ------------------------------------------------------------------ E4M3
def test_e4m3_known_values_roundtrip():
    # exact values of the reference test (tests/test_quantizer.py:10-16)
    vals = np.array([0.0, 0.5, 1.0, 1.5, 2.0, -3.5, 448.0, -448.0, 2.0 ** -6, 2.0 ** -9, 0.875],
                    dtype=np.float32)
    np.testing.assert_array_equal(Q.e4m3_decode(Q.e4m3_encode(vals)), vals)
    # and their codes, from the e4m3fn bit layout (sign|eeee|mmm, bias 7)
    assert Q.e4m3_encode(np.float32(448.0)) == 0x7E
    assert Q.e4m3_encode(np.float32(-448.0)) == 0xFE
    assert Q.e4m3_encode(np.float32(1.0)) == 0x38
    assert Q.e4m3_encode(np.float32(2.0 ** -9)) == 0x01
    assert Q.e4m3_encode(np.float32(2.0 ** -6)) == 0x08
    assert Q.e4m3_encode(np.float32(-0.0)) == 0x80


def test_e4m3_decode_exhaustive_closed_form():
    codes = np.arange(256, dtype=np.uint8)
    got = Q.e4m3_decode(codes)
    for c in range(256):
        s = -1.0 if c & 0x80 else 1.0
        e, m = (c >> 3) & 0xF, c & 7
        want = s * (2.0 ** (e - 7) * (1 + m / 8) if e else m * 2.0 ** -9)
        assert got[c] == np.float32(want), c


def test_e4m3_vs_torch_reference_test():
    # the reference's own oracle test (tests/test_quantizer.py:19-27)
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(4096).astype(np.float32) * 100).clip(-448, 448)
    ours = Q.e4m3_decode(Q.e4m3_encode(x))
    ref = torch.tensor(x).to(torch.float8_e4m3fn).float().numpy()
    np.testing.assert_array_equal(ours, ref)


def _strided_fp32(lo_bits, hi_bits, stride):
    b = np.arange(lo_bits, hi_bits, stride, dtype=np.uint64).astype(np.uint32)
    return b.view(np.float32)


def test_e4m3_encode_sweep_vs_torch_outside_quirk_band():
    """Every 61st fp32 bit pattern of [0, 448] (both signs): equal to torch's
    round-to-nearest-even e4m3fn cast except inside [7.5*2^-9, 2^-6), where the
    reference clips the subnormal code to 7 (quantizer.py:48-49)."""
    torch = pytest.importorskip("torch")
    pos = _strided_fp32(0, int(np.float32(448.0).view(np.uint32)) + 1, 61)
    x = np.concatenate([pos, -pos])
    ours = Q.e4m3_encode(x)
    ref = torch.tensor(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    band = (np.abs(x) >= 7.5 * 2.0 ** -9) & (np.abs(x) < 2.0 ** -6)
    np.testing.assert_array_equal(ours[~band], ref[~band])
    assert np.all((ours[band] & 0x7F) == 0x07)
    assert np.all(ref[band] & 0x7F == 0x08)


def test_e4m3_rne_sat_vs_torch_and_saturation():
    torch = pytest.importorskip("torch")
    pos = _strided_fp32(0, int(np.float32(448.0).view(np.uint32)) + 1, 67)
    x = np.concatenate([pos, -pos])
    np.testing.assert_array_equal(
        Q.e4m3_encode_rne_sat(x), torch.tensor(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy())
    big = np.array([448.0, 449.0, 470.0, 1e6, np.inf, -500.0], dtype=np.float32)
    np.testing.assert_array_equal(Q.e4m3_encode_rne_sat(big),
                                  np.array([0x7E, 0x7E, 0x7E, 0x7E, 0x7E, 0xFE], np.uint8))
    assert Q.e4m3_encode_rne_sat(np.float32(np.nan)) & 0x7F == 0x7F


# ------------------------------------------------------------ FP8 blocks
def test_fp8_block_brute_force_tiny():
    rng = np.random.default_rng(5)
    w = (rng.standard_normal((5, 7)) * 3).astype(np.float32)
    q, s = Q.quantize_fp8_block(w, bs=4)
    assert q.shape == (5, 7) and s.shape == (2, 2)
    for bi in range(2):
        for bj in range(2):
            blk = w[4 * bi:4 * bi + 4, 4 * bj:4 * bj + 4]
            amax = np.float32(np.abs(blk).max())
            sc = np.float32(1.0) if amax == 0 else np.float32(amax / np.float32(448.0))
            assert s[bi, bj] == sc
            for r in range(blk.shape[0]):
                for c in range(blk.shape[1]):
                    assert q[4 * bi + r, 4 * bj + c] == Q.e4m3_encode(np.float32(blk[r, c] / sc))


def test_fp8_block_quant_error_and_nondivisible():
    # reference tests/test_quantizer.py:30-45
    rng = np.random.default_rng(1)
    w = rng.standard_normal((256, 384)).astype(np.float32)
    q, s = Q.quantize_fp8_block(w, 128)
    wd = Q.dequantize_fp8_block(q, s, 128)
    assert np.abs(wd - w).mean() / np.abs(w).mean() < 0.05
    w2 = np.random.default_rng(2).standard_normal((100, 200)).astype(np.float32)
    q2, s2 = Q.quantize_fp8_block(w2, 128)
    assert Q.dequantize_fp8_block(q2, s2, 128).shape == w2.shape
    # the block holding the maximum decodes it exactly to 448 * scale
    i = np.unravel_index(np.abs(w).argmax(), w.shape)
    assert abs(int(q[i]) & 0x7F) == 0x7E


def test_fp8_inline_layout_and_roundtrip():
    rng = np.random.default_rng(9)
    w = (rng.standard_normal((3, 256)) * 0.1).astype(np.float16).astype(np.float32)
    p = Q.quantize_fp8_inline(w)
    assert p.shape == (3, Q.fp8_inline_row_bytes(256)) == (3, 264)
    # scale sits right after its 128 codes (fastllm_fp8_block128.cu:84-88)
    s0 = p[0, 128:132].view(np.float32)[0]
    assert s0 == np.float32(np.abs(w[0, :128]).max() / np.float32(448.0))
    wd = Q.dequantize_fp8_inline(p, 256)
    assert np.abs(wd - w).max() <= np.abs(w).max() / 16  # 3 mantissa bits


# ------------------------------------------------------------------ INT4
def test_int4_group_error_bound():
    # reference tests/test_quantizer.py:48-56
    rng = np.random.default_rng(3)
    w = rng.standard_normal((64, 256)).astype(np.float32)
    p, s, z = Q.quantize_int4_group(w, 128)
    wd = Q.dequantize_int4_group(p, s, z, 128)
    step = (w.reshape(64, 2, 128).max(-1) - w.reshape(64, 2, 128).min(-1)) / 15.0
    assert (np.abs(wd - w).reshape(64, 2, 128).max(-1) <= step * 0.5 + 1e-6).all()


def test_int4_variants_brute_force_tiny():
    rng = np.random.default_rng(11)
    w = (rng.standard_normal((3, 16)) * 0.3).astype(np.float32)
    w[1, :8] = 0.25  # constant group -> scale 1 branch
    p3, s3, z3 = Q.quantize_int4_group(w, 8)
    q9, s9, z9 = Q.quantize_int4_marlin(w, 8)
    p13, s13, z13 = Q.quantize_int4_rowmajor(w, 8)
    for r in range(3):
        for gi in range(2):
            g = w[r, 8 * gi:8 * gi + 8]
            lo, hi = np.float32(g.min()), np.float32(g.max())
            s = np.float32((hi - lo) / np.float32(15.0))
            s = np.float32(1.0) if s == 0 else s
            zi = min(max(np.rint(np.float32(-lo / s)), 0), 15)
            assert s3[r, gi] == s and z3[r, gi] == lo and s9[r, gi] == s and z9[r, gi] == zi
            assert s13[r, gi] == np.float16(s) and z13[r, gi] == np.float16(zi)
            for i in range(8):
                c = 8 * gi + i
                q3 = min(max(np.rint(np.float32(np.float32(g[i] - lo) / s)), 0), 15)
                q9_ = min(max(np.rint(np.float32(g[i] / s)) + zi, 0), 15)
                q13 = min(max(np.rint(np.float32(np.float32(g[i] / s) + np.float32(zi))), 0), 15)
                nib = (c % 2) * 4
                assert (p3[r, c // 2] >> nib) & 0xF == q3
                assert q9[r, c] == q9_
                assert (p13[r, c // 2] >> nib) & 0xF == q13


def test_int4_variant_disagreement_counts():
    """Config-1 shape, N(0,0.02) seed 0: the three RTN variants disagree on
    exactly the element counts measured independently of this oracle
    (marlin vs rowmajor codes: 2 for fp32 input / 359 for fp16-cast input;
    group vs marlin codes: 773,237 / 773,125)."""
    rng = np.random.default_rng(0)
    W = (rng.standard_normal((3072, 1024)) * 0.02).astype(np.float32)
    for w, n913, n39 in ((W, 2, 773237), (W.astype(np.float16), 359, 773125)):
        q9, _, _ = Q.quantize_int4_marlin(w, 128)
        q13 = Q._unpack_pairs(Q.quantize_int4_rowmajor(w, 128)[0]).astype(np.uint8)
        q3 = Q._unpack_pairs(Q.quantize_int4_group(w, 128)[0]).astype(np.uint8)
        assert int((q9 != q13).sum()) == n913
        assert int((q3 != q9).sum()) == n39


def test_rowmajor_batched_equals_per_matrix():
    rng = np.random.default_rng(4)
    W = (rng.standard_normal((3, 32, 256)) * 0.1).astype(np.float16)
    pb, sb, zb = Q.quantize_int4_rowmajor(W, 128)
    for e in range(3):
        p, s, z = Q.quantize_int4_rowmajor(W[e], 128)
        np.testing.assert_array_equal(pb[e], p)
        np.testing.assert_array_equal(sb[e], s)
        np.testing.assert_array_equal(zb[e], z)


def test_pack_gptq_brute_force():
    rng = np.random.default_rng(6)
    q = rng.integers(0, 16, size=(8, 24)).astype(np.uint8)
    words = Q.pack_gptq(q)
    assert words.shape == (3, 8)
    for kw in range(3):
        for n in range(8):
            want = 0
            for i in range(8):
                want |= int(q[n, 8 * kw + i]) << (4 * i)
            assert int(words[kw, n]) == want


def test_marlin_permutation_brute_force():
    """Scale position 8i+j of each 64-chunk holds column 8j+i; zero word w of a
    chunk holds, in slot s, column 8*zpi[s] + w with zpi = [0,2,4,6,1,3,5,7]
    (docs/fastllm-internals.md:449-503); reading back through
    marlin_dequant recovers the unpermuted values."""
    rng = np.random.default_rng(8)
    N, G, gs = 128, 2, 32
    scale = rng.random((N, G)).astype(np.float32) + 0.5
    zero = rng.integers(0, 16, size=(N, G))
    s_out, z_out = Q.marlin_scales_zeros(scale, zero)
    zpi = [0, 2, 4, 6, 1, 3, 5, 7]
    for g in range(G):
        for c in range(N // 64):
            for i in range(8):
                for j in range(8):
                    assert s_out[g, 64 * c + 8 * i + j] == np.float16(scale[64 * c + 8 * j + i, g])
            for w in range(8):
                word = int(z_out[g, 8 * c + w])
                for s in range(8):
                    assert (word >> (4 * s)) & 0xF == zero[64 * c + 8 * zpi[s] + w, g]
    q = rng.integers(0, 16, size=(N, G * gs)).astype(np.uint8)
    deq = Q.marlin_dequant(q, s_out, z_out, gs)
    want = (q.reshape(N, G, gs).astype(np.float32) - zero[:, :, None]) * \
        scale.astype(np.float16).astype(np.float32)[:, :, None]
    np.testing.assert_array_equal(deq, want.reshape(N, G * gs))


def test_moe_tile_pack_brute_force():
    """The MoE tile layout against its per-nibble definition: weight (R, k)
    sits in block (R // 16, k // 128), lane c + 16 q (c = R % 16,
    q = k % 128 // 32), u32 j = k % 32 // 8, nibble slot
    {0,4,1,5,2,6,3,7}[k % 8]."""
    rng = np.random.default_rng(11)
    rows, in_f, gs = 32, 256, 64
    packed = rng.integers(0, 256, size=(rows, in_f // 2)).astype(np.uint8)
    sc = (rng.random((rows, in_f // gs)) + 0.5).astype(np.float16)
    ze = rng.integers(0, 16, size=(rows, in_f // gs)).astype(np.float16)
    qt, sz = Q.moe_tile_pack(packed, sc, ze)
    assert qt.shape == (rows // 16, in_f // 128, 1024) and sz.shape == (rows // 16, in_f // gs, 16)
    slot_of = [0, 4, 1, 5, 2, 6, 3, 7]
    for R in range(rows):
        for k in range(in_f):
            want = (int(packed[R, k // 2]) >> (4 * (k % 2))) & 0xF
            kb, q, j, r = k // 128, (k % 128) // 32, (k % 32) // 8, k % 8
            byte = 16 * (R % 16 + 16 * q) + 4 * j + slot_of[r] // 2
            got = (int(qt[R // 16, kb, byte]) >> (4 * (slot_of[r] % 2))) & 0xF
            assert got == want
        for g in range(in_f // gs):
            v = int(sz[R // 16, g, R % 16])
            assert v & 0xFFFF == int(sc[R, g].view(np.uint16))
            assert v >> 16 == int(ze[R, g].view(np.uint16))
