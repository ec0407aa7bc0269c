"""Block codecs: the oracle's dequantizers and the converter's quantizers.

No golden vectors for these formats exist in the reference (k-quants are never
exercised by its tests).  What pins them here:
  * f16: exhaustive over all 65536 bit patterns against numpy's IEEE binary16.
  * Q8_0: closed form on hand-built blocks.
  * Q4_K / Q5_K / Q6_K: hand-built blocks where a single sub-block scale is
    non-zero, so a wrong nibble/bit interleave, a wrong 6-bit scale unpacking
    (including the high bits of scales 4..7) or a wrong sign fails.
  * Product quantizer -> oracle dequantizer round trips within the format's
    resolution, and product dequantizer == oracle dequantizer bit for bit.
"""
import numpy as np
import pytest

import malaga_amd as M
import oracle as O

F32, F16, Q8_0, Q4_K, Q5_K, Q6_K = 0, 1, 8, 12, 13, 14


def test_f16_exhaustive():
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    blocks = bits.view(np.uint8)
    got = O.dequant(F16, blocks, 65536)
    same = (got == ref) | (np.isnan(got) & np.isnan(ref))
    assert same.all()


def test_f32_to_f16_round_to_nearest_even():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.normal(0, 1, 20000), rng.normal(0, 1e-5, 2000), rng.normal(0, 3e4, 2000),
                        [65504, 65519.9, 65520, 1e-8, -0.0, 5.9604645e-08, 2.9802322e-08]]).astype(np.float32)
    ref = x.astype(np.float16).view(np.uint16)
    got = np.array([O.f2h(float(v)) for v in x], dtype=np.uint16)
    np.testing.assert_array_equal(got, ref)


def half_bits(v: float) -> bytes:
    return np.array([v], dtype=np.float16).tobytes()


def test_q8_0_closed_form():
    d = 0.0137
    q = np.arange(-16, 16, dtype=np.int8) * 4 - 1
    blk = half_bits(d) + q.tobytes()
    got = O.dequant(Q8_0, np.frombuffer(blk, np.uint8), 32)
    np.testing.assert_array_equal(got, np.float32(np.float16(d)) * q.astype(np.float32))


def pack_k4_scales(sc, mn):
    """6-bit scale/min table of Q4_K/Q5_K (8 pairs in 12 bytes), written from the format spec."""
    s = [0] * 12
    for j in range(8):
        if j < 4:
            s[j] = sc[j] & 63
            s[j + 4] = mn[j] & 63
        else:
            s[j + 4] = (sc[j] & 15) | ((mn[j] & 15) << 4)
            s[j - 4] |= (sc[j] >> 4) << 6
            s[j] |= (mn[j] >> 4) << 6
    return bytes(s)


@pytest.mark.parametrize("sub", range(8))
def test_q4_k_single_subblock(sub):
    rng = np.random.default_rng(sub)
    d, dmin = 0.25, 0.125
    sc = [0] * 8
    mn = [0] * 8
    sc[sub] = 37 + sub   # >= 16 exercises the high bits of the packing
    mn[sub] = 50 - sub
    nib = rng.integers(0, 16, 256)
    qs = bytearray(128)
    for g in range(4):            # byte l of group g: low nibble -> value 64g + l, high -> 64g + 32 + l
        for l in range(32):
            qs[32 * g + l] = nib[64 * g + l] | (nib[64 * g + 32 + l] << 4)
    blk = half_bits(d) + half_bits(dmin) + pack_k4_scales(sc, mn) + bytes(qs)
    got = O.dequant(Q4_K, np.frombuffer(blk, np.uint8), 256)
    exp = np.zeros(256, np.float32)
    exp[:] = 0.0
    r = slice(32 * sub, 32 * sub + 32)
    exp[r] = np.float32(d * sc[sub]) * nib[r].astype(np.float32) - np.float32(dmin * mn[sub])
    np.testing.assert_allclose(got, exp, rtol=0, atol=1e-6)


@pytest.mark.parametrize("sub", [0, 3, 4, 7])
def test_q5_k_single_subblock(sub):
    rng = np.random.default_rng(10 + sub)
    d, dmin = 0.5, 0.25
    sc, mn = [0] * 8, [0] * 8
    sc[sub], mn[sub] = 21 + 5 * sub, 9 + 7 * sub
    val = rng.integers(0, 32, 256)
    qh = bytearray(32)
    qs = bytearray(128)
    for g in range(4):
        for l in range(32):
            lo, hi = val[64 * g + l], val[64 * g + 32 + l]
            qs[32 * g + l] = (lo & 15) | ((hi & 15) << 4)
            qh[l] |= ((lo >> 4) << (2 * g)) | ((hi >> 4) << (2 * g + 1))
    blk = half_bits(d) + half_bits(dmin) + pack_k4_scales(sc, mn) + bytes(qh) + bytes(qs)
    got = O.dequant(Q5_K, np.frombuffer(blk, np.uint8), 256)
    exp = np.zeros(256, np.float32)
    r = slice(32 * sub, 32 * sub + 32)
    exp[r] = np.float32(d * sc[sub]) * val[r].astype(np.float32) - np.float32(dmin * mn[sub])
    np.testing.assert_allclose(got, exp, rtol=0, atol=1e-6)


@pytest.mark.parametrize("sub", [0, 5, 8, 15])
def test_q6_k_single_group(sub):
    rng = np.random.default_rng(20 + sub)
    d = 0.03125
    sc = np.zeros(16, np.int8)
    sc[sub] = -23 if sub % 2 else 45
    val = rng.integers(0, 64, 256)  # stored 6-bit values (value - 32 is the level)
    ql = bytearray(128)
    qh = bytearray(64)
    for h in range(2):               # 128-value halves; within a half, position 32*k + l
        for l in range(32):
            v = [val[128 * h + 32 * k + l] for k in range(4)]
            ql[64 * h + l] = (v[0] & 15) | ((v[2] & 15) << 4)
            ql[64 * h + 32 + l] = (v[1] & 15) | ((v[3] & 15) << 4)
            qh[32 * h + l] = (v[0] >> 4) | ((v[1] >> 4) << 2) | ((v[2] >> 4) << 4) | ((v[3] >> 4) << 6)
    blk = bytes(ql) + bytes(qh) + sc.tobytes() + half_bits(d)
    got = O.dequant(Q6_K, np.frombuffer(blk, np.uint8), 256)
    exp = np.zeros(256, np.float32)
    r = slice(16 * sub, 16 * sub + 16)
    exp[r] = np.float32(d) * np.float32(sc[sub]) * (val[r] - 32).astype(np.float32)
    np.testing.assert_allclose(got, exp, rtol=0, atol=1e-6)


@pytest.mark.parametrize("t,rel", [(Q8_0, 0.006), (Q4_K, 0.08), (Q5_K, 0.04), (Q6_K, 0.02), (F16, 1e-3)])
def test_quantizer_roundtrip(t, rel):
    rng = np.random.default_rng(t)
    x = rng.normal(0, 0.02, 256 * 64).astype(np.float32)
    blocks = M.quantize(t, x)
    assert blocks.size == M.type_bytes(t, x.size)
    y = O.dequant(t, blocks, x.size)
    err = np.sqrt(np.mean((x - y) ** 2)) / np.sqrt(np.mean(x ** 2))
    assert err < rel, err
    # product and oracle dequantizers agree bit for bit
    np.testing.assert_array_equal(M.dequantize(t, blocks, x.size), y)


def test_q8_0_quantizer_closed_form():
    rng = np.random.default_rng(5)
    x = rng.normal(0, 1, 32 * 40).astype(np.float32)
    x[:32] = 0  # all-zero block: d = 0, q = 0
    blocks = M.quantize(Q8_0, x).reshape(-1, 34)
    amax = np.abs(x.reshape(-1, 32)).max(1)
    d = amax / np.float32(127)
    np.testing.assert_array_equal(blocks[:, :2].copy().view(np.float16)[:, 0], d.astype(np.float16))
    inv = np.where(d != 0, 1 / d, 0).astype(np.float32)
    v = x.reshape(-1, 32) * inv[:, None]
    q = (np.sign(v) * np.floor(np.abs(v) + 0.5)).astype(np.int8)
    np.testing.assert_array_equal(blocks[:, 2:].view(np.int8), q)


@pytest.mark.parametrize("t", [F32, F16, Q8_0, Q4_K, Q5_K, Q6_K])
def test_oracle_gemv_is_a_dot_of_dequantized_rows(t):
    rng = np.random.default_rng(3)
    N, K = 7, 512
    w = rng.normal(0, 0.05, (N, K)).astype(np.float32)
    blocks = M.quantize(t, w)
    x = rng.normal(0, 1, (2, K)).astype(np.float32)
    y = O.gemv(t, blocks, N, K, x)
    wd = O.dequant(t, blocks, N * K).reshape(N, K).astype(np.float64)
    np.testing.assert_allclose(y, (x.astype(np.float64) @ wd.T).astype(np.float32), rtol=1e-6, atol=1e-6)
