"""Pins for the oracle's Q4_K functions (CPU only).

Each check is independent of the oracle's own code: numpy's float16
conversion (exhaustive), the Q4_K scale layout written as a bit map, hand-built
blocks whose weights are exact small numbers, numpy float64 products, and
planted mistakes that must be caught.
"""
import numpy as np
import pytest

import oracle


def _block(d_bits, dmin_bits, scales12, qs128):
    b = np.zeros(144, np.uint8)
    b[0], b[1] = d_bits & 0xFF, d_bits >> 8
    b[2], b[3] = dmin_bits & 0xFF, dmin_bits >> 8
    b[4:16] = scales12
    b[16:] = qs128
    return b


def test_f16_decode_exhaustive_against_numpy():
    """Every one of the 65536 half bit patterns (unpack2x16float semantics)."""
    bits = np.arange(65536, dtype=np.uint16)
    got = oracle.f16_to_f32(bits)
    ref = bits.view(np.float16).astype(np.float32)
    same = (got.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(got) & np.isnan(ref))
    assert same.all()


def test_f16_encode_matches_numpy_rounding():
    rng = np.random.default_rng(1)
    vals = (rng.standard_normal(20000) * 10.0 ** rng.integers(-9, 6, 20000)).astype(np.float32)
    edge = np.array([65504, 65519.996, 65520, 2.0 ** -24, 2.0 ** -25, 1.5 * 2.0 ** -25,
                     2.0 ** -14, 2.0 ** -14 - 2.0 ** -26, 0.0, -0.0, 1.0 + 2.0 ** -11,
                     1.0 + 3 * 2.0 ** -11], np.float32)
    vals = np.concatenate([vals, edge, -edge])
    with np.errstate(over="ignore"):
        ref = vals.astype(np.float16).view(np.uint16)
    got = np.array([oracle.f32_to_f16(v) for v in vals], np.uint16)
    np.testing.assert_array_equal(got, ref)


# The packed scale bytes as a bit map (ggml's Q4_K layout, the one
# shader_q4k_matvec.wgsl:87-113 decodes): (byte, bit) -> (field, j, bit).
def _layout():
    m = {}
    for j in range(4):
        for bit in range(6):
            m[(j, bit)] = ("sc", j, bit)          # low 6 bits of bytes 0-3: scales 0-3
            m[(j + 4, bit)] = ("m", j, bit)       # low 6 bits of bytes 4-7: mins 0-3
        for bit in range(4):
            m[(j + 8, bit)] = ("sc", j + 4, bit)      # low nibble of bytes 8-11: scales 4-7
            m[(j + 8, bit + 4)] = ("m", j + 4, bit)   # high nibble of bytes 8-11: mins 4-7
        m[(j, 6)] = ("sc", j + 4, 4)    # top 2 bits of bytes 0-3: scales 4-7 bits 4,5
        m[(j, 7)] = ("sc", j + 4, 5)
        m[(j + 4, 6)] = ("m", j + 4, 4)  # top 2 bits of bytes 4-7: mins 4-7 bits 4,5
        m[(j + 4, 7)] = ("m", j + 4, 5)
    return m


def test_scale_unpack_against_bit_map():
    layout = _layout()
    assert len(layout) == 96  # every bit of the 12 bytes has exactly one meaning
    for (byte, bit), (field, j, fbit) in layout.items():
        s = np.zeros(12, np.uint8)
        s[byte] = 1 << bit
        for jj in range(8):
            sc, mn = oracle.q4k_scale_min(s, jj)
            want_sc = (1 << fbit) if (field == "sc" and jj == j) else 0
            want_m = (1 << fbit) if (field == "m" and jj == j) else 0
            assert (sc, mn) == (want_sc, want_m), (byte, bit, jj)


def test_scale_unpack_hand_example():
    # scales 0..7 = 1, 2, ..., 8 style values chosen to use the high bits.
    sc = [5, 17, 33, 63, 0, 47, 18, 61]
    mn = [62, 1, 16, 48, 63, 32, 7, 40]
    s = np.zeros(12, np.uint8)
    for j in range(4):
        s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    for j in range(8):
        assert oracle.q4k_scale_min(s, j) == (sc[j], mn[j])


def _hand_block():
    """d = 1, dmin = 0.5, sub-block j: scale j+1, min 2j+1; quants chosen so
    weight i of the block is recoverable from its value."""
    sc = [j + 1 for j in range(8)]
    mn = [2 * j + 1 for j in range(8)]
    s = np.zeros(12, np.uint8)
    for j in range(4):
        s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    # quant of weight i; the sub-block offset makes halves 32 apart differ
    q = np.array([(i * 7 + 3 + 5 * (i // 32)) % 16 for i in range(256)], np.uint8)
    qs = np.zeros(128, np.uint8)
    for it in range(4):
        for i in range(32):
            qs[it * 32 + i] = q[it * 64 + i] | (q[it * 64 + 32 + i] << 4)
    w = np.array([q[i] * sc[i // 32] - 0.5 * mn[i // 32] for i in range(256)], np.float32)
    return _block(0x3C00, 0x3800, s, qs), w


def test_dequant_hand_block_exact():
    blk, w = _hand_block()
    np.testing.assert_array_equal(oracle.q4k_dequant(blk, 1, 256)[0], w)
    two = np.concatenate([blk, blk])
    np.testing.assert_array_equal(oracle.q4k_dequant(two, 1, 512)[0], np.concatenate([w, w]))
    np.testing.assert_array_equal(oracle.q4k_dequant(two, 2, 256), np.stack([w, w]))


def test_planted_nibble_swap_is_caught():
    """Swapping which nibble feeds which sub-block changes the weights."""
    blk, w = _hand_block()
    bad = blk.copy()
    bad[16:] = ((blk[16:] >> 4) | (blk[16:] << 4)) & 0xFF
    assert not np.array_equal(oracle.q4k_dequant(bad, 1, 256)[0], w)


def test_dequant_subnormal_scales():
    """d and dmin as f16 subnormals (unpack2x16float keeps their exact value)."""
    blk, _ = _hand_block()
    blk[0:2] = [0x01, 0x00]   # d = 2^-24
    blk[2:4] = [0x00, 0x02]   # dmin = 2^-15 (0x0200 subnormal)
    w = oracle.q4k_dequant(blk, 1, 256)[0]
    sc1, m1 = oracle.q4k_scale_min(blk[4:16], 0)
    q0 = blk[16] & 0xF
    assert w[0] == np.float32(q0 * (2.0 ** -24 * sc1)) - np.float32(2.0 ** -15 * m1)


def test_quantize_round_trip_error_bound():
    """scripts/quantize.py's scheme, bounded from its definition: with
    es = d*sc the effective step and em = dmin*m the effective min,
    |es - range/15| <= d/2 and |em - (-min)| <= dmin/2 (when min <= 0), so a
    weight is off by at most half a step, or, where the top quant clips,
    15*d/2 + dmin/2; a sub-block with min > 0 also loses its offset (em = 0)."""
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((6, 1024)) * 0.03).astype(np.float32)
    x[0, :256] = np.linspace(-1, 1, 256)
    x[1, :32] = 0.25                    # constant, positive sub-block
    x[2, 256:512] = np.abs(x[2, 256:512])  # all-positive block
    q = oracle.q4k_quantize(x)
    w = oracle.q4k_dequant(q, 6, 1024).astype(np.float64)
    blocks = q.reshape(-1, 144)
    for r in range(6):
        for blk in range(4):
            b = blocks[r * 4 + blk]
            d = np.frombuffer(b[0:2].tobytes(), np.float16)[0].astype(np.float64)
            dmin = np.frombuffer(b[2:4].tobytes(), np.float16)[0].astype(np.float64)
            # d and dmin are the f16 roundings of max scale / 63, max min / 63
            v = x[r, blk * 256:(blk + 1) * 256].astype(np.float32).reshape(8, 32)
            rs = np.where(v.max(1) > v.min(1), (v.max(1) - v.min(1)) / np.float32(15), 0)
            rm = -v.min(1)
            want_d = np.float16(rs.max() / np.float32(63) if rs.max() > 0 else 1.0)
            want_dm = np.float16(rm.max() / np.float32(63) if rm.max() > 0 else 1.0)
            assert (np.float16(d), np.float16(dmin)) == (want_d, want_dm), (r, blk)
            for j in range(8):
                sc, mn = oracle.q4k_scale_min(b[4:16], j)
                seg = slice(blk * 256 + j * 32, blk * 256 + j * 32 + 32)
                xs = x[r, seg].astype(np.float64)
                bound = max(d * sc / 2, 7.5 * d + dmin / 2) + max(0.0, xs.min())
                err = np.abs(w[r, seg] - xs).max()
                assert err <= bound * (1 + 1e-3) + 1e-7, (r, blk, j, err, bound)


def test_matvec_f64_against_numpy():
    blocks = oracle.q4k_random_blocks(3, 40, 768)
    x = oracle.normal(7, (3, 768))
    w = oracle.q4k_dequant(blocks, 40, 768).astype(np.float64)
    want = x.astype(np.float64) @ w.T
    np.testing.assert_allclose(oracle.q4k_matvec_f64(blocks, x, 40), want, rtol=1e-12, atol=1e-12)


def _bound(blocks, x, N):
    """sum_k (|w_k| + 2 |dmin*min_k|) |x_k|: the scale of the f32 rounding
    error of any summation order of the product."""
    K = x.shape[1]
    w = oracle.q4k_dequant(blocks, N, K).astype(np.float64)
    zq = blocks.reshape(-1, 144).copy()
    zq[:, 16:] = 0
    mins = -oracle.q4k_dequant(zq.reshape(-1), N, K).astype(np.float64)
    return np.abs(x.astype(np.float64)) @ (np.abs(w) + 2 * np.abs(mins)).T


def test_matvec_shader_order_within_f32_bound():
    blocks = oracle.q4k_random_blocks(4, 64, 2048)
    x = oracle.normal(8, (2, 2048))
    got = oracle.q4k_matvec_wgsl(blocks, x, 64).astype(np.float64)
    ref = oracle.q4k_matvec_f64(blocks, x, 64)
    assert (np.abs(got - ref) <= 1e-5 * _bound(blocks, x, 64)).all()


def test_planted_dmin_sign_is_caught():
    """w = q*d1 + m1 (wrong sign of the min) must fail the f64 pin."""
    blocks = oracle.q4k_random_blocks(9, 8, 256)
    x = oracle.normal(10, (1, 256))
    w = oracle.q4k_dequant(blocks, 8, 256).astype(np.float64)
    zq = blocks.reshape(-1, 144).copy()
    zq[:, 16:] = 0
    mins = -oracle.q4k_dequant(zq.reshape(-1), 8, 256).astype(np.float64)
    wrong = (w + 2 * mins) @ x[0].astype(np.float64)
    assert np.abs(wrong - oracle.q4k_matvec_f64(blocks, x, 8)[0]).max() > 1e-3
