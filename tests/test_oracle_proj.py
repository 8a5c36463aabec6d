"""CPU pins of the projection references (oracle/proj.py): known answers that a dropped
term, a transposed operand or a wrong block offset fails."""
import numpy as np

from oracle import bf16, proj
from oracle.inputs import Gen


def test_gemv_one_hot_picks_a_column_and_is_linear():
    g = Gen(11)
    n_in, n_out = 40, 7
    w = g.normal_bf16(1, (n_out, n_in))
    x = np.zeros(n_in, np.uint16)
    x[13] = bf16.from_f32(np.array([2.0], np.float32))[0]
    y, mag = proj.gemv_ref(x, w)
    np.testing.assert_array_equal(y, 2.0 * bf16.to_f32(w[:, 13]).astype(np.float64))   # w[o][13], not w[13][o]
    np.testing.assert_array_equal(mag, np.abs(y))
    x2 = g.normal_bf16(2, (n_in,))
    y2, _ = proj.gemv_ref(x2, w)
    # additivity over a split of the inputs
    xa, xb = x2.copy(), x2.copy()
    xa[n_in // 2:] = 0
    xb[:n_in // 2] = 0
    np.testing.assert_allclose(proj.gemv_ref(xa, w)[0] + proj.gemv_ref(xb, w)[0], y2, rtol=1e-12, atol=1e-12)


def test_in_proj_rows_are_gemvs_and_split_layout():
    class Cfg:
        h_k, h_v, d_k, d_v = 1, 2, 4, 4

    g = Gen(12)
    K, B = 16, 3
    N = 2 * 1 * 4 + 2 * 4 + 2 * 4 + 2 * 2          # C=16, Z=8, a=2, b=2 -> 28
    h = g.normal_bf16(1, (B, K))
    w = g.normal_bf16(2, (N, K))
    y, _ = proj.in_proj_ref(h, w)
    for r in range(B):
        np.testing.assert_allclose(y[r], proj.gemv_ref(h[r], w)[0], rtol=1e-15)
    x, z, a, b = proj.in_proj_split(Cfg, np.arange(B * N).reshape(B, N))
    assert x.shape == (B, 16) and z.shape == (B, 2, 4) and a.shape == (B, 2) and b.shape == (B, 2)
    assert x[1, 0] == N and z[1, 0, 0] == N + 16 and a[1, 0] == N + 24 and b[1, 1] == N + 27


def test_q8_formats_and_known_answers():
    d = proj.half_exact(np.array([[1.5, 0.25]], np.float32))
    qs = np.zeros((1, 2, 32), np.int8)
    qs[0, 0, :] = 1
    qs[0, 1, 0] = -127
    qs[0, 1, 31] = 5
    pk = proj.pack_q8_0(d, qs)
    assert pk.size == 68
    assert pk[0:2].view("<f2")[0] == 1.5 and pk[34:36].view("<f2")[0] == 0.25        # scale first
    assert pk[2:34].view(np.int8).tolist() == [1] * 32
    assert pk[36] == np.uint8(129) and pk[67] == 5                                    # -127, then the last quant
    xd = proj.half_exact(np.array([[2.0, 3.0]], np.float32))
    xq = np.ones((1, 2, 32), np.int8)
    px = proj.pack_q8_1(xd, xq, proj.half_exact(np.array([[7.0, 9.0]], np.float32)))
    assert px.size == 72 and px[2:4].view("<f2")[0] == 7.0 and px[4:36].view(np.int8).tolist() == [1] * 32
    y, sc = proj.q8_0_ref(d, qs, xd, xq)
    # block 0: 1.5 * 2 * 32; block 1: 0.25 * 3 * (-127 + 5)
    assert y[0, 0] == 1.5 * 2 * 32 + 0.25 * 3 * (-122)
    assert sc[0, 0] == (1.5 * 2 + 0.25 * 3) * 32 * 127 * 127


def test_q8_blocks_distribution():
    d, q = proj.q8_blocks(5, 1, 4, 8)
    dv = d.view(np.float16).astype(np.float64)
    assert dv.min() >= 1 / 1024 and dv.max() <= 2047 / 1024
    assert np.all(np.abs(dv * 1024 - np.round(dv * 1024)) == 0)      # exact multiples of 1/1024
    assert q.min() >= -127 and q.max() <= 127 and q.dtype == np.int8


def test_q8_1_quantize_known_answers():
    # One block with max|x| = 127 (d = 1): ties go away from zero (2.5 -> 3, -2.5 -> -3, a
    # round-half-even mistake gives 2 and -2), 126.5 -> 127; a second, all-zero block is all
    # zero bytes (d = 0, q = 0, not a division by zero); a third with max|x| = 63.5 (d = 0.5).
    x = np.zeros(96, np.float32)
    x[:5] = [2.5, -2.5, 127.0, -126.5, 0.49999997]
    x[64:67] = [63.5, -1.25, 0.25]
    d, s, q = proj.q8_1_unpack(proj.q8_1_quantize(x))
    np.testing.assert_array_equal(d.view(np.float16), np.array([1.0, 0.0, 0.5], np.float16))
    np.testing.assert_array_equal(q[0][:5], [3, -3, 127, -127, 0])
    assert not q[0][5:].any() and not q[1].any() and d[1] == 0 and s[1] == 0
    np.testing.assert_array_equal(q[2][:3], [127, -3, 1])                   # 63.5/0.5, -2.5 -> -3, 0.5 -> 1
    assert s.view(np.float16)[0] == np.float16(2.5 - 2.5 + 127.0 - 126.5 + 0.49999997)
    # block layout: d at bytes 0-1, s at 2-3, qs at 4-35 of each 36-byte block
    b = proj.q8_1_quantize(x)
    assert b.size == 3 * 36 and b[36 + 4:72].sum() == 0 and b[72:74].view("<u2")[0] == np.float16(0.5).view(np.uint16)


def test_q8_1_quantize_bounds_and_sum():
    g = Gen(41)
    nb = 4000
    scale = np.exp(g.normal(1, (nb, 1)) * 2).astype(np.float32)           # magnitudes over ~7 decades, sums in fp16 range
    x = (g.normal(2, (nb, 32)) * scale).astype(np.float32)
    d, s, q = proj.q8_1_unpack(proj.q8_1_quantize(x.reshape(-1)))
    d32 = np.abs(x).max(axis=1) / np.float32(127.0)
    assert np.abs(q).max() <= 127 and (np.abs(q).max(axis=1) == 127).all()  # the largest value maps to +-127
    err = np.abs(x.astype(np.float64) - q.astype(np.float64) * d32[:, None].astype(np.float64))
    assert (err <= 0.5 * d32[:, None] * (1 + 2.0 ** -20)).all()             # round to nearest in units of d
    np.testing.assert_array_equal(d, d32.astype(np.float16).view(np.uint16))
    ref = x.astype(np.float64).sum(axis=1)
    assert np.abs(ref).max() < 60000
    # fp32 summation error, then one fp16 rounding (relative 2^-11, or half the subnormal step)
    tol = 32 * 2.0 ** -23 * np.abs(x).astype(np.float64).sum(axis=1) + np.abs(ref) * 2.0 ** -11 + 2.0 ** -25
    assert (np.abs(s.view(np.float16).astype(np.float64) - ref) <= tol).all()


def test_q8_1_quantize_range_clamps():
    # Block 0: max|x| = 1e7, so max|x| / 127 = 78740.16 exceeds fp16's 65504: d is stored as
    # 65504 and the codes saturate (1e7 / 65504 = 152.7 -> 127, 3 * 65504 -> 3 exactly); the sum
    # 1e7 - 1e7 + 196512 = 196512 is stored as 65504, not inf. Block 1: a sum past fp32's range
    # (two 3e38) is stored as 65504 too. Block 2: max|x| = 127 * 65504 exactly, the largest
    # block the clamp leaves alone (d = 65504 from the division itself, codes unsaturated).
    x = np.zeros(96, np.float32)
    x[:4] = [1e7, -1e7, 3 * 65504.0, -65504.0 * 0.5]
    x[32:34] = [3e38, 3e38]
    x[64:66] = [127 * 65504.0, -2 * 65504.0]
    d, s, q = proj.q8_1_unpack(proj.q8_1_quantize(x))
    h = d.view(np.float16)
    assert np.isfinite(h).all() and np.isfinite(s.view(np.float16)).all()
    assert h[0] == np.float16(65504.0) and h[1] == np.float16(65504.0) and h[2] == np.float16(65504.0)
    np.testing.assert_array_equal(q[0][:4], [127, -127, 3, -1])            # -0.5 rounds away from zero
    assert s.view(np.float16)[0] == np.float16(65504.0) and s.view(np.float16)[1] == np.float16(65504.0)
    np.testing.assert_array_equal(q[1][:2], [127, 127])
    np.testing.assert_array_equal(q[2][:2], [127, -2])
    # below the bound nothing changes: the unclamped rule on a block with max|x| = 8e6
    y = np.zeros(32, np.float32)
    y[:3] = [8e6, -4e6, 1.0]
    dy, _, qy = proj.q8_1_unpack(proj.q8_1_quantize(y))
    d32 = np.float32(8e6) / np.float32(127.0)
    assert dy[0] == d32.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(qy[0][:3], [127, np.int8(np.round(np.float32(-4e6) / d32)), 0])
