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
