"""GPU parity of the projections feeding the layer (gemv.hip, gdn_inproj.hip) against the
double references of oracle/proj.py.

Tolerances, from the reference's own tests: bf16 GEMV |y - ref| <= 2e-5 x sum|x w| per row
(tests/test_bf16_gemv.cu:11); Q8_0 |y - ref| <= 1e-5 x sum|d_w d_x| 32 127^2 (tests/
test_mmvq_wave.cu:57-59). Bitwise: the pair product equals the single product and split(64)
(test_bf16_gemv.cu:41-43); a Q8_0 column does not change with the number of columns launched
(test_mmvq_wave.cu:4); in the input projection the bf16 pieces are RNE of the fp32 result
and the fp32 result is within the GEMV tolerance.
"""
import numpy as np
import pytest

import baloon_amd as bx
from oracle import bf16, inputs, proj
from oracle.inputs import Gen
from tests.common import dev, host

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    return torch


def _ok(name, got, ref, mag, tol):
    err = np.abs(got.astype(np.float64) - ref) / (tol * mag + 1e-30)
    assert float(err.max(initial=0.0)) <= 1.0, f"{name}: worst err/tol {float(err.max()):.3f}"


@pytest.mark.parametrize("nin", [2560, 5120, 100, 63, 64, 65])
def test_bf16_gemv_family(nin):
    torch = _torch()
    g = Gen(0x6D4E0100 + nin)
    for nout in (1, 48, 64, 130, 1000):
        x = g.normal_bf16(1, (nin,))
        w = bf16.from_f32((g.normal(2 + nout, (nout, nin)) * 0.05).astype(np.float32))
        w2 = bf16.from_f32((g.normal(3 + nout, (nout + 17, nin)) * 0.05).astype(np.float32))
        ref, mag = proj.gemv_ref(x, w)
        ref2, mag2 = proj.gemv_ref(x, w2)
        dx, dw, dw2 = dev(x), dev(w), dev(w2)
        y = torch.empty(nout, dtype=torch.float32, device="cuda")
        assert bx.ix_bf16_gemv(dx, dw, y, nin, nout) == 0
        ye = host(y).copy()
        _ok(f"gemv nin={nin} nout={nout}", ye, ref, mag, 2e-5)
        assert bx.ix_bf16_gemv_split(dx, dw, y, nin, nout, 64) == 0
        yw = host(y).copy()
        np.testing.assert_array_equal(yw, ye)                      # split(64) is the wave-per-row kernel
        for tpr in (32, 128, 256):
            assert bx.ix_bf16_gemv_split(dx, dw, y, nin, nout, tpr) == 0
            _ok(f"split({tpr}) nin={nin} nout={nout}", host(y), ref, mag, 2e-5)
        y1 = torch.empty(nout, dtype=torch.float32, device="cuda")
        y2 = torch.empty(nout + 17, dtype=torch.float32, device="cuda")
        assert bx.ix_bf16_gemv_pair(dx, dw, y1, nout, dw2, y2, nout + 17, nin) == 0
        np.testing.assert_array_equal(host(y1), yw)               # pair == standalone, bitwise
        _ok(f"pair.y2 nin={nin} nout={nout}", host(y2), ref2, mag2, 2e-5)


@pytest.mark.parametrize("n_in", [32, 96, 256, 2048, 4096, 7 * 32])
def test_mmvq_q8_0(n_in):
    torch = _torch()
    nb = n_in // 32
    for n_out in (1, 3, 4, 5, 100, 333):
        seed = 0x6D4E0200 + n_in * 7 + n_out
        wd, wq = proj.q8_blocks(seed, 1, n_out, nb)
        xd, xq = proj.q8_blocks(seed, 5, 8, nb)
        ref, sc = proj.q8_0_ref(wd, wq, xd, xq)
        dw = dev(proj.pack_q8_0(wd, wq))
        dxq = dev(proj.pack_q8_1(xd, xq))
        y = torch.empty(8, n_out, dtype=torch.float32, device="cuda")
        outs = {}
        for nc in (8, 1, 3):
            y.fill_(float("nan"))
            assert bx.ix_mmvq_q8_0(dw, dxq, y, n_in, n_out, nc) == 0
            got = host(y)[:nc].copy()
            outs[nc] = got
            err = np.abs(got.astype(np.float64) - ref[:nc]) / sc[:nc]
            assert float(err.max()) <= 1e-5, (n_in, n_out, nc, float(err.max()))
        np.testing.assert_array_equal(outs[1][0], outs[8][0])     # column 0 independent of ncols
        np.testing.assert_array_equal(outs[3], outs[8][:3])


@pytest.mark.parametrize("kw,B,hidden", [
    ({}, 64, 2048),                                  # the bench shape (Qwen3-Next GDN layer)
    ({}, 1, 256),
    ({}, 70, 128),                                   # a second, partial row tile
    (dict(h_k=2, h_v=4), 5, 384),                    # N = 1544: a partial column tile
    (dict(h_k=4, h_v=12, head_map=1), 17, 512),
    ({}, 3, 64),                                     # one k stage (fewer than the ring holds)
    ({}, 9, 192),                                    # three k stages
])
def test_in_proj(kw, B, hidden):
    torch = _torch()
    cfg = bx.make_cfg(**kw)
    N = bx.ix_gdn_in_proj_width(cfg)
    C, Z = cfg.channels, cfg.h_v * cfg.d_v
    assert N == C + Z + 2 * cfg.h_v
    g = Gen(0x6D4E0300 + B + hidden)
    h = g.normal_bf16(1, (B, hidden))
    w = bf16.from_f32((g.normal(2, (N, hidden)) * 0.05).astype(np.float32))
    ref, mag = proj.in_proj_ref(h, w)
    dh, dw = dev(h), dev(w)
    pieces = [torch.zeros(B, C, dtype=torch.bfloat16, device="cuda"),
              torch.zeros(B, cfg.h_v, cfg.d_v, dtype=torch.bfloat16, device="cuda"),
              torch.zeros(B, cfg.h_v, dtype=torch.bfloat16, device="cuda"),
              torch.zeros(B, cfg.h_v, dtype=torch.bfloat16, device="cuda")]
    y = torch.full((B, N), float("nan"), dtype=torch.float32, device="cuda")
    assert bx.ix_gdn_in_proj(cfg, B, hidden, dh, dw, *pieces, y) == 0
    torch.cuda.synchronize()
    yf = host(y)
    _ok(f"in_proj B={B} K={hidden}", yf, ref, mag, 2e-5)
    for got, want in zip(pieces, proj.in_proj_split(cfg, yf)):
        np.testing.assert_array_equal(host(got), bf16.from_f32(np.ascontiguousarray(want)))
    # without the fp32 output the bf16 pieces are the same
    again = [torch.zeros_like(t) for t in pieces]
    assert bx.ix_gdn_in_proj(cfg, B, hidden, dh, dw, *again, None) == 0
    torch.cuda.synchronize()
    for p0, p1 in zip(pieces, again):
        np.testing.assert_array_equal(host(p0), host(p1))


def test_in_proj_feeds_decode():
    # The projection's pieces drive the gated decode directly (through GdnLayer) ...
    torch = _torch()
    cfg = bx.make_cfg()
    B, hidden = 4, 256
    N = bx.ix_gdn_in_proj_width(cfg)
    g = Gen(0x6D4E0399)
    h = g.normal_bf16(1, (B, hidden))
    w = bf16.from_f32((g.normal(2, (N, hidden)) * 0.05).astype(np.float32))
    x = torch.empty(B, cfg.channels, dtype=torch.bfloat16, device="cuda")
    z = torch.empty(B, cfg.h_v, cfg.d_v, dtype=torch.bfloat16, device="cuda")
    a = torch.empty(B, cfg.h_v, dtype=torch.bfloat16, device="cuda")
    b = torch.empty(B, cfg.h_v, dtype=torch.bfloat16, device="cuda")
    assert bx.ix_gdn_in_proj(cfg, B, hidden, dev(h), dev(w), x, z, a, b) == 0
    layer = bx.GdnLayer(B, cfg)
    lp = inputs.layer_params(cfg, 0x6D4E0398)                 # non-zero conv weights and gates
    layer.conv_w.copy_(dev(lp["w"]).view(torch.bfloat16))
    layer.A_log.copy_(dev(lp["A_log"]))
    layer.dt_bias.copy_(dev(lp["dt_bias"]))
    yb = torch.empty(B, cfg.h_v, cfg.d_v, dtype=torch.bfloat16, device="cuda")
    y = torch.empty(B, cfg.h_v, cfg.d_v, dtype=torch.float32, device="cuda")
    n_in = cfg.h_v * cfg.d_v
    yq = torch.empty(B * n_in // 32 * 36, dtype=torch.uint8, device="cuda")
    layer.decode(x, a, b, z=z, y=y, y_bf16=yb, y_q8_1=yq)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(yb.float()).all())
    np.testing.assert_array_equal(host(yb), bf16.from_f32(host(y)))
    # ... and its q8_1 output drives a Q8_0 out-projection (the quantiser's own bytes).
    np.testing.assert_array_equal(host(yq), proj.q8_1_quantize(host(y).reshape(-1)))
    n_out = 64
    wd, wq = proj.q8_blocks(0x6D4E039A, 1, n_out, n_in // 32)
    out = torch.empty(B, n_out, dtype=torch.float32, device="cuda")
    assert bx.ix_mmvq_q8_0(dev(proj.pack_q8_0(wd, wq)), yq, out, n_in, n_out, B) == 0
    torch.cuda.synchronize()
    xd, _, xq = proj.q8_1_unpack(host(yq))
    assert (xd != 0).all()                                   # every block is a real one
    ref, sc = proj.q8_0_ref(wd, wq, xd.reshape(B, -1), xq.reshape(B, n_in // 32, 32))
    assert float(np.max(np.abs(host(out).astype(np.float64) - ref) / sc)) <= 1e-5
