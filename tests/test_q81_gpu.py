"""q8_1 output of the GDN path (GPU): the standalone quantiser against the CPU restatement
(oracle/proj.py q8_1_quantize) byte for byte; the gated calls' fused y_q8_1 against the
standalone quantiser applied to their own fp32 y, byte for byte over more than 1e7 values (the
rule of QFUSE_PARITY_NOTES.md:2-3: every q8_1 producer shares one division,
src/ix_q81_div.h:1-9); and the quantised GDN output fed to the Q8_0 out-projection product."""
import numpy as np
import pytest

import baloon_amd as bx
import oracle
from oracle import inputs, proj
from oracle.inputs import Gen
from tests.common import dev, host, state_to_dev
from tests.test_gated_gpu import EPS, Layer

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    return torch


def quantize(x_dev):
    torch = _torch()
    n = x_dev.numel()
    out = torch.full((n // 32 * 36,), 0xA5, dtype=torch.uint8, device="cuda")
    assert bx.ix_q8_1_quantize(x_dev, out, n) == 0
    torch.cuda.synchronize()
    return host(out)


@pytest.mark.parametrize("nb", [1, 2, 1001, 200003])
def test_quantize_matches_oracle(nb):
    g = Gen(0x6D4E0500 + nb)
    scale = np.exp(g.normal(1, (nb, 1)) * 2).astype(np.float32)
    x = (g.normal(2, (nb, 32)) * scale).astype(np.float32)
    if nb > 2:
        x[1] = 0.0                                                     # an all-zero block
        x[2] = 0.0
        x[2, :4] = [127.0, 2.5, -2.5, -0.5]                            # exact ties: d = 1
        x[3] = 0.0
        x[3, :2] = [1e-44, -1e-45]                                     # d = max/127 underflows to 0
    if nb > 6:
        x[4] = 0.0
        x[4, :4] = [1e7, -1e7, 3 * 65504.0, -0.5 * 65504.0]            # d clamped to 65504, codes saturate
        x[5] = 0.0
        x[5, :2] = [3e38, 3e38]                                        # fp32 sum overflows: s clamped
        x[6] = 0.0
        x[6, :2] = [127 * 65504.0, -2 * 65504.0]                       # the largest unclamped d
    got = quantize(dev(x.reshape(-1)))
    want = proj.q8_1_quantize(x.reshape(-1))
    np.testing.assert_array_equal(got, want)


def test_quantize_validation():
    torch = _torch()
    x = torch.zeros(64, dtype=torch.float32, device="cuda")
    y = torch.zeros(72, dtype=torch.uint8, device="cuda")
    INVALID = 1
    assert bx.ix_q8_1_quantize(x, y, 0) == INVALID
    assert bx.ix_q8_1_quantize(x, y, 48) == INVALID                   # not a multiple of 32
    assert bx.ix_q8_1_quantize(None, y, 64) == INVALID
    assert bx.ix_q8_1_quantize(x, y[1:], 64) == INVALID               # 4-byte alignment of the blocks


def _gated_decode_q81(cfg, B, seed, ws):
    torch = _torch()
    run = Layer(cfg, B, seed, ws)
    t = inputs.token_inputs(cfg, seed, B)
    g = inputs.out_gate_inputs(cfg, seed, B)
    y = torch.empty(B, cfg.h_v, cfg.d_v, dtype=torch.float32, device="cuda")
    yq = torch.full((B * cfg.h_v * cfg.d_v // 32 * 36,), 0xA5, dtype=torch.uint8, device="cuda")
    args = (cfg, B, dev(t["x"]), run.d_cs, run.d_w, dev(t["a"]), dev(t["b"]), run.d_A, run.d_dt, run.d_st)
    gate = bx.out_gate(dev(g["z"]), dev(g["nrm"]), EPS, y, None, yq)
    assert bx.ix_gdn_decode_gated(*args, gate=gate, workspace=run.ws) == 0
    torch.cuda.synchronize()
    return y, host(yq)


@pytest.mark.parametrize("ws", [True, False], ids=["head_kernel", "group_kernel"])
@pytest.mark.parametrize("kw,B", [({}, 64), ({}, 1), (dict(h_k=2, h_v=18), 3)])
def test_decode_fused_equals_separate(kw, B, ws):
    cfg = bx.make_cfg(**kw)
    y, yq = _gated_decode_q81(cfg, B, inputs.seed_for(2) + 501 + B, ws)
    np.testing.assert_array_equal(yq, quantize(y.reshape(-1)))
    np.testing.assert_array_equal(yq, proj.q8_1_quantize(host(y).reshape(-1)))


def test_prefill_fused_equals_separate_over_1e7_values():
    # T = 4096 tokens x 32 heads x 128 = 16.8 M values through the prefill's gated epilogue.
    torch = _torch()
    cfg = bx.make_cfg()
    seed = inputs.seed_for(3) + 503
    T = 4096
    cu = np.array([0, 1500, 1501, T], np.int32)
    n = cu.size - 1
    p = inputs.layer_params(cfg, seed)
    tok = inputs.token_inputs(cfg, seed, T)
    st = inputs.initial_states(cfg, seed, n)
    g = inputs.out_gate_inputs(cfg, seed, T)
    need = bx.ix_gdn_prefill_gated_workspace_size(cfg, n, T)
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    y = torch.empty(T, cfg.h_v, cfg.d_v, dtype=torch.float32, device="cuda")
    yq = torch.full((T * cfg.h_v * cfg.d_v // 32 * 36,), 0xA5, dtype=torch.uint8, device="cuda")
    args = (cfg, n, T, dev(cu), dev(tok["x"]), dev(st["conv_state"]), dev(p["w"]), dev(tok["a"]), dev(tok["b"]),
            dev(p["A_log"]), dev(p["dt_bias"]), state_to_dev(st["state"]))
    gate = bx.out_gate(dev(g["z"]), dev(g["nrm"]), EPS, y, None, yq)
    assert bx.ix_gdn_prefill_gated(*args, gate=gate, workspace=ws, workspace_bytes=need) == 0
    torch.cuda.synchronize()
    got = host(yq)
    assert y.numel() >= 10_000_000
    np.testing.assert_array_equal(got, quantize(y.reshape(-1)))
    np.testing.assert_array_equal(got, proj.q8_1_quantize(host(y).reshape(-1)))


def test_gdn_output_feeds_q8_0_product():
    # The gated decode's q8_1 output is the activation of the Q8_0 out-projection
    # (n_in = h_v * d_v): checked against the double reference of the product on the decoded
    # blocks (tests/mmvq_wave_ref.h:37-47 norm, 1e-5 of the scale), and against the fp32 y.
    torch = _torch()
    cfg = bx.make_cfg()
    B, n_out = 8, 333
    y, yq = _gated_decode_q81(cfg, B, inputs.seed_for(2) + 509, True)
    n_in = cfg.h_v * cfg.d_v
    wd, wq = proj.q8_blocks(0x6D4E0509, 1, n_out, n_in // 32)
    out = torch.empty(B, n_out, dtype=torch.float32, device="cuda")
    assert bx.ix_mmvq_q8_0(dev(proj.pack_q8_0(wd, wq)), dev(yq), out, n_in, n_out, B) == 0
    torch.cuda.synchronize()
    xd, _, xq = proj.q8_1_unpack(yq)
    ref, sc = proj.q8_0_ref(wd, wq, xd.reshape(B, -1), xq.reshape(B, n_in // 32, 32))
    got = host(out).astype(np.float64)
    assert float(np.max(np.abs(got - ref) / sc)) <= 1e-5
    # Only the activations' quantisation separates it from the fp32 y: per value
    # |y - q d16| <= d32 / 2 + 127 |d32 - d16| <= (1/2 + 127 * 2^-11) d32 < 0.57 d16.
    wf = (wq.astype(np.float64) * wd.view(np.float16).astype(np.float64)[..., None]).reshape(n_out, n_in)
    exact = host(y).reshape(B, n_in).astype(np.float64) @ wf.T
    bound = (np.abs(wf) @ np.repeat(xd.view(np.float16).astype(np.float64).reshape(B, -1), 32, axis=1).T).T * 0.57
    assert (np.abs(ref - exact) <= bound + 1e-9).all()
