"""GPU parity of the gated output norm fused into the layer calls (ix_gdn_decode_gated,
ix_gdn_prefill_gated): y = o / sqrt(mean(o^2) + eps) * ssm_norm * sigmoid(z) per (row, head),
the semantics of ix_gdn_out_norm (src/ix_gdn.cu:87-100).

Tolerances (written here): y within max|d|/max|ref| <= 1e-5 of the double oracle applied to
the kernel's own fp32 outputs (the reference's out_norm bound, tests/test_gdn.cu:51); y within
1e-4 of the oracle's end-to-end y (norm of the double recurrence's outputs), the state bound;
bf16 y bit-exact RNE of the fp32 y; the recurrence (o, state, conv state) bit-identical to the
ungated call of the same kernel; the counter sections of the decode workspace left zero.
"""
import numpy as np
import pytest

import baloon_amd as bx
import oracle
from oracle import bf16, inputs
from tests.common import NT, TOL_O_ABS, TOL_STATE_REL, dev, host, state_from_dev, state_to_dev

pytestmark = pytest.mark.gpu
EPS = 1e-6
TOL_Y_OWN = 1e-5
TOL_Y_E2E = 1e-4


def _torch():
    import torch
    return torch


def counters_zero(ws, cfg, B):
    w = host(ws)
    assert w.size >= B * cfg.h_k * 4                  # one int32 counter per (sequence, q/k head)
    return not w.any()


class Layer:
    def __init__(self, cfg, B, seed, ws=True):
        torch = _torch()
        self.cfg, self.B, self.seed = cfg, B, seed
        self.p = inputs.layer_params(cfg, seed)
        st = inputs.initial_states(cfg, seed, B)
        self.cs, self.st = st["conv_state"], st["state"].astype(np.float64)
        self.d_w, self.d_A, self.d_dt = dev(self.p["w"]), dev(self.p["A_log"]), dev(self.p["dt_bias"])
        self.d_cs, self.d_st = dev(st["conv_state"]), state_to_dev(st["state"])
        self.ws = torch.zeros(bx.ix_gdn_decode_workspace_size(cfg, B), dtype=torch.uint8, device="cuda") if ws else None

    def decode(self, t, g, gated=True, want_o=True):
        torch = _torch()
        cfg, B = self.cfg, self.B
        o = torch.empty(B, cfg.h_v, cfg.d_v, dtype=torch.float32, device="cuda") if want_o else None
        y = torch.full((B, cfg.h_v, cfg.d_v), float("nan"), dtype=torch.float32, device="cuda")
        yb = torch.zeros(B, cfg.h_v, cfg.d_v, dtype=torch.bfloat16, device="cuda")
        args = (cfg, B, dev(t["x"]), self.d_cs, self.d_w, dev(t["a"]), dev(t["b"]), self.d_A, self.d_dt, self.d_st)
        if gated:
            d_z, d_n = dev(g["z"]), dev(g["nrm"])
            gate = bx.out_gate(d_z, d_n, EPS, y, yb)
            assert bx.ix_gdn_decode_gated(*args, o=o, gate=gate, workspace=self.ws) == 0
        else:
            assert bx.ix_gdn_decode(*args, o=o, workspace=self.ws) == 0
        torch.cuda.synchronize()
        return (host(o) if want_o else None), host(y), host(yb)

    def oracle_step(self, t):
        cfg, B = self.cfg, self.B
        self.cs, self.st, ro = oracle.decode(cfg, B, t["x"], self.cs, self.p["w"], t["a"], t["b"], self.p["A_log"],
                                             self.p["dt_bias"], self.st, nthreads=NT)
        return ro


WS = [pytest.param(True, id="workspace"), pytest.param(False, id="no_workspace")]


@pytest.mark.parametrize("ws", WS)
@pytest.mark.parametrize("kw,B", [({}, 16), ({}, 1), (dict(h_k=4, h_v=12, head_map=1), 3),
                                  (dict(h_k=3, h_v=8), 2), (dict(h_k=1, h_v=16), 2), (dict(h_k=2, h_v=18), 2)])
def test_decode_gated_matches_out_norm(kw, B, ws):
    cfg = bx.make_cfg(**kw)
    seed = inputs.seed_for(2) + 31 + B
    g_run, p_run = Layer(cfg, B, seed, ws), Layer(cfg, B, seed, ws)
    for k in range(3):
        t = inputs.token_inputs(cfg, seed, B, step=k)
        g = inputs.out_gate_inputs(cfg, seed, B, step=k)
        o, y, yb = g_run.decode(t, g)
        o_plain, _, _ = p_run.decode(t, g, gated=False)
        ro = g_run.oracle_step(t)
        np.testing.assert_array_equal(o, o_plain)                    # the recurrence is unchanged
        assert float(np.max(np.abs(o - ro))) <= TOL_O_ABS
        own = oracle.rel_err(y, oracle.gated_out(o, g["z"], g["nrm"], EPS))
        assert own <= TOL_Y_OWN, f"step {k}: y vs norm of own o {own}"
        e2e = oracle.rel_err(y, oracle.gated_out(ro, g["z"], g["nrm"], EPS))
        assert e2e <= TOL_Y_E2E, f"step {k}: y vs oracle {e2e}"
        np.testing.assert_array_equal(yb, bf16.from_f32(y))
    np.testing.assert_array_equal(host(g_run.d_st), host(p_run.d_st))
    np.testing.assert_array_equal(host(g_run.d_cs), g_run.cs)
    assert oracle.rel_err(state_from_dev(g_run.d_st), g_run.st) <= TOL_STATE_REL
    if ws:
        assert counters_zero(g_run.ws, cfg, B)


def test_decode_gated_kernels_agree_and_o_optional():
    # Both kernels give the same y within fp32 rounding of their (differently ordered) o; the
    # workspace kernel's y does not depend on which workgroup of a group finishes last, so
    # repeated runs are bit-identical; o may be omitted.
    cfg = bx.make_cfg()
    B, seed = 8, inputs.seed_for(2) + 77
    runs = [Layer(cfg, B, seed, True), Layer(cfg, B, seed, True), Layer(cfg, B, seed, False)]
    t = inputs.token_inputs(cfg, seed, B)
    g = inputs.out_gate_inputs(cfg, seed, B)
    _, y0, yb0 = runs[0].decode(t, g)
    _, y1, yb1 = runs[1].decode(t, g, want_o=False)
    _, y2, _ = runs[2].decode(t, g)
    np.testing.assert_array_equal(y0, y1)
    np.testing.assert_array_equal(yb0, yb1)
    assert oracle.rel_err(y2, y0) <= TOL_Y_OWN


def test_prefill_gated_matches_out_norm():
    torch = _torch()
    cfg = bx.make_cfg()
    seed = inputs.seed_for(3) + 41
    cu = np.array([0, 70, 71, 150, 350], np.int32)
    n, T = cu.size - 1, int(cu[-1])
    p = inputs.layer_params(cfg, seed)
    tok = inputs.token_inputs(cfg, seed, T)
    st = inputs.initial_states(cfg, seed, n)
    g = inputs.out_gate_inputs(cfg, seed, T)
    d_w, d_A, d_dt, d_cu = dev(p["w"]), dev(p["A_log"]), dev(p["dt_bias"]), dev(cu)
    d_z, d_n = dev(g["z"]), dev(g["nrm"])
    need = bx.ix_gdn_prefill_gated_workspace_size(cfg, n, T)
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    res = []
    for with_o in (True, False, None):          # gated with o, gated without o, plain
        d_cs, d_st = dev(st["conv_state"]), state_to_dev(st["state"])
        o = torch.empty(T, cfg.h_v, cfg.d_v, dtype=torch.float32, device="cuda") if with_o in (True, None) else None
        y = torch.full((T, cfg.h_v, cfg.d_v), float("nan"), dtype=torch.float32, device="cuda")
        yb = torch.zeros(T, cfg.h_v, cfg.d_v, dtype=torch.bfloat16, device="cuda")
        args = (cfg, n, T, d_cu, dev(tok["x"]), d_cs, d_w, dev(tok["a"]), dev(tok["b"]), d_A, d_dt, d_st)
        if with_o is None:
            rc = bx.ix_gdn_prefill(*args, o=o, workspace=ws, workspace_bytes=need)
        else:
            rc = bx.ix_gdn_prefill_gated(*args, o=o, gate=bx.out_gate(d_z, d_n, EPS, y, yb), workspace=ws,
                                         workspace_bytes=need)
        assert rc == 0
        torch.cuda.synchronize()
        res.append((host(o) if o is not None else None, host(y), host(yb), host(d_cs), host(d_st)))
    (o, y, yb, cs, s), (_, y_no, yb_no, cs_no, s_no), (o_pl, _, _, cs_pl, s_pl) = res
    np.testing.assert_array_equal(o, o_pl)
    np.testing.assert_array_equal(s, s_pl)
    np.testing.assert_array_equal(cs, cs_pl)
    np.testing.assert_array_equal(y, y_no)
    np.testing.assert_array_equal(yb, yb_no)
    np.testing.assert_array_equal(yb, bf16.from_f32(y))
    assert oracle.rel_err(y, oracle.gated_out(o, g["z"], g["nrm"], EPS)) <= TOL_Y_OWN
    _, _, ro = oracle.prefill(cfg, cu, tok["x"], st["conv_state"], p["w"], tok["a"], tok["b"], p["A_log"],
                              p["dt_bias"], st["state"], nthreads=NT)
    assert oracle.rel_err(y, oracle.gated_out(ro, g["z"], g["nrm"], EPS)) <= TOL_Y_E2E
    # Without o, a workspace of a few chunks' windows (the norm's fp32 input held one window at
    # a time) gives the same y and states bit for bit.
    for window in (1, 2):
        wneed = bx.ix_gdn_prefill_window_workspace_size(cfg, n, T, window, gated=True)
        assert 0 < wneed < need
        wws = torch.empty(wneed, dtype=torch.uint8, device="cuda")
        d_cs, d_st = dev(st["conv_state"]), state_to_dev(st["state"])
        y_w = torch.full((T, cfg.h_v, cfg.d_v), float("nan"), dtype=torch.float32, device="cuda")
        yb_w = torch.zeros(T, cfg.h_v, cfg.d_v, dtype=torch.bfloat16, device="cuda")
        rc = bx.ix_gdn_prefill_gated(cfg, n, T, d_cu, dev(tok["x"]), d_cs, d_w, dev(tok["a"]), dev(tok["b"]), d_A,
                                     d_dt, d_st, o=None, gate=bx.out_gate(d_z, d_n, EPS, y_w, yb_w), workspace=wws,
                                     workspace_bytes=wneed)
        assert rc == 0
        torch.cuda.synchronize()
        np.testing.assert_array_equal(host(y_w), y_no, err_msg=f"window {window}")
        np.testing.assert_array_equal(host(yb_w), yb_no)
        np.testing.assert_array_equal(host(d_st), s_no)
        np.testing.assert_array_equal(host(d_cs), cs_no)
