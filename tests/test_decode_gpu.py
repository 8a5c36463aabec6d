"""GPU parity of the fused batched decode (ix_gdn_decode) against the oracle.

Tolerances (written here, from the benchmark's acceptance rule): fp32 outputs within 1e-3
absolute of the double oracle; bf16 outputs bit-exact round-to-nearest-even of the kernel's
own fp32 outputs, and within 1e-3 absolute of the oracle beyond bf16's own half-ulp
rounding; fp32 state max|d|/max|ref| <= 1e-4 after the steps (the reference's norm,
tests/test_gdn.cu:10-13); conv state bit-exact. Both kernels are covered: with a counter workspace (many short
workgroups, the q/k conv history written by the last member of each group) and without.
"""
import os

import numpy as np
import pytest

import baloon_amd as bx
import oracle
from oracle import bf16, inputs
from tests.common import (NT, TOL_O_ABS, TOL_STATE_REL, bf16_excess_err, dev, extreme_gates, extreme_params, host,
                          state_from_dev, state_to_dev)

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    return torch


class Run:
    """Device copies of one layer's parameters and states, plus the oracle's copies."""

    def __init__(self, cfg, B, seed, state_std=0.02, conv_std=1.0, ws=True, extreme=False):
        torch = _torch()
        self.cfg, self.B, self.seed = cfg, B, seed
        self.p = inputs.layer_params(cfg, seed)
        if extreme:
            self.p = extreme_params(self.p)
        s = inputs.initial_states(cfg, seed, B, state_std=state_std, conv_std=conv_std)
        self.cs, self.st = s["conv_state"], s["state"].astype(np.float64)
        self.d_w, self.d_A, self.d_dt = dev(self.p["w"]), dev(self.p["A_log"]), dev(self.p["dt_bias"])
        self.d_cs, self.d_st = dev(s["conv_state"]), state_to_dev(s["state"])
        self.ws = (torch.zeros(bx.ix_gdn_decode_workspace_size(cfg, B), dtype=torch.uint8, device="cuda")
                   if ws else None)

    def step(self, t, step_idx):
        torch = _torch()
        cfg, B = self.cfg, self.B
        o = torch.empty(B, cfg.h_v, cfg.d_v, dtype=torch.float32, device="cuda")
        ob = torch.empty(B, cfg.h_v, cfg.d_v, dtype=torch.bfloat16, device="cuda")
        rc = bx.ix_gdn_decode(cfg, B, dev(t["x"]), self.d_cs, self.d_w, dev(t["a"]), dev(t["b"]), self.d_A,
                              self.d_dt, self.d_st, o, ob, self.ws)
        assert rc == 0
        self.cs, self.st, ro = oracle.decode(cfg, B, t["x"], self.cs, self.p["w"], t["a"], t["b"], self.p["A_log"],
                                             self.p["dt_bias"], self.st, nthreads=NT)
        torch.cuda.synchronize()
        return host(o), host(ob), ro

    def check_outputs(self, o, ob, ro, where=""):
        err = float(np.max(np.abs(o - ro)))
        assert err <= TOL_O_ABS, f"{where} o abs err {err}"
        np.testing.assert_array_equal(ob, bf16.from_f32(o), err_msg=f"{where} bf16 o is not RNE(fp32 o)")
        ex = bf16_excess_err(ob, ro)
        assert ex <= TOL_O_ABS, f"{where} bf16 o err beyond rounding {ex}"

    def check_states(self, where=""):
        rel = oracle.rel_err(state_from_dev(self.d_st), self.st)
        assert rel <= TOL_STATE_REL, f"{where} state rel err {rel}"
        np.testing.assert_array_equal(host(self.d_cs), self.cs)
        if self.ws is not None:
            assert int(self.ws.count_nonzero()) == 0, "counter workspace not left zeroed"


def run_steps(cfg, B, steps, seed, check_every=1, extreme=False, **kw):
    r = Run(cfg, B, seed, extreme=extreme, **kw)
    for s in range(steps):
        t = inputs.token_inputs(cfg, seed, B, step=s)
        if extreme:
            t = extreme_gates(cfg, t, seed + s)
        o, ob, ro = r.step(t, s)
        if (s + 1) % check_every == 0 or s == steps - 1:
            r.check_outputs(o, ob, ro, f"step {s}")
    r.check_states(f"after {steps} steps")
    return r


WS = [pytest.param(True, id="workspace"), pytest.param(False, id="no_workspace")]


@pytest.mark.parametrize("ws", WS)
def test_config1_single_token(ws):
    # B=1, 16 q/k heads, 32 v heads, d=128, fused conv over 8192 channels.
    run_steps(oracle.make_cfg(), 1, 1, inputs.seed_for(1), ws=ws)


@pytest.mark.parametrize("B", [1, 2, 3, 4, 5])
def test_small_batches(B):
    # Configuration 1's batch and its neighbours, over several carried steps: at small B the
    # workspace kernel runs fewer workgroups than the chip has CUs (B <= 4 on 256 CUs: the
    # 512-thread workgroups; B = 5: the 256-thread ones), and each group counter and conv
    # history still has to come out right every step.
    run_steps(oracle.make_cfg(), B, 6, inputs.seed_for(1) + 200 + B, ws=True)


@pytest.mark.parametrize("ws", WS)
def test_config2_batch64_256_steps(ws):
    # Configuration 2 as stated: B=64 independent sequences, 256 consecutive decode steps with
    # state carry-over; outputs checked every 32 steps, states and conv states at the end.
    run_steps(oracle.make_cfg(), 64, 256, inputs.seed_for(2), check_every=32, ws=ws)


@pytest.mark.parametrize("ws", WS)
def test_extreme_gates(ws):
    # Gate logits past softplus's threshold on both sides (a + dt_bias > 20: softplus(x) = x,
    # a log decay near -400 whose exp underflows to 0 with A_log = ln 16; a + dt_bias < -20:
    # decay ~1) and beta logits at +-30, at seeded positions among ordinary tokens.
    run_steps(oracle.make_cfg(), 4, 12, inputs.seed_for(2) + 300, extreme=True, ws=ws)


@pytest.mark.parametrize("ws", WS)
def test_long_carry_256_steps_small_batch(ws):
    run_steps(oracle.make_cfg(), 2, 256, inputs.seed_for(2) + 100, check_every=32, ws=ws)


@pytest.mark.parametrize("kw", [
    dict(head_map=1),
    dict(conv_act=1),
    dict(q_scale=128 ** -0.5),
    dict(d_conv=2),
    dict(d_conv=3),
    dict(h_k=3, h_v=8),              # uneven modulo groups (3, 3, 2 heads per src)
    dict(h_k=4, h_v=2),              # src 2, 3 own no v head; their q/k conv state still rolls
    dict(h_k=2, h_v=6, head_map=1),  # 3 v heads per src: two passes of the 2-tile workgroup
    dict(h_k=1, h_v=5),
    dict(l2_eps=1e-3),
    dict(h_k=1, h_v=16),             # 16 v heads on one q/k head: the configuration limit
    dict(h_k=2, h_v=32, head_map=1), # 16 per source with the contiguous map
    dict(h_k=2, h_v=18),             # 9 per source (more than 8) with modulo pairing
])
@pytest.mark.parametrize("ws", WS)
def test_variants(kw, ws):
    cfg = oracle.make_cfg(**kw)
    run_steps(cfg, 3, 4, inputs.seed_for(1) + 7 * len(kw), ws=ws)


def test_config0_golden_identity_conv():
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "config0.npz"))
    torch = _torch()
    cfg = bx.make_cfg(h_k=1, h_v=1, d_conv=2)
    C = cfg.channels
    d_w, d_A, d_dt = dev(g["w"]), dev(g["A_log"]), dev(g["dt_bias"])
    d_st = state_to_dev(g["state0"])
    d_cs = torch.zeros(1, C, 1, dtype=torch.bfloat16, device="cuda")
    o = torch.empty(1, 1, 128, dtype=torch.float32, device="cuda")
    ws = torch.zeros(bx.ix_gdn_decode_workspace_size(cfg, 1), dtype=torch.uint8, device="cuda")
    outs = []
    for t in range(g["x"].shape[0]):
        assert bx.ix_gdn_decode(cfg, 1, dev(g["x"][t:t + 1]), d_cs, d_w, dev(g["a"][t:t + 1]), dev(g["b"][t:t + 1]),
                                d_A, d_dt, d_st, o, None, ws) == 0
        outs.append(host(o).copy())
    torch.cuda.synchronize()
    got = np.concatenate(outs)
    assert float(np.max(np.abs(got - g["o"]))) <= TOL_O_ABS
    assert oracle.rel_err(state_from_dev(d_st), g["state"]) <= TOL_STATE_REL


def test_deterministic_and_null_outputs():
    torch = _torch()
    cfg = bx.make_cfg()
    seed = inputs.seed_for(2) + 5
    res = []
    for _ in range(2):
        r = Run(cfg, 8, seed)
        t = inputs.token_inputs(cfg, seed, 8)
        o = torch.empty(8, 32, 128, dtype=torch.float32, device="cuda")
        assert bx.ix_gdn_decode(cfg, 8, dev(t["x"]), r.d_cs, r.d_w, dev(t["a"]), dev(t["b"]), r.d_A, r.d_dt,
                                r.d_st, o, None, r.ws) == 0
        torch.cuda.synchronize()
        res.append((host(o).copy(), host(r.d_st).copy()))
    np.testing.assert_array_equal(res[0][0], res[1][0])
    np.testing.assert_array_equal(res[0][1], res[1][1])
    # no outputs at all: state still advances identically
    r = Run(cfg, 8, seed)
    t = inputs.token_inputs(cfg, seed, 8)
    assert bx.ix_gdn_decode(cfg, 8, dev(t["x"]), r.d_cs, r.d_w, dev(t["a"]), dev(t["b"]), r.d_A, r.d_dt,
                            r.d_st, None, None, r.ws) == 0
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(r.d_st), res[0][1])


def test_bf16_output_is_rne_of_fp32_output():
    torch = _torch()
    cfg = bx.make_cfg()
    seed = inputs.seed_for(1) + 3
    r = Run(cfg, 4, seed)
    t = inputs.token_inputs(cfg, seed, 4)
    o = torch.empty(4, 32, 128, dtype=torch.float32, device="cuda")
    ob = torch.empty(4, 32, 128, dtype=torch.bfloat16, device="cuda")
    assert bx.ix_gdn_decode(cfg, 4, dev(t["x"]), r.d_cs, r.d_w, dev(t["a"]), dev(t["b"]), r.d_A, r.d_dt, r.d_st,
                            o, ob, r.ws) == 0
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(ob), bf16.from_f32(host(o)))


def test_workspace_and_group_kernels_agree():
    # Same inputs through both kernels: conv states bit-identical, outputs and states within
    # fp32 rounding of each other (their reductions are ordered differently).
    cfg = bx.make_cfg()
    seed = inputs.seed_for(2) + 17
    ra, rb = Run(cfg, 16, seed, ws=True), Run(cfg, 16, seed, ws=False)
    for k in range(3):
        t = inputs.token_inputs(cfg, seed, 16, step=k)
        oa, _, ro = ra.step(t, k)
        ob, _, _ = rb.step(t, k)
        assert float(np.max(np.abs(oa - ob))) <= 1e-5
    np.testing.assert_array_equal(host(ra.d_cs), host(rb.d_cs))
    assert oracle.rel_err(host(ra.d_st), host(rb.d_st)) <= 1e-5


@pytest.mark.parametrize("ws", WS)
def test_graph_replays_match_eager(ws):
    # K decode calls captured once in a HIP graph (each records one kernel and no memset) and
    # replayed three times, the states restored by eager copies between replays: every replay
    # gives the eager calls' outputs and states bit for bit.
    torch = _torch()
    cfg = bx.make_cfg()
    B, K, seed = 3, 4, inputs.seed_for(1) + 41
    r = Run(cfg, B, seed, ws=ws)
    toks = [inputs.token_inputs(cfg, seed, B, step=k) for k in range(K)]
    d_toks = [(dev(t["x"]), dev(t["a"]), dev(t["b"])) for t in toks]
    outs = [torch.empty(B, cfg.h_v, cfg.d_v, dtype=torch.float32, device="cuda") for _ in range(K)]
    cs0, st0 = r.d_cs.clone(), r.d_st.clone()

    def calls(stream):
        for k, (x, a, b) in enumerate(d_toks):
            assert bx.ix_gdn_decode(cfg, B, x, r.d_cs, r.d_w, a, b, r.d_A, r.d_dt, r.d_st, outs[k], None, r.ws,
                                    stream) == 0

    calls(torch.cuda.current_stream())
    torch.cuda.synchronize()
    eager = ([host(o).copy() for o in outs], host(r.d_cs).copy(), host(r.d_st).copy())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        calls(torch.cuda.current_stream())
    for rep in range(3):
        r.d_cs.copy_(cs0)
        r.d_st.copy_(st0)
        for o in outs:
            o.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for k in range(K):
            np.testing.assert_array_equal(host(outs[k]), eager[0][k], err_msg=f"replay {rep} output {k}")
        np.testing.assert_array_equal(host(r.d_cs), eager[1], err_msg=f"replay {rep} conv state")
        np.testing.assert_array_equal(host(r.d_st), eager[2], err_msg=f"replay {rep} state")
        if ws:
            assert int(r.ws.count_nonzero()) == 0, "counters not left zeroed"
