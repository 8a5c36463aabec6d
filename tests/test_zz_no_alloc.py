"""GPU check of ix_gdn_decode_noalloc, the decode entry point that allocates nothing.

It runs the kernel ix_gdn_decode runs with a counter workspace, with the counters in the
library's static per-GPU array instead. So on the same inputs its outputs, state and conv
state must be bit-identical to ix_gdn_decode with a workspace, and within the decode
tolerances of the double oracle (fp32 o within 1e-3 absolute, state max|d|/max|ref| <= 1e-4,
conv state bit-exact). Two no-allocation calls run back to back, the second on a smaller
batch: the first call must leave the shared counters at zero for the second to be right.
In a fresh process (tests/noalloc_graph_child.py) the library's first call is made under
HIP graph capture; the graph's replays must match eager ix_gdn_decode bit for bit, and eager
no-allocation calls must leave the device's free memory unchanged.
"""
import ctypes
import os
import subprocess
import sys

import numpy as np
import pytest

import baloon_amd as bx
import oracle
from oracle import inputs
from tests.common import NT, TOL_O_ABS, TOL_STATE_REL, dev, host, state_from_dev, state_to_dev

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    return torch


def _outputs(cfg, B):
    torch = _torch()
    return (torch.full((B, cfg.h_v, cfg.d_v), float("nan"), dtype=torch.float32, device="cuda"),
            torch.zeros(B, cfg.h_v, cfg.d_v, dtype=torch.bfloat16, device="cuda"))


def test_noalloc_matches_workspace_decode_on_two_calls():
    torch = _torch()
    cfg = bx.make_cfg()
    cases = [(64, inputs.seed_for(2) + 500), (5, inputs.seed_for(2) + 501)]     # the second smaller
    runs = []
    for B, seed in cases:
        p = inputs.layer_params(cfg, seed)
        s = inputs.initial_states(cfg, seed, B)
        t = inputs.token_inputs(cfg, seed, B)
        d = dict(p=p, s=s, t=t, B=B, w=dev(p["w"]), A=dev(p["A_log"]), dt=dev(p["dt_bias"]), x=dev(t["x"]),
                 a=dev(t["a"]), b=dev(t["b"]))
        d["cs_n"], d["st_n"] = dev(s["conv_state"]), state_to_dev(s["state"])
        d["cs_w"], d["st_w"] = dev(s["conv_state"]), state_to_dev(s["state"])
        d["o_n"], d["ob_n"] = _outputs(cfg, B)
        d["o_w"], d["ob_w"] = _outputs(cfg, B)
        runs.append(d)
    # the two no-allocation calls, back to back on one stream
    for d in runs:
        rc = bx.ix_gdn_decode_noalloc(cfg, d["B"], d["x"], d["cs_n"], d["w"], d["a"], d["b"], d["A"], d["dt"],
                                      d["st_n"], d["o_n"], d["ob_n"])
        assert rc == 0, rc
    torch.cuda.synchronize()
    for d in runs:
        B = d["B"]
        ws = torch.zeros(bx.ix_gdn_decode_workspace_size(cfg, B), dtype=torch.uint8, device="cuda")
        assert bx.ix_gdn_decode(cfg, B, d["x"], d["cs_w"], d["w"], d["a"], d["b"], d["A"], d["dt"], d["st_w"],
                                d["o_w"], d["ob_w"], ws) == 0
        torch.cuda.synchronize()
        for n, w in (("o", "o"), ("ob", "ob"), ("st", "st"), ("cs", "cs")):
            np.testing.assert_array_equal(host(d[f"{n}_n"]), host(d[f"{w}_w"]), err_msg=f"B={B} {n}")
        cs_r, st_r, o_r = oracle.decode(cfg, B, d["t"]["x"], d["s"]["conv_state"], d["p"]["w"], d["t"]["a"],
                                        d["t"]["b"], d["p"]["A_log"], d["p"]["dt_bias"], d["s"]["state"], nthreads=NT)
        assert float(np.max(np.abs(host(d["o_n"]) - o_r))) <= TOL_O_ABS
        assert oracle.rel_err(state_from_dev(d["st_n"]), st_r) <= TOL_STATE_REL
        np.testing.assert_array_equal(host(d["cs_n"]), cs_r)


def test_noalloc_rejects_batches_beyond_its_array():
    # 65536 counters: B * h_k above that is refused before any launch.
    L = bx.lib()
    p = ctypes.c_void_p(1 << 20)
    big = bx.make_cfg(h_k=2, h_v=4)
    args = (p, p, p, p, p, p, p, p, None, None, None)
    assert L.ix_gdn_decode_noalloc(ctypes.byref(big), 32769, *args) == bx.HIP_ERROR_INVALID_VALUE
    assert L.ix_gdn_decode_noalloc(ctypes.byref(bx.make_cfg(d_k=64)), 1, *args) == bx.HIP_ERROR_INVALID_VALUE


def test_noalloc_first_call_under_graph_capture_in_a_fresh_process():
    child = os.path.join(os.path.dirname(os.path.abspath(__file__)), "noalloc_graph_child.py")
    r = subprocess.run([sys.executable, "-u", child], capture_output=True, text=True, timeout=110)
    print(r.stdout)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok"), r.stdout + r.stderr
    assert r.stdout.count("bit-identical to eager ix_gdn_decode") == 3
