#!/usr/bin/env python3
"""Benchmark of the GDN path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--batch 64] [--layers 4] [--no-cpu]

Headline workload (configuration 2 of the benchmark set): batched GDN decode, B = 64
independent sequences, 16 q/k heads and 32 v heads, d_k = d_v = 128, fp32 state 128 MiB per
layer, fused conv (4 taps over 8192 channels), one ix_gdn_decode launch per step. A "step" is
one decode token for all B sequences of one layer; steps rotate over --layers independent
layers (state, conv state, weights), so the working set (4 x 128 MiB) exceeds the 256 MB
Infinity Cache and the state really streams from HBM. Inputs are resident in HBM before the
timed region, which is bracketed by HIP events on the launch stream.

Also reported on the same line: decode latency at B = 1 (configuration 1), eager and as a
captured HIP graph; the gated decode, the speculative window and the input projection at the
decode batch; chunked prefill of one 4096-token sequence (configuration 3) with its MFMA
roofline fraction; the measured in-place HBM ceiling of the box.

The cpu_baseline leg is the only code here that uses oracle/ (the CPU restatement of the
reference's recurrence, test infrastructure). It generates the seeded inputs every GPU leg
runs on (oracle/inputs.py, the generator the tests use), replays each timed decode and
prefill sequence on this host's cores -- those replays are the CPU baseline -- and checks the
GPU's results against them: the states after the timed region and the last outputs of every
decode leg, the prefill's outputs and final state, one window and one projection call. A
mismatch is a failed gate: the bench then prints no JSON line and exits with status 3.
Nothing from oracle/ runs inside a timed GPU region.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E spec
MFMA_BF16_PEAK_TFLOPS = 2500.0 # MI355X dense bf16 spec
STATE_TILE = 128 * 128 * 4     # bytes per (sequence, v head)
PREFILL_FLOP_PER_TOKEN = 5_767_168     # 2C^2(3d_k+2d_v) + 6 C d_k d_v per (v head, chunk of 64) / 64, x 32 heads
TOL_O_ABS = 1e-3               # fp32 outputs vs the double oracle (bf16 outputs: beyond their own rounding)
TOL_STATE_REL = 1e-4           # fp32 state: max|d| / max|ref|
TOL_Y_REL = 1e-4               # gated output norm, end to end
TOL_PROJ = 2e-5                # projection: |y - ref| <= 2e-5 * sum |h w| per output
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "decode_traffic.json")


def parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--layers", type=int, default=4)
    ap.add_argument("--inputs", type=int, default=8, help="distinct token input sets cycled through")
    ap.add_argument("--no-cpu", action="store_true",
                    help="skip the single-core CPU samples (the multi-core replays, which gate the run, always run)")
    ap.add_argument("--legs", default="all",
                    help="comma-separated subset of decode,gated,window,in_proj,latency,prefill,prefill_varlen,"
                         "legacy,ceiling for "
                         "profiling passes; the result line needs all of them (the default)")
    a = ap.parse_args()
    known = ("decode", "gated", "window", "in_proj", "latency", "prefill", "prefill_varlen", "legacy", "ceiling")
    a.legs = set(known) if a.legs == "all" else set(a.legs.split(","))
    if not a.legs <= set(known):
        ap.error(f"--legs: unknown {sorted(a.legs - set(known))}")
    return a


def cpu_share() -> int:
    """Host threads for the CPU legs: the GPU box's CPU share is 16 whatever nproc shows."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


# ---------------------------------------------------------------------------------------------
# host <-> device plumbing
# ---------------------------------------------------------------------------------------------

def to_dev(a):
    import torch
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16).cuda()
    return torch.from_numpy(a.copy()).cuda()


def to_host(t) -> np.ndarray:
    import torch
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def state_dev(st):
    """[..][h_v][d_k][d_v] -> the library's [..][h_v][d_v][d_k] layout on the device."""
    return to_dev(np.ascontiguousarray(np.swapaxes(np.asarray(st, np.float32), -1, -2)))


def state_host(t) -> np.ndarray:
    return np.ascontiguousarray(np.swapaxes(to_host(t), -1, -2))


def bf16_f32(bits) -> np.ndarray:
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


_HEAT = {}


def heat(ms=40.0):
    """Brings the GPU to its loaded clocks: about `ms` of in-place streaming over a scratch
    buffer that nothing measured or checked reads. Started from idle, the first tens of
    milliseconds of a workload run up to ~8% slower while the clocks rise (the same decode
    launches took 46.9 us in their first 12 ms and 45.3 us after), so every timed region below
    is measured at the clocks a continuously loaded GPU runs at."""
    import torch
    if "buf" not in _HEAT:
        _HEAT["buf"] = torch.ones(64 << 20, dtype=torch.float32, device="cuda")      # 256 MiB
    buf = _HEAT["buf"]
    end = time.perf_counter() + ms / 1e3
    while time.perf_counter() < end:
        for _ in range(8):
            buf.mul_(1.0)
        torch.cuda.synchronize()


def timed(stream, fn, n):
    """n calls of fn(i) between HIP events recorded on `stream`, right after heat(); every
    status checked after. The start event is queued behind a last ~0.5 ms of the heat work,
    so that the GPU reaches it with the first calls already queued: the region times the
    GPU's work, not the host's latency in issuing the first call."""
    import torch

    import baloon_amd as bx
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    heat()
    with torch.cuda.stream(stream):
        for _ in range(4):
            _HEAT["buf"].mul_(1.0)
    e0.record(stream)
    rcs = [fn(i) for i in range(n)]
    e1.record(stream)
    torch.cuda.synchronize()
    for rc in rcs:
        bx.check("launch", rc)
    return e0.elapsed_time(e1) / 1e3          # seconds


# ---------------------------------------------------------------------------------------------
# cpu_baseline leg: the only user of oracle/ (inputs, CPU replays, the correctness gate)
# ---------------------------------------------------------------------------------------------

class CpuBaselineLeg:
    def __init__(self):
        import oracle
        from oracle import bf16, inputs, proj
        self.oracle, self.inputs, self.bf16, self.proj = oracle, inputs, bf16, proj
        self.nt = cpu_share()
        self.cfg = oracle.make_cfg()
        self.failures = []
        self.record = {}

    # ---- inputs ----
    def decode_data(self, B, L, P):
        """Per-layer parameters, the initial states (shared by the layers) and P token input
        sets for configuration 2, from seed 0x6D4E0002 (layer l: + l)."""
        inp, cfg = self.inputs, self.cfg
        seed = inp.seed_for(2)
        st = inp.initial_states(cfg, seed, B)
        return dict(
            params=[inp.layer_params(cfg, seed + l) for l in range(L)],
            state0=st["state"], cs0=st["conv_state"],
            tokens=[inp.token_inputs(cfg, seed, B, step=i) for i in range(P)],
            gate=inp.out_gate_inputs(cfg, seed, B),
        )

    def window_tokens(self, B, K):
        t = self.inputs.token_inputs(self.cfg, self.inputs.seed_for(2) + 0x51, B * K)
        return {k: v.reshape(B, K, -1) for k, v in t.items()}

    def proj_data(self, B, hidden, N):
        g = self.inputs.Gen(self.inputs.seed_for(2) + 0x61)
        h = g.normal_bf16(1, (B, hidden))
        w = self.bf16.from_f32((g.normal(2, (N, hidden)) * 0.05).astype(np.float32))
        return h, w

    def prefill_data(self, T):
        """Configuration 3's inputs (seed 0x6D4E0003), generated once."""
        if self.record.get("prefill_data", (None,))[0] != T:
            inp, cfg = self.inputs, self.cfg
            seed = inp.seed_for(3)
            self.record["prefill_data"] = (T, dict(params=inp.layer_params(cfg, seed),
                                                   tokens=inp.token_inputs(cfg, seed, T)))
        return self.record["prefill_data"][1]

    def latency_data(self):
        inp, cfg = self.inputs, self.cfg
        seed = inp.seed_for(1)
        st = inp.initial_states(cfg, seed, 1)
        return dict(params=inp.layer_params(cfg, seed), state0=st["state"], cs0=st["conv_state"],
                    tokens=[inp.token_inputs(cfg, seed, 1, step=i) for i in range(8)])

    # ---- checks ----
    def fail(self, what):
        self.failures.append(what)
        print(f"bench gate FAILED: {what}", file=sys.stderr)

    def check_bf16_out(self, what, bits, ref, tol=TOL_O_ABS):
        """bf16 outputs within tol of the double reference beyond bf16's own half-ulp rounding."""
        ref = np.asarray(ref, np.float64)
        got32 = bf16_f32(bits)
        got = got32.astype(np.float64)

        def binade(v):   # 2^e with 2^e <= |v| < 2^(e+1)
            return (np.abs(v).view(np.uint32) & np.uint32(0x7F800000)).view(np.float32).astype(np.float64)

        # half a bf16 ulp, of whichever of ref and the output lies in the higher binade (the
        # rounding may cross a power of two)
        half = np.maximum(np.maximum(binade(ref.astype(np.float32)), binade(got32)) * 2.0 ** -8, 2.0 ** -133)
        err = float(np.max(np.abs(got - ref) - half)) if ref.size else 0.0
        if not err <= tol:
            self.fail(f"{what}: bf16 output error beyond rounding {err:.3g} > {tol}")
        return err

    def check_state(self, what, got, ref):
        rel = self.oracle.rel_err(got, ref)
        if not rel <= TOL_STATE_REL:
            self.fail(f"{what}: state rel err {rel:.3g} > {TOL_STATE_REL}")
        return rel

    def check_equal(self, what, got, ref):
        if not np.array_equal(got, ref):
            self.fail(f"{what}: not bit-identical")

    # ---- decode replay (the CPU baseline and the decode gate) ----
    def replay_decode(self, D, order, L, P, B, nthreads):
        """The timed GPU sequence launch by launch: launch i is one step of layer order[i] % L
        with token set order[i] % P. Returns per-layer (conv state, state), the last output
        and the seconds spent in the oracle."""
        o_ = self.oracle
        cs = [D["cs0"].copy() for _ in range(L)]
        st = [D["state0"].astype(np.float64) for _ in range(L)]
        o_last, sec = None, 0.0
        for i in order:
            l, t, p = i % L, D["tokens"][i % P], D["params"][i % L]
            t0 = time.perf_counter()
            cs[l], st[l], o_last = o_.decode(self.cfg, B, t["x"], cs[l], p["w"], t["a"], t["b"], p["A_log"],
                                             p["dt_bias"], st[l], nthreads=nthreads)
            sec += time.perf_counter() - t0
        return cs, st, o_last, sec

    def gate_decode(self, D, order, args, res, gated_res=None):
        L, P, B = args.layers, args.inputs, args.batch
        cs, st, o_last, sec = self.replay_decode(D, order, L, P, B, self.nt)
        self.record["decode"] = dict(tokens_per_s=B * len(order) / sec, steps=len(order), sec=sec)
        errs = []
        for l in range(L):
            self.check_equal(f"decode layer {l} conv state", res["cs"][l], cs[l])
            errs.append(self.check_state(f"decode layer {l}", res["st"][l], st[l]))
        e_o = self.check_bf16_out("decode last o", res["out"], o_last)
        out = dict(state_rel_err=max(errs), o_err=e_o)
        if gated_res is not None:
            for l in range(L):
                self.check_equal(f"gated decode layer {l} state vs ungated", gated_res["st"][l], res["st"][l])
                self.check_equal(f"gated decode layer {l} conv state vs ungated", gated_res["cs"][l], res["cs"][l])
            g = D["gate"]
            y_ref = self.oracle.gated_out(o_last, g["z"], g["nrm"], 1e-6)
            y = bf16_f32(gated_res["out"]).astype(np.float64)
            half = np.abs(y_ref) * 2.0 ** -8
            y_err = float(np.max(np.maximum(np.abs(y - y_ref) - half, 0.0)) / max(np.max(np.abs(y_ref)), 1e-30))
            if not y_err <= TOL_Y_REL:
                self.fail(f"gated decode last y: rel err beyond bf16 rounding {y_err:.3g} > {TOL_Y_REL}")
            out["y_rel_err"] = y_err
        return out

    def cpu_decode_1core(self, D, args, budget_s=6.0, max_steps=16):
        """Single-thread rate on a bounded sample: launches of layer 0 until the budget is used."""
        cs, st = D["cs0"].copy(), D["state0"].astype(np.float64)
        p, steps, t0 = D["params"][0], 0, time.perf_counter()
        while steps < max_steps:
            t = D["tokens"][steps % args.inputs]
            cs, st, _ = self.oracle.decode(self.cfg, args.batch, t["x"], cs, p["w"], t["a"], t["b"], p["A_log"],
                                           p["dt_bias"], st, nthreads=1)
            steps += 1
            if time.perf_counter() - t0 >= budget_s:
                break
        return args.batch * steps / (time.perf_counter() - t0), steps

    # ---- window, projection and prefill gates ----
    def gate_window(self, D, W, B, K, o_win, cs_after, st_after, o_exact=None):
        cs, st = D["cs0"].copy(), D["state0"].astype(np.float64)
        p = D["params"][0]
        errs = []
        for t in range(K):
            cs, st, ro = self.oracle.decode(self.cfg, B, W["x"][:, t], cs, p["w"], W["a"][:, t], W["b"][:, t],
                                            p["A_log"], p["dt_bias"], st, nthreads=self.nt)
            errs.append(self.check_bf16_out(f"window token {t} o", o_win[:, t], ro))
            if o_exact is not None:
                errs.append(self.check_bf16_out(f"window (exact verify) token {t} o", o_exact[:, t], ro))
        self.check_equal("window commit conv state", cs_after, cs)
        rel = self.check_state("window commit", st_after, st)
        return dict(o_err=max(errs), state_rel_err=rel)

    def gate_proj(self, h, w, y):
        ref, mag = self.proj.in_proj_ref(h, w)
        err = float(np.max(np.abs(y.astype(np.float64) - ref) / np.maximum(mag, 1e-30)))
        if not err <= TOL_PROJ:
            self.fail(f"in_proj: error {err:.3g} x magnitude > {TOL_PROJ}")
        return err

    def gate_prefill(self, D, T, cs_gpu, st_gpu, o_gpu):
        cfg, inp = self.cfg, self.inputs
        st0 = inp.initial_states(cfg, inp.seed_for(3), 1, state_std=0.0, conv_std=0.0)
        p, tok = D["params"], D["tokens"]
        t0 = time.perf_counter()
        cs, st, o = self.oracle.prefill(cfg, [0, T], tok["x"], st0["conv_state"], p["w"], tok["a"], tok["b"],
                                        p["A_log"], p["dt_bias"], st0["state"], nthreads=self.nt)
        sec = time.perf_counter() - t0
        self.record["prefill"] = dict(tokens_per_s=T / sec, T=T, sec=sec)
        self.check_equal("prefill conv state", cs_gpu, cs)
        rel = self.check_state("prefill", st_gpu, st)
        e_o = self.check_bf16_out("prefill o", o_gpu, o)
        return dict(state_rel_err=rel, o_err=e_o)

    def varlen_data(self):
        """Configuration 4's packed prefill inputs (seed 0x6D4E0004): 32 sequences of lengths
        U[1, 2048], initial states N(0, 0.02)."""
        if "varlen_data" not in self.record:
            inp, cfg = self.inputs, self.cfg
            seed = inp.seed_for(4)
            cu = inp.varlen(seed, 32, 1, 2048)
            T = int(cu[-1])
            self.record["varlen_data"] = dict(cu=cu, T=T, params=inp.layer_params(cfg, seed),
                                              tokens=inp.token_inputs(cfg, seed, T),
                                              st0=inp.initial_states(cfg, seed, 32))
        return self.record["varlen_data"]

    def gate_prefill_varlen(self, V, cs_gpu, st_gpu, o_gpu):
        p, tok, st0 = V["params"], V["tokens"], V["st0"]
        t0 = time.perf_counter()
        cs, st, o = self.oracle.prefill(self.cfg, V["cu"], tok["x"], st0["conv_state"], p["w"], tok["a"], tok["b"],
                                        p["A_log"], p["dt_bias"], st0["state"], nthreads=self.nt)
        sec = time.perf_counter() - t0
        self.record["prefill_varlen"] = dict(tokens_per_s=V["T"] / sec, sec=sec)
        self.check_equal("varlen prefill conv state", cs_gpu, cs)
        rel = self.check_state("varlen prefill", st_gpu, st)
        e_o = self.check_bf16_out("varlen prefill o", o_gpu, o)
        return dict(state_rel_err=rel, o_err=e_o)

    def legacy_data(self):
        """The reference acceptance test's shapes (tests/test_gdn.cu:16-55): step S=128,
        h_k=16, h_v=48; conv over 8192+5 channels, d_conv 4; l2 33 x 128; out_norm 48 x 128;
        beta over 48 heads; the test's distributions, from the portable generator."""
        g = self.inputs.Gen(0x6D4E0100)
        S, hk, hv, C, dc = 128, 16, 48, 8192 + 5, 4
        return dict(
            S=S, hk=hk, hv=hv, C=C, dc=dc,
            st=g.normal_f32(1, (S * hv * S,), 0.1), q=g.normal_f32(2, (hk * S,), 0.1),
            k=g.normal_f32(3, (hk * S,), 0.1), v=g.normal_f32(4, (hv * S,)),
            gate=-np.abs(g.normal_f32(5, (hv,))), beta=(0.5 + 0.4 * np.tanh(g.normal(6, (hv,)))).astype(np.float32),
            cs=g.normal_f32(7, (C * (dc - 1),)), x=g.normal_f32(8, (C,)), w=g.normal_f32(9, (C * dc,)),
            l2=g.normal_f32(10, (33 * 128,)), o=g.normal_f32(11, (hv * S,)), z=g.normal_f32(12, (hv * S,)),
            nrm=(1.0 + 0.1 * g.normal(13, (S,))).astype(np.float32), b=g.normal_f32(14, (hv,), 3.0))

    def gate_legacy(self, L, got):
        """The reference test's norm max|gpu - ref| <= tol * max|ref| and tolerances
        (tests/test_gdn.cu:10-13, :30-31, :40-41, :46, :51, :55)."""
        o_ = self.oracle
        errs = {}

        def rel(name, g, r, tol):
            r = np.asarray(r, np.float64)
            e = float(np.max(np.abs(np.asarray(g, np.float64) - r)) / max(float(np.max(np.abs(r))), 1e-30))
            errs[name] = e
            if not e <= tol:
                self.fail(f"legacy {name}: rel err {e:.3g} > {tol}")

        rs, ro = o_.step(L["st"], L["q"], L["k"], L["v"], L["gate"], L["beta"], L["S"], L["hk"], L["hv"])
        rel("step.o", got["step_o"], ro, 1e-4)
        rel("step.state", got["step_st"], rs, 1e-4)
        rcs, rout = o_.conv_step(L["cs"], L["x"], L["w"], L["C"], L["dc"])
        rel("conv.out", got["conv_out"], rout, 1e-5)
        self.check_equal("legacy conv.state", got["conv_cs"], rcs)
        rel("l2", got["l2"], o_.l2_norm(L["l2"], 33, 128, 1e-6), 1e-6)
        rel("out_norm", got["out_norm"], o_.out_norm(L["o"], L["z"], L["nrm"], L["hv"], L["S"], 1e-6), 1e-5)
        rel("beta", got["beta"], o_.beta_gate(L["b"]), 1e-6)
        return errs

    def cpu_prefill_1core(self, D, Tp=256):
        cfg, inp = self.cfg, self.inputs
        st0 = inp.initial_states(cfg, inp.seed_for(3), 1, state_std=0.0, conv_std=0.0)
        p, tok = D["params"], D["tokens"]
        t0 = time.perf_counter()
        self.oracle.prefill(cfg, [0, Tp], tok["x"][:Tp], st0["conv_state"], p["w"], tok["a"][:Tp], tok["b"][:Tp],
                            p["A_log"], p["dt_bias"], st0["state"], nthreads=1)
        return Tp / (time.perf_counter() - t0)


# ---------------------------------------------------------------------------------------------
# GPU legs
# ---------------------------------------------------------------------------------------------

def decode_leg(args, D, gated=False):
    """B-sequence decode over rotated layers; gated=True times ix_gdn_decode_gated (the same
    step with the gated output norm fused in, y written as bf16). Launch i runs layer i % L
    with token set i % P; the warmup launches i < W, then the timed launches i < K."""
    import torch

    import baloon_amd as bx

    cfg = bx.make_cfg()
    B, L, P = args.batch, args.layers, args.inputs
    hv = cfg.h_v
    st0 = np.ascontiguousarray(np.swapaxes(D["state0"], -1, -2))
    layers = []
    for l in range(L):
        p = D["params"][l]
        layers.append(dict(w=to_dev(p["w"]), A_log=to_dev(p["A_log"]), dt=to_dev(p["dt_bias"]), state=to_dev(st0),
                           cs=to_dev(D["cs0"])))
    ins = [dict(x=to_dev(t["x"]), a=to_dev(t["a"]), b=to_dev(t["b"])) for t in D["tokens"]]
    out = torch.empty(B, hv, 128, dtype=torch.bfloat16, device="cuda")
    ws = torch.zeros(bx.ix_gdn_decode_workspace_size(cfg, B), dtype=torch.uint8, device="cuda")
    z, nrm = to_dev(D["gate"]["z"]), to_dev(D["gate"]["nrm"])
    gate = bx.out_gate(z, nrm, 1e-6, None, out)
    stream = torch.cuda.current_stream()
    lib, cfg_ref, gate_ref, s_ptr = bx.lib(), ctypes.byref(cfg), ctypes.byref(gate), stream.cuda_stream

    def launch(i):
        Ly, In = layers[i % L], ins[i % P]
        if gated:
            return lib.ix_gdn_decode_gated(cfg_ref, B, In["x"].data_ptr(), Ly["cs"].data_ptr(), Ly["w"].data_ptr(),
                                           In["a"].data_ptr(), In["b"].data_ptr(), Ly["A_log"].data_ptr(),
                                           Ly["dt"].data_ptr(), Ly["state"].data_ptr(), None, None, gate_ref,
                                           ws.data_ptr(), s_ptr)
        return lib.ix_gdn_decode(cfg_ref, B, In["x"].data_ptr(), Ly["cs"].data_ptr(), Ly["w"].data_ptr(),
                                 In["a"].data_ptr(), In["b"].data_ptr(), Ly["A_log"].data_ptr(), Ly["dt"].data_ptr(),
                                 Ly["state"].data_ptr(), None, out.data_ptr(), ws.data_ptr(), s_ptr)

    for i in range(args.warmup):
        bx.check("ix_gdn_decode", launch(i))
    sec = timed(stream, launch, args.steps)            # the timed region: K back-to-back launches
    K = args.steps
    avg_launch_s = sec / K
    state_bytes = 2 * B * hv * STATE_TILE
    achieved = state_bytes / avg_launch_s / 1e9
    res = dict(
        tokens_per_s=B * K / sec, ms_per_step=sec * 1e3 / K, avg_kernel_us=avg_launch_s * 1e6,
        state_bytes_per_launch=state_bytes,
        roofline=dict(bound="hbm", achieved=round(achieved, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                      frac=round(achieved / HBM_PEAK_GBS, 4)),
        cs=[to_host(Ly["cs"]) for Ly in layers], st=[state_host(Ly["state"]) for Ly in layers], out=to_host(out),
    )
    del layers, ins
    torch.cuda.empty_cache()
    return res


def window_leg(args, D, W, O, K=4, iters=64):
    """Speculative window at B = 64: verify K draft tokens on the matrix cores
    (ix_gdn_decode_window_mfma; the bit-exact ix_gdn_decode_window is timed beside it), then
    ix_gdn_commit_window with all K accepted (the most state work), layers rotated as in the
    decode leg. One verify of each kind and a commit on layer 0 are checked against the CPU
    replay first."""
    import torch

    import baloon_amd as bx

    cfg = bx.make_cfg()
    B, L = args.batch, args.layers
    hv = cfg.h_v
    st0 = np.ascontiguousarray(np.swapaxes(D["state0"], -1, -2))
    layers = [dict(w=to_dev(p["w"]), A_log=to_dev(p["A_log"]), dt=to_dev(p["dt_bias"]), state=to_dev(st0),
                   cs=to_dev(D["cs0"])) for p in D["params"][:L]]
    x, a, b = to_dev(W["x"]), to_dev(W["a"]), to_dev(W["b"])
    o = torch.empty(B, K, hv, 128, dtype=torch.bfloat16, device="cuda")
    rec = torch.empty(bx.ix_gdn_window_record_size(cfg, B, K), dtype=torch.uint8, device="cuda")
    acc = torch.full((B,), K, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream()

    def verify(i):
        Ly = layers[i % L]
        return bx.ix_gdn_decode_window_mfma(cfg, B, K, x, Ly["cs"], Ly["w"], a, b, Ly["A_log"], Ly["dt"],
                                            Ly["state"], None, o, rec, stream)

    def verify_exact(i):
        Ly = layers[i % L]
        return bx.ix_gdn_decode_window(cfg, B, K, x, Ly["cs"], Ly["w"], a, b, Ly["A_log"], Ly["dt"], Ly["state"],
                                       None, o, rec, stream)

    def commit(i):
        Ly = layers[i % L]
        return bx.ix_gdn_commit_window(cfg, B, K, acc, x, rec, Ly["cs"], Ly["state"], stream)

    bx.check("ix_gdn_decode_window", verify_exact(0))
    torch.cuda.synchronize()
    o_exact = to_host(o)
    bx.check("ix_gdn_decode_window_mfma", verify(0))
    bx.check("ix_gdn_commit_window", commit(0))
    torch.cuda.synchronize()
    gate = O.gate_window(D, W, B, K, to_host(o), to_host(layers[0]["cs"]), state_host(layers[0]["state"]),
                         o_exact=o_exact)
    # one launch committing the window in all L layers (ix_gdn_commit_window_layers): checked
    # bit for bit against one ix_gdn_commit_window per layer on copies of the states first
    copies = [dict(cs=Ly["cs"].clone(), st=Ly["state"].clone()) for Ly in layers]
    for Cp in copies:
        bx.check("ix_gdn_commit_window", bx.ix_gdn_commit_window(cfg, B, K, acc, x, rec, Cp["cs"], Cp["st"], stream))
    t_x, t_rec = bx.layer_pointer_table([x] * L), bx.layer_pointer_table([rec] * L)
    t_cs, t_st = bx.layer_pointer_table([Ly["cs"] for Ly in layers]), bx.layer_pointer_table([Ly["state"] for Ly in layers])

    def commit_layers(i):
        return bx.ix_gdn_commit_window_layers(cfg, B, K, acc, t_x, t_rec, t_cs, t_st, stream)

    bx.check("ix_gdn_commit_window_layers", commit_layers(0))
    torch.cuda.synchronize()
    for l, Cp in enumerate(copies):
        O.check_equal(f"commit_window_layers layer {l} conv state", to_host(layers[l]["cs"]), to_host(Cp["cs"]))
        O.check_equal(f"commit_window_layers layer {l} state", to_host(layers[l]["state"]), to_host(Cp["st"]))
    del copies
    out = {}
    for name, fn in (("verify", verify), ("verify_exact", verify_exact), ("commit", commit),
                     ("commit_layers", commit_layers)):
        for i in range(8):
            bx.check(name, fn(i))
        out[name] = timed(stream, fn, iters) * 1e6 / iters
    sb = B * hv * STATE_TILE
    del layers
    torch.cuda.empty_cache()
    return dict(K=K, B=B, verify_us=round(out["verify"], 2), verify_exact_us=round(out["verify_exact"], 2),
                commit_us=round(out["commit"], 2), verify_state_gbs=round(sb / out["verify"] / 1e3, 1),
                commit_state_gbs=round(2 * sb / out["commit"] / 1e3, 1),
                commit_layers=dict(layers=L, us=round(out["commit_layers"], 2),
                                   state_gbs=round(2 * sb * L / out["commit_layers"] / 1e3, 1),
                                   note="one ix_gdn_commit_window_layers launch for all layers"),
                us_per_token_window=round((out["verify"] + out["commit"]) / K, 2), check=gate)


def in_proj_leg(args, O, hidden=2048, iters=100):
    """The layer's input projection at the decode batch: [x | z | a | b] = h W^T for B = 64
    rows, hidden 2048 (Qwen3-Next), N = 12352 outputs. Weight-streaming bound: 8 rotated copies
    of W (405 MB, more than the 256 MB MALL). One call is checked against the double reference."""
    import torch

    import baloon_amd as bx

    cfg = bx.make_cfg()
    B = args.batch
    N = bx.ix_gdn_in_proj_width(cfg)
    h_np, w_np = O.proj_data(B, hidden, N)
    h, w0 = to_dev(h_np), to_dev(w_np)
    nw = 8
    ws = [w0] + [w0.clone() for _ in range(nw - 1)]
    x = torch.empty(B, cfg.channels, dtype=torch.bfloat16, device="cuda")
    z = torch.empty(B, cfg.h_v, cfg.d_v, dtype=torch.bfloat16, device="cuda")
    a = torch.empty(B, cfg.h_v, dtype=torch.bfloat16, device="cuda")
    b = torch.empty(B, cfg.h_v, dtype=torch.bfloat16, device="cuda")
    y = torch.empty(B, N, dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream()
    bx.check("ix_gdn_in_proj", bx.ix_gdn_in_proj(cfg, B, hidden, h, ws[0], x, z, a, b, y, stream))
    torch.cuda.synchronize()
    err = O.gate_proj(h_np, w_np, to_host(y))
    for i in range(8):
        bx.check("ix_gdn_in_proj", bx.ix_gdn_in_proj(cfg, B, hidden, h, ws[i % nw], x, z, a, b, None, stream))
    us = timed(stream, lambda i: bx.ix_gdn_in_proj(cfg, B, hidden, h, ws[i % nw], x, z, a, b, None, stream),
               iters) * 1e6 / iters
    wbytes = N * hidden * 2
    del ws
    torch.cuda.empty_cache()
    return dict(B=B, hidden=hidden, N=N, us=round(us, 2), weight_gbs=round(wbytes / us / 1e3, 1),
                tflops=round(2.0 * B * hidden * N / us / 1e6, 2), check=dict(err_x_magnitude=err))


def latency_leg(O, iters=200, graph_steps=32, graph_replays=20):
    """Configuration 1: one decode token at B = 1 (2 MiB state), microseconds per call: eager
    back-to-back launches, and the same launches captured once in a HIP graph and replayed
    (launch-free; the calls record one kernel each and no memset)."""
    import torch

    import baloon_amd as bx

    cfg = bx.make_cfg()
    D = O.latency_data()
    p = D["params"]
    w, A_log, dt = to_dev(p["w"]), to_dev(p["A_log"]), to_dev(p["dt_bias"])
    st, cs = state_dev(D["state0"]), to_dev(D["cs0"])
    toks = [dict(x=to_dev(t["x"]), a=to_dev(t["a"]), b=to_dev(t["b"])) for t in D["tokens"]]
    o = torch.empty(1, cfg.h_v, 128, dtype=torch.bfloat16, device="cuda")
    ws = torch.zeros(bx.ix_gdn_decode_workspace_size(cfg, 1), dtype=torch.uint8, device="cuda")

    def call(i, stream):
        t = toks[i % len(toks)]
        return bx.ix_gdn_decode(cfg, 1, t["x"], cs, w, t["a"], t["b"], A_log, dt, st, None, o, ws, stream)

    stream = torch.cuda.current_stream()
    for i in range(20):
        bx.check("ix_gdn_decode", call(i, stream))
    eager_us = timed(stream, lambda i: call(i, stream), iters) * 1e6 / iters

    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(stream)
    with torch.cuda.stream(side):
        bx.check("ix_gdn_decode", call(0, side))
    stream.wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        cap = torch.cuda.current_stream()
        for i in range(graph_steps):
            bx.check("ix_gdn_decode", call(i, cap))
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    heat()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(graph_replays):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    graph_us = e0.elapsed_time(e1) * 1e3 / (graph_replays * graph_steps)
    return round(eager_us, 2), round(graph_us, 2)


def prefill_leg(O, T=4096, iters=30):
    """Configuration 3: ix_gdn_prefill of one T-token sequence from a zero state. Each call
    gets its own state and conv state, zeroed before the timed region (like every other
    input, they are resident in HBM when it starts; the kernels' work does not depend on
    their values), and the outputs and states of the last timed call are checked against the
    CPU replay."""
    import torch

    import baloon_amd as bx

    cfg = bx.make_cfg()
    D = O.prefill_data(T)
    p, tok = D["params"], D["tokens"]
    w, A_log, dt = to_dev(p["w"]), to_dev(p["A_log"]), to_dev(p["dt_bias"])
    x, a, b = to_dev(tok["x"]), to_dev(tok["a"]), to_dev(tok["b"])
    cu = torch.tensor([0, T], dtype=torch.int32, device="cuda")
    warm = 2
    sts = [torch.zeros(1, cfg.h_v, 128, 128, device="cuda") for _ in range(warm + iters)]
    css = [torch.zeros(1, cfg.channels, cfg.d_conv - 1, dtype=torch.bfloat16, device="cuda") for _ in range(warm + iters)]
    o = torch.empty(T, cfg.h_v, 128, dtype=torch.bfloat16, device="cuda")
    need = bx.ix_gdn_prefill_workspace_size(cfg, 1, T)
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream()

    def run(i):
        return bx.ix_gdn_prefill(cfg, 1, T, cu, x, css[i], w, a, b, A_log, dt, sts[i], None, o, ws, need, stream)

    for i in range(warm):
        bx.check("ix_gdn_prefill", run(i))
    sec = timed(stream, lambda i: run(warm + i), iters) / iters
    tflops = PREFILL_FLOP_PER_TOKEN * T / sec / 1e12
    check = O.gate_prefill(D, T, to_host(css[-1]), state_host(sts[-1]), to_host(o))
    # The same call with a workspace of 16-chunk windows (1024 tokens): bounded memory, same
    # results bit for bit.
    wchunks = 16
    wneed = bx.ix_gdn_prefill_window_workspace_size(cfg, 1, T, wchunks)
    wws = torch.empty(wneed, dtype=torch.uint8, device="cuda")
    full_st, full_cs = sts[-1].clone(), css[-1].clone()
    for st_, cs_ in zip(sts, css):
        st_.zero_()
        cs_.zero_()
    ow = torch.empty_like(o)

    def run_w(i):
        return bx.ix_gdn_prefill(cfg, 1, T, cu, x, css[i], w, a, b, A_log, dt, sts[i], None, ow, wws, wneed, stream)

    for i in range(warm):
        bx.check("ix_gdn_prefill", run_w(i))
    wsec = timed(stream, lambda i: run_w(warm + i), iters) / iters
    same = bool(torch.equal(ow, o)) and bool(torch.equal(sts[-1], full_st)) and bool(torch.equal(css[-1], full_cs))
    if not same:
        raise SystemExit("prefill: the windowed run differs from the one-window run")
    del ws, wws
    torch.cuda.empty_cache()
    return dict(T=T, tokens_per_s=round(T / sec, 1), us_per_call=round(sec * 1e6, 1),
                mfma=dict(bound="mfma", achieved=round(tflops, 2), peak=MFMA_BF16_PEAK_TFLOPS, unit="TFLOP/s",
                          frac=round(tflops / MFMA_BF16_PEAK_TFLOPS, 5)),
                workspace_mib=round(need / 2 ** 20, 1),
                windowed=dict(window_tokens=wchunks * 64, us_per_call=round(wsec * 1e6, 1),
                              workspace_mib=round(wneed / 2 ** 20, 1), bit_identical=same),
                check=check)


def prefill_varlen_leg(O, iters=5):
    """Configuration 4's prefill as serving batches it: 32 sequences of lengths U[1, 2048]
    (35,129 tokens) packed by cu_seqlens into one ix_gdn_prefill call, initial states
    N(0, 0.02). Each timed call gets its own copy of the initial states, prepared before the
    timed region; the last timed call's outputs and states are checked against the CPU
    replay."""
    import torch

    import baloon_amd as bx

    cfg = bx.make_cfg()
    V = O.varlen_data()
    p, tok, T, n = V["params"], V["tokens"], V["T"], len(V["cu"]) - 1
    w, A_log, dt = to_dev(p["w"]), to_dev(p["A_log"]), to_dev(p["dt_bias"])
    x, a, b = to_dev(tok["x"]), to_dev(tok["a"]), to_dev(tok["b"])
    cu = to_dev(V["cu"])
    warm = 1
    st0, cs0 = state_dev(V["st0"]["state"]), to_dev(V["st0"]["conv_state"])
    sts = [st0.clone() for _ in range(warm + iters)]
    css = [cs0.clone() for _ in range(warm + iters)]
    o = torch.empty(T, cfg.h_v, 128, dtype=torch.bfloat16, device="cuda")
    need = bx.ix_gdn_prefill_workspace_size(cfg, n, T)
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream()

    def run(i):
        return bx.ix_gdn_prefill(cfg, n, T, cu, x, css[i], w, a, b, A_log, dt, sts[i], None, o, ws, need, stream)

    for i in range(warm):
        bx.check("ix_gdn_prefill", run(i))
    sec = timed(stream, lambda i: run(warm + i), iters) / iters
    tflops = PREFILL_FLOP_PER_TOKEN * T / sec / 1e12
    check = O.gate_prefill_varlen(V, to_host(css[-1]), state_host(sts[-1]), to_host(o))
    del ws, sts, css
    torch.cuda.empty_cache()
    return dict(n_seq=n, T=T, tokens_per_s=round(T / sec, 1), us_per_call=round(sec * 1e6, 1),
                mfma=dict(bound="mfma", achieved=round(tflops, 2), peak=MFMA_BF16_PEAK_TFLOPS, unit="TFLOP/s",
                          frac=round(tflops / MFMA_BF16_PEAK_TFLOPS, 5)),
                workspace_mib=round(need / 2 ** 20, 1), check=check)


def legacy_leg(O, iters=200):
    """The five reference launchers at the reference acceptance test's shapes
    (tests/test_gdn.cu:16-55), microseconds per call (back-to-back calls between HIP events;
    the step updates its state in place call after call). One call of each is checked first,
    against the CPU oracle, with the test's norm and tolerances. The step's state traffic is
    S * h_v * S fp32 read and written once: 6.29 MB per call."""
    import torch

    import baloon_amd as bx

    L = O.legacy_data()
    S, hk, hv, C, dc = L["S"], L["hk"], L["hv"], L["C"], L["dc"]
    st, q, k, v, g, bt = (to_dev(L[n]) for n in ("st", "q", "k", "v", "gate", "beta"))
    so = torch.empty(hv * S, dtype=torch.float32, device="cuda")
    cs, x, w = to_dev(L["cs"]), to_dev(L["x"]), to_dev(L["w"])
    cout = torch.empty(C, dtype=torch.float32, device="cuda")
    l2 = to_dev(L["l2"])
    o, z, nrm = to_dev(L["o"]), to_dev(L["z"]), to_dev(L["nrm"])
    y = torch.empty(hv * S, dtype=torch.float32, device="cuda")
    b = to_dev(L["b"])
    stream = torch.cuda.current_stream()
    calls = {
        "step": lambda i: bx.ix_gdn_step(st, q, k, v, g, bt, so, S, hk, hv, stream),
        "conv_step": lambda i: bx.ix_gdn_conv_step(cs, x, w, cout, C, dc, stream),
        "l2_norm": lambda i: bx.ix_gdn_l2_norm(l2, 33, 128, 1e-6, stream),
        "out_norm": lambda i: bx.ix_gdn_out_norm(o, z, nrm, y, hv, S, 1e-6, stream),
        "beta_gate": lambda i: bx.ix_gdn_beta_gate(b, hv, stream),
    }
    for name, fn in calls.items():
        bx.check(name, fn(0))
    torch.cuda.synchronize()
    check = O.gate_legacy(L, dict(step_o=to_host(so), step_st=to_host(st), conv_out=to_host(cout),
                                  conv_cs=to_host(cs), l2=to_host(l2), out_norm=to_host(y), beta=to_host(b)))
    us = {}
    for name, fn in calls.items():
        for i in range(5):
            bx.check(name, fn(i))
        us[name] = round(timed(stream, fn, iters) * 1e6 / iters, 2)
    state_bytes = 2 * S * hv * S * 4
    return dict(step_us=us["step"], step_state_gbs=round(state_bytes / us["step"] / 1e3, 1),
                conv_step_us=us["conv_step"], l2_norm_us=us["l2_norm"], out_norm_us=us["out_norm"],
                beta_gate_us=us["beta_gate"],
                shapes="step S=128 h_k=16 h_v=48; conv C=8197 d_conv=4; l2 33x128; out_norm 48x128; beta 48",
                check=check)


def hbm_ceiling(nbuf=4, mib=128, iters=20):
    """Measured in-place read+write rate of the box: torch's x.mul_(1) over nbuf rotated
    128 MiB buffers (the decode state's traffic pattern, MALL defeated)."""
    import torch
    bufs = [torch.ones(mib << 18, dtype=torch.float32, device="cuda") for _ in range(nbuf)]
    for b in bufs:
        b.mul_(1.0)
    torch.cuda.synchronize()
    heat()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(iters):
        bufs[i % nbuf].mul_(1.0)
    e1.record()
    torch.cuda.synchronize()
    sec = e0.elapsed_time(e1) / 1e3 / iters
    del bufs
    return round(2 * (mib << 20) / sec / 1e9, 1)


def replayed_traffic(args):
    """HBM bytes per launch of the headline decode kernel from the committed rocprofv3 --pmc
    (FETCH_SIZE, WRITE_SIZE) runs of this workload; not measured in this run."""
    if not os.path.exists(TRAFFIC_FILE) or args.batch != 64 or args.layers != 4:
        return None, None
    t = json.load(open(TRAFFIC_FILE))
    return t["bytes_per_launch"], f"replayed from {os.path.relpath(TRAFFIC_FILE, ROOT)} ({t['source']})"


def partial_run(args, O):
    """A subset of the legs (--legs), for profiling passes: each leg runs and is gated as in the
    full run, and one JSON object with their results is printed (not the result line)."""
    out = {}
    D = O.decode_data(args.batch, args.layers, args.inputs) if args.legs & {"decode", "gated", "window"} else None
    if "decode" in args.legs or "gated" in args.legs:
        order = list(range(args.warmup)) + list(range(args.steps))
        d = decode_leg(args, D) if "decode" in args.legs else None
        dg = decode_leg(args, D, gated=True) if "gated" in args.legs else None
        if d is not None:
            out["decode"] = dict(avg_kernel_us=round(d["avg_kernel_us"], 2), roofline=d["roofline"],
                                 check=O.gate_decode(D, order, args, d, dg))
        if dg is not None:
            out["decode_gated"] = dict(avg_kernel_us=round(dg["avg_kernel_us"], 2))
    if "window" in args.legs:
        out["spec_window"] = window_leg(args, D, O.window_tokens(args.batch, 4), O)
    if "in_proj" in args.legs:
        out["in_proj"] = in_proj_leg(args, O)
    if "latency" in args.legs:
        out["decode_b1_us_per_token"], out["decode_b1_us_per_token_graph"] = latency_leg(O)
    if "prefill" in args.legs:
        out["prefill"] = prefill_leg(O)
    if "prefill_varlen" in args.legs:
        out["prefill_varlen"] = prefill_varlen_leg(O)
    if "legacy" in args.legs:
        out["legacy"] = legacy_leg(O)
    if "ceiling" in args.legs:
        out["hbm_inplace_ceiling_gbs"] = hbm_ceiling()
    if O.failures:
        print(f"bench.py: {len(O.failures)} correctness check(s) failed", file=sys.stderr)
        sys.exit(3)
    print(json.dumps(dict(partial_legs=sorted(args.legs), **out)))


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE {world}); "
              "the GDN path is benchmarked on a single MI355X", file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    torch.cuda.synchronize()
    O = CpuBaselineLeg()
    legs = args.legs
    if legs != {"decode", "gated", "window", "in_proj", "latency", "prefill", "prefill_varlen", "legacy", "ceiling"}:
        partial_run(args, O)
        return
    D = O.decode_data(args.batch, args.layers, args.inputs)

    d = decode_leg(args, D)
    dg = decode_leg(args, D, gated=True)
    win = window_leg(args, D, O.window_tokens(args.batch, 4), O)
    ip = in_proj_leg(args, O)
    lat_eager, lat_graph = latency_leg(O)
    pf = prefill_leg(O)
    pv = prefill_varlen_leg(O)
    leg = legacy_leg(O)
    ceiling = hbm_ceiling()

    # the CPU replay of the timed decode sequence: the CPU baseline, and the decode gate
    order = list(range(args.warmup)) + list(range(args.steps))
    dcheck = O.gate_decode(D, order, args, d, dg)
    cpu = dict(value=round(O.record["decode"]["tokens_per_s"], 1), unit="tokens/s", cores=O.nt, kind="port",
               nproc=os.cpu_count(),
               sample=(f"the benchmark's own decode sequence: {len(order)} steps of B={args.batch} "
                       f"({args.layers} layers) in {O.record['decode']['sec']:.1f} s on {O.nt} threads "
                       "(oracle/gdn_oracle.c, double)"),
               prefill_tokens_per_s=round(O.record["prefill"]["tokens_per_s"], 1),
               prefill_sample=f"one sequence of {pf['T']} tokens, token-by-token recurrence on {O.nt} threads",
               prefill_varlen_tokens_per_s=round(O.record["prefill_varlen"]["tokens_per_s"], 1),
               prefill_varlen_sample=f"configuration 4's {pv['n_seq']} sequences ({pv['T']} tokens) on {O.nt} threads")
    if not args.no_cpu:
        v1, n1 = O.cpu_decode_1core(D, args)
        cpu.update(value_1core=round(v1, 1), sample_1core=f"{n1} steps of B={args.batch} on 1 thread",
                   prefill_tokens_per_s_1core=round(O.cpu_prefill_1core(O.prefill_data(pf["T"])), 1))
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                cpu["cpu_model"] = ln.split(":", 1)[1].strip()
                break
    except OSError:
        pass

    if O.failures:
        print(f"bench.py: {len(O.failures)} correctness check(s) failed; no result line", file=sys.stderr)
        sys.exit(3)
    traffic, traffic_src = replayed_traffic(args)
    roofline = dict(d["roofline"], traffic=traffic, traffic_source=traffic_src)
    line = {
        "metric": "GDN decode tokens/s + state HBM GB/s (%peak) at B=64; prefill tok/s T=4096",
        "value": round(d["tokens_per_s"], 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(d["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded generator of oracle/inputs.py)",
        "config": {"workload": "C2 batched GDN decode: B=64, h_k=16, h_v=32, d=128, fused conv k=4, "
                               f"{args.layers} layers rotated (state {args.layers}x128 MiB)",
                   "B": args.batch, "layers": args.layers, "parallelism": "single-gpu"},
        "avg_kernel_us": round(d["avg_kernel_us"], 2),
        "state_gbs": d["roofline"]["achieved"],
        "hbm_inplace_ceiling_gbs": ceiling,
        "decode_b1_us_per_token": lat_eager,
        "decode_b1_us_per_token_graph": lat_graph,
        "decode_gated": {"avg_kernel_us": round(dg["avg_kernel_us"], 2), "state_gbs": dg["roofline"]["achieved"],
                         "note": "same step with the gated RMS output norm fused in (bf16 y instead of bf16 o)"},
        "spec_window": win,
        "in_proj": ip,
        "prefill": pf,
        "prefill_varlen": pv,
        "legacy": leg,
        "correctness": dict(gated="every leg checked against the CPU replay (oracle/); tolerances: fp32 o 1e-3 "
                                  "abs beyond bf16 rounding, state max|d|/max|ref| 1e-4, conv state bit-exact",
                            decode=dcheck),
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
