#!/usr/bin/env python3
"""Benchmark of the GDN path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--batch 64] [--layers 4] [--no-cpu]

Headline workload (configuration 2 of the benchmark set): batched GDN decode, B = 64
independent sequences, 16 q/k heads and 32 v heads, d_k = d_v = 128, fp32 state 128 MiB per
layer, fused conv (4 taps over 8192 channels), one ix_gdn_decode launch per step. A "step" is
one decode token for all B sequences of one layer; steps rotate over --layers independent
layers (state, conv state, weights), so the working set (4 x 128 MiB) exceeds the 256 MB
Infinity Cache and the state really streams from HBM. Inputs are synthetic and resident in
HBM before the timed region, which is bracketed by HIP events on the launch stream.

Also reported on the same line: decode latency at B = 1 (configuration 1), chunked prefill
of one 4096-token sequence (configuration 3) with its MFMA roofline fraction, the measured
in-place HBM ceiling of the box, and the CPU oracle (a C port of the reference's recurrence)
timed on this host over bounded samples of the same workloads.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E spec
STATE_TILE = 128 * 128 * 4     # bytes per (sequence, v head)


def parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--layers", type=int, default=4)
    ap.add_argument("--inputs", type=int, default=8, help="distinct input sets cycled through")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="budget per CPU baseline leg")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    return ap.parse_args()


def decode_bench(args, gated=False):
    """B-sequence decode over rotated layers; gated=True times ix_gdn_decode_gated (the same
    step with the gated output norm fused in, y written as bf16)."""
    import torch

    import baloon_amd as bx

    cfg = bx.make_cfg()
    B, L, P = args.batch, args.layers, args.inputs
    C, hv = cfg.channels, cfg.h_v
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(0x6D4E0002)
    layers = []
    for _ in range(L):
        layers.append(dict(
            w=(torch.randn(C, cfg.d_conv, generator=g, device=dev) * 0.1).to(torch.bfloat16),
            A_log=torch.rand(hv, generator=g, device=dev) * float(torch.log(torch.tensor(16.0))),
            dt=torch.randn(hv, generator=g, device=dev) * 0.1,
            state=torch.randn(B, hv, 128, 128, generator=g, device=dev) * 0.02,
            cs=torch.randn(B, C, cfg.d_conv - 1, generator=g, device=dev).to(torch.bfloat16),
        ))
    ins = [dict(x=torch.randn(B, C, generator=g, device=dev).to(torch.bfloat16),
                a=torch.randn(B, hv, generator=g, device=dev).to(torch.bfloat16),
                b=torch.randn(B, hv, generator=g, device=dev).to(torch.bfloat16)) for _ in range(P)]
    o = torch.empty(B, hv, 128, dtype=torch.bfloat16, device=dev)
    ws = torch.zeros(bx.ix_gdn_decode_workspace_size(cfg, B), dtype=torch.uint8, device=dev)   # stream-ordered: shared
    z = torch.randn(B, hv, 128, generator=g, device=dev).to(torch.bfloat16)
    nrm = 1.0 + 0.1 * torch.randn(128, generator=g, device=dev)
    y = torch.empty(B, hv, 128, dtype=torch.bfloat16, device=dev)
    gate = bx.out_gate(z, nrm, 1e-6, None, y)
    stream = torch.cuda.current_stream()
    lib = bx.lib()
    import ctypes
    cfg_ref = ctypes.byref(cfg)
    s_ptr = stream.cuda_stream

    gate_ref = ctypes.byref(gate)

    def launch(i):
        Ly, In = layers[i % L], ins[i % P]
        if gated:
            return lib.ix_gdn_decode_gated(cfg_ref, B, In["x"].data_ptr(), Ly["cs"].data_ptr(), Ly["w"].data_ptr(),
                                           In["a"].data_ptr(), In["b"].data_ptr(), Ly["A_log"].data_ptr(),
                                           Ly["dt"].data_ptr(), Ly["state"].data_ptr(), None, None, gate_ref,
                                           ws.data_ptr(), s_ptr)
        return lib.ix_gdn_decode(cfg_ref, B, In["x"].data_ptr(), Ly["cs"].data_ptr(), Ly["w"].data_ptr(),
                                 In["a"].data_ptr(), In["b"].data_ptr(), Ly["A_log"].data_ptr(), Ly["dt"].data_ptr(),
                                 Ly["state"].data_ptr(), None, o.data_ptr(), ws.data_ptr(), s_ptr)

    for i in range(args.warmup):
        bx.check("ix_gdn_decode", launch(i))
    torch.cuda.synchronize()
    K = args.steps
    # Timed region: K back-to-back launches on `stream`, bracketed by HIP events recorded on
    # that same stream. Every launch's status is checked after the region.
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    rcs = []
    torch.cuda.synchronize()
    t0.record(stream)
    for i in range(K):
        rcs.append(launch(i))
    t1.record(stream)
    torch.cuda.synchronize()
    for rc in rcs:
        bx.check("ix_gdn_decode", rc)
    total_ms = t0.elapsed_time(t1)
    avg_launch_s = total_ms / K / 1e3          # average launch duration seen by the stream
    state_bytes = 2 * B * hv * STATE_TILE
    achieved = state_bytes / avg_launch_s / 1e9
    traffic = None
    tf = os.path.join(ROOT, "profiles", "decode_traffic.json")
    if os.path.exists(tf) and B == 64 and L == 4:
        traffic = json.load(open(tf))["bytes_per_launch"]      # PMC-measured HBM bytes per launch
    return dict(
        tokens_per_s=B * K / (total_ms / 1e3),
        ms_per_step=total_ms / K,
        avg_kernel_us=avg_launch_s * 1e6,
        state_bytes_per_launch=state_bytes,
        roofline=dict(bound="hbm", achieved=round(achieved, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                      frac=round(achieved / HBM_PEAK_GBS, 4), traffic=traffic),
    )


def window_bench(args, K=4, iters=64):
    """Speculative window at B = 64: ix_gdn_decode_window over K draft tokens, then
    ix_gdn_commit_window with all K accepted (the most state work), layers rotated as in the
    decode leg. Reports microseconds per call and the state GB/s of each (verify reads the
    state once, commit reads and writes it once)."""
    import torch

    import baloon_amd as bx

    cfg = bx.make_cfg()
    B, L = args.batch, args.layers
    C, hv = cfg.channels, cfg.h_v
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(0x6D4E0005)
    layers = [dict(w=(torch.randn(C, cfg.d_conv, generator=g, device=dev) * 0.1).to(torch.bfloat16),
                   A_log=torch.rand(hv, generator=g, device=dev) * 2.77,
                   dt=torch.randn(hv, generator=g, device=dev) * 0.1,
                   state=torch.randn(B, hv, 128, 128, generator=g, device=dev) * 0.02,
                   cs=torch.randn(B, C, cfg.d_conv - 1, generator=g, device=dev).to(torch.bfloat16))
              for _ in range(L)]
    x = torch.randn(B, K, C, generator=g, device=dev).to(torch.bfloat16)
    a = torch.randn(B, K, hv, generator=g, device=dev).to(torch.bfloat16)
    b = torch.randn(B, K, hv, generator=g, device=dev).to(torch.bfloat16)
    o = torch.empty(B, K, hv, 128, dtype=torch.bfloat16, device=dev)
    rec = torch.empty(bx.ix_gdn_window_record_size(cfg, B, K), dtype=torch.uint8, device=dev)
    acc = torch.full((B,), K, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream()

    def verify(i):
        Ly = layers[i % L]
        return bx.ix_gdn_decode_window(cfg, B, K, x, Ly["cs"], Ly["w"], a, b, Ly["A_log"], Ly["dt"], Ly["state"],
                                       None, o, rec, stream)

    def commit(i):
        Ly = layers[i % L]
        return bx.ix_gdn_commit_window(cfg, B, K, acc, x, rec, Ly["cs"], Ly["state"], stream)

    out = {}
    for name, fn in (("verify", verify), ("commit", commit)):
        for i in range(8):
            bx.check(name, fn(i))
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        rcs = [fn(i) for i in range(iters)]
        e1.record(stream)
        torch.cuda.synchronize()
        for rc in rcs:
            bx.check(name, rc)
        out[name] = e0.elapsed_time(e1) * 1e3 / iters
    sb = B * hv * STATE_TILE
    return dict(K=K, B=B, verify_us=round(out["verify"], 2), commit_us=round(out["commit"], 2),
                verify_state_gbs=round(sb / out["verify"] / 1e3, 1),
                commit_state_gbs=round(2 * sb / out["commit"] / 1e3, 1),
                us_per_token_window=round((out["verify"] + out["commit"]) / K, 2))


def in_proj_bench(args, hidden=2048, iters=100):
    """The layer's input projection at the decode batch: y = h W^T for B = 64 rows, hidden
    2048 (Qwen3-Next), N = 12352 outputs (x | z | a | b). Weight-streaming bound: reports
    microseconds per call, the weight bytes' GB/s and TFLOP/s."""
    import torch

    import baloon_amd as bx

    cfg = bx.make_cfg()
    B = args.batch
    N = bx.ix_gdn_in_proj_width(cfg)
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(0x6D4E0006)
    nw = 8                                                    # rotated weight copies: 8 x 50.6 MB exceeds the 256 MB MALL
    ws = [(torch.randn(N, hidden, generator=g, device=dev) * 0.05).to(torch.bfloat16) for _ in range(nw)]
    h = torch.randn(B, hidden, generator=g, device=dev).to(torch.bfloat16)
    x = torch.empty(B, cfg.channels, dtype=torch.bfloat16, device=dev)
    z = torch.empty(B, cfg.h_v, cfg.d_v, dtype=torch.bfloat16, device=dev)
    a = torch.empty(B, cfg.h_v, dtype=torch.bfloat16, device=dev)
    b = torch.empty(B, cfg.h_v, dtype=torch.bfloat16, device=dev)
    stream = torch.cuda.current_stream()
    for i in range(8):
        bx.check("ix_gdn_in_proj", bx.ix_gdn_in_proj(cfg, B, hidden, h, ws[i % nw], x, z, a, b, None, stream))
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    rcs = [bx.ix_gdn_in_proj(cfg, B, hidden, h, ws[i % nw], x, z, a, b, None, stream) for i in range(iters)]
    e1.record(stream)
    torch.cuda.synchronize()
    for rc in rcs:
        bx.check("ix_gdn_in_proj", rc)
    us = e0.elapsed_time(e1) * 1e3 / iters
    wbytes = N * hidden * 2
    return dict(B=B, hidden=hidden, N=N, us=round(us, 2), weight_gbs=round(wbytes / us / 1e3, 1),
                tflops=round(2.0 * B * hidden * N / us / 1e6, 2))


def decode_latency(iters=200):
    """Configuration 1: one decode token at B = 1 (2 MiB state), microseconds per call."""
    import torch

    import baloon_amd as bx

    cfg = bx.make_cfg()
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(0x6D4E0001)
    C, hv = cfg.channels, cfg.h_v
    w = (torch.randn(C, cfg.d_conv, generator=g, device=dev) * 0.1).to(torch.bfloat16)
    A_log = torch.rand(hv, generator=g, device=dev) * 2.77
    dt = torch.randn(hv, generator=g, device=dev) * 0.1
    st = torch.randn(1, hv, 128, 128, generator=g, device=dev) * 0.02
    cs = torch.randn(1, C, cfg.d_conv - 1, generator=g, device=dev).to(torch.bfloat16)
    x = torch.randn(1, C, generator=g, device=dev).to(torch.bfloat16)
    a = torch.randn(1, hv, generator=g, device=dev).to(torch.bfloat16)
    b = torch.randn(1, hv, generator=g, device=dev).to(torch.bfloat16)
    o = torch.empty(1, hv, 128, dtype=torch.bfloat16, device=dev)
    ws = torch.zeros(bx.ix_gdn_decode_workspace_size(cfg, 1), dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream()
    for _ in range(20):
        bx.check("ix_gdn_decode", bx.ix_gdn_decode(cfg, 1, x, cs, w, a, b, A_log, dt, st, None, o, ws, stream))
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    rcs = [bx.ix_gdn_decode(cfg, 1, x, cs, w, a, b, A_log, dt, st, None, o, ws, stream) for _ in range(iters)]
    e1.record(stream)
    torch.cuda.synchronize()
    for rc in rcs:
        bx.check("ix_gdn_decode", rc)
    return round(e0.elapsed_time(e1) * 1e3 / iters, 2)


PREFILL_FLOP_PER_TOKEN = 5_767_168     # 2C^2(3d_k+2d_v) + 6 C d_k d_v per (v head, chunk of 64) / 64, x 32 heads
MFMA_BF16_PEAK_TFLOPS = 2500.0


def prefill_bench(T=4096, iters=10):
    """Configuration 3: ix_gdn_prefill of one T-token sequence from a zero state."""
    import torch

    import baloon_amd as bx

    cfg = bx.make_cfg()
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(0x6D4E0003)
    C, hv = cfg.channels, cfg.h_v
    w = (torch.randn(C, cfg.d_conv, generator=g, device=dev) * 0.1).to(torch.bfloat16)
    A_log = torch.rand(hv, generator=g, device=dev) * 2.77
    dt = torch.randn(hv, generator=g, device=dev) * 0.1
    x = torch.randn(T, C, generator=g, device=dev).to(torch.bfloat16)
    a = torch.randn(T, hv, generator=g, device=dev).to(torch.bfloat16)
    b = torch.randn(T, hv, generator=g, device=dev).to(torch.bfloat16)
    cu = torch.tensor([0, T], dtype=torch.int32, device=dev)
    st = torch.zeros(1, hv, 128, 128, device=dev)
    cs = torch.zeros(1, C, cfg.d_conv - 1, dtype=torch.bfloat16, device=dev)
    o = torch.empty(T, hv, 128, dtype=torch.bfloat16, device=dev)
    need = bx.ix_gdn_prefill_workspace_size(cfg, 1, T)
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream()

    def run():
        st.zero_()
        cs.zero_()
        return bx.ix_gdn_prefill(cfg, 1, T, cu, x, cs, w, a, b, A_log, dt, st, None, o, ws, need, stream)

    for _ in range(2):
        bx.check("ix_gdn_prefill", run())
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    # the zero fills of the state and conv state (2.1 MB) are inside the region
    e0.record(stream)
    rcs = [run() for _ in range(iters)]
    e1.record(stream)
    torch.cuda.synchronize()
    for rc in rcs:
        bx.check("ix_gdn_prefill", rc)
    sec = e0.elapsed_time(e1) / 1e3 / iters
    tflops = PREFILL_FLOP_PER_TOKEN * T / sec / 1e12
    return dict(T=T, tokens_per_s=round(T / sec, 1), us_per_call=round(sec * 1e6, 1),
                mfma=dict(bound="mfma", achieved=round(tflops, 2), peak=MFMA_BF16_PEAK_TFLOPS, unit="TFLOP/s",
                          frac=round(tflops / MFMA_BF16_PEAK_TFLOPS, 5)),
                workspace_mib=round(need / 2 ** 20, 1))


def hbm_ceiling(nbuf=4, mib=128, iters=20):
    """Measured in-place read+write rate of the box: torch's x.mul_(1) over nbuf rotated
    128 MiB buffers (the decode state's traffic pattern, MALL defeated)."""
    import torch
    bufs = [torch.ones(mib << 18, dtype=torch.float32, device="cuda") for _ in range(nbuf)]
    for b in bufs:
        b.mul_(1.0)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(iters):
        bufs[i % nbuf].mul_(1.0)
    e1.record()
    torch.cuda.synchronize()
    sec = e0.elapsed_time(e1) / 1e3 / iters
    del bufs
    return round(2 * (mib << 20) / sec / 1e9, 1)


def cpu_baseline(args):
    """Oracle (C port of the reference's double recurrence, tests/test_gdn.cu:22-26, extended
    with the fused conv/gates/L2) timed on this host's cores over a bounded sample of the same
    workload: B = 64 sequences, decode steps until the time budget is used."""
    import numpy as np

    import oracle
    from oracle import inputs

    cfg = oracle.make_cfg()
    B = args.batch
    seed = inputs.seed_for(2)
    p = inputs.layer_params(cfg, seed)
    s = inputs.initial_states(cfg, seed, B)
    toks = [inputs.token_inputs(cfg, seed, B, step=i) for i in range(2)]
    ncores = min(16, os.cpu_count() or 1)
    out = {}
    for cores in sorted({1, ncores}):
        cs, st = s["conv_state"], s["state"].astype(np.float64)
        steps, t0 = 0, time.perf_counter()
        while True:
            t = toks[steps % 2]
            cs, st, _ = oracle.decode(cfg, B, t["x"], cs, p["w"], t["a"], t["b"], p["A_log"], p["dt_bias"], st,
                                      nthreads=cores)
            steps += 1
            el = time.perf_counter() - t0
            if el >= args.cpu_seconds or steps >= 256:
                break
        out[cores] = (B * steps / el, steps, el)
    best = max(out)
    v, steps, el = out[best]
    # prefill: token-by-token recurrence of one sequence (configuration 3's shape), bounded sample
    Tp = 256
    tok = inputs.token_inputs(cfg, inputs.seed_for(3), Tp)
    st0 = inputs.initial_states(cfg, inputs.seed_for(3), 1, state_std=0.0, conv_std=0.0)
    pre = {}
    for cores in sorted({1, ncores}):
        t0 = time.perf_counter()
        oracle.prefill(cfg, [0, Tp], tok["x"], st0["conv_state"], p["w"], tok["a"], tok["b"], p["A_log"],
                       p["dt_bias"], st0["state"], nthreads=cores)
        pre[cores] = Tp / (time.perf_counter() - t0)
    cpu_model = ""
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                cpu_model = ln.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return dict(value=round(v, 1), unit="tokens/s", cores=best, kind="port", nproc=os.cpu_count(),
                cpu_model=cpu_model,
                sample=f"B={B} decode, {steps} steps in {el:.1f} s on {best} threads (oracle/gdn_oracle.c, double)",
                value_1core=round(out[1][0], 1),
                prefill_tokens_per_s=round(pre[best], 1), prefill_tokens_per_s_1core=round(pre[1], 1),
                prefill_sample=f"one sequence of {Tp} tokens, token-by-token recurrence")


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
    d = decode_bench(args)
    dg = decode_bench(args, gated=True)
    win = window_bench(args)
    ip = in_proj_bench(args)
    lat = decode_latency()
    pf = prefill_bench()
    ceiling = hbm_ceiling()
    cpu = None if args.no_cpu else cpu_baseline(args)
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
        "data": "synthetic",
        "config": {"workload": "C2 batched GDN decode: B=64, h_k=16, h_v=32, d=128, fused conv k=4, "
                               f"{args.layers} layers rotated (state {args.layers}x128 MiB)",
                   "B": args.batch, "layers": args.layers, "parallelism": "single-gpu"},
        "avg_kernel_us": round(d["avg_kernel_us"], 2),
        "state_gbs": d["roofline"]["achieved"],
        "hbm_inplace_ceiling_gbs": ceiling,
        "decode_b1_us_per_token": lat,
        "decode_gated": {"avg_kernel_us": round(dg["avg_kernel_us"], 2), "state_gbs": dg["roofline"]["achieved"],
                         "note": "same step with the gated RMS output norm fused in (bf16 y instead of bf16 o)"},
        "spec_window": win,
        "in_proj": ip,
        "prefill": pf,
        "roofline": d["roofline"],
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
