"""Writes tests/golden/config0.npz: configuration 0 of the benchmark set, computed by the
oracle (oracle/gdn_oracle.c). The reference ships no golden vectors for this path, so this
fixture is a regression anchor for the oracle and a fixed parity target for the GPU.

Configuration 0: one sequence, one q/k head and one v head, d_k = d_v = 128, 64 decode
tokens; q, k, v bf16 ~ N(0,1) (q, k L2-normalised inside the step); a ~ N(0,1),
A_log ~ U(ln 1, ln 16), dt_bias ~ N(0, 0.1), b ~ N(0,1); initial state fp32 ~ N(0, 0.02).
The fused path always convolves, so the conv is the identity here: d_conv = 2 with taps
[0, 1] (bf16 1.0 is exact), which passes x through bit for bit.

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle  # noqa: E402
from oracle import bf16, inputs  # noqa: E402

T = 64


def config0_cfg():
    return oracle.make_cfg(h_k=1, h_v=1, d_k=128, d_v=128, d_conv=2)


def config0_inputs():
    cfg = config0_cfg()
    seed = inputs.seed_for(0)
    p = inputs.layer_params(cfg, seed)
    w = np.zeros((cfg.channels, 2), np.float32)
    w[:, 1] = 1.0
    p["w"] = bf16.from_f32(w)
    tok = inputs.token_inputs(cfg, seed, T)
    st = inputs.initial_states(cfg, seed, 1, state_std=0.02, conv_std=0.0)
    return cfg, p, tok, st


def main():
    cfg, p, tok, st = config0_inputs()
    cs, state, o = oracle.prefill(cfg, [0, T], tok["x"], st["conv_state"], p["w"], tok["a"], tok["b"],
                                  p["A_log"], p["dt_bias"], st["state"])
    out = os.path.join(HERE, "config0.npz")
    np.savez_compressed(out, x=tok["x"], a=tok["a"], b=tok["b"], w=p["w"], A_log=p["A_log"],
                        dt_bias=p["dt_bias"], state0=st["state"], o=o, state=state)
    print(f"wrote {out}: o {o.shape}, state {state.shape}")


if __name__ == "__main__":
    main()
