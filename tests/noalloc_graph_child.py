"""Child process of tests/test_zz_no_alloc.py (not collected by pytest): the first
ix_gdn_decode_noalloc call of a fresh process made under HIP graph capture.

Captures two ix_gdn_decode_noalloc calls (two tokens) into a torch CUDA graph -- the
library's first call on the device, so its symbol lookup happens during the capture --
replays the graph three times, with eager work and a synchronisation between replays, and
checks the state, conv state and outputs after every replay bit for bit against the same
tokens run eagerly through ix_gdn_decode with a caller workspace. Then checks that an eager
ix_gdn_decode_noalloc call leaves the device's free memory unchanged. Prints "ok" last.
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)


def main():
    import torch

    import baloon_amd as bx
    from oracle import inputs
    from tests.common import dev, host, state_to_dev

    cfg = bx.make_cfg()
    B, seed = 8, inputs.seed_for(2) + 520
    p = inputs.layer_params(cfg, seed)
    s = inputs.initial_states(cfg, seed, B)
    toks = [inputs.token_inputs(cfg, seed, B, step=i) for i in range(2)]
    w, A, dt = dev(p["w"]), dev(p["A_log"]), dev(p["dt_bias"])
    xs = [dict(x=dev(t["x"]), a=dev(t["a"]), b=dev(t["b"])) for t in toks]
    cs_g, st_g = dev(s["conv_state"]), state_to_dev(s["state"])
    cs_e, st_e = dev(s["conv_state"]), state_to_dev(s["state"])
    o_g = torch.empty(2, B, cfg.h_v, cfg.d_v, dtype=torch.float32, device="cuda")
    o_e = torch.empty_like(o_g)
    ws = torch.zeros(bx.ix_gdn_decode_workspace_size(cfg, B), dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            cap = torch.cuda.current_stream()
            for i in range(2):
                t = xs[i]
                rc = bx.ix_gdn_decode_noalloc(cfg, B, t["x"], cs_g, w, t["a"], t["b"], A, dt, st_g, o_g[i], None,
                                              s=cap)
                assert rc == 0, f"capture call {i}: {rc}"
    torch.cuda.synchronize()
    for r in range(3):
        graph.replay()
        torch.cuda.synchronize()
        for i in range(2):                          # the eager reference: the same two tokens
            t = xs[i]
            assert bx.ix_gdn_decode(cfg, B, t["x"], cs_e, w, t["a"], t["b"], A, dt, st_e, o_e[i], None, ws) == 0
        _ = torch.ones(1024, device="cuda").sum()   # unrelated eager work between the replays
        torch.cuda.synchronize()
        for name, g, e in (("state", st_g, st_e), ("conv state", cs_g, cs_e), ("o", o_g, o_e)):
            assert np.array_equal(host(g), host(e)), f"replay {r}: {name} differs from the eager decode"
        print(f"replay {r}: bit-identical to eager ix_gdn_decode", flush=True)

    free0, _ = torch.cuda.mem_get_info()
    t = xs[0]
    for _ in range(4):
        assert bx.ix_gdn_decode_noalloc(cfg, B, t["x"], cs_g, w, t["a"], t["b"], A, dt, st_g, o_g[0], None) == 0
    torch.cuda.synchronize()
    free1, _ = torch.cuda.mem_get_info()
    assert free1 == free0, f"device free memory changed by {free0 - free1} bytes over eager no-allocation calls"
    print("ok", flush=True)


if __name__ == "__main__":
    main()
