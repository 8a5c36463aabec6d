"""GPU parity of the speculative-window calls (ix_gdn_decode_window, ix_gdn_commit_window).

Two verify paths. The exact one (ix_gdn_decode_window) must give outputs bit-identical to K
ix_gdn_decode calls on the same states (the kernels share the column math). The matrix-core
one (ix_gdn_decode_window_mfma) computes the same outputs in the K-token space from S^T k and
S^T q: within 1e-4 absolute of the decode calls' outputs (fp32 and split-bf16 rounding), and
its window record must be bit-identical to the exact path's. Either verify must leave both
states untouched, and commit with n accepted tokens must leave the states bit-identical to n
decode calls; against the double oracle the decode tolerances hold (fp32 outputs 1e-3
absolute, state max|d|/max|ref| <= 1e-4, conv state bit-exact). Accepted counts are clamped
to [0, K].
"""
import numpy as np
import pytest

import baloon_amd as bx
import oracle
from oracle import bf16, inputs
from tests.common import (NT, TOL_O_ABS, TOL_STATE_REL, dev, extreme_gates, extreme_params, host, state_from_dev,
                          state_to_dev)

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    return torch


TOL_MFMA_VS_DECODE = 1e-4
MODES = [pytest.param("exact", id="exact"), pytest.param("mfma", id="mfma")]


def window_case(cfg, B, K, accepted, seed, extreme=False, mode="exact"):
    torch = _torch()
    p = inputs.layer_params(cfg, seed)
    st = inputs.initial_states(cfg, seed, B)
    tok = inputs.token_inputs(cfg, seed, B * K)                      # row b*K + t
    if extreme:
        p, tok = extreme_params(p), extreme_gates(cfg, tok, seed)
    x = tok["x"].reshape(B, K, -1)
    a = tok["a"].reshape(B, K, -1)
    b = tok["b"].reshape(B, K, -1)
    d_w, d_A, d_dt = dev(p["w"]), dev(p["A_log"]), dev(p["dt_bias"])
    d_x, d_a, d_b = dev(x), dev(a), dev(b)

    # verify
    d_cs, d_st = dev(st["conv_state"]), state_to_dev(st["state"])
    cs0, st0 = host(d_cs).copy(), host(d_st).copy()
    # zeroed: the record's sections are padded to 256 bytes, and the comparison below of the
    # two verifies' records covers the padding too
    rec = torch.zeros(bx.ix_gdn_window_record_size(cfg, B, K), dtype=torch.uint8, device="cuda")
    o_win = torch.full((B, K, cfg.h_v, cfg.d_v), float("nan"), dtype=torch.float32, device="cuda")
    ob_win = torch.zeros(B, K, cfg.h_v, cfg.d_v, dtype=torch.bfloat16, device="cuda")
    verify = bx.ix_gdn_decode_window if mode == "exact" else bx.ix_gdn_decode_window_mfma
    assert verify(cfg, B, K, d_x, d_cs, d_w, d_a, d_b, d_A, d_dt, d_st, o_win, ob_win, rec) == 0
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(d_st), st0)                    # verify changes no state
    np.testing.assert_array_equal(host(d_cs), cs0)
    o_win = host(o_win)
    np.testing.assert_array_equal(host(ob_win), bf16.from_f32(o_win))
    if mode == "mfma":                                                # the same record as the exact verify
        rec_exact = torch.zeros_like(rec)
        assert bx.ix_gdn_decode_window(cfg, B, K, d_x, d_cs, d_w, d_a, d_b, d_A, d_dt, d_st, None, None,
                                       rec_exact) == 0
        torch.cuda.synchronize()
        np.testing.assert_array_equal(host(rec), host(rec_exact), err_msg="window record")

    # the same tokens through K decode calls, keeping the states after each
    l_cs, l_st = dev(st["conv_state"]), state_to_dev(st["state"])
    ws = torch.zeros(bx.ix_gdn_decode_workspace_size(cfg, B), dtype=torch.uint8, device="cuda")
    od = torch.empty(B, cfg.h_v, cfg.d_v, dtype=torch.float32, device="cuda")
    after = [(cs0, st0)]
    for t in range(K):
        assert bx.ix_gdn_decode(cfg, B, dev(x[:, t]), l_cs, d_w, dev(a[:, t]), dev(b[:, t]), d_A, d_dt, l_st, od,
                                None, ws) == 0
        torch.cuda.synchronize()
        if mode == "exact":
            np.testing.assert_array_equal(o_win[:, t], host(od), err_msg=f"window output t={t}")
        else:
            err = float(np.max(np.abs(o_win[:, t] - host(od))))
            assert err <= TOL_MFMA_VS_DECODE, f"window output t={t}: {err} from the decode call's"
        after.append((host(l_cs).copy(), host(l_st).copy()))

    # commit
    acc = np.asarray(accepted, np.int32)
    assert bx.ix_gdn_commit_window(cfg, B, K, dev(acc), d_x, rec, d_cs, d_st) == 0
    torch.cuda.synchronize()
    cs1, st1 = host(d_cs), host(d_st)
    for bi in range(B):
        n = int(min(max(acc[bi], 0), K))
        np.testing.assert_array_equal(cs1[bi], after[n][0][bi], err_msg=f"conv state b={bi} n={n}")
        np.testing.assert_array_equal(st1[bi], after[n][1][bi], err_msg=f"state b={bi} n={n}")

    # against the double oracle: outputs of the whole window, states after each prefix
    rcs, rst = st["conv_state"], st["state"].astype(np.float64)
    ref = [(rcs, rst)]
    for t in range(K):
        rcs, rst, ro = oracle.decode(cfg, B, x[:, t], rcs, p["w"], a[:, t], b[:, t], p["A_log"], p["dt_bias"], rst,
                                     nthreads=NT)
        assert float(np.max(np.abs(o_win[:, t] - ro))) <= TOL_O_ABS
        ref.append((rcs, rst))
    for bi in range(B):
        n = int(min(max(acc[bi], 0), K))
        np.testing.assert_array_equal(cs1[bi], ref[n][0][bi])
        got = np.swapaxes(st1[bi], -1, -2)
        assert oracle.rel_err(got, ref[n][1][bi]) <= TOL_STATE_REL


@pytest.mark.parametrize("K,accepted", [
    (4, [0, 1, 2, 3, 4, 4]),
    (1, [1, 0, -2, 7, 1, 1]),
    (8, [8, 5, 0, 13, 3, -1]),
    (16, [16, 3, 0, 16, 15, 7]),                      # the largest window
    (5, [5, 2, 0, 7, 5, 1]),                          # size class 8 partly filled (k and q share a tile)
    (12, [12, 9, 0, 13, 4, 12]),                      # size class 16 partly filled (separate k, q tiles)
])
@pytest.mark.parametrize("mode", MODES)
def test_window_verify_and_commit(K, accepted, mode):
    window_case(bx.make_cfg(), 6, K, accepted, inputs.seed_for(2) + 50 + K, mode=mode)


@pytest.mark.parametrize("kw", [dict(head_map=1, h_k=4, h_v=12), dict(d_conv=2), dict(d_conv=3, conv_act=1),
                                dict(h_k=3, h_v=8, q_scale=0.125), dict(h_k=1, h_v=16), dict(h_k=2, h_v=18),
                                dict(h_k=2, h_v=32, head_map=1)])
@pytest.mark.parametrize("mode", MODES)
def test_window_variants(kw, mode):
    window_case(bx.make_cfg(**kw), 3, 3, [3, 1, 2], inputs.seed_for(2) + 60 + len(kw) + kw.get("h_v", 0), mode=mode)


@pytest.mark.parametrize("mode", MODES)
def test_window_extreme_gates(mode):
    # gate logits past softplus's threshold on both sides, beta logits at +-30, A_log = ln 16
    window_case(bx.make_cfg(), 6, 8, [8, 5, 0, 3, 7, 1], inputs.seed_for(2) + 90, extreme=True, mode=mode)


def test_window_mfma_at_bench_shape():
    # configuration 2's batch, K = 4, all accepted: the shape the benchmark times
    window_case(bx.make_cfg(), 64, 4, [4] * 64, inputs.seed_for(2) + 95, mode="mfma")


def test_window_then_decode_continues():
    # After a commit the states continue under ix_gdn_decode like any others.
    torch = _torch()
    cfg = bx.make_cfg()
    B, K, seed = 4, 3, inputs.seed_for(2) + 71
    p = inputs.layer_params(cfg, seed)
    st = inputs.initial_states(cfg, seed, B)
    tok = inputs.token_inputs(cfg, seed, B * K)
    x, a, b = (tok[n].reshape(B, K, -1) for n in ("x", "a", "b"))
    d_w, d_A, d_dt = dev(p["w"]), dev(p["A_log"]), dev(p["dt_bias"])
    d_cs, d_st = dev(st["conv_state"]), state_to_dev(st["state"])
    rec = torch.empty(bx.ix_gdn_window_record_size(cfg, B, K), dtype=torch.uint8, device="cuda")
    assert bx.ix_gdn_decode_window(cfg, B, K, dev(x), d_cs, d_w, dev(a), dev(b), d_A, d_dt, d_st, None, None,
                                   rec) == 0
    acc = np.array([2, 0, 3, 1], np.int32)
    assert bx.ix_gdn_commit_window(cfg, B, K, dev(acc), dev(x), rec, d_cs, d_st) == 0
    rcs, rst = st["conv_state"].copy(), st["state"].astype(np.float64)
    for bi in range(B):
        for t in range(int(acc[bi])):
            c1, s1, _ = oracle.decode(cfg, 1, x[bi:bi + 1, t], rcs[bi:bi + 1], p["w"], a[bi:bi + 1, t],
                                      b[bi:bi + 1, t], p["A_log"], p["dt_bias"], rst[bi:bi + 1])
            rcs[bi], rst[bi] = c1[0], s1[0]
    ws = torch.zeros(bx.ix_gdn_decode_workspace_size(cfg, B), dtype=torch.uint8, device="cuda")
    od = torch.empty(B, cfg.h_v, cfg.d_v, dtype=torch.float32, device="cuda")
    for k in range(4):
        t = inputs.token_inputs(cfg, seed, B, step=100 + k)
        assert bx.ix_gdn_decode(cfg, B, dev(t["x"]), d_cs, d_w, dev(t["a"]), dev(t["b"]), d_A, d_dt, d_st, od, None,
                                ws) == 0
        rcs, rst, ro = oracle.decode(cfg, B, t["x"], rcs, p["w"], t["a"], t["b"], p["A_log"], p["dt_bias"], rst,
                                     nthreads=NT)
        torch.cuda.synchronize()
        assert float(np.max(np.abs(host(od) - ro))) <= TOL_O_ABS
    np.testing.assert_array_equal(host(d_cs), rcs)
    assert oracle.rel_err(state_from_dev(d_st), rst) <= TOL_STATE_REL


@pytest.mark.parametrize("kw", [dict(), dict(d_conv=3, h_k=2, h_v=6, head_map=1)])
def test_commit_layers_matches_per_layer_commits(kw):
    # ix_gdn_commit_window_layers over 4 layers (each with its own parameters, window inputs,
    # record, conv state and state) must leave every layer bit-identical to one
    # ix_gdn_commit_window call per layer; a fifth table entry with a null state is skipped.
    torch = _torch()
    cfg = bx.make_cfg(**kw)
    B, K, nl = 6, 4, 4
    acc = dev(np.array([0, 1, 2, 3, 4, 9], np.int32))
    layers = []
    for l in range(nl):
        seed = inputs.seed_for(2) + 700 + 13 * l
        p = inputs.layer_params(cfg, seed)
        st = inputs.initial_states(cfg, seed, B)
        tok = inputs.token_inputs(cfg, seed, B * K)
        x, a, b = (dev(tok[n].reshape(B, K, -1)) for n in ("x", "a", "b"))
        cs, s = dev(st["conv_state"]), state_to_dev(st["state"])
        rec = torch.zeros(bx.ix_gdn_window_record_size(cfg, B, K), dtype=torch.uint8, device="cuda")
        assert bx.ix_gdn_decode_window_mfma(cfg, B, K, x, cs, dev(p["w"]), a, b, dev(p["A_log"]),
                                            dev(p["dt_bias"]), s, None, None, rec) == 0
        layers.append(dict(x=x, rec=rec, cs1=cs.clone(), st1=s.clone(), cs2=cs.clone(), st2=s.clone()))
    for L in layers:
        assert bx.ix_gdn_commit_window(cfg, B, K, acc, L["x"], L["rec"], L["cs1"], L["st1"]) == 0
    spare_cs, spare_x, spare_rec = layers[0]["cs2"].clone(), layers[0]["x"], layers[0]["rec"]
    spare_before = host(spare_cs).copy()
    tables = [bx.layer_pointer_table([L[n] for L in layers] + [extra])
              for n, extra in (("x", spare_x), ("rec", spare_rec), ("cs2", spare_cs))]
    st_table = torch.tensor([L["st2"].data_ptr() for L in layers] + [0], dtype=torch.int64).cuda()
    assert bx.ix_gdn_commit_window_layers(cfg, B, K, acc, tables[0], tables[1], tables[2], st_table) == 0
    torch.cuda.synchronize()
    for l, L in enumerate(layers):
        np.testing.assert_array_equal(host(L["cs2"]), host(L["cs1"]), err_msg=f"layer {l} conv state")
        np.testing.assert_array_equal(host(L["st2"]), host(L["st1"]), err_msg=f"layer {l} state")
    np.testing.assert_array_equal(host(spare_cs), spare_before, err_msg="the skipped entry was written")

