"""GPU parity of the chunked prefill (ix_gdn_prefill) against the oracle's token-by-token
recurrence (oracle.prefill, double precision).

Tolerances, from the benchmark's acceptance rule: fp32 outputs within 1e-3 absolute of
the oracle; bf16 outputs exactly RNE of the kernel's own fp32 outputs; fp32 state
max|d|/max|ref| <= 1e-4 after the sequence (the reference's norm, tests/test_gdn.cu:10-13);
conv state bit-exact. Inputs come from the portable generator (oracle/inputs.py).
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


def gpu_prefill(cfg, cu, tok, p, st, outputs=("o", "ob"), window=None):
    """Runs ix_gdn_prefill on copies of the states; returns (conv_state, state, o, o_bf16). With
    window, the workspace holds windows of that many chunks only."""
    torch = _torch()
    cu = np.asarray(cu, np.int32)
    n, T = cu.size - 1, int(tok["x"].shape[0])
    d_cs, d_st = dev(st["conv_state"]), state_to_dev(st["state"])
    o = torch.full((T, cfg.h_v, cfg.d_v), float("nan"), dtype=torch.float32, device="cuda") if "o" in outputs else None
    ob = torch.zeros(T, cfg.h_v, cfg.d_v, dtype=torch.bfloat16, device="cuda") if "ob" in outputs else None
    need = (bx.ix_gdn_prefill_workspace_size(cfg, n, T) if window is None
            else bx.ix_gdn_prefill_window_workspace_size(cfg, n, T, window))
    assert need > 0
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    rc = bx.ix_gdn_prefill(cfg, n, T, dev(cu), dev(tok["x"]), d_cs, dev(p["w"]), dev(tok["a"]), dev(tok["b"]),
                           dev(p["A_log"]), dev(p["dt_bias"]), d_st, o, ob, ws, need)
    assert rc == 0, rc
    torch.cuda.synchronize()
    return (host(d_cs), state_from_dev(d_st), None if o is None else host(o), None if ob is None else host(ob))


def oracle_prefill(cfg, cu, tok, p, st):
    return oracle.prefill(cfg, cu, tok["x"], st["conv_state"], p["w"], tok["a"], tok["b"], p["A_log"],
                          p["dt_bias"], st["state"], nthreads=NT)


def check(cfg, cu, seed, state_std=0.02, conv_std=1.0, extreme=False):
    cu = np.asarray(cu, np.int32)
    n, T = cu.size - 1, int(cu[-1])
    p = inputs.layer_params(cfg, seed)
    tok = inputs.token_inputs(cfg, seed, max(T, 1))
    tok = {k: v[:T] for k, v in tok.items()}
    if extreme:
        p, tok = extreme_params(p), extreme_gates(cfg, tok, seed)
    st = inputs.initial_states(cfg, seed, n, state_std=state_std, conv_std=conv_std)
    cs, s, o, ob = gpu_prefill(cfg, cu, tok, p, st)
    rcs, rs, ro = oracle_prefill(cfg, cu, tok, p, st)
    np.testing.assert_array_equal(cs, rcs)
    rel = oracle.rel_err(s, rs)
    assert rel <= TOL_STATE_REL, f"state rel err {rel}"
    if T:
        err = float(np.max(np.abs(o - ro)))
        assert err <= TOL_O_ABS, f"o abs err {err}"
        np.testing.assert_array_equal(ob, bf16.from_f32(o))
    return rel


@pytest.mark.parametrize("T", [1, 5, 63, 64, 65, 200])
def test_single_sequence_lengths(T):
    check(oracle.make_cfg(), [0, T], inputs.seed_for(3) + T)


def test_varlen_with_empty_and_short_sequences():
    check(oracle.make_cfg(), [0, 0, 1, 65, 195, 198, 198, 260], inputs.seed_for(4))


@pytest.mark.parametrize("n", [1100, 4400])
def test_more_sequences_than_one_plan_pass(n):
    # The offsets are scanned in passes of 1024 threads, the running maximum and chunk count
    # carried between passes (two and five passes here). Most sequences are empty or a few
    # tokens long; a few span several chunks around pass boundaries.
    lens = np.floor(inputs.Gen(inputs.seed_for(4) + n).uniform(0x51, (n,)) * 5).astype(np.int64)
    for b in (1024, 4096):
        if b < n:
            lens[b - 4:b + 3] = [70, 0, 130, 1, 64, 0, 65]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    check(oracle.make_cfg(h_k=1, h_v=1), cu, inputs.seed_for(4) + n, state_std=0.0)


@pytest.mark.parametrize("kw", [
    dict(head_map=1),
    dict(conv_act=1),
    dict(q_scale=128 ** -0.5),
    dict(d_conv=2),
    dict(d_conv=3),
    dict(h_k=3, h_v=8),
    dict(h_k=4, h_v=2),
    dict(h_k=2, h_v=6, head_map=1),
    dict(h_k=1, h_v=1),
    dict(h_k=1, h_v=16),             # 16 v heads on one q/k head: the configuration limit
    dict(h_k=2, h_v=32, head_map=1), # 16 per source with the contiguous map
    dict(h_k=2, h_v=18),             # 9 per source (more than 8) with modulo pairing
])
def test_variants(kw):
    check(oracle.make_cfg(**kw), [0, 70, 71, 150], inputs.seed_for(3) + 11 * len(kw))


@pytest.mark.parametrize("frac", [0.05, 0.2])
def test_extreme_gates(frac):
    # Gate logits past softplus's threshold on both sides and beta logits at +-30 at seeded
    # positions (tests/common.py extreme_gates), A_log = ln 16 on every other head: decays
    # that underflow to 0 next to decays of ~1 inside one chunk, over several chunks.
    cfg = oracle.make_cfg()
    seed = inputs.seed_for(3) + int(frac * 100)
    cu = np.asarray([0, 260, 333], np.int32)
    p = extreme_params(inputs.layer_params(cfg, seed))
    tok = extreme_gates(cfg, inputs.token_inputs(cfg, seed, 333), seed, frac)
    st = inputs.initial_states(cfg, seed, 2)
    cs, s, o, ob = gpu_prefill(cfg, cu, tok, p, st)
    rcs, rs, ro = oracle_prefill(cfg, cu, tok, p, st)
    np.testing.assert_array_equal(cs, rcs)
    rel = oracle.rel_err(s, rs)
    assert rel <= TOL_STATE_REL, f"state rel err {rel}"
    err = float(np.max(np.abs(o - ro)))
    assert err <= TOL_O_ABS, f"o abs err {err}"
    np.testing.assert_array_equal(ob, bf16.from_f32(o))


@pytest.mark.parametrize("beta_logit", [None, 30.0])
def test_no_decay(beta_logit):
    # Every gate logit at -30: softplus(a + dt_bias) ~ 1e-13, so the decay is 1 to fp32
    # precision and A = beta (k_t . k_s) keeps its full weight across the whole chunk; the
    # blocks of T = (I + A)^-1 below the diagonal are then as large as they get (with
    # beta = 1 too in the second case). Several chunks, two sequences.
    cfg = oracle.make_cfg()
    seed = inputs.seed_for(3) + 41
    cu = np.asarray([0, 200, 333], np.int32)
    p = inputs.layer_params(cfg, seed)
    tok = dict(inputs.token_inputs(cfg, seed, 333))
    tok["a"] = bf16.from_f32(np.full(tok["a"].shape, -30.0, np.float32))
    if beta_logit is not None:
        tok["b"] = bf16.from_f32(np.full(tok["b"].shape, beta_logit, np.float32))
    st = inputs.initial_states(cfg, seed, 2)
    cs, s, o, ob = gpu_prefill(cfg, cu, tok, p, st)
    rcs, rs, ro = oracle_prefill(cfg, cu, tok, p, st)
    np.testing.assert_array_equal(cs, rcs)
    rel = oracle.rel_err(s, rs)
    assert rel <= TOL_STATE_REL, f"state rel err {rel}"
    err = float(np.max(np.abs(o - ro)))
    assert err <= TOL_O_ABS, f"o abs err {err}"
    np.testing.assert_array_equal(ob, bf16.from_f32(o))
    print(f"no decay, beta logit {beta_logit}: state rel err {rel:.3g}, o abs err {err:.3g}")


def test_zero_initial_state_config3_shape_short():
    check(oracle.make_cfg(), [0, 300], inputs.seed_for(3), state_std=0.0, conv_std=0.0)


def test_config3_full_T4096():
    # configuration 3: one sequence of 4096 tokens from a zero state.
    rel = check(oracle.make_cfg(), [0, 4096], inputs.seed_for(3), state_std=0.0, conv_std=0.0)
    print(f"T=4096 state rel err {rel:.2e}")


def test_prefill_matches_gpu_decode_loop():
    # The same tokens through T single-token decodes on the GPU give the same result.
    torch = _torch()
    cfg = bx.make_cfg()
    seed, T = inputs.seed_for(3) + 99, 70
    p = inputs.layer_params(cfg, seed)
    tok = inputs.token_inputs(cfg, seed, T)
    st = inputs.initial_states(cfg, seed, 1)
    cs, s, o, _ = gpu_prefill(cfg, [0, T], tok, p, st)
    d_cs, d_st = dev(st["conv_state"]), state_to_dev(st["state"])
    d_w, d_A, d_dt = dev(p["w"]), dev(p["A_log"]), dev(p["dt_bias"])
    od = torch.empty(1, cfg.h_v, cfg.d_v, dtype=torch.float32, device="cuda")
    ws = torch.zeros(bx.ix_gdn_decode_workspace_size(cfg, 1), dtype=torch.uint8, device="cuda")
    outs = []
    for t in range(T):
        assert bx.ix_gdn_decode(cfg, 1, dev(tok["x"][t:t + 1]), d_cs, d_w, dev(tok["a"][t:t + 1]),
                                dev(tok["b"][t:t + 1]), d_A, d_dt, d_st, od, None, ws) == 0
        outs.append(host(od)[0].copy())
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(d_cs), cs)
    assert float(np.max(np.abs(np.stack(outs) - o))) <= TOL_O_ABS
    assert oracle.rel_err(s, state_from_dev(d_st)) <= TOL_STATE_REL


def test_config4_varlen_prefill_then_decode():
    # configuration 4 as stated: 32 sequences with lengths ~ U[1, 2048] packed by cu_seqlens,
    # initial states N(0, 0.02), then 32 decode steps per sequence from the carried conv and
    # recurrent states; outputs of every decode step checked, states at the end.
    torch = _torch()
    cfg = bx.make_cfg()
    seed, n, steps = inputs.seed_for(4), 32, 32
    cu = inputs.varlen(seed, n, 1, 2048)
    T = int(cu[-1])
    p = inputs.layer_params(cfg, seed)
    tok = inputs.token_inputs(cfg, seed, T)
    st = inputs.initial_states(cfg, seed, n)
    cs, s, o, _ = gpu_prefill(cfg, cu, tok, p, st)
    rcs, rs, ro = oracle_prefill(cfg, cu, tok, p, st)
    np.testing.assert_array_equal(cs, rcs)
    assert oracle.rel_err(s, rs) <= TOL_STATE_REL
    assert float(np.max(np.abs(o - ro))) <= TOL_O_ABS
    d_cs, d_st = dev(cs), state_to_dev(s)
    d_w, d_A, d_dt = dev(p["w"]), dev(p["A_log"]), dev(p["dt_bias"])
    od = torch.empty(n, cfg.h_v, cfg.d_v, dtype=torch.float32, device="cuda")
    ws = torch.zeros(bx.ix_gdn_decode_workspace_size(cfg, n), dtype=torch.uint8, device="cuda")
    for k in range(steps):
        t = inputs.token_inputs(cfg, seed, n, step=1000 + k)
        assert bx.ix_gdn_decode(cfg, n, dev(t["x"]), d_cs, d_w, dev(t["a"]), dev(t["b"]), d_A, d_dt, d_st, od,
                                None, ws) == 0
        rcs, rs, rod = oracle.decode(cfg, n, t["x"], rcs, p["w"], t["a"], t["b"], p["A_log"], p["dt_bias"], rs,
                                     nthreads=NT)
        torch.cuda.synchronize()
        assert float(np.max(np.abs(host(od) - rod))) <= TOL_O_ABS, k
    np.testing.assert_array_equal(host(d_cs), rcs)
    assert oracle.rel_err(state_from_dev(d_st), rs) <= TOL_STATE_REL


@pytest.mark.parametrize("window", [1, 2, 3])
@pytest.mark.parametrize("cu", [[0, 300], [0, 0, 1, 65, 195, 198, 198, 260], [10, 290]], ids=["one", "varlen", "offset"])
def test_windows_match_one_window(cu, window):
    # A workspace for windows of a few chunks runs the batch window by window; every chunk's
    # arithmetic is the same, so the results are bit-identical to the one-window run,
    # including a sequence split across windows and conv history carried between them.
    cfg = bx.make_cfg()
    seed = inputs.seed_for(3) + 71 + window
    n, T = len(cu) - 1, 300
    p = inputs.layer_params(cfg, seed)
    tok = inputs.token_inputs(cfg, seed, T)
    st = inputs.initial_states(cfg, seed, n)
    full = gpu_prefill(cfg, cu, tok, p, st)
    win = gpu_prefill(cfg, cu, tok, p, st, window=window)
    for a, b in zip(full, win):
        np.testing.assert_array_equal(a, b)


def test_windows_with_many_sequences():
    # 600 short sequences, a third of them empty, in windows of two chunks: each window's chain
    # workgroups walk its chunks across sequence boundaries, in 8 groups cut at sequence starts
    # (h_v * 8 = 32 strips), resuming states and histories the previous windows left.
    cfg = bx.make_cfg(h_k=2, h_v=4)
    rng = np.random.default_rng(inputs.seed_for(4) + 9)
    lens = rng.integers(1, 100, 600)
    lens[rng.random(600) < 0.3] = 0
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    n, T = 600, int(cu[-1])
    seed = inputs.seed_for(4) + 10
    p = inputs.layer_params(cfg, seed)
    tok = inputs.token_inputs(cfg, seed, T)
    st = inputs.initial_states(cfg, seed, n)
    full = gpu_prefill(cfg, cu, tok, p, st)
    win = gpu_prefill(cfg, cu, tok, p, st, window=2)
    for a, b in zip(full, win):
        np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("case", range(6))
def test_random_batches(case):
    # Seeded random batches: head layout, sequence count and lengths (empty ones included),
    # initial state scale and window size drawn per case; against the oracle, and the windowed
    # run bit-identical to the one-window run.
    rng = np.random.default_rng(inputs.seed_for(4) + 1000 + case)
    h_k, h_v = [(1, 1), (1, 2), (2, 4), (2, 6), (4, 8), (3, 3)][case]
    cfg = bx.make_cfg(h_k=h_k, h_v=h_v, head_map=int(rng.integers(0, 2)), conv_act=int(rng.integers(0, 2)))
    n = int(rng.integers(1, 10))
    lens = rng.integers(0, 200, n)
    lens[rng.random(n) < 0.2] = 0
    lens[-1] = max(int(lens[-1]), 1)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    T = int(cu[-1])
    seed = inputs.seed_for(4) + 2000 + case
    p = inputs.layer_params(cfg, seed)
    tok = inputs.token_inputs(cfg, seed, T)
    st = inputs.initial_states(cfg, seed, n, state_std=float(rng.choice([0.0, 0.02, 0.5])))
    full = gpu_prefill(cfg, cu, tok, p, st)
    cs, s, o, ob = full
    rcs, rs, ro = oracle_prefill(cfg, cu, tok, p, st)
    np.testing.assert_array_equal(cs, rcs)
    assert oracle.rel_err(s, rs) <= TOL_STATE_REL
    assert float(np.max(np.abs(o - ro))) <= TOL_O_ABS
    np.testing.assert_array_equal(ob, bf16.from_f32(o))
    win = gpu_prefill(cfg, cu, tok, p, st, window=int(rng.integers(1, 4)))
    for a, b in zip(full, win):
        np.testing.assert_array_equal(a, b)


def test_state_only_and_repeatable():
    cfg = bx.make_cfg()
    seed = inputs.seed_for(3) + 5
    cu = [0, 100, 229]
    p = inputs.layer_params(cfg, seed)
    tok = inputs.token_inputs(cfg, seed, 229)
    st = inputs.initial_states(cfg, seed, 2)
    a = gpu_prefill(cfg, cu, tok, p, st)
    b = gpu_prefill(cfg, cu, tok, p, st, outputs=())
    np.testing.assert_array_equal(a[0], b[0])
    np.testing.assert_array_equal(a[1], b[1])        # deterministic, outputs optional


def test_non_monotone_cu_seqlens_is_clamped_in_bounds():
    # A decreasing offset is clamped to a running maximum (an empty sequence); nothing is
    # read or written outside the buffers and the other sequences are unaffected.
    cfg = bx.make_cfg(h_k=2, h_v=4)
    seed = inputs.seed_for(4) + 1
    p = inputs.layer_params(cfg, seed)
    tok = inputs.token_inputs(cfg, seed, 90)
    st = inputs.initial_states(cfg, seed, 3)
    cs, s, o, _ = gpu_prefill(cfg, [0, 40, 30, 90], tok, p, st)
    rcs, rs, ro = oracle_prefill(cfg, [0, 40, 40, 90], tok, p, st)
    np.testing.assert_array_equal(cs, rcs)
    assert oracle.rel_err(s, rs) <= TOL_STATE_REL
    assert float(np.max(np.abs(o - ro))) <= TOL_O_ABS


@pytest.mark.parametrize("cu,T", [([10, 70], 100), ([-5, 200], 100), ([50, 20], 100), ([30, 30], 40)])
def test_single_sequence_bounds_are_clamped(cu, T):
    # One sequence takes its bounds straight from cu (there is no plan pass for n_seq = 1),
    # with the plan's clamping: lo = clamp(cu[0], 0, T), hi = max(clamp(cu[1], 0, T), lo).
    # Tokens outside [lo, hi) are neither read into the state nor written to o.
    cfg = bx.make_cfg(h_k=2, h_v=4)
    seed = inputs.seed_for(4) + 11 + cu[0] + 7 * cu[1]
    p = inputs.layer_params(cfg, seed)
    tok = inputs.token_inputs(cfg, seed, T)
    st = inputs.initial_states(cfg, seed, 1)
    cs, s, o, _ = gpu_prefill(cfg, cu, tok, p, st)
    lo = min(max(cu[0], 0), T)
    hi = max(min(max(cu[1], 0), T), lo)
    assert np.isnan(o[:lo]).all() and np.isnan(o[hi:]).all()
    if hi == lo:
        np.testing.assert_array_equal(cs, st["conv_state"])
        np.testing.assert_array_equal(s, st["state"].astype(s.dtype))
        return
    sub = {k: v[lo:hi] for k, v in tok.items()}
    rcs, rs, ro = oracle_prefill(cfg, [0, hi - lo], sub, p, st)
    np.testing.assert_array_equal(cs, rcs)
    assert oracle.rel_err(s, rs) <= TOL_STATE_REL
    assert float(np.max(np.abs(o[lo:hi] - ro))) <= TOL_O_ABS
