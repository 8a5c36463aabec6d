"""Pins for the CPU oracle (runs without a GPU).

The reference ships no golden vectors for the GDN path (its test regenerates inputs from
std::mt19937, tests/test_gdn.cu:15), and no reference code can run here (CUDA-only, and
src/ix_compat.h:4-6 refuses any non-Iluvatar build). So every oracle function is pinned by
checks that a plausible mistake would fail: known answers, invariants, one-hot layout
probes, brute force against a differently-structured formulation, and composition of the
fused oracle from the legacy ones.
"""
import math

import numpy as np
import pytest

import oracle
from oracle import bf16, inputs


def rng(seed):
    return np.random.default_rng(seed)


def as_heads(st, S, h_v):
    """Legacy state [S(i)][h_v][S(j)] -> [h_v][i][j]."""
    return np.asarray(st).reshape(S, h_v, S).transpose(1, 0, 2)


# ------------------------------------------------------------------------------------------
# legacy step: tests/test_gdn.cu:22-26
# ------------------------------------------------------------------------------------------

def _rand_step(r, S, hk, hv):
    st = (r.standard_normal(S * hv * S) * 0.1).astype(np.float32)
    q = (r.standard_normal(hk * S) * 0.1).astype(np.float32)
    k = (r.standard_normal(hk * S) * 0.1).astype(np.float32)
    v = r.standard_normal(hv * S).astype(np.float32)
    gate = (-np.abs(r.standard_normal(hv))).astype(np.float32)
    beta = (0.5 + 0.4 * np.tanh(r.standard_normal(hv))).astype(np.float32)
    return st, q, k, v, gate, beta


def test_step_beta_zero_is_pure_decay():
    S, hk, hv = 16, 2, 4
    st, q, k, v, gate, _ = _rand_step(rng(1), S, hk, hv)
    beta = np.zeros(hv, np.float32)
    rs, ro = oracle.step(st, q, k, v, gate, beta, S, hk, hv)
    M0, M1 = as_heads(st.astype(np.float64), S, hv), as_heads(rs, S, hv)
    for h in range(hv):
        g = math.exp(float(gate[h]))
        src = h % hk
        np.testing.assert_allclose(M1[h], g * M0[h], rtol=1e-14, atol=0)
        np.testing.assert_allclose(ro[h * S:(h + 1) * S], g * M0[h].T @ q[src * S:(src + 1) * S].astype(np.float64),
                                   rtol=1e-12, atol=1e-15)


def test_step_zero_state_is_outer_product():
    S, hk, hv = 8, 3, 6
    _, q, k, v, gate, beta = _rand_step(rng(2), S, hk, hv)
    rs, ro = oracle.step(np.zeros(S * hv * S, np.float32), q, k, v, gate, beta, S, hk, hv)
    M = as_heads(rs, S, hv)
    for h in range(hv):
        src = h % hk
        kk = k[src * S:(src + 1) * S].astype(np.float64)
        qq = q[src * S:(src + 1) * S].astype(np.float64)
        vv = v[h * S:(h + 1) * S].astype(np.float64)
        np.testing.assert_allclose(M[h], float(beta[h]) * np.outer(kk, vv), rtol=1e-12, atol=1e-16)
        np.testing.assert_allclose(ro[h * S:(h + 1) * S], float(beta[h]) * (kk @ qq) * vv, rtol=1e-10, atol=1e-16)


def test_step_unit_key_full_beta_stores_v_exactly():
    # With beta = 1 and |k| = 1 the post-update S'^T k equals v for ANY decay -- but only if
    # the decay is applied before the k^T S read (src/ix_gdn.cu:49-50).
    S, hk, hv = 12, 2, 4
    st, q, k, v, gate, _ = _rand_step(rng(3), S, hk, hv)
    for src in range(hk):
        seg = k[src * S:(src + 1) * S].astype(np.float64)
        k[src * S:(src + 1) * S] = (seg / np.linalg.norm(seg)).astype(np.float32)
    beta = np.ones(hv, np.float32)
    gate[:] = -0.7
    rs, _ = oracle.step(st, q, k, v, gate, beta, S, hk, hv)
    M = as_heads(rs, S, hv)
    for h in range(hv):
        kk = k[(h % hk) * S:(h % hk + 1) * S].astype(np.float64)   # |k|^2 = 1 + O(1e-7) after fp32 rounding
        np.testing.assert_allclose(M[h].T @ kk, v[h * S:(h + 1) * S], rtol=0, atol=1e-5)


def test_step_one_hot_layout_and_pairing():
    # A single 1 at state element (h0, i0, j0) = index (i0*h_v + h0)*S + j0 (src/ix_gdn.cu:47-48),
    # beta = 0, gate = 0: o[h0][j0] = q[src][i0] and nothing else moves.
    S, hk, hv = 6, 2, 5
    for (h0, i0, j0) in [(0, 0, 0), (3, 2, 5), (4, 5, 1)]:
        st = np.zeros(S * hv * S, np.float32)
        st[(i0 * hv + h0) * S + j0] = 1.0
        q = np.arange(1, hk * S + 1, dtype=np.float32)
        k = np.zeros(hk * S, np.float32)
        v = np.zeros(hv * S, np.float32)
        rs, ro = oracle.step(st, q, k, v, np.zeros(hv, np.float32), np.zeros(hv, np.float32), S, hk, hv)
        expect = np.zeros(hv * S)
        expect[h0 * S + j0] = q[(h0 % hk) * S + i0]      # modulo pairing, src/ix_gdn.cu:38
        np.testing.assert_array_equal(ro, expect)
        np.testing.assert_array_equal(rs, st.astype(np.float64))


def test_step_modulo_not_division_pairing():
    # h_k=2, h_v=4: head 1 pairs with src 1 (mod), not src 0 (h // 2).
    S, hk, hv = 4, 2, 4
    q = np.concatenate([np.ones(S), 2 * np.ones(S)]).astype(np.float32)
    k = np.concatenate([np.ones(S), 3 * np.ones(S)]).astype(np.float32)
    v = np.ones(hv * S, np.float32)
    beta = np.ones(hv, np.float32)
    _, ro = oracle.step(np.zeros(S * hv * S, np.float32), q, k, v, np.zeros(hv, np.float32), beta, S, hk, hv)
    kq = [S * 1.0 * 1.0, S * 3.0 * 2.0]
    for h in range(hv):
        np.testing.assert_allclose(ro[h * S:(h + 1) * S], kq[h % hk])


@pytest.mark.parametrize("S,hk,hv", [(2, 1, 1), (3, 2, 3), (4, 3, 6), (4, 4, 4)])
def test_step_brute_force_product_form(S, hk, hv):
    # Independent formulation: S' = (I - beta k k^T)(g S) + beta k v^T, o = S'^T q.
    r = rng(10 + S + hk)
    st, q, k, v, gate, beta = _rand_step(r, S, hk, hv)
    rs, ro = oracle.step(st, q, k, v, gate, beta, S, hk, hv)
    M0, M1 = as_heads(st.astype(np.float64), S, hv), as_heads(rs, S, hv)
    for h in range(hv):
        src = h % hk
        kk = k[src * S:(src + 1) * S].astype(np.float64)
        qq = q[src * S:(src + 1) * S].astype(np.float64)
        vv = v[h * S:(h + 1) * S].astype(np.float64)
        g, b = math.exp(float(gate[h])), float(beta[h])
        Sn = (np.eye(S) - b * np.outer(kk, kk)) @ (g * M0[h]) + b * np.outer(kk, vv)
        np.testing.assert_allclose(M1[h], Sn, rtol=1e-12, atol=1e-14)
        np.testing.assert_allclose(ro[h * S:(h + 1) * S], Sn.T @ qq, rtol=1e-11, atol=1e-14)


# ------------------------------------------------------------------------------------------
# conv, l2, beta, out_norm: tests/test_gdn.cu:36-54
# ------------------------------------------------------------------------------------------

@pytest.mark.parametrize("dc", [2, 3, 4])
def test_conv_tap_order_and_exact_shift(dc):
    C = 7
    r = rng(dc)
    cs = r.standard_normal(C * (dc - 1)).astype(np.float32)
    x = r.standard_normal(C).astype(np.float32)
    for tap in range(dc):
        w = np.zeros(C * dc, np.float32)
        w[np.arange(C) * dc + tap] = 1.0
        cs2, out = oracle.conv_step(cs, x, w, C, dc)
        hist = cs.reshape(C, dc - 1)
        expect = x if tap == dc - 1 else hist[:, tap]          # oldest first, x last
        np.testing.assert_array_equal(out, expect.astype(np.float64))
        shifted = np.concatenate([hist[:, 1:], x[:, None]], axis=1).ravel()
        np.testing.assert_array_equal(cs2, shifted)


def test_conv_state_holds_last_inputs():
    C, dc = 5, 4
    r = rng(7)
    cs = r.standard_normal(C * (dc - 1)).astype(np.float32)
    w = r.standard_normal(C * dc).astype(np.float32)
    xs = [r.standard_normal(C).astype(np.float32) for _ in range(dc - 1)]
    for x in xs:
        cs, _ = oracle.conv_step(cs, x, w, C, dc)
    np.testing.assert_array_equal(cs.reshape(C, dc - 1), np.stack(xs, axis=1))


@pytest.mark.parametrize("cols", [1, 7, 64, 65, 128, 1024])
def test_l2_invariant(cols):
    rows, eps = 5, 1e-6
    x = rng(cols).standard_normal(rows * cols).astype(np.float32)
    r = oracle.l2_norm(x, rows, cols, eps).reshape(rows, cols)
    xs = x.reshape(rows, cols).astype(np.float64)
    s = (xs * xs).sum(1)
    np.testing.assert_allclose((r * r).sum(1), s / (s + eps), rtol=1e-6)
    ratio = r / xs                                              # one float inverse per row
    np.testing.assert_allclose(ratio, ratio[:, :1] * np.ones_like(ratio), rtol=2e-7, atol=0)


def test_beta_and_softplus_closed_forms():
    b = np.array([0.0, 1.0, -1.0, 30.0, -30.0], np.float32)
    r = oracle.beta_gate(b)
    assert r[0] == 0.5
    assert abs(r[1] + r[2] - 1.0) < 1e-15                      # sigmoid(-x) = 1 - sigmoid(x)
    assert abs(r[1] - 0.7310585786300049) < 1e-15
    assert abs(oracle.softplus(0.0) - math.log(2.0)) < 1e-15
    assert oracle.softplus(20.5) == 20.5                        # threshold 20, src/ix_gdn.cu:22
    assert abs(oracle.softplus(-30.0) - math.exp(-30.0)) < 1e-25
    assert abs(oracle.gate(0.0, 0.0, 0.0) + math.log(2.0)) < 1e-15   # decay = 1/2
    al = float(np.float32(math.log(4.0)))                       # A_log is an fp32 parameter
    assert abs(oracle.gate(al, 0.5, -0.5) + math.exp(al) * math.log(2.0)) < 1e-12


def test_out_norm_constant_row():
    hv, S, eps = 3, 16, 1e-6
    c = np.array([0.5, -2.0, 3.0])
    o = np.repeat(c, S).astype(np.float32)
    z = np.zeros(hv * S, np.float32)
    nrm = np.linspace(0.5, 1.5, S).astype(np.float32)
    y = oracle.out_norm(o, z, nrm, hv, S, eps).reshape(hv, S)
    for h in range(hv):
        np.testing.assert_allclose(y[h], c[h] / math.sqrt(c[h] ** 2 + eps) * nrm * 0.5, rtol=2e-7)


def test_out_norm_mean_of_squares_and_gate_sign():
    # Half the row at a, half at b: mean(o^2) = (a^2 + b^2) / 2 (a sum or a wrong divisor fails);
    # z = +-ln 3 gives sigmoid 3/4 and 1/4 (a sign error in the gate swaps them).
    S, eps = 8, 0.0
    a, b = 3.0, 4.0
    o = np.array([a] * 4 + [b] * 4, np.float32)
    z = np.array([math.log(3.0), -math.log(3.0)] * 4, np.float32)
    nrm = np.full(S, 2.0, np.float32)
    y = oracle.out_norm(o, z, nrm, 1, S, eps)
    rms = math.sqrt((a * a + b * b) / 2)
    want = o / rms * 2.0 * np.array([0.75, 0.25] * 4)
    np.testing.assert_allclose(y, want, rtol=1e-6)


def test_gated_out_rows_and_bf16_gate():
    # gated_out normalises each (row, head) of [rows][h_v][d_v] on its own, with z given as
    # bf16 bits: constant rows c give sign(c) * nrm * sigmoid(z) (eps = 0).
    rows, hv, S = 2, 3, 16
    c = np.array([[1.0, -2.0, 0.5], [4.0, -0.25, 8.0]])
    o = np.repeat(c[..., None], S, axis=-1)
    zf = np.array([0.0, 1.0, -1.0], np.float32)
    z_bits = np.broadcast_to(bf16.from_f32(zf)[None, :, None], (rows, hv, S)).copy()
    nrm = np.linspace(0.5, 1.5, S).astype(np.float32)
    y = oracle.gated_out(o, z_bits, nrm, 0.0)
    sig = 1.0 / (1.0 + np.exp(-zf.astype(np.float64)))
    want = np.sign(c)[..., None] * nrm[None, None, :] * sig[None, :, None]
    np.testing.assert_allclose(y, want, rtol=1e-6)


# ------------------------------------------------------------------------------------------
# fused decode and prefill (extensions)
# ------------------------------------------------------------------------------------------

def _small_cfg(**kw):
    base = dict(h_k=2, h_v=4, d_k=8, d_v=8, d_conv=4)
    base.update(kw)
    return oracle.make_cfg(**base)


def _fused_inputs(cfg, B, seed):
    p = inputs.layer_params(cfg, seed)
    t = inputs.token_inputs(cfg, seed, B)
    s = inputs.initial_states(cfg, seed, B)
    return p, t, s


@pytest.mark.parametrize("head_map", [0, 1])
def test_decode_composes_legacy_functions(head_map):
    # ixo_decode == legacy conv_step -> L2 -> gate/beta closed forms -> legacy step.
    cfg = _small_cfg(head_map=head_map)
    B, C, dk, hk, hv, dc = 3, cfg.channels, cfg.d_k, cfg.h_k, cfg.h_v, cfg.d_conv
    p, t, s = _fused_inputs(cfg, B, 21)
    cs_o, st_o, o_o = oracle.decode(cfg, B, t["x"], s["conv_state"], p["w"], t["a"], t["b"], p["A_log"],
                                    p["dt_bias"], s["state"])
    w32 = bf16.to_f32(p["w"]).ravel()
    for b in range(B):
        cs32 = bf16.to_f32(s["conv_state"][b]).ravel()
        cs2, y = oracle.conv_step(cs32, bf16.to_f32(t["x"][b]), w32, C, dc)
        np.testing.assert_array_equal(bf16.from_f32(cs2).reshape(C, dc - 1), cs_o[b])
        q = y[:hk * dk].reshape(hk, dk)
        k = y[hk * dk:2 * hk * dk].reshape(hk, dk)
        v = y[2 * hk * dk:].reshape(hv, dk)
        qn = q / np.sqrt((q * q).sum(1, keepdims=True) + cfg.l2_eps)
        kn = k / np.sqrt((k * k).sum(1, keepdims=True) + cfg.l2_eps)
        # map every v head onto its own (q, k) copy so the legacy modulo step sees src = h
        srcs = [oracle.src_head(cfg, h) for h in range(hv)]
        qh, kh = qn[srcs].ravel(), kn[srcs].ravel()
        a = bf16.to_f32(t["a"][b]).astype(np.float64)
        bb = bf16.to_f32(t["b"][b]).astype(np.float64)
        gate = np.array([oracle.gate(float(p["A_log"][h]), a[h], float(p["dt_bias"][h])) for h in range(hv)])
        beta = 1.0 / (1.0 + np.exp(-bb))
        leg = s["state"][b].transpose(1, 0, 2).ravel()            # [h][i][j] -> [i][h][j]
        rs, ro = oracle.step(leg, qh, kh, v.ravel(), gate, beta, dk, hv, hv)
        np.testing.assert_allclose(as_heads(rs, dk, hv), st_o[b], rtol=1e-5, atol=1e-7)
        np.testing.assert_allclose(ro.reshape(hv, dk), o_o[b], rtol=1e-5, atol=1e-7)


def _identity_conv_case(cfg, B, seed):
    """Inputs whose conv output is x itself: every tap weight 0 except the current input's,
    which is 1 (both exact in bf16), and a zero recurrent state."""
    p, t, s = _fused_inputs(cfg, B, seed)
    w = np.zeros((cfg.channels, cfg.d_conv), np.float32)
    w[:, -1] = 1.0
    p["w"] = bf16.from_f32(w)
    s["state"] = np.zeros_like(s["state"])
    return p, t, s


@pytest.mark.parametrize("act", [0, 1])
def test_decode_activation_closed_form(act):
    # With a zero state the step gives S' = beta k^ v^T and o = beta (k^ . q^) v, where v is
    # the conv output after the activation and q^, k^ the normalised activated q, k rows. An
    # identity conv makes that output act(x): x itself, or SiLU(x) = x / (1 + e^-x). The x
    # rows include 0 (SiLU(0) = 0) and +-12 (SiLU(12) = 12 - 7.4e-5, SiLU(-12) = -7.4e-5).
    cfg = _small_cfg(conv_act=act, h_k=2, h_v=4)
    B = 2
    p, t, s = _identity_conv_case(cfg, B, 61)
    xf = bf16.to_f32(t["x"]).astype(np.float64)
    xf[:, 3] = 0.0
    xf[:, 5] = 12.0
    xf[:, -2] = -12.0
    t["x"] = bf16.from_f32(xf.astype(np.float32))
    xf = bf16.to_f32(t["x"]).astype(np.float64)
    _, st, o = oracle.decode(cfg, B, t["x"], s["conv_state"], p["w"], t["a"], t["b"], p["A_log"], p["dt_bias"],
                             s["state"])
    y = xf / (1.0 + np.exp(-xf)) if act else xf
    if act:
        assert y[0, 3] == 0.0 and abs(y[0, 5] - (12.0 - 12.0 * math.exp(-12.0) / (1 + math.exp(-12.0)))) < 1e-12
    dk, hk = cfg.d_k, cfg.h_k
    for b in range(B):
        q = y[b, :hk * dk].reshape(hk, dk)
        k = y[b, hk * dk:2 * hk * dk].reshape(hk, dk)
        v = y[b, 2 * hk * dk:].reshape(cfg.h_v, cfg.d_v)
        qn = q / np.sqrt((q * q).sum(1, keepdims=True) + cfg.l2_eps)
        kn = k / np.sqrt((k * k).sum(1, keepdims=True) + cfg.l2_eps)
        beta = 1.0 / (1.0 + np.exp(-bf16.to_f32(t["b"][b]).astype(np.float64)))
        for h in range(cfg.h_v):
            src = h % hk
            np.testing.assert_allclose(st[b, h], beta[h] * np.outer(kn[src], v[h]), rtol=1e-12, atol=1e-15)
            np.testing.assert_allclose(o[b, h], beta[h] * (kn[src] @ qn[src]) * v[h], rtol=1e-10, atol=1e-14)


def test_decode_q_scale_is_linear_in_o_only():
    # q_scale multiplies the normalised q (1 in the reference): the outputs scale by it and
    # the states do not move. A power of two scales exactly; 1/sqrt(128) within rounding.
    cfg1 = _small_cfg()
    B = 3
    p, t, s = _fused_inputs(cfg1, B, 71)
    ref = oracle.decode(cfg1, B, t["x"], s["conv_state"], p["w"], t["a"], t["b"], p["A_log"], p["dt_bias"],
                        s["state"])
    for qs, exact in ((0.25, True), (128 ** -0.5, False), (-2.0, True)):
        cfg = _small_cfg(q_scale=qs)
        cs, st, o = oracle.decode(cfg, B, t["x"], s["conv_state"], p["w"], t["a"], t["b"], p["A_log"],
                                  p["dt_bias"], s["state"])
        np.testing.assert_array_equal(cs, ref[0])
        np.testing.assert_array_equal(st, ref[1])
        want = np.float64(np.float32(qs)) * ref[2]
        if exact:
            np.testing.assert_array_equal(o, want)
        else:
            np.testing.assert_allclose(o, want, rtol=1e-13, atol=1e-16)


def test_decode_batch_rows_independent():
    cfg = _small_cfg()
    B = 4
    p, t, s = _fused_inputs(cfg, B, 5)
    full = oracle.decode(cfg, B, t["x"], s["conv_state"], p["w"], t["a"], t["b"], p["A_log"], p["dt_bias"],
                         s["state"], nthreads=3)
    for b in range(B):
        one = oracle.decode(cfg, 1, t["x"][b:b + 1], s["conv_state"][b:b + 1], p["w"], t["a"][b:b + 1],
                            t["b"][b:b + 1], p["A_log"], p["dt_bias"], s["state"][b:b + 1])
        for got, ref in zip(full, one):
            np.testing.assert_array_equal(got[b:b + 1], ref)


def test_decode_head_maps_agree_when_ratio_is_one():
    p0 = _small_cfg(h_k=4, h_v=4)
    p1 = _small_cfg(h_k=4, h_v=4, head_map=1)
    p, t, s = _fused_inputs(p0, 2, 9)
    r0 = oracle.decode(p0, 2, t["x"], s["conv_state"], p["w"], t["a"], t["b"], p["A_log"], p["dt_bias"], s["state"])
    r1 = oracle.decode(p1, 2, t["x"], s["conv_state"], p["w"], t["a"], t["b"], p["A_log"], p["dt_bias"], s["state"])
    for a, b in zip(r0, r1):
        np.testing.assert_array_equal(a, b)
    assert [oracle.src_head(_small_cfg(h_k=2, h_v=6), h) for h in range(6)] == [0, 1, 0, 1, 0, 1]
    assert [oracle.src_head(_small_cfg(h_k=2, h_v=6, head_map=1), h) for h in range(6)] == [0, 0, 0, 1, 1, 1]


def test_prefill_equals_token_loop_and_splits():
    cfg = _small_cfg()
    T = 9
    p = inputs.layer_params(cfg, 31)
    tok = inputs.token_inputs(cfg, 31, T)
    s = inputs.initial_states(cfg, 31, 1)
    cs, st = s["conv_state"], s["state"]
    outs = []
    for t in range(T):
        cs, st, o = oracle.decode(cfg, 1, tok["x"][t:t + 1], cs, p["w"], tok["a"][t:t + 1], tok["b"][t:t + 1],
                                  p["A_log"], p["dt_bias"], st)
        outs.append(o[0])
    cs_p, st_p, o_p = oracle.prefill(cfg, [0, T], tok["x"], s["conv_state"], p["w"], tok["a"], tok["b"],
                                     p["A_log"], p["dt_bias"], s["state"])
    np.testing.assert_array_equal(cs_p, cs)
    np.testing.assert_array_equal(st_p, st)
    np.testing.assert_array_equal(o_p, np.stack(outs))
    # split [0,4) + [4,9) carried through the states gives the same result
    cs_a, st_a, o_a = oracle.prefill(cfg, [0, 4], tok["x"][:4], s["conv_state"], p["w"], tok["a"][:4], tok["b"][:4],
                                     p["A_log"], p["dt_bias"], s["state"])
    cs_b, st_b, o_b = oracle.prefill(cfg, [0, 5], tok["x"][4:], cs_a, p["w"], tok["a"][4:], tok["b"][4:],
                                     p["A_log"], p["dt_bias"], st_a)
    np.testing.assert_array_equal(np.concatenate([o_a, o_b]), o_p)
    np.testing.assert_array_equal(st_b, st_p)


def test_prefill_varlen_sequences_independent():
    cfg = _small_cfg()
    cu = np.array([0, 3, 3, 8], np.int32)          # includes an empty sequence
    p = inputs.layer_params(cfg, 41)
    tok = inputs.token_inputs(cfg, 41, int(cu[-1]))
    s = inputs.initial_states(cfg, 41, 3)
    cs, st, o = oracle.prefill(cfg, cu, tok["x"], s["conv_state"], p["w"], tok["a"], tok["b"], p["A_log"],
                               p["dt_bias"], s["state"])
    for i in range(3):
        lo, hi = int(cu[i]), int(cu[i + 1])
        cs1, st1, o1 = oracle.prefill(cfg, [0, hi - lo], tok["x"][lo:hi], s["conv_state"][i:i + 1], p["w"],
                                      tok["a"][lo:hi], tok["b"][lo:hi], p["A_log"], p["dt_bias"], s["state"][i:i + 1])
        np.testing.assert_array_equal(cs[i:i + 1], cs1)
        np.testing.assert_array_equal(st[i:i + 1], st1)
        np.testing.assert_array_equal(o[lo:hi], o1)
    np.testing.assert_array_equal(st[1], s["state"][1].astype(np.float64))   # empty sequence untouched


# ------------------------------------------------------------------------------------------
# generator and bf16 helpers
# ------------------------------------------------------------------------------------------

def test_bf16_round_to_nearest_even():
    vals = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 1.0 + 2 ** -8 + 2 ** -20, -2.5, np.inf, -np.inf], np.float32)
    got = bf16.to_f32(bf16.from_f32(vals))
    expect = np.array([1.0, 1.0, 1.0 + 2 ** -6, 1.0 + 2 ** -7, -2.5, np.inf, -np.inf], np.float32)
    np.testing.assert_array_equal(got, expect)
    assert bf16.from_f32(np.array([np.nan], np.float32))[0] == 0x7FC0
    u = np.arange(0, 65536, dtype=np.uint32).astype(np.uint16)
    f = bf16.to_f32(u)
    finite = np.isfinite(f)
    np.testing.assert_array_equal(bf16.from_f32(f)[finite], u[finite])   # bf16 -> f32 -> bf16 is identity


def test_generator_is_deterministic_and_sane():
    g1, g2 = inputs.Gen(inputs.seed_for(2)), inputs.Gen(inputs.seed_for(2))
    a, b = g1.normal(3, (50000,)), g2.normal(3, (50000,))
    np.testing.assert_array_equal(a, b)
    assert abs(a.mean()) < 0.03 and abs(a.std() - 1.0) < 0.02
    assert not np.array_equal(a, g1.normal(4, (50000,)))
    u = g1.uniform(5, (50000,), 2.0, 3.0)
    assert u.min() >= 2.0 and u.max() < 3.0 and abs(u.mean() - 2.5) < 0.01
    np.testing.assert_array_equal(g1.normal(3, (10,)), a[:10])        # prefix stable
