"""GPU parity of the five legacy entry points against the oracle -- the checks of the
reference's acceptance test tests/test_gdn.cu:16-55, same shapes and tolerances
(max|gpu-ref| <= tol * max|ref|, :10-13), plus ragged shapes the API allows.
Inputs come from the portable generator instead of std::mt19937 (:15)."""
import numpy as np
import pytest

import baloon_amd as bx
import oracle
from oracle import inputs
from tests.common import dev, host

pytestmark = pytest.mark.gpu


def _sync():
    import torch
    torch.cuda.synchronize()


def gen(seed):
    return inputs.Gen(seed)


@pytest.mark.parametrize("S,hk,hv", [(128, 16, 48), (128, 48, 48), (128, 16, 32), (100, 16, 48), (7, 3, 5),
                                     (64, 1, 1), (128, 1, 1)])
def test_step(S, hk, hv):
    # tests/test_gdn.cu:16-32: state N*0.1, q,k N*0.1, v N, gate -|N|, beta 0.5+0.4 tanh(N); tol 1e-4.
    g = gen(100 + S + hk + hv)
    st = g.normal_f32(1, (S * hv * S,), 0.1)
    q = g.normal_f32(2, (hk * S,), 0.1)
    k = g.normal_f32(3, (hk * S,), 0.1)
    v = g.normal_f32(4, (hv * S,))
    gate = -np.abs(g.normal_f32(5, (hv,)))
    beta = (0.5 + 0.4 * np.tanh(g.normal(6, (hv,)))).astype(np.float32)
    rs, ro = oracle.step(st, q, k, v, gate, beta, S, hk, hv)
    ds, dq, dk, dv, dg, db = map(dev, (st, q, k, v, gate, beta))
    import torch
    do = torch.empty(hv * S, dtype=torch.float32, device="cuda")
    assert bx.ix_gdn_step(ds, dq, dk, dv, dg, db, do, S, hk, hv) == 0
    _sync()
    assert oracle.chk(host(do), ro, 1e-4), oracle.rel_err(host(do), ro)
    assert oracle.chk(host(ds), rs, 1e-4), oracle.rel_err(host(ds), rs)


def test_step_repeated_tokens_carry_state():
    S, hk, hv, T = 128, 16, 32, 16
    g = gen(7)
    st = g.normal_f32(1, (S * hv * S,), 0.1)
    rs = st.astype(np.float64)
    ds = dev(st)
    import torch
    do = torch.empty(hv * S, dtype=torch.float32, device="cuda")
    for t in range(T):
        q = g.normal_f32(10 + t, (hk * S,), 0.1)
        k = g.normal_f32(40 + t, (hk * S,), 0.1)
        v = g.normal_f32(70 + t, (hv * S,))
        gate = -np.abs(g.normal_f32(100 + t, (hv,))) * 0.1
        beta = (0.5 + 0.4 * np.tanh(g.normal(130 + t, (hv,)))).astype(np.float32)
        rs, ro = oracle.step(rs, q, k, v, gate, beta, S, hk, hv)
        assert bx.ix_gdn_step(ds, dev(q), dev(k), dev(v), dev(gate), dev(beta), do, S, hk, hv) == 0
        _sync()
        assert oracle.chk(host(do), ro, 1e-4), (t, oracle.rel_err(host(do), ro))
    assert oracle.chk(host(ds), rs, 1e-4), oracle.rel_err(host(ds), rs)


@pytest.mark.parametrize("C,dc", [(8192 + 5, 4), (8192, 4), (1000, 2), (333, 3), (1, 4)])
def test_conv(C, dc):
    # tests/test_gdn.cu:33-41: out tol 1e-5, state exact.
    g = gen(200 + C + dc)
    cs = g.normal_f32(1, (C * (dc - 1),))
    x = g.normal_f32(2, (C,))
    w = g.normal_f32(3, (C * dc,))
    rcs, ro = oracle.conv_step(cs, x, w, C, dc)
    dcs, dx, dw = dev(cs), dev(x), dev(w)
    import torch
    dout = torch.empty(C, dtype=torch.float32, device="cuda")
    assert bx.ix_gdn_conv_step(dcs, dx, dw, dout, C, dc) == 0
    _sync()
    assert oracle.chk(host(dout), ro, 1e-5), oracle.rel_err(host(dout), ro)
    np.testing.assert_array_equal(host(dcs), rcs)


@pytest.mark.parametrize("cols", [128, 100, 7, 64, 65, 1024, 1])
def test_l2_norm(cols):
    # tests/test_gdn.cu:42-46: rows 33, eps 1e-6, tol 1e-6.
    rows, eps = 33, 1e-6
    x = gen(300 + cols).normal_f32(1, (rows * cols,))
    r = oracle.l2_norm(x, rows, cols, eps)
    dx = dev(x)
    assert bx.ix_gdn_l2_norm(dx, rows, cols, eps) == 0
    _sync()
    assert oracle.chk(host(dx), r, 1e-6), oracle.rel_err(host(dx), r)


@pytest.mark.parametrize("S", [128, 100, 65, 1, 300])
def test_out_norm(S):
    # tests/test_gdn.cu:47-52: h_v 48, eps 1e-6, ssm_norm 1 + 0.1 N, tol 1e-5.
    hv, eps = 48, 1e-6
    g = gen(400 + S)
    o = g.normal_f32(1, (hv * S,))
    z = g.normal_f32(2, (hv * S,))
    nrm = (1.0 + 0.1 * g.normal(3, (S,))).astype(np.float32)
    r = oracle.out_norm(o, z, nrm, hv, S, eps)
    import torch
    dy = torch.empty(hv * S, dtype=torch.float32, device="cuda")
    assert bx.ix_gdn_out_norm(dev(o), dev(z), dev(nrm), dy, hv, S, eps) == 0
    _sync()
    assert oracle.chk(host(dy), r, 1e-5), oracle.rel_err(host(dy), r)


@pytest.mark.parametrize("n", [48, 1, 1000])
def test_beta_gate(n):
    # tests/test_gdn.cu:53-55: logits 3 N, tol 1e-6.
    b = (3.0 * gen(500 + n).normal(1, (n,))).astype(np.float32)
    r = oracle.beta_gate(b)
    db = dev(b)
    assert bx.ix_gdn_beta_gate(db, n) == 0
    _sync()
    assert oracle.chk(host(db), r, 1e-6), oracle.rel_err(host(db), r)


def test_invalid_shapes_return_invalid_value_and_leave_buffers():
    import torch
    st = torch.ones(16, device="cuda")
    assert bx.ix_gdn_step(st, st, st, st, st, st, st, 129, 1, 1) == bx.HIP_ERROR_INVALID_VALUE
    assert bx.ix_gdn_l2_norm(st, 1, 1025, 1e-6) == bx.HIP_ERROR_INVALID_VALUE
    assert bx.ix_gdn_conv_step(st, st, st, st, 4, 1) == bx.HIP_ERROR_INVALID_VALUE
    _sync()
    assert torch.all(st == 1).item()
