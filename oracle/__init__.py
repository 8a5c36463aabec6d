"""CPU oracle for the GDN path -- TEST INFRASTRUCTURE ONLY.

This package is the checker the HIP library is compared against. Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may import it; the
product path (``baloon_amd``) never does.

* ``liboracle.so`` (built from ``gdn_oracle.c`` by ``make -C oracle``) restates the
  reference's double-precision host references, tests/test_gdn.cu:22-54, plus closed-form
  extensions for the fused decode and the token-by-token prefill.
* :mod:`oracle.inputs` is the portable seeded input generator (splitmix64 + Box-Muller).
* :mod:`oracle.bf16` holds exact bf16 <-> fp32 conversions (round to nearest even).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

from . import bf16, inputs  # noqa: F401  (re-exported helpers)

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None


class Cfg(ctypes.Structure):
    """Mirror of ``ixo_cfg`` / ``ix_gdn_cfg`` (same field order)."""

    _fields_ = [
        ("h_k", ctypes.c_int), ("h_v", ctypes.c_int),
        ("d_k", ctypes.c_int), ("d_v", ctypes.c_int),
        ("d_conv", ctypes.c_int), ("head_map", ctypes.c_int), ("conv_act", ctypes.c_int),
        ("q_scale", ctypes.c_float), ("l2_eps", ctypes.c_float),
    ]

    @property
    def channels(self) -> int:
        return 2 * self.h_k * self.d_k + self.h_v * self.d_v


def make_cfg(h_k=16, h_v=32, d_k=128, d_v=128, d_conv=4, head_map=0, conv_act=0,
             q_scale=1.0, l2_eps=1e-6) -> Cfg:
    return Cfg(h_k, h_v, d_k, d_v, d_conv, head_map, conv_act, q_scale, l2_eps)


def build(force: bool = False) -> str:
    """Compile liboracle.so with make (gcc)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-C", _HERE] + (["-B"] if force else []), check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        I = ctypes.c_int
        F = ctypes.c_float
        sig = {
            "ixo_step": [P, P, P, P, P, P, P, I, I, I],
            "ixo_conv_step": [P, P, P, P, I, I],
            "ixo_l2_norm": [P, P, I, I, F],
            "ixo_out_norm": [P, P, P, P, I, I, F],
            "ixo_beta_gate": [P, P, I],
            "ixo_decode": [P, I, P, P, P, P, P, P, P, P, P, I],
            "ixo_prefill": [P, I, P, P, P, P, P, P, P, P, P, P, I],
            "ixo_src_head": [P, I],
        }
        for name, args in sig.items():
            fn = getattr(_lib, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int if name == "ixo_src_head" else None
        _lib.ixo_mix_counter.argtypes = [ctypes.c_uint64, ctypes.c_uint64, P]
        _lib.ixo_mix_counter.restype = None
        for name in ("ixo_gate", "ixo_sigmoid", "ixo_softplus"):
            getattr(_lib, name).restype = ctypes.c_double
        _lib.ixo_gate.argtypes = [F, ctypes.c_double, F]
        _lib.ixo_sigmoid.argtypes = [ctypes.c_double]
        _lib.ixo_softplus.argtypes = [ctypes.c_double]
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _u16(a):
    return np.ascontiguousarray(a, dtype=np.uint16)


# ---- legacy entry points -------------------------------------------------------------------

def step(state, q, k, v, gate, beta, S, h_k, h_v):
    """tests/test_gdn.cu:22-26. Returns (state', o) in float64; state layout [S][h_v][S]."""
    rs = np.array(state, dtype=np.float64, copy=True)
    ro = np.zeros(h_v * S, dtype=np.float64)
    q, k, v, gate, beta = map(_f32, (q, k, v, gate, beta))
    lib().ixo_step(_p(rs), _p(q), _p(k), _p(v), _p(gate), _p(beta), _p(ro), S, h_k, h_v)
    return rs, ro


def conv_step(conv_state, x, w, C, d_conv):
    """tests/test_gdn.cu:36-37. Returns (conv_state' float32, out float64)."""
    cs = np.array(conv_state, dtype=np.float32, copy=True)
    out = np.zeros(C, dtype=np.float64)
    x, w = _f32(x), _f32(w)
    lib().ixo_conv_step(_p(cs), _p(x), _p(w), _p(out), C, d_conv)
    return cs, out


def l2_norm(x, rows, cols, eps):
    """tests/test_gdn.cu:45."""
    x = _f32(x)
    r = np.zeros(rows * cols, dtype=np.float64)
    lib().ixo_l2_norm(_p(x), _p(r), rows, cols, eps)
    return r


def out_norm(o, z, nrm, h_v, S, eps):
    """tests/test_gdn.cu:49-50."""
    o, z, nrm = _f32(o), _f32(z), _f32(nrm)
    r = np.zeros(h_v * S, dtype=np.float64)
    lib().ixo_out_norm(_p(o), _p(z), _p(nrm), _p(r), h_v, S, eps)
    return r


def gated_out(o, z_bits, nrm, eps):
    """The gated output norm of every (row, head) of o [..][h_v][d_v]: ixo_out_norm
    (tests/test_gdn.cu:49-50) over the rows, with o taken to fp32 and z from bf16 bits.
    Returns float64 of o's shape."""
    o = np.asarray(o)
    S = o.shape[-1]
    rows = o.size // S
    z = bf16.to_f32(np.asarray(z_bits, dtype=np.uint16)).reshape(-1)
    return out_norm(o.astype(np.float32).reshape(-1), z, nrm, rows, S, eps).reshape(o.shape)


def beta_gate(b):
    """tests/test_gdn.cu:54."""
    b = _f32(b)
    r = np.zeros(b.size, dtype=np.float64)
    lib().ixo_beta_gate(_p(b), _p(r), b.size)
    return r


# ---- fused layer extensions ------------------------------------------------------------------

def decode(cfg: Cfg, B, x, conv_state, w, a, b, A_log, dt_bias, state, nthreads=1):
    """One decode token for B sequences. bf16 arrays are uint16 bit patterns.

    Returns (conv_state' uint16, state' float64 [B][h_v][d_k][d_v], o float64 [B][h_v][d_v]).
    """
    cs = np.array(conv_state, dtype=np.uint16, copy=True)
    st = np.array(state, dtype=np.float64, copy=True)
    o = np.zeros((B, cfg.h_v, cfg.d_v), dtype=np.float64)
    x, w, a, b = map(_u16, (x, w, a, b))
    A_log, dt_bias = _f32(A_log), _f32(dt_bias)
    lib().ixo_decode(ctypes.byref(cfg), B, _p(x), _p(cs), _p(w), _p(a), _p(b), _p(A_log), _p(dt_bias),
                     _p(st), _p(o), nthreads)
    return cs, st, o


def prefill(cfg: Cfg, cu_seqlens, x, conv_state, w, a, b, A_log, dt_bias, state, nthreads=1):
    """Token-by-token recurrence over packed sequences (cu_seqlens offsets).

    Returns (conv_state', state' float64 [n_seq][h_v][d_k][d_v], o float64 [T][h_v][d_v]).
    """
    cu = np.ascontiguousarray(cu_seqlens, dtype=np.int32)
    n_seq = cu.size - 1
    T = int(cu[-1])
    cs = np.array(conv_state, dtype=np.uint16, copy=True)
    st = np.array(state, dtype=np.float64, copy=True)
    o = np.zeros((T, cfg.h_v, cfg.d_v), dtype=np.float64)
    x, w, a, b = map(_u16, (x, w, a, b))
    A_log, dt_bias = _f32(A_log), _f32(dt_bias)
    lib().ixo_prefill(ctypes.byref(cfg), n_seq, _p(cu), _p(x), _p(cs), _p(w), _p(a), _p(b), _p(A_log),
                      _p(dt_bias), _p(st), _p(o), nthreads)
    return cs, st, o


def src_head(cfg: Cfg, h: int) -> int:
    return lib().ixo_src_head(ctypes.byref(cfg), h)


def gate(A_log: float, a: float, dt_bias: float) -> float:
    return lib().ixo_gate(A_log, a, dt_bias)


def sigmoid(x: float) -> float:
    return lib().ixo_sigmoid(x)


def softplus(x: float) -> float:
    return lib().ixo_softplus(x)


def rel_err(got, ref) -> float:
    """The reference's comparison norm, max|got-ref| / max|ref| (tests/test_gdn.cu:10-13)."""
    got = np.asarray(got, dtype=np.float64).ravel()
    ref = np.asarray(ref, dtype=np.float64).ravel()
    if ref.size == 0:
        return 0.0
    return float(np.max(np.abs(got - ref)) / max(np.max(np.abs(ref)), 1e-30))


def chk(got, ref, tol) -> bool:
    """tests/test_gdn.cu:10-13: max|got-ref| <= tol * max|ref|."""
    got = np.asarray(got, dtype=np.float64).ravel()
    ref = np.asarray(ref, dtype=np.float64).ravel()
    mx = float(np.max(np.abs(got - ref))) if ref.size else 0.0
    sc = max(float(np.max(np.abs(ref))) if ref.size else 0.0, 1e-30)
    return mx <= tol * sc
