"""Portable seeded input generator (test infrastructure).

A counter-based splitmix64 generator: value i of tensor ``tid`` under ``seed`` is
``mix(mix(seed ^ mix(tid)) + i)``, so any slice of any tensor is reproducible without
generating the rest, and the same bits come out on every machine. Uniforms take the top 53
bits; normals use Box-Muller in double on two consecutive counters, then round to the target
dtype (bf16 round-to-nearest-even, or fp32).

Distributions follow the benchmark configurations: q, k, v, x ~ N(0,1) bf16; gate logit
a ~ N(0,1) and beta logit b ~ N(0,1) (bf16); A_log ~ U(ln 1, ln 16); dt_bias ~ N(0, 0.1);
state ~ N(0, 0.02) fp32; conv weights ~ N(0, 0.1) bf16.
"""
from __future__ import annotations

import ctypes
import math

import numpy as np

from . import bf16

_M = np.uint64(0xFFFFFFFFFFFFFFFF)


def _mix(z: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = (z + np.uint64(0x9E3779B97F4A7C15)) & _M
        z = ((z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)) & _M
        z = ((z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)) & _M
        return z ^ (z >> np.uint64(31))


def seed_for(config_id: int) -> int:
    """Seed convention of the benchmark configurations: 0x6D4E0000 + config id."""
    return 0x6D4E0000 + int(config_id)


class Gen:
    _CHUNK = 1 << 22          # normals per pass: bounded temporaries, same values

    def __init__(self, seed: int):
        self.seed = np.uint64(seed)

    def _key(self, tid: int) -> np.uint64:
        return _mix(np.array([self.seed ^ _mix(np.array([np.uint64(tid)]))[0]], dtype=np.uint64))[0]

    @staticmethod
    def _bits_at(key: np.uint64, start: int, n: int) -> np.ndarray:
        """mix(i + key) for counters i = start .. start + n - 1."""
        if n >= 1 << 16:                 # the same integers from the C oracle library, much faster
            from . import lib
            out = np.empty(n, dtype=np.uint64)
            with np.errstate(over="ignore"):
                k = int((key + np.uint64(start)) & _M)
            lib().ixo_mix_counter(k, n, out.ctypes.data_as(ctypes.c_void_p))
            return out
        with np.errstate(over="ignore"):
            return _mix((np.arange(start, start + n, dtype=np.uint64) + key) & _M)

    def _bits(self, tid: int, n: int) -> np.ndarray:
        return self._bits_at(self._key(tid), 0, n)

    def uniform(self, tid: int, shape, lo=0.0, hi=1.0) -> np.ndarray:
        n = int(np.prod(shape))
        u = (self._bits(tid, n) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
        return (lo + (hi - lo) * u).reshape(shape)

    def _normal_into(self, tid: int, n: int, std, mean, out: np.ndarray, convert) -> np.ndarray:
        key = self._key(tid)
        for lo in range(0, n, self._CHUNK):
            m = min(self._CHUNK, n - lo)
            b = self._bits_at(key, 2 * lo, 2 * m)      # normal i uses counters 2i and 2i + 1
            u1 = (b[0::2] >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
            u2 = (b[1::2] >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
            z = np.sqrt(-2.0 * np.log1p(-u1)) * np.cos(2.0 * math.pi * u2)
            out[lo:lo + m] = convert(mean + std * z)
        return out

    def normal(self, tid: int, shape, std=1.0, mean=0.0) -> np.ndarray:
        n = int(np.prod(shape))
        return self._normal_into(tid, n, std, mean, np.empty(n, np.float64), lambda v: v).reshape(shape)

    def normal_bf16(self, tid: int, shape, std=1.0) -> np.ndarray:
        n = int(np.prod(shape))
        return self._normal_into(tid, n, std, 0.0, np.empty(n, np.uint16),
                                 lambda v: bf16.from_f32(v.astype(np.float32))).reshape(shape)

    def normal_f32(self, tid: int, shape, std=1.0) -> np.ndarray:
        n = int(np.prod(shape))
        return self._normal_into(tid, n, std, 0.0, np.empty(n, np.float32),
                                 lambda v: v.astype(np.float32)).reshape(shape)


# Tensor ids (stable; step-dependent tensors add step * 0x100).
T_X, T_CS, T_W, T_A, T_B, T_ALOG, T_DT, T_STATE, T_LEN, T_Z, T_NRM = range(1, 12)


def layer_params(cfg, seed: int) -> dict:
    """Per-layer parameters: conv weights [C][d_conv] bf16, A_log and dt_bias [h_v] fp32."""
    g = Gen(seed)
    C = cfg.channels
    return {
        "w": g.normal_bf16(T_W, (C, cfg.d_conv), 0.1),
        "A_log": g.uniform(T_ALOG, (cfg.h_v,), 0.0, math.log(16.0)).astype(np.float32),
        "dt_bias": g.normal_f32(T_DT, (cfg.h_v,), 0.1),
    }


def token_inputs(cfg, seed: int, rows: int, step: int = 0) -> dict:
    """Per-token inputs for ``rows`` tokens: x [rows][C], a, b [rows][h_v] (bf16 bits)."""
    g = Gen(seed)
    C = cfg.channels
    return {
        "x": g.normal_bf16(T_X + 0x100 * step, (rows, C)),
        "a": g.normal_bf16(T_A + 0x100 * step, (rows, cfg.h_v)),
        "b": g.normal_bf16(T_B + 0x100 * step, (rows, cfg.h_v)),
    }


def out_gate_inputs(cfg, seed: int, rows: int, step: int = 0) -> dict:
    """Gated output norm inputs: z [rows][h_v][d_v] ~ N(0,1) bf16 and the norm weight
    ssm_norm [d_v] = 1 + 0.1 N(0,1) fp32 (the distribution of tests/test_gdn.cu:48)."""
    g = Gen(seed)
    return {
        "z": g.normal_bf16(T_Z + 0x100 * step, (rows, cfg.h_v, cfg.d_v)),
        "nrm": (1.0 + g.normal(T_NRM, (cfg.d_v,), 0.1)).astype(np.float32),
    }


def initial_states(cfg, seed: int, n_seq: int, state_std=0.02, conv_std=1.0) -> dict:
    """Recurrent state [n][h_v][d_k][d_v] fp32 and conv state [n][C][d_conv-1] bf16."""
    g = Gen(seed)
    C = cfg.channels
    st = (g.normal_f32(T_STATE, (n_seq, cfg.h_v, cfg.d_k, cfg.d_v), state_std) if state_std
          else np.zeros((n_seq, cfg.h_v, cfg.d_k, cfg.d_v), np.float32))
    cs = (g.normal_bf16(T_CS, (n_seq, C, cfg.d_conv - 1), conv_std) if conv_std
          else np.zeros((n_seq, C, cfg.d_conv - 1), np.uint16))
    return {"state": st, "conv_state": cs}


def varlen(seed: int, n_seq: int, lo: int, hi: int) -> np.ndarray:
    """cu_seqlens for n_seq lengths ~ U{lo..hi}."""
    g = Gen(seed)
    lens = lo + np.floor(g.uniform(T_LEN, (n_seq,)) * (hi - lo + 1)).astype(np.int64)
    return np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
