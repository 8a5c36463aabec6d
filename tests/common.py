"""Shared helpers for the GDN tests: numpy <-> device tensors and the comparison norms."""
from __future__ import annotations

import os

import numpy as np

import oracle
from oracle import bf16, inputs

TOL_O_ABS = 1e-3       # fp32 outputs vs the double oracle, absolute
TOL_STATE_REL = 1e-4   # fp32 state vs the double oracle, max|d| / max|ref|
# Oracle threads: the GPU box's CPU share is 16 whatever os.cpu_count() reports there.
NT = max(1, min(16, len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)))


def extreme_gates(cfg, tok, seed, frac=0.2):
    """Drive the gate and beta logits of token inputs past the reference's thresholds.

    In each of a and b, a fraction ``frac`` of the entries is set to a large positive value
    and another ``frac`` to a large negative one, at seeded positions: a = +25 puts
    a + dt_bias above softplus's threshold 20 (softplus(x) = x there, src/ix_gdn.cu:22) and,
    with A_log up to ln 16, a log decay near -400 whose exp underflows to 0 in fp32;
    a = -25 puts it below -20 (softplus ~ e^x, decay ~1); b = +-30 gives beta = 1 and
    beta ~ 1e-13. Returns a copy of tok with a and b replaced (bf16 bits)."""
    g = inputs.Gen(seed ^ 0x5EED)
    out = dict(tok)
    for name, big, tid in (("a", 25.0, 0x401), ("b", 30.0, 0x402)):
        v = bf16.to_f32(tok[name]).astype(np.float32)
        u = g.uniform(tid, v.shape)
        v = np.where(u < frac, np.float32(big), np.where(u < 2 * frac, np.float32(-big), v)).astype(np.float32)
        out[name] = bf16.from_f32(v)
    return out


def extreme_params(p):
    """Layer parameters with A_log = ln 16 (the top of its range) on every other v head."""
    q = dict(p)
    al = np.array(p["A_log"], dtype=np.float32, copy=True)
    al[::2] = np.float32(np.log(16.0))
    q["A_log"] = al
    return q


def dev(a, dtype=None):
    """numpy array -> contiguous cuda tensor. uint16 arrays become bfloat16 (bit-exact)."""
    import torch
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16).cuda()
    t = torch.from_numpy(a.copy())
    if dtype is not None:
        t = t.to(dtype)
    return t.cuda()


def host(t) -> np.ndarray:
    """cuda tensor -> numpy (bfloat16 -> uint16 bits)."""
    import torch
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def state_to_dev(st):
    """Oracle state [..][h_v][d_k][d_v] -> device tensor in the library's [..][h_v][d_v][d_k] layout."""
    return dev(np.ascontiguousarray(np.swapaxes(np.asarray(st, dtype=np.float32), -1, -2)))


def state_from_dev(t) -> np.ndarray:
    """Device state [..][h_v][d_v][d_k] -> numpy in the oracle's [..][h_v][d_k][d_v] layout."""
    return np.ascontiguousarray(np.swapaxes(host(t), -1, -2))


def bf16_excess_err(got_bits: np.ndarray, ref_f64: np.ndarray) -> float:
    """max(|bf16 - ref| - half a bf16 ulp): the error beyond bf16's own rounding."""
    ref = np.asarray(ref_f64, dtype=np.float64)
    got32 = bf16.to_f32(got_bits)
    got = got32.astype(np.float64)

    def binade(v):   # 2^e with 2^e <= |v| < 2^(e+1)
        return (np.abs(v).view(np.uint32) & np.uint32(0x7F800000)).view(np.float32).astype(np.float64)

    # half a bf16 ulp of whichever of ref and the output lies in the higher binade (the rounding
    # may cross a power of two)
    half = np.maximum(np.maximum(binade(ref.astype(np.float32)), binade(got32)) * 2.0 ** -8, 2.0 ** -133)
    return float(np.max(np.abs(got - ref) - half)) if ref.size else 0.0


def bf16_ulp_diff(got_bits: np.ndarray, ref_f64: np.ndarray) -> int:
    """Max distance in bf16 ulps between bf16 outputs and RNE(fp32(ref))."""
    ref_bits = bf16.from_f32(np.asarray(ref_f64, dtype=np.float32)).astype(np.int32)
    g = np.asarray(got_bits).astype(np.int32)

    def ordered(u):  # map bf16 bit patterns to a monotonic integer line
        return np.where(u & 0x8000, -(u & 0x7FFF), u & 0x7FFF)

    return int(np.max(np.abs(ordered(g) - ordered(ref_bits)))) if g.size else 0


__all__ = ["oracle", "bf16", "inputs", "dev", "host", "state_to_dev", "state_from_dev", "bf16_ulp_diff", "bf16_excess_err",
           "extreme_gates", "extreme_params", "NT", "TOL_O_ABS", "TOL_STATE_REL"]
