"""CPU references for the projections feeding the GDN layer (test infrastructure only).

Restates the reference's double-precision host checks:
  * bf16 GEMV: tests/test_bf16_gemv.cu:21-22 -- y[o] = sum_i x[i] w[o][i] in double, with the
    per-row magnitude sum_i |x[i] w[o][i]| that scales the tolerance (:11, 2e-5 x magnitude);
  * Q8_0 x q8_1: tests/mmvq_wave_ref.h:37-47 -- y[c][r] = sum over blocks of
    d_w * d_x * (integer dot of the block's 32 int8 pairs) in double, with the scale
    sum |d_w d_x| * 32 * 127 * 127 of tests/test_mmvq_wave.cu:57-58 (tolerance 1e-5 x scale);
  * the block formats of src/ix_mmvq_wave.cu:22-25: Q8_0 = fp16 d + 32 int8 (34 bytes),
    q8_1 = fp16 d, fp16 s + 32 int8 (36 bytes), little endian, packed back to back;
  * the q8_1 quantiser (q8_1_quantize below): the reference fixes the division every q8_1
    producer uses (src/ix_q81_div.h:1-9: d = amax / 127, q = roundf(x / d), IEEE division,
    no fast-math) but ships no quantiser, so the rest follows the published q8_1 quantiser of
    ggml (llama.cpp, ggml-cuda/quantize.cu, MIT): d = max|x| / 127, q = 0 for an all-zero
    block, s = the sum of the block's values, d and s stored as fp16.
The layer's input projection is the same GEMV for B rows, split into the pieces
x | z | a | b (include/ix_gdn.h).
"""
from __future__ import annotations

import numpy as np

from . import bf16
from .inputs import Gen


def gemv_ref(x_bits, w_bits):
    """x [n_in] and w [n_out][n_in] as bf16 bits -> (y, magnitude), float64 [n_out]."""
    x = bf16.to_f32(np.asarray(x_bits, np.uint16)).astype(np.float64)
    w = bf16.to_f32(np.asarray(w_bits, np.uint16)).astype(np.float64)
    return w @ x, np.abs(w) @ np.abs(x)


def in_proj_ref(h_bits, w_bits):
    """h [B][K], W [N][K] bf16 bits -> (y, magnitude), float64 [B][N]."""
    h = bf16.to_f32(np.asarray(h_bits, np.uint16)).astype(np.float64)
    w = bf16.to_f32(np.asarray(w_bits, np.uint16)).astype(np.float64)
    return h @ w.T, np.abs(h) @ np.abs(w).T


def in_proj_split(cfg, y):
    """Split [B][N] columns into the layer's pieces x [B][C], z [B][h_v][d_v], a, b [B][h_v]."""
    C = 2 * cfg.h_k * cfg.d_k + cfg.h_v * cfg.d_v
    Z = cfg.h_v * cfg.d_v
    B = y.shape[0]
    return (y[:, :C], y[:, C:C + Z].reshape(B, cfg.h_v, cfg.d_v), y[:, C + Z:C + Z + cfg.h_v],
            y[:, C + Z + cfg.h_v:C + Z + 2 * cfg.h_v])


# ---- Q8_0 / q8_1 ---------------------------------------------------------------------------

def half_exact(v):
    """float values that are exactly representable in fp16 -> fp16 bits."""
    return np.asarray(v, np.float16).view(np.uint16)


def q8_blocks(seed, tid, rows, nb):
    """Random blocks like tests/test_mmvq_wave.cu:30-31: scales (1 + u % 2047) / 1024 (exact in
    fp16), quants uniform in [-127, 127]. Returns (d bits uint16 [rows][nb], qs int8 [rows][nb][32])."""
    g = Gen(seed)
    u = (g._bits(tid, rows * nb) % np.uint64(2047)).astype(np.float64)
    d = half_exact(((1.0 + u) / 1024.0).astype(np.float32)).reshape(rows, nb)
    q = ((g._bits(tid + 1, rows * nb * 32) % np.uint64(255)).astype(np.int64) - 127).astype(np.int8)
    return d, q.reshape(rows, nb, 32)


def pack_q8_0(d, qs) -> np.ndarray:
    """[rows][nb] blocks -> bytes: per block fp16 d then 32 int8 (34 bytes)."""
    rows, nb = d.shape
    out = np.zeros((rows, nb, 34), np.uint8)
    out[..., 0:2] = d.astype("<u2")[..., None].view(np.uint8)
    out[..., 2:34] = qs.view(np.uint8)
    return out.reshape(-1)


def pack_q8_1(d, qs, s=None) -> np.ndarray:
    """[cols][nb] blocks -> bytes: per block fp16 d, fp16 s, then 32 int8 (36 bytes)."""
    cols, nb = d.shape
    s = np.zeros_like(d) if s is None else s
    out = np.zeros((cols, nb, 36), np.uint8)
    out[..., 0:2] = d.astype("<u2")[..., None].view(np.uint8)
    out[..., 2:4] = s.astype("<u2")[..., None].view(np.uint8)
    out[..., 4:36] = qs.view(np.uint8)
    return out.reshape(-1)


def q8_0_ref(wd, wq, xd, xq):
    """y [ncols][n_out] and scale [ncols][n_out] in float64."""
    dw = wd.view(np.float16).astype(np.float64)                   # [n_out][nb]
    dx = xd.view(np.float16).astype(np.float64)                   # [nc][nb]
    dots = np.einsum("rbk,cbk->crb", wq.astype(np.int64), xq.astype(np.int64))   # exact integers
    y = np.einsum("crb,rb,cb->cr", dots.astype(np.float64), dw, dx)
    sc = np.einsum("rb,cb->cr", np.abs(dw), np.abs(dx)) * 32 * 127 * 127
    return y, sc


HALF_MAX = np.float32(65504.0)        # largest finite fp16 value


def q8_1_quantize(x) -> np.ndarray:
    """fp32 values [n] (n % 32 == 0) -> q8_1 bytes [n / 32 * 36], per 32 consecutive values:
    d = max|x| / 127 in fp32 (IEEE division, src/ix_q81_div.h:8-9), qs = roundf(x / d) with the
    quotient in fp32 and ties away from zero (0 when d = 0: an all-zero block, or one whose d
    underflows), s = the fp32 sum taken in
    xor-butterfly order (offsets 16, 8, 4, 2, 1: the order of a 32-lane butterfly, in which
    every lane ends with the same bits), d and s rounded to fp16.
    Pinning: the division and rounding rule is the reference's (ix_q81_div.h); the block
    layout its Q8_0 product's (src/ix_mmvq_wave.cu:20-24); the q = 0 rule and the s term are
    ggml's. The Q8_0 product reads only d and qs, so s is "parity unpinned" against the
    reference (checked here against a float64 sum and the butterfly order only).
    Range: d is clamped to fp16's largest finite value 65504 (with the codes then saturating
    at +-127) and s to [-65504, 65504] before the fp16 conversion; below max|x| = 127 * 65504
    the clamps change nothing. The reference names such a clamp (q8_1_finite,
    ix_q81_div.h:9) without defining it: this rule is the library's own, parity unpinned,
    pinned by the known answers in tests/test_oracle_proj.py."""
    x = np.asarray(x, np.float32).reshape(-1, 32)
    amax = np.abs(x).max(axis=1)
    d = np.minimum((amax / np.float32(127.0)).astype(np.float32), HALF_MAX).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        t = (x / d[:, None]).astype(np.float32)
        r = np.sign(t).astype(np.float64) * np.floor(np.abs(t).astype(np.float64) + 0.5)
    q = np.where(d[:, None] == 0, 0.0, np.clip(r, -127.0, 127.0)).astype(np.int8)
    s = x.copy()
    idx = np.arange(32)
    with np.errstate(over="ignore"):
        for off in (16, 8, 4, 2, 1):
            s = (s + s[:, idx ^ off]).astype(np.float32)
    dh = d.astype(np.float16).view(np.uint16)[:, None]
    sh = np.clip(s[:, 0], -HALF_MAX, HALF_MAX).astype(np.float16).view(np.uint16)[:, None]
    return pack_q8_1(dh, q[:, None, :], sh)


def q8_1_unpack(b):
    """q8_1 bytes -> (d bits uint16 [nb], s bits uint16 [nb], qs int8 [nb][32])."""
    b = np.asarray(b, np.uint8).reshape(-1, 36)
    return b[:, 0:2].copy().view("<u2")[:, 0], b[:, 2:4].copy().view("<u2")[:, 0], b[:, 4:36].copy().view(np.int8)
