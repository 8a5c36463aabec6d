"""baloon_amd -- MI355X-native gated delta-rule (GDN) path.

The product is ``libixgdn.so`` (HIP, gfx950), whose C ABI is ``include/ix_gdn.h``. This
module binds it with ctypes and mirrors the reference's launcher interface
(src/ix_gdn.cu:108-136): the same names, the same argument order and meaning, and the same
error behaviour -- every call returns a ``hipError_t`` code (0 = success), with
``hipErrorInvalidValue`` (1) for shapes the reference rejects.

PyTorch is only plumbing here: tensors supply device memory and the current stream. Every
tensor argument must live on the GPU; the functions pass raw device pointers to the C ABI.
There is no CPU fallback: if the library is missing, :func:`lib` raises.
"""
from __future__ import annotations

import ctypes
import os

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libixgdn.so")

HIP_SUCCESS = 0
HIP_ERROR_INVALID_VALUE = 1
HIP_ERROR_NOT_SUPPORTED = 801

HEAD_MOD = 0   # src = h mod h_k (reference pairing, src/ix_gdn.cu:38)
HEAD_DIV = 1   # src = h / (h_v / h_k)
ACT_NONE = 0   # conv output used as is (reference, src/ix_gdn.cu:64-67)
ACT_SILU = 1

# Every symbol include/ix_gdn.h declares.
EXPORTS = (
    "ix_gdn_step", "ix_gdn_conv_step", "ix_gdn_l2_norm", "ix_gdn_beta_gate", "ix_gdn_out_norm",
    "ix_gdn_channels", "ix_gdn_decode_workspace_size", "ix_gdn_decode", "ix_gdn_prefill_workspace_size",
    "ix_gdn_prefill", "ix_gdn_decode_gated", "ix_gdn_prefill_gated_workspace_size", "ix_gdn_prefill_gated",
    "ix_gdn_prefill_window_workspace_size",
    "ix_gdn_window_record_size", "ix_gdn_decode_window", "ix_gdn_decode_window_mfma", "ix_gdn_commit_window",
    "ix_bf16_gemv", "ix_bf16_gemv_pair", "ix_bf16_gemv_split", "ix_mmvq_q8_0", "ix_gdn_in_proj_width", "ix_gdn_in_proj",
    "ix_gdn_version", "ix_gdn_decode_noalloc", "ix_q8_1_quantize", "ix_gdn_commit_window_layers",
)


class IxGdnError(RuntimeError):
    def __init__(self, name: str, code: int):
        super().__init__(f"{name} returned hipError_t {code}")
        self.code = code


class Cfg(ctypes.Structure):
    """``ix_gdn_cfg`` (include/ix_gdn.h)."""

    _fields_ = [
        ("h_k", ctypes.c_int), ("h_v", ctypes.c_int),
        ("d_k", ctypes.c_int), ("d_v", ctypes.c_int),
        ("d_conv", ctypes.c_int), ("head_map", ctypes.c_int), ("conv_act", ctypes.c_int),
        ("q_scale", ctypes.c_float), ("l2_eps", ctypes.c_float),
    ]

    @property
    def channels(self) -> int:
        return 2 * self.h_k * self.d_k + self.h_v * self.d_v


class OutGate(ctypes.Structure):
    """``ix_gdn_out_gate`` (include/ix_gdn.h): y = o / sqrt(mean(o^2) + eps) * ssm_norm * sigmoid(z)."""

    _fields_ = [
        ("z", ctypes.c_void_p), ("ssm_norm", ctypes.c_void_p), ("eps", ctypes.c_float),
        ("y", ctypes.c_void_p), ("y_bf16", ctypes.c_void_p), ("y_q8_1", ctypes.c_void_p),
    ]


def make_cfg(h_k=16, h_v=32, d_k=128, d_v=128, d_conv=4, head_map=HEAD_MOD, conv_act=ACT_NONE,
             q_scale=1.0, l2_eps=1e-6) -> Cfg:
    """Layer description; defaults are the reference's semantics at the Qwen3-Next shape."""
    return Cfg(h_k, h_v, d_k, d_v, d_conv, head_map, conv_act, q_scale, l2_eps)


_lib = None


def lib() -> ctypes.CDLL:
    """Load libixgdn.so (built by ``python -m baloon_amd.build``); raise if it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m baloon_amd.build`")
    L = ctypes.CDLL(LIB_PATH)
    P, I, F, Z, LL = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_size_t, ctypes.c_longlong
    sig = {
        "ix_gdn_step": ([P, P, P, P, P, P, P, I, I, I, P], I),
        "ix_gdn_conv_step": ([P, P, P, P, I, I, P], I),
        "ix_gdn_l2_norm": ([P, I, I, F, P], I),
        "ix_gdn_beta_gate": ([P, I, P], I),
        "ix_gdn_out_norm": ([P, P, P, P, I, I, F, P], I),
        "ix_gdn_channels": ([P], I),
        "ix_gdn_decode_workspace_size": ([P, I], Z),
        "ix_gdn_decode": ([P, I, P, P, P, P, P, P, P, P, P, P, P, P], I),
        "ix_gdn_prefill_workspace_size": ([P, I, I], Z),
        "ix_gdn_prefill": ([P, I, I, P, P, P, P, P, P, P, P, P, P, P, P, Z, P], I),
        "ix_gdn_decode_gated": ([P, I, P, P, P, P, P, P, P, P, P, P, P, P, P], I),
        "ix_gdn_prefill_gated_workspace_size": ([P, I, I], Z),
        "ix_gdn_prefill_window_workspace_size": ([P, I, I, I, I], Z),
        "ix_gdn_prefill_gated": ([P, I, I, P, P, P, P, P, P, P, P, P, P, P, P, P, Z, P], I),
        "ix_gdn_window_record_size": ([P, I, I], Z),
        "ix_gdn_decode_window": ([P, I, I, P, P, P, P, P, P, P, P, P, P, P, P], I),
        "ix_gdn_decode_window_mfma": ([P, I, I, P, P, P, P, P, P, P, P, P, P, P, P], I),
        "ix_gdn_commit_window": ([P, I, I, P, P, P, P, P, P], I),
        "ix_bf16_gemv": ([P, P, P, LL, LL, P], I),
        "ix_bf16_gemv_pair": ([P, P, P, LL, P, P, LL, LL, P], I),
        "ix_bf16_gemv_split": ([P, P, P, LL, LL, I, P], I),
        "ix_mmvq_q8_0": ([P, P, P, I, I, I, P], I),
        "ix_gdn_in_proj_width": ([P], I),
        "ix_gdn_in_proj": ([P, I, I, P, P, P, P, P, P, P, P], I),
        "ix_gdn_version": ([], ctypes.c_char_p),
        "ix_gdn_decode_noalloc": ([P, I, P, P, P, P, P, P, P, P, P, P, P], I),
        "ix_q8_1_quantize": ([P, P, LL, P], I),
        "ix_gdn_commit_window_layers": ([P, I, I, I, P, P, P, P, P, P], I),
    }
    for name, (args, res) in sig.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = res
    _lib = L
    return L


def _ptr(t) -> int | None:
    """Device pointer of a CUDA tensor (None for None)."""
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("baloon_amd: tensors must be on the GPU")
    if not t.is_contiguous():
        raise ValueError("baloon_amd: tensors must be contiguous")
    return t.data_ptr()


def _stream(s) -> int | None:
    if s is None:
        import torch
        return torch.cuda.current_stream().cuda_stream
    return getattr(s, "cuda_stream", s)


def check(name: str, code: int) -> None:
    if code != HIP_SUCCESS:
        raise IxGdnError(name, code)


# ---- legacy entry points (src/ix_gdn.cu:108-136), return hipError_t --------------------------

def ix_gdn_step(state, q, k, v, gate, beta, o, S, h_k, h_v, s=None) -> int:
    return lib().ix_gdn_step(_ptr(state), _ptr(q), _ptr(k), _ptr(v), _ptr(gate), _ptr(beta), _ptr(o),
                             S, h_k, h_v, _stream(s))


def ix_gdn_conv_step(conv_state, x, kW, out, channels, d_conv, s=None) -> int:
    return lib().ix_gdn_conv_step(_ptr(conv_state), _ptr(x), _ptr(kW), _ptr(out), channels, d_conv, _stream(s))


def ix_gdn_l2_norm(x, rows, cols, eps, s=None) -> int:
    return lib().ix_gdn_l2_norm(_ptr(x), rows, cols, eps, _stream(s))


def ix_gdn_beta_gate(beta, h_v, s=None) -> int:
    return lib().ix_gdn_beta_gate(_ptr(beta), h_v, _stream(s))


def ix_gdn_out_norm(o, z, ssm_norm, y, h_v, S, eps, s=None) -> int:
    return lib().ix_gdn_out_norm(_ptr(o), _ptr(z), _ptr(ssm_norm), _ptr(y), h_v, S, eps, _stream(s))


# ---- fused layer entry points ------------------------------------------------------------------

def ix_gdn_decode_workspace_size(cfg: Cfg, B: int) -> int:
    return lib().ix_gdn_decode_workspace_size(ctypes.byref(cfg), B)


def ix_gdn_decode(cfg: Cfg, B, x, conv_state, conv_w, a, b, A_log, dt_bias, state, o=None, o_bf16=None,
                  workspace=None, s=None) -> int:
    """One decode token for B sequences. bf16 tensors may be torch.bfloat16 or int16/uint16 bits.

    state is [B][h_v][d_v][d_k] fp32 (each head's state stored column by column). workspace,
    if given, is a device buffer of ix_gdn_decode_workspace_size(cfg, B) bytes, zero-filled
    once (the calls keep its counters at zero); it selects the faster many-workgroup kernel."""
    return lib().ix_gdn_decode(ctypes.byref(cfg), B, _ptr(x), _ptr(conv_state), _ptr(conv_w), _ptr(a), _ptr(b),
                               _ptr(A_log), _ptr(dt_bias), _ptr(state), _ptr(o), _ptr(o_bf16), _ptr(workspace),
                               _stream(s))


def ix_gdn_decode_noalloc(cfg: Cfg, B, x, conv_state, conv_w, a, b, A_log, dt_bias, state, o=None, o_bf16=None,
                          s=None) -> int:
    """ix_gdn_decode without a workspace and without any allocation: the group counters live
    in a library-owned static device array (B * h_k <= 65536). Calls on one GPU must be
    ordered (they share the array)."""
    return lib().ix_gdn_decode_noalloc(ctypes.byref(cfg), B, _ptr(x), _ptr(conv_state), _ptr(conv_w), _ptr(a),
                                       _ptr(b), _ptr(A_log), _ptr(dt_bias), _ptr(state), _ptr(o), _ptr(o_bf16),
                                       _stream(s))


def ix_gdn_prefill_workspace_size(cfg: Cfg, n_seq: int, total_T: int) -> int:
    return lib().ix_gdn_prefill_workspace_size(ctypes.byref(cfg), n_seq, total_T)


def ix_gdn_prefill(cfg: Cfg, n_seq, total_T, cu_seqlens, x, conv_state, conv_w, a, b, A_log, dt_bias, state,
                   o=None, o_bf16=None, workspace=None, workspace_bytes=0, s=None) -> int:
    return lib().ix_gdn_prefill(ctypes.byref(cfg), n_seq, total_T, _ptr(cu_seqlens), _ptr(x), _ptr(conv_state),
                                _ptr(conv_w), _ptr(a), _ptr(b), _ptr(A_log), _ptr(dt_bias), _ptr(state), _ptr(o),
                                _ptr(o_bf16), _ptr(workspace), workspace_bytes, _stream(s))


def out_gate(z, ssm_norm, eps, y=None, y_bf16=None, y_q8_1=None) -> OutGate:
    """The gate description of the gated calls, from device tensors (z bf16, ssm_norm fp32;
    y_q8_1 a byte buffer of 36 bytes per 32 outputs)."""
    return OutGate(_ptr(z), _ptr(ssm_norm), eps, _ptr(y), _ptr(y_bf16), _ptr(y_q8_1))


def ix_gdn_decode_gated(cfg: Cfg, B, x, conv_state, conv_w, a, b, A_log, dt_bias, state, o=None, o_bf16=None,
                        gate: OutGate | None = None, workspace=None, s=None) -> int:
    """ix_gdn_decode plus the gated RMS output norm of each (sequence, v head) in the same launch."""
    g = ctypes.byref(gate) if gate is not None else None
    return lib().ix_gdn_decode_gated(ctypes.byref(cfg), B, _ptr(x), _ptr(conv_state), _ptr(conv_w), _ptr(a),
                                     _ptr(b), _ptr(A_log), _ptr(dt_bias), _ptr(state), _ptr(o), _ptr(o_bf16), g,
                                     _ptr(workspace), _stream(s))


def ix_gdn_prefill_gated_workspace_size(cfg: Cfg, n_seq: int, total_T: int) -> int:
    return lib().ix_gdn_prefill_gated_workspace_size(ctypes.byref(cfg), n_seq, total_T)


def ix_gdn_prefill_window_workspace_size(cfg: Cfg, n_seq: int, total_T: int, window_chunks: int,
                                         gated: bool = False) -> int:
    """Workspace bytes for the (gated) prefill run in windows of window_chunks 64-token chunks."""
    return lib().ix_gdn_prefill_window_workspace_size(ctypes.byref(cfg), n_seq, total_T, window_chunks,
                                                      1 if gated else 0)


def ix_gdn_prefill_gated(cfg: Cfg, n_seq, total_T, cu_seqlens, x, conv_state, conv_w, a, b, A_log, dt_bias, state,
                         o=None, o_bf16=None, gate: OutGate | None = None, workspace=None, workspace_bytes=0,
                         s=None) -> int:
    """ix_gdn_prefill plus the gated RMS output norm of every (token, v head) row."""
    g = ctypes.byref(gate) if gate is not None else None
    return lib().ix_gdn_prefill_gated(ctypes.byref(cfg), n_seq, total_T, _ptr(cu_seqlens), _ptr(x),
                                      _ptr(conv_state), _ptr(conv_w), _ptr(a), _ptr(b), _ptr(A_log), _ptr(dt_bias),
                                      _ptr(state), _ptr(o), _ptr(o_bf16), g, _ptr(workspace), workspace_bytes,
                                      _stream(s))


def ix_gdn_window_record_size(cfg: Cfg, B: int, K: int) -> int:
    return lib().ix_gdn_window_record_size(ctypes.byref(cfg), B, K)


def ix_gdn_decode_window(cfg: Cfg, B, K, x, conv_state, conv_w, a, b, A_log, dt_bias, state, o=None, o_bf16=None,
                         record=None, s=None) -> int:
    """Verify K draft tokens per sequence (x [B][K][C]); the states are read, not written."""
    return lib().ix_gdn_decode_window(ctypes.byref(cfg), B, K, _ptr(x), _ptr(conv_state), _ptr(conv_w), _ptr(a),
                                      _ptr(b), _ptr(A_log), _ptr(dt_bias), _ptr(state), _ptr(o), _ptr(o_bf16),
                                      _ptr(record), _stream(s))


def ix_gdn_decode_window_mfma(cfg: Cfg, B, K, x, conv_state, conv_w, a, b, A_log, dt_bias, state, o=None,
                              o_bf16=None, record=None, s=None) -> int:
    """ix_gdn_decode_window on the matrix cores: outputs to fp32 rounding of the exact verify,
    the same record."""
    return lib().ix_gdn_decode_window_mfma(ctypes.byref(cfg), B, K, _ptr(x), _ptr(conv_state), _ptr(conv_w),
                                           _ptr(a), _ptr(b), _ptr(A_log), _ptr(dt_bias), _ptr(state), _ptr(o),
                                           _ptr(o_bf16), _ptr(record), _stream(s))


def ix_gdn_commit_window(cfg: Cfg, B, K, accepted, x, record, conv_state, state, s=None) -> int:
    """Advance each sequence's states by its accepted prefix of the verified window."""
    return lib().ix_gdn_commit_window(ctypes.byref(cfg), B, K, _ptr(accepted), _ptr(x), _ptr(record),
                                      _ptr(conv_state), _ptr(state), _stream(s))


def layer_pointer_table(tensors):
    """Device array (int64 tensor on the GPU) of the device pointers of a list of tensors, the
    per-layer table ix_gdn_commit_window_layers reads."""
    import torch
    ptrs = [_ptr(t) or 0 for t in tensors]
    return torch.tensor(ptrs, dtype=torch.int64).cuda()


def ix_gdn_commit_window_layers(cfg: Cfg, B, K, accepted, xs, records, conv_states, states, s=None) -> int:
    """ix_gdn_commit_window for every layer in one launch. xs, records, conv_states and states
    are the per-layer pointer tables (int64 device tensors, see layer_pointer_table), which
    must stay alive until the launch has run, or per-layer lists of tensors: then the tables
    are built here and the call waits for its launch, so that they outlive it."""
    import torch

    def is_table(v):
        return isinstance(v, torch.Tensor) and v.dtype == torch.int64 and v.dim() == 1
    built = not all(is_table(v) for v in (xs, records, conv_states, states))
    tx, tr, tc, ts = (v if is_table(v) else layer_pointer_table(v) for v in (xs, records, conv_states, states))
    n = tx.numel()
    if not (tr.numel() == tc.numel() == ts.numel() == n):
        return HIP_ERROR_INVALID_VALUE
    rc = lib().ix_gdn_commit_window_layers(ctypes.byref(cfg), n, B, K, _ptr(accepted), _ptr(tx), _ptr(tr),
                                           _ptr(tc), _ptr(ts), _stream(s))
    if built and rc == HIP_SUCCESS:
        torch.cuda.synchronize()
    return rc


# ---- projections ----------------------------------------------------------------------------

def ix_bf16_gemv(x, w, y, n_in, n_out, s=None) -> int:
    return lib().ix_bf16_gemv(_ptr(x), _ptr(w), _ptr(y), n_in, n_out, _stream(s))


def ix_bf16_gemv_pair(x, w1, y1, n_out1, w2, y2, n_out2, n_in, s=None) -> int:
    return lib().ix_bf16_gemv_pair(_ptr(x), _ptr(w1), _ptr(y1), n_out1, _ptr(w2), _ptr(y2), n_out2, n_in, _stream(s))


def ix_bf16_gemv_split(x, w, y, n_in, n_out, threads_per_row, s=None) -> int:
    return lib().ix_bf16_gemv_split(_ptr(x), _ptr(w), _ptr(y), n_in, n_out, threads_per_row, _stream(s))


def ix_mmvq_q8_0(weights, x_q8_1, y, n_in, n_out, ncols, s=None) -> int:
    return lib().ix_mmvq_q8_0(_ptr(weights), _ptr(x_q8_1), _ptr(y), n_in, n_out, ncols, _stream(s))


def ix_q8_1_quantize(x, y_q8_1, n, s=None) -> int:
    """q8_1 blocks (36 bytes per 32 values) of n fp32 values: the activation format of ix_mmvq_q8_0."""
    return lib().ix_q8_1_quantize(_ptr(x), _ptr(y_q8_1), n, _stream(s))


def ix_gdn_in_proj_width(cfg: Cfg) -> int:
    return lib().ix_gdn_in_proj_width(ctypes.byref(cfg))


def ix_gdn_in_proj(cfg: Cfg, B, hidden, h, w, x, z, a, b, y=None, s=None) -> int:
    """[x | z | a | b] = h W^T for B rows: h [B][hidden], W [N][hidden] bf16 -> bf16 pieces."""
    return lib().ix_gdn_in_proj(ctypes.byref(cfg), B, hidden, _ptr(h), _ptr(w), _ptr(x), _ptr(z), _ptr(a), _ptr(b),
                                _ptr(y), _stream(s))


def version() -> str:
    return lib().ix_gdn_version().decode()


from .layer import GdnLayer  # noqa: E402,F401
