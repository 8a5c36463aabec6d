"""The C ABI boundary, checked without a GPU: the library loads, exports every symbol that
include/ix_gdn.h declares, and rejects the shapes the reference rejects (src/ix_gdn.cu:110,
:117, :122, :127, :133) before touching the device. No kernel is launched here."""
import ctypes
import os
import re

import pytest

import baloon_amd as bx

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "ix_gdn.h")
INVALID = bx.HIP_ERROR_INVALID_VALUE


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\*?\s*(ix_[a-z0-9_]+)\s*\(",
                                 text, flags=re.M)))


def test_header_declares_expected_entry_points():
    assert declared_functions() == sorted(bx.EXPORTS)


def test_library_exports_every_declared_symbol():
    L = bx.lib()
    for name in declared_functions():
        assert hasattr(L, name), name
    assert bx.version().startswith("ixgdn")


# SGPR spills go to VGPR lanes (v_writelane / v_readlane), not scratch. The prefill's chain
# kernel carries a few (its SGPR working set is the chunk geometry and many workspace base
# addresses); it is bounded here at its current count so that a regression fails. Every other
# kernel must have none.
SGPR_SPILL_BOUND = {"chain_kernel": 16, "tri_kernel": 32}


def resource_lines():
    report = os.path.join(ROOT, "baloon_amd", "_build", "resource_usage.txt")
    if not os.path.exists(report):
        pytest.skip("library built without the resource report")
    out = []
    for ln in open(report):
        if ln.strip():
            out.append(dict(kv.split("=", 1) for kv in ln.split() if "=" in kv))
    assert out, "empty resource report"
    return out


def test_resource_usage_has_no_scratch():
    for f in resource_lines():
        for key in ("ScratchSize", "VGPRsSpill", "SGPRsSpill"):
            assert key in f, (key, f)          # a renamed key must not pass silently
        assert f["ScratchSize"] == "0", f
        assert f["VGPRsSpill"] == "0", f


def test_sgpr_spills_bounded():
    seen = []
    for f in resource_lines():
        n = int(f["SGPRsSpill"])
        bound = next((b for k, b in SGPR_SPILL_BOUND.items() if k in f["name"]), 0)
        assert n <= bound, f"{f['name']}: {n} SGPRs spilled (bound {bound})"
        if n:
            seen.append((f["name"], n))
    print("SGPR spills:", seen)


NULL = None


@pytest.mark.parametrize("S,hk,hv", [(0, 1, 1), (129, 1, 1), (-1, 1, 1), (128, 0, 1), (128, 1, 0)])
def test_step_rejects_bad_shapes(S, hk, hv):
    assert bx.lib().ix_gdn_step(NULL, NULL, NULL, NULL, NULL, NULL, NULL, S, hk, hv, NULL) == INVALID


@pytest.mark.parametrize("C,dc", [(0, 4), (-3, 4), (8, 1), (8, 0)])
def test_conv_rejects_bad_shapes(C, dc):
    assert bx.lib().ix_gdn_conv_step(NULL, NULL, NULL, NULL, C, dc, NULL) == INVALID


@pytest.mark.parametrize("rows,cols", [(0, 8), (4, 0), (4, 1025), (-1, 8)])
def test_l2_rejects_bad_shapes(rows, cols):
    assert bx.lib().ix_gdn_l2_norm(NULL, rows, cols, ctypes.c_float(1e-6), NULL) == INVALID


def test_beta_rejects_null_and_bad_count():
    assert bx.lib().ix_gdn_beta_gate(NULL, 4, NULL) == INVALID
    assert bx.lib().ix_gdn_beta_gate(ctypes.c_void_p(16), 0, NULL) == INVALID


@pytest.mark.parametrize("hv,S", [(0, 8), (4, 0)])
def test_out_norm_rejects_bad_shapes(hv, S):
    assert bx.lib().ix_gdn_out_norm(NULL, NULL, NULL, NULL, hv, S, ctypes.c_float(1e-6), NULL) == INVALID


def test_fused_cfg_validation():
    L = bx.lib()
    good = bx.make_cfg()
    assert L.ix_gdn_channels(ctypes.byref(good)) == 8192
    bad = [bx.make_cfg(d_k=64), bx.make_cfg(d_conv=1), bx.make_cfg(d_conv=5), bx.make_cfg(h_k=0),
           bx.make_cfg(head_map=2), bx.make_cfg(h_k=3, h_v=32, head_map=bx.HEAD_DIV), bx.make_cfg(conv_act=7)]
    for c in bad:
        rc = L.ix_gdn_decode(ctypes.byref(c), 1, *([ctypes.c_void_p(256)] * 8), NULL, NULL, NULL, NULL)
        assert rc == INVALID
    p = ctypes.c_void_p(256)
    assert L.ix_gdn_decode(ctypes.byref(good), 0, p, p, p, p, p, p, p, p, NULL, NULL, NULL, NULL) == INVALID
    assert L.ix_gdn_decode(ctypes.byref(good), 1, NULL, p, p, p, p, p, p, p, NULL, NULL, NULL, NULL) == INVALID
    assert L.ix_gdn_decode(ctypes.byref(good), 1, p, p, p, p, p, p, p, ctypes.c_void_p(260), NULL, NULL,
                           NULL, NULL) == INVALID           # state must be 16-byte aligned
    assert L.ix_gdn_decode(None, 1, p, p, p, p, p, p, p, p, NULL, NULL, NULL, NULL) == INVALID


def test_prefill_validation_without_launch():
    L = bx.lib()
    cfg = bx.make_cfg()
    need = bx.ix_gdn_prefill_workspace_size(cfg, 2, 100)
    assert need > 0 and need % 256 == 0
    assert bx.ix_gdn_prefill_workspace_size(cfg, 0, 100) == 0
    assert bx.ix_gdn_prefill_workspace_size(cfg, 2, -1) == 0
    assert bx.ix_gdn_prefill_workspace_size(bx.make_cfg(d_k=64), 2, 100) == 0
    assert bx.ix_gdn_prefill_workspace_size(cfg, 2, 200) > need       # grows with tokens
    small = bx.ix_gdn_prefill_window_workspace_size(cfg, 2, 100, 1)   # windows of one chunk
    assert 0 < small < need and small % 256 == 0
    assert bx.ix_gdn_prefill_window_workspace_size(cfg, 2, 100, 10 ** 6) == need
    assert bx.ix_gdn_prefill_window_workspace_size(cfg, 2, 100, 0) == 0
    assert bx.ix_gdn_prefill_window_workspace_size(cfg, 0, 100, 1) == 0
    assert bx.ix_gdn_prefill_window_workspace_size(cfg, 2, 100, 1, gated=True) > small
    # the window operands do not grow with tokens; only the chunk tables do (16 bytes a chunk)
    assert bx.ix_gdn_prefill_window_workspace_size(cfg, 2, 64 * 1000, 1) - small <= 1000 * 16 + 512
    # the default size: windows of at most 80 chunks
    at80 = bx.ix_gdn_prefill_window_workspace_size(cfg, 1, 64 * 79, 80)
    assert bx.ix_gdn_prefill_workspace_size(cfg, 1, 64 * 79) == at80        # one window
    for T in (64 * 1000, 64 * 100000):
        big = bx.ix_gdn_prefill_workspace_size(cfg, 1, T)
        assert big == bx.ix_gdn_prefill_window_workspace_size(cfg, 1, T, 80)
        assert big - at80 <= (T // 64) * 16 + 512
        assert bx.ix_gdn_prefill_gated_workspace_size(cfg, 1, T) == \
            bx.ix_gdn_prefill_window_workspace_size(cfg, 1, T, 80, gated=True)
    p = ctypes.c_void_p(1 << 20)

    def call(n_seq, T, ws, nbytes, c=cfg):
        return L.ix_gdn_prefill(ctypes.byref(c), n_seq, T, p, p, p, p, p, p, p, p, p, NULL, NULL, ws, nbytes, NULL)

    assert call(2, 100, p, small - 1) == INVALID                     # below one chunk's window
    assert call(2, 100, ctypes.c_void_p((1 << 20) + 64), need) == INVALID   # not 256-byte aligned
    assert call(2, 100, NULL, need) == INVALID                       # no workspace
    assert call(0, 100, p, need) == INVALID
    assert call(2, -5, p, need) == INVALID
    assert call(2, 100, p, need, bx.make_cfg(head_map=5)) == INVALID
    assert call(2, 0, NULL, 0) == bx.HIP_SUCCESS                     # nothing to consume: no launch


def test_head_group_limit():
    # at most 16 v heads per q/k head in the fused kernels
    L = bx.lib()
    p = ctypes.c_void_p(256)
    ok, bad = bx.make_cfg(h_k=2, h_v=32), bx.make_cfg(h_k=1, h_v=17)
    assert L.ix_gdn_decode(ctypes.byref(bad), 1, p, p, p, p, p, p, p, p, NULL, NULL, NULL, NULL) == INVALID
    assert bx.ix_gdn_prefill_workspace_size(ok, 1, 64) > 0
    assert bx.ix_gdn_prefill_workspace_size(bad, 1, 64) == 0


def test_gated_validation_without_launch():
    L = bx.lib()
    cfg = bx.make_cfg()
    p = ctypes.c_void_p(1 << 20)
    ok = bx.OutGate(1 << 20, 1 << 20, 1e-6, 1 << 20, None)

    def dec(gate, c=cfg):
        g = ctypes.byref(gate) if gate is not None else None
        return L.ix_gdn_decode_gated(ctypes.byref(c), 1, p, p, p, p, p, p, p, p, NULL, NULL, g, NULL, NULL)

    assert dec(None) == INVALID                                                  # gate required
    assert dec(bx.OutGate(None, 1 << 20, 1e-6, 1 << 20, None)) == INVALID      # no z
    assert dec(bx.OutGate(1 << 20, None, 1e-6, 1 << 20, None)) == INVALID      # no ssm_norm
    assert dec(bx.OutGate(1 << 20, 1 << 20, 1e-6, None, None)) == INVALID      # no output
    assert dec(bx.OutGate(1 << 20, (1 << 20) + 2, 1e-6, 1 << 20, None)) == INVALID   # ssm_norm alignment
    assert dec(bx.OutGate((1 << 20) + 1, 1 << 20, 1e-6, None, 1 << 20)) == INVALID   # z alignment
    assert dec(bx.OutGate(1 << 20, 1 << 20, 1e-6, None, None, (1 << 20) + 2)) == INVALID   # y_q8_1 alignment
    assert dec(ok, bx.make_cfg(d_conv=7)) == INVALID

    need = bx.ix_gdn_prefill_workspace_size(cfg, 2, 100)
    gneed = bx.ix_gdn_prefill_gated_workspace_size(cfg, 2, 100)
    assert gneed >= need + 100 * 32 * 128 * 4 and gneed % 256 == 0
    assert bx.ix_gdn_prefill_gated_workspace_size(cfg, 0, 100) == 0

    def pre(gate, nbytes):
        g = ctypes.byref(gate) if gate is not None else None
        return L.ix_gdn_prefill_gated(ctypes.byref(cfg), 2, 100, p, p, p, p, p, p, p, p, p, NULL, NULL, g, p,
                                      nbytes, NULL)

    assert pre(None, gneed) == INVALID
    gsmall = bx.ix_gdn_prefill_window_workspace_size(cfg, 2, 100, 1, gated=True)
    assert pre(ok, gsmall - 1) == INVALID                  # needs room for one window's fp32 norm input
    assert pre(bx.OutGate(1 << 20, 1 << 20, 1e-6, None, None), gneed) == INVALID


def test_decode_workspace_sections():
    # one int32 counter per (sequence, q/k head), rounded up to 256 bytes
    r = lambda n: (n + 255) // 256 * 256
    for kw in ({}, dict(h_k=2, h_v=18), dict(h_k=3, h_v=8)):
        cfg = bx.make_cfg(**kw)
        for B in (1, 3, 64):
            assert bx.ix_gdn_decode_workspace_size(cfg, B) == r(B * cfg.h_k * 4)


def test_window_validation_without_launch():
    L = bx.lib()
    cfg = bx.make_cfg()
    p = ctypes.c_void_p(1 << 20)
    r = bx.ix_gdn_window_record_size(cfg, 2, 4)
    rows = 8
    rr = lambda n: (n + 255) // 256 * 256
    assert r == rr(rows * 16 * 128 * 4) + rr(rows * 32 * 128 * 4) + 2 * rr(rows * 32 * 4)
    for B, K in [(0, 4), (2, 0), (2, 17), (-1, 1)]:
        assert bx.ix_gdn_window_record_size(cfg, B, K) == 0

    def verify(K, c=cfg, rec=p, state=p, fn=L.ix_gdn_decode_window):
        return fn(ctypes.byref(c), 2, K, p, p, p, p, p, p, p, state, NULL, NULL, rec, NULL)

    def verify_mfma(K, c=cfg, rec=p, state=p):
        return verify(K, c, rec, state, L.ix_gdn_decode_window_mfma)

    def commit(K, c=cfg, acc=p, rec=p):
        return L.ix_gdn_commit_window(ctypes.byref(c), 2, K, acc, p, rec, p, p, NULL)

    for f in (verify, verify_mfma, commit):
        assert f(0) == INVALID and f(17) == INVALID
        assert f(4, c=bx.make_cfg(h_k=4, h_v=2)) == INVALID            # a q/k head feeds no v head
        assert f(4, rec=ctypes.c_void_p((1 << 20) + 16)) == INVALID     # record not 256-byte aligned
        assert f(4, rec=NULL) == INVALID
    assert verify(4, state=ctypes.c_void_p((1 << 20) + 8)) == INVALID  # state not 16-byte aligned
    assert verify_mfma(4, state=ctypes.c_void_p((1 << 20) + 8)) == INVALID
    assert commit(4, acc=NULL) == INVALID


def test_projection_validation_without_launch():
    L = bx.lib()
    p = ctypes.c_void_p(1 << 20)
    for nin, nout in [(0, 4), (4, 0), (-1, 4)]:
        assert L.ix_bf16_gemv(p, p, p, nin, nout, NULL) == INVALID
    assert L.ix_bf16_gemv_pair(p, p, p, 0, p, p, 0, 8, NULL) == INVALID
    assert L.ix_bf16_gemv_pair(p, p, p, 4, p, p, 4, 0, NULL) == INVALID
    for tpr in (0, -64, 48, 2048):
        assert L.ix_bf16_gemv_split(p, p, p, 8, 4, tpr, NULL) == INVALID
    for n_in, n_out, nc in [(0, 1, 1), (33, 1, 1), (32, 0, 1), (32, 1, 0), (32, 1, 9)]:
        assert L.ix_mmvq_q8_0(p, p, p, n_in, n_out, nc, NULL) == INVALID
    assert L.ix_mmvq_q8_0(NULL, p, p, 32, 1, 1, NULL) == INVALID
    assert L.ix_mmvq_q8_0(ctypes.c_void_p((1 << 20) + 1), p, p, 32, 1, 1, NULL) == INVALID     # Q8_0 is 2-byte aligned
    cfg = bx.make_cfg()
    assert bx.ix_gdn_in_proj_width(cfg) == 8192 + 4096 + 64
    assert bx.ix_gdn_in_proj_width(bx.make_cfg(d_k=64)) == 0
    ok = (p, p, p, p, p, p, NULL, NULL)
    for B, K in [(0, 2048), (4, 0), (4, 100), (4, 2050)]:
        assert L.ix_gdn_in_proj(ctypes.byref(cfg), B, K, *ok) == INVALID
    assert L.ix_gdn_in_proj(ctypes.byref(cfg), 4, 2048, ctypes.c_void_p((1 << 20) + 8), p, p, p, p, p, NULL,
                            NULL) == INVALID                                    # h must be 16-byte aligned


def test_q8_1_validation_without_launch():
    L = bx.lib()
    a = 1 << 20
    assert L.ix_q8_1_quantize(a, a, 0, None) == INVALID
    assert L.ix_q8_1_quantize(a, a, 48, None) == INVALID          # not whole blocks
    assert L.ix_q8_1_quantize(None, a, 64, None) == INVALID
    assert L.ix_q8_1_quantize(a + 2, a, 64, None) == INVALID      # fp32 alignment
    assert L.ix_q8_1_quantize(a, a + 2, 64, None) == INVALID      # block alignment


def test_commit_layers_validation_without_launch():
    # ix_gdn_commit_window_layers refuses bad counts and null tables before any launch.
    cfg = bx.make_cfg()
    L = bx.lib()
    p = ctypes.c_void_p(1 << 20)
    args = (p, p, p, p, p, None)
    assert L.ix_gdn_commit_window_layers(ctypes.byref(cfg), 0, 2, 4, *args) == bx.HIP_ERROR_INVALID_VALUE
    assert L.ix_gdn_commit_window_layers(ctypes.byref(cfg), 2, 2, 17, *args) == bx.HIP_ERROR_INVALID_VALUE
    assert L.ix_gdn_commit_window_layers(ctypes.byref(cfg), 2, 0, 4, *args) == bx.HIP_ERROR_INVALID_VALUE
    assert L.ix_gdn_commit_window_layers(ctypes.byref(cfg), 2, 2, 4, None, p, p, p, p, None) == \
        bx.HIP_ERROR_INVALID_VALUE
    assert L.ix_gdn_commit_window_layers(ctypes.byref(cfg), 2, 2, 4, p, p, p, None, p, None) == \
        bx.HIP_ERROR_INVALID_VALUE
    assert L.ix_gdn_commit_window_layers(ctypes.byref(bx.make_cfg(d_k=64)), 2, 2, 4, *args) == \
        bx.HIP_ERROR_INVALID_VALUE
