"""GdnLayer: device-resident parameters and per-sequence states for one GDN layer.

A thin host object over the C ABI: it owns the conv weights, A_log, dt_bias, the recurrent
state block [n][h_v][d_v][d_k] fp32 (each head's state stored column by column), the conv
state [n][C][d_conv-1] bf16, the gated output norm's weight ssm_norm [d_v] fp32 and the
zeroed decode workspace, and calls ``ix_gdn_decode`` / ``ix_gdn_prefill`` (or their gated
variants, when a gate input z is passed) on the current stream. Allocation happens here, at
construction (and for the prefill workspace, on first use of a given size), never inside the
library calls.
"""
from __future__ import annotations

import torch

from . import (Cfg, check, ix_gdn_decode, ix_gdn_decode_gated, ix_gdn_decode_workspace_size, ix_gdn_prefill,
               ix_gdn_prefill_gated, ix_gdn_prefill_gated_workspace_size, ix_gdn_prefill_workspace_size, make_cfg,
               out_gate)


class GdnLayer:
    def __init__(self, n_slots: int, cfg: Cfg | None = None, device="cuda"):
        self.cfg = cfg or make_cfg()
        c = self.cfg
        self.n_slots = n_slots
        self.device = torch.device(device)
        C = c.channels
        self.conv_w = torch.zeros(C, c.d_conv, dtype=torch.bfloat16, device=self.device)
        self.A_log = torch.zeros(c.h_v, dtype=torch.float32, device=self.device)
        self.dt_bias = torch.zeros(c.h_v, dtype=torch.float32, device=self.device)
        self.state = torch.zeros(n_slots, c.h_v, c.d_v, c.d_k, dtype=torch.float32, device=self.device)
        self.conv_state = torch.zeros(n_slots, C, c.d_conv - 1, dtype=torch.bfloat16, device=self.device)
        self.ssm_norm = torch.ones(c.d_v, dtype=torch.float32, device=self.device)
        self.norm_eps = 1e-6
        self.decode_ws = torch.zeros(ix_gdn_decode_workspace_size(c, n_slots), dtype=torch.uint8, device=self.device)
        self._ws = None

    def decode(self, x, a, b, o=None, o_bf16=None, z=None, y=None, y_bf16=None, y_q8_1=None, stream=None):
        """One token for all n_slots sequences: x [n][C] bf16, a, b [n][h_v] bf16. With z
        [n][h_v][d_v] bf16 the gated output norm is fused in and written to y, y_bf16 and/or
        y_q8_1 (uint8, 36 bytes per 32 outputs: the activation format of ix_mmvq_q8_0)."""
        args = (self.cfg, self.n_slots, x, self.conv_state, self.conv_w, a, b, self.A_log, self.dt_bias, self.state,
                o, o_bf16)
        if z is None:
            check("ix_gdn_decode", ix_gdn_decode(*args, self.decode_ws, stream))
        else:
            g = out_gate(z, self.ssm_norm, self.norm_eps, y, y_bf16, y_q8_1)
            check("ix_gdn_decode_gated", ix_gdn_decode_gated(*args, g, self.decode_ws, stream))

    def prefill(self, cu_seqlens, x, a, b, o=None, o_bf16=None, z=None, y=None, y_bf16=None, y_q8_1=None,
                stream=None):
        """Packed prefill of n_slots sequences (cu_seqlens int32 [n+1] on the device); z, y,
        y_bf16, y_q8_1 as in decode, with [total_T] rows."""
        total_T = x.shape[0]
        size = ix_gdn_prefill_workspace_size if z is None else ix_gdn_prefill_gated_workspace_size
        need = size(self.cfg, self.n_slots, total_T)
        if self._ws is None or self._ws.numel() < need:
            self._ws = torch.empty(max(need, 256), dtype=torch.uint8, device=self.device)
        args = (self.cfg, self.n_slots, total_T, cu_seqlens, x, self.conv_state, self.conv_w, a, b, self.A_log,
                self.dt_bias, self.state, o, o_bf16)
        if z is None:
            check("ix_gdn_prefill", ix_gdn_prefill(*args, self._ws, self._ws.numel(), stream))
        else:
            g = out_gate(z, self.ssm_norm, self.norm_eps, y, y_bf16, y_q8_1)
            check("ix_gdn_prefill_gated", ix_gdn_prefill_gated(*args, g, self._ws, self._ws.numel(), stream))
