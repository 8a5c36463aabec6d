"""GdnLayer: device-resident parameters and per-sequence states for one GDN layer.

A thin host object over the C ABI: it owns the conv weights, A_log, dt_bias, the recurrent
state block [n][h_v][d_v][d_k] fp32 (each head's state stored column by column), the conv
state [n][C][d_conv-1] bf16 and the zeroed decode counter workspace, and calls
``ix_gdn_decode`` / ``ix_gdn_prefill`` on the current stream. Allocation happens here, at
construction (and for the prefill workspace, on first use of a given size), never inside the
library calls.
"""
from __future__ import annotations

import torch

from . import (Cfg, check, ix_gdn_decode, ix_gdn_decode_workspace_size, ix_gdn_prefill,
               ix_gdn_prefill_workspace_size, make_cfg)


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
        self.decode_ws = torch.zeros(ix_gdn_decode_workspace_size(c, n_slots), dtype=torch.uint8, device=self.device)
        self._ws = None

    def decode(self, x, a, b, o=None, o_bf16=None, stream=None):
        """One token for all n_slots sequences: x [n][C] bf16, a, b [n][h_v] bf16."""
        check("ix_gdn_decode", ix_gdn_decode(self.cfg, self.n_slots, x, self.conv_state, self.conv_w, a, b,
                                             self.A_log, self.dt_bias, self.state, o, o_bf16, self.decode_ws,
                                             stream))

    def prefill(self, cu_seqlens, x, a, b, o=None, o_bf16=None, stream=None):
        """Packed prefill of n_slots sequences (cu_seqlens int32 [n+1] on the device)."""
        total_T = x.shape[0]
        need = ix_gdn_prefill_workspace_size(self.cfg, self.n_slots, total_T)
        if self._ws is None or self._ws.numel() < need:
            self._ws = torch.empty(max(need, 256), dtype=torch.uint8, device=self.device)
        check("ix_gdn_prefill", ix_gdn_prefill(self.cfg, self.n_slots, total_T, cu_seqlens, x, self.conv_state,
                                               self.conv_w, a, b, self.A_log, self.dt_bias, self.state, o, o_bf16,
                                               self._ws, self._ws.numel(), stream))
