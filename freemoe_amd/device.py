"""A MoE layer resident in HBM, driven through libfmx (tests and bench plumbing).

Holds the packed expert slots, the device slot table (arrays of slot
addresses, so kernels find routed experts without a host round trip), the
router and norm weights, and the fmx_moe_layer descriptor that points at them.
torch provides the device memory and the stream; every computation is a
libfmx call.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import fmx
from .workloads import LayerWeights


def to_device(a: np.ndarray, device) -> torch.Tensor:
    a = np.ascontiguousarray(a)
    if not a.flags.writeable:  # a read-only memory map (a checkpoint's bytes)
        a = a.copy()
    return torch.from_numpy(a).to(device)


def pack(type_id: int, raw: torch.Tensor, rows: int, cols: int, stream=None) -> torch.Tensor:
    """Raw GGUF blocks (device uint8) -> packed device layout."""
    out = torch.empty(fmx.packed_bytes(type_id, rows, cols), dtype=torch.uint8, device=raw.device)
    fmx.call("fmx_pack", type_id, raw.data_ptr(), out.data_ptr(), rows, cols, fmx.stream_handle(stream))
    return out


class DeviceLayer:
    def __init__(self, lw: LayerWeights, device="cuda", stream=None):
        self.w = lw
        self.device = torch.device(device)
        H, F, E = lw.hidden, lw.ffn, lw.experts
        self.norm = to_device(lw.norm_weight, self.device)
        self.router = to_device(lw.router_bytes, self.device)
        if lw.router_type != fmx.FMX_TYPE_F32:
            self.router = pack(lw.router_type, self.router, E, H, stream)
        self.router_bias = None if lw.router_bias is None else to_device(lw.router_bias, self.device)
        self.gate, self.up, self.down = [], [], []
        for e in range(E):
            self.gate.append(pack(lw.gate_type, to_device(lw.gate[e], self.device), F, H, stream))
            self.up.append(pack(lw.up_type, to_device(lw.up[e], self.device), F, H, stream))
            self.down.append(pack(lw.down_type, to_device(lw.down[e], self.device), H, F, stream))
        self.slots = torch.tensor([[t.data_ptr() for t in arr] for arr in (self.gate, self.up, self.down)],
                                  dtype=torch.int64, device=self.device)
        self.desc = fmx.MoELayer(
            H, F, E, lw.top_k, self.norm.data_ptr(), lw.rms_eps, lw.norm_bias, lw.router_type,
            self.router.data_ptr(), fmx.ptr(self.router_bias), int(lw.weights_norm), int(lw.epsilon_additive),
            lw.weights_epsilon, lw.weights_scale, lw.gate_type, lw.up_type, lw.down_type,
            self.slots[0].data_ptr(), self.slots[1].data_ptr(), self.slots[2].data_ptr())
        self.workspace = None
        self.prefill_workspace = None

    def weight_bytes_per_expert(self) -> int:
        return sum(fmx.raw_row_bytes(t, c) * r for t, r, c in (
            (self.w.gate_type, self.w.ffn, self.w.hidden), (self.w.up_type, self.w.ffn, self.w.hidden),
            (self.w.down_type, self.w.hidden, self.w.ffn)))

    def ensure_workspace(self, tokens: int) -> torch.Tensor:
        need = fmx.lib().fmx_moe_workspace_bytes(ctypes.byref(self.desc), tokens)
        if need == 0:
            raise fmx.FmxError(1, "fmx_moe_workspace_bytes")
        if self.workspace is None or self.workspace.numel() < need:
            self.workspace = torch.zeros(need, dtype=torch.uint8, device=self.device)
        return self.workspace

    def route(self, x: torch.Tensor, stream=None):
        t = x.shape[0]
        H, E, K = self.w.hidden, self.w.experts, self.w.top_k
        h = torch.empty((t, H), dtype=torch.float32, device=self.device)
        logits = torch.empty((t, E), dtype=torch.float32, device=self.device)
        ids = torch.empty((t, K), dtype=torch.int32, device=self.device)
        wts = torch.empty((t, K), dtype=torch.float32, device=self.device)
        ws = self.ensure_workspace(t)
        fmx.call("fmx_moe_route", ctypes.byref(self.desc), x.data_ptr(), t, h.data_ptr(), logits.data_ptr(),
                 ids.data_ptr(), wts.data_ptr(), ws.data_ptr(), ws.numel(), fmx.stream_handle(stream))
        return h, logits, ids, wts

    def decode(self, x: torch.Tensor, out=None, ids=None, wts=None, stream=None):
        t = x.shape[0]
        K = self.w.top_k
        out = torch.empty_like(x) if out is None else out
        ids = torch.empty((t, K), dtype=torch.int32, device=self.device) if ids is None else ids
        wts = torch.empty((t, K), dtype=torch.float32, device=self.device) if wts is None else wts
        ws = self.ensure_workspace(t)
        fmx.call("fmx_moe_decode", ctypes.byref(self.desc), x.data_ptr(), out.data_ptr(), t, ids.data_ptr(),
                 wts.data_ptr(), ws.data_ptr(), ws.numel(), fmx.stream_handle(stream))
        return out, ids, wts

    def prefill(self, x: torch.Tensor, out=None, ids=None, wts=None, stream=None, kernel_ms=None):
        """The whole layer over all rows of x at once (grouped GEMMs). With
        kernel_ms (a list), runs fmx_moe_prefill_timed and appends the gate/up
        and down GEMMs' own milliseconds (synchronises the stream)."""
        t = x.shape[0]
        K = self.w.top_k
        out = torch.empty_like(x) if out is None else out
        ids = torch.empty((t, K), dtype=torch.int32, device=self.device) if ids is None else ids
        wts = torch.empty((t, K), dtype=torch.float32, device=self.device) if wts is None else wts
        need = fmx.lib().fmx_moe_prefill_workspace_bytes(ctypes.byref(self.desc), t)
        if need == 0:
            raise fmx.FmxError(1, "fmx_moe_prefill_workspace_bytes")
        if self.prefill_workspace is None or self.prefill_workspace.numel() < need:
            self.prefill_workspace = torch.zeros(need, dtype=torch.uint8, device=self.device)
        ws = self.prefill_workspace
        if kernel_ms is None:
            fmx.call("fmx_moe_prefill", ctypes.byref(self.desc), x.data_ptr(), out.data_ptr(), t, ids.data_ptr(),
                     wts.data_ptr(), ws.data_ptr(), ws.numel(), fmx.stream_handle(stream))
        else:
            ms = (ctypes.c_double * 2)()
            fmx.call("fmx_moe_prefill_timed", ctypes.byref(self.desc), x.data_ptr(), out.data_ptr(), t,
                     ids.data_ptr(), wts.data_ptr(), ws.data_ptr(), ws.numel(), fmx.stream_handle(stream), ms)
            kernel_ms.extend([ms[0], ms[1]])
        return out, ids, wts

    def prefill_status(self, stream=None) -> int:
        return fmx.lib().fmx_moe_status(self.prefill_workspace.data_ptr(), fmx.stream_handle(stream))

    def status(self, stream=None) -> int:
        ws = self.ensure_workspace(1)
        return fmx.lib().fmx_moe_status(ws.data_ptr(), fmx.stream_handle(stream))
