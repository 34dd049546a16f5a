"""Static-tape incremental decode (lm/eval/graph_decode.py:15-64 semantics).

The tape holds refined, pre-rotated keys and refined values, [B, h, P_max, dh].
One ``step`` = dm_decode_step: project the token, read tape rows
[max(0, pos-W+1), pos) plus the raw self pair (split-P streaming kernel +
LSE merge), refine_kv, and write the refined pair into slot ``pos``.
"""

import ctypes

import torch

from . import _lib as L
from .engine import PackedWeights, check_supported


class StaticTape:
    """noalloc=True steps through dm_decode_step_noalloc: no workspace tensor, the
    library's static scratch instead (for graph capture / serving loops); steps whose
    scratch would exceed _lib.DM_DECODE_SCRATCH_MAX are refused at construction."""

    def __init__(self, attn_or_cfg, B, P_max, device="cuda", dtype=torch.bfloat16, sd=None, noalloc=False):
        cfg = attn_or_cfg.cfg if hasattr(attn_or_cfg, "cfg") else attn_or_cfg
        check_supported(cfg)
        self.cfg, self.B, self.P = cfg, B, P_max
        self.device, self.dtype = torch.device(device), dtype
        h, dh = cfg.n_heads, cfg.head_dim
        self.K = torch.zeros(B, h, P_max, dh, device=self.device, dtype=dtype)
        self.V = torch.zeros_like(self.K)
        self.conf = L.make_config(cfg, B, dtype)
        nbytes = L.lib().dm_decode_workspace_bytes(ctypes.byref(self.conf), P_max)
        if nbytes == 0:
            raise L.DMError("dm_decode_workspace_bytes rejected the configuration")
        self.noalloc = noalloc
        if noalloc:
            if nbytes > L.DM_DECODE_SCRATCH_MAX:
                raise L.DMError(f"decode scratch {nbytes} bytes > the static {L.DM_DECODE_SCRATCH_MAX}")
            self.workspace = None
        else:
            self.workspace = torch.empty(nbytes, device=self.device, dtype=torch.uint8)
        self.o_cat = torch.empty(B, cfg.d_model, device=self.device, dtype=dtype)
        self.y = torch.empty(B, cfg.d_model, device=self.device, dtype=dtype)
        self.w = PackedWeights(cfg, self.device, dtype, with_transposes=False)
        self._attn = attn_or_cfg if hasattr(attn_or_cfg, "named_parameters") else None
        self._ver = None
        if sd is not None:
            self.w.pack(sd)

    def _refresh(self):
        if self._attn is None:
            return
        ver = self._attn._param_version()
        if ver != self._ver:
            self.w.pack(dict(self._attn.named_parameters()))
            self._ver = ver

    def step(self, xhat, pos, cos, sin, with_wo=False):
        """xhat [B, d] (pre-normed, storage dtype). Returns (o_cat [B,d], y or None).

        pos: the absolute position (int), or a one-element int32 tensor on the device that
        the kernels read at run time (lm/eval/graph_decode.py:24: one captured graph serves
        every position); the caller keeps it inside [0, P_max)."""
        self._refresh()
        xhat = xhat.contiguous()
        assert xhat.dtype == self.dtype and xhat.shape == (self.B, self.cfg.d_model)
        cos = cos.to(device=self.device, dtype=torch.float32).contiguous()
        sin = sin.to(device=self.device, dtype=torch.float32).contiguous()
        a = L.dm_decode_args()
        if isinstance(pos, torch.Tensor):
            if pos.dtype != torch.int32 or pos.numel() != 1 or pos.device.type != self.device.type:
                raise ValueError("a device position is a one-element int32 tensor on the tape's device")
            if cos.shape[0] < self.P:
                raise ValueError(f"RoPE table has {cos.shape[0]} rows; a device position needs {self.P}")
            a.pos, a.pos_dev = 0, L.ptr(pos)
        else:
            if cos.shape[0] <= pos:
                raise ValueError(f"RoPE table has {cos.shape[0]} rows, pos={pos}")
            a.pos = pos
        a.tape_T = self.P
        a.xhat, a.K_tape, a.V_tape = L.ptr(xhat), L.ptr(self.K), L.ptr(self.V)
        a.o_cat = L.ptr(self.o_cat)
        a.y = L.ptr(self.y) if with_wo else None
        ws = self.w.struct(with_attn_norm=False)
        if self.noalloc:
            L.check(L.lib().dm_decode_step_noalloc(ctypes.byref(self.conf), ctypes.byref(ws), L.ptr(cos),
                                                   L.ptr(sin), ctypes.byref(a), L.stream_ptr()))
        else:
            a.workspace, a.workspace_bytes = L.ptr(self.workspace), self.workspace.numel()
            L.check(L.lib().dm_decode_step(ctypes.byref(self.conf), ctypes.byref(ws), L.ptr(cos),
                                           L.ptr(sin), ctypes.byref(a), L.stream_ptr()))
        return self.o_cat, (self.y if with_wo else None)
