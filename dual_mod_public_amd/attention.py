"""DualModAttention on the HIP path — same parameters and call signatures as
models/dualmod/attention.py:86-588, so reference state dicts load unchanged.

``forward`` runs the exact chunked scan (K = c per chunk, equal to the
sequential scan by nilpotency, scan_cell_fwd.py:1-10) in libdm_hip.so;
``decode_step`` runs the static-tape decode kernels. Knobs outside the HIP
path's set raise NotImplementedError at construction (engine.check_supported).
"""

import math

import torch
import torch.nn as nn

from . import _lib as L
from .config import DualModConfig
from .engine import HipSweepCell, check_supported, uniform_chunks
from .lowrank import LoRAGate, LoRALinear


class RMSNorm(nn.Module):
    """attention.py:74-83. Inside the attention path the kernels apply it (norm_ctx); the
    trunk's attn_norm / mlp_norm / norm_f call ``forward``: fp32 statistics, result in the
    input's dtype."""

    def __init__(self, d, eps=1e-5):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(d))
        self.eps = eps

    def forward(self, x):
        xf = x.float()
        return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps) * self.weight.float()).to(x.dtype)


def _forward_only(name, module, *tensors):
    """attend_one / refine_kv run the HIP kernels without an autograd graph: a call that would
    need gradients (grad mode on, and an input or a parameter that requires them) raises instead
    of returning a result that silently has none."""
    if not torch.is_grad_enabled():
        return
    params = module.parameters() if module is not None else ()
    if any(t is not None and t.requires_grad for t in tensors) or any(p.requires_grad for p in params):
        raise NotImplementedError(f"{name} is forward-only on the HIP path (no autograd); "
                                  "differentiate through forward() or call it under torch.no_grad()")


class DualModAttention(nn.Module):
    CHUNK = 64   # chunk length of the exact forward (cells of K = c sweeps)

    def __init__(self, cfg: DualModConfig):
        super().__init__()
        check_supported(cfg)
        self.cfg = cfg
        d = cfg.d_model
        self.n_heads = cfg.n_heads
        self.head_dim = cfg.head_dim
        self.scale = 1.0 / math.sqrt(cfg.head_dim)
        self.wq = nn.Linear(d, d, bias=False)
        self.wk = nn.Linear(d, d, bias=False)
        self.wv = nn.Linear(d, d, bias=False)
        self.wo = nn.Linear(d, d, bias=False)
        # ctx_rank / gate_rank > 0: factored operators with the reference's parameter
        # names (attention.py:24-75, 125-152, 182-183); the kernels get their dense products
        def ctx_mat(bias=False):
            if cfg.ctx_rank > 0:
                return LoRALinear(d, cfg.ctx_rank, d, bias=bias)
            return nn.Linear(d, d, bias=bias)

        def gate():
            if cfg.gate_rank > 0:
                return LoRAGate(2 * d, cfg.gate_rank, d)
            return nn.Linear(2 * d, d, bias=True)

        self.w_kctx = ctx_mat()
        self.w_gk = gate()
        self.w_vctx = ctx_mat()
        self.w_gv = gate()
        if cfg.ctx_mod in ("mult", "mult_res"):
            self.v_gate = ctx_mat(bias=True)
            self.v_map = ctx_mat()
        elif cfg.ctx_mod == "fusion":
            # attention.py:173-174, 198-200: v_in = u + silu(v_pre([xhat, u])), zero-initialised
            self.v_pre = nn.Linear(2 * d, d, bias=False)
            nn.init.zeros_(self.v_pre.weight)
        self.norm_ctx = RMSNorm(d)
        # per-head RMS-norm gains (attention.py:113-114, 145-148, 165-166)
        if getattr(cfg, "v_norm", "none") == "rms":
            self.v_gain = nn.Parameter(torch.ones(cfg.n_heads))
        if getattr(cfg, "k_ctx_norm", "none") == "rms":
            self.k_gain = nn.Parameter(torch.full((cfg.n_heads,), float(getattr(cfg, "k_gain_init", 1.75))))
        if getattr(cfg, "v_ctx_norm", "none") == "rms":
            self.ctx_gain = nn.Parameter(torch.ones(cfg.n_heads))
        self._cells = {}
        self._packed_version = None

    # ---- HIP cell cache --------------------------------------------------------
    def _param_version(self):
        return tuple((p.data_ptr(), p._version) for p in self.parameters())

    def _hip_cell(self, B, cache_T, dtype):
        key = (B, cache_T, dtype)
        cell = self._cells.get(key)
        ver = self._param_version()
        if cell is None:
            dev = self.wq.weight.device
            cell = HipSweepCell(self.cfg, B, cache_T, device=dev, dtype=dtype)
            self._cells[key] = cell
            cell._ver = None
        if cell._ver != ver:
            cell.pack(dict(self.named_parameters()))
            cell._ver = ver
        return cell

    # ---- full-sequence forward (attention.py:438-447, mode "sequential") --------
    def forward(self, xhat, cos, sin, collect=None, n_sweeps=None):
        """xhat [B,T,d] pre-normed; cos/sin rows 0..T-1. Returns W_O o_cat [B,T,d].

        Runs the chunked scan with chunks of CHUNK rows: n_sweeps=None gives K = c
        sweeps per chunk, equal to the exact sequential scan (nilpotency,
        scan_cell_fwd.py:1-10); n_sweeps < c gives the chunked Jacobi result at that
        K. Differentiable: the backward is the HIP reverse scan with exact recompute."""
        if collect is not None:
            raise NotImplementedError("telemetry collection is not supported on the HIP path")
        from .autograd import dm_layer
        B, T, d = xhat.shape
        cell = self._hip_cell(B, T, xhat.dtype)
        params = dict(self.named_parameters())
        return dm_layer(xhat, cell, params, cos[:T], sin[:T], uniform_chunks(T, self.CHUNK, n_sweeps),
                        normalize=False, residual=False)

    # ---- the per-position step as two calls (attention.py:283-434) --------------
    def attend_one(self, q_r, k_self_r, v_self, K_past, V_past, need_probs=False, collect=None):
        """attention.py:283-312 on the HIP decode read (dm_attend_one): q_r, k_self_r, v_self
        [B,h,1,dh]; K_past / V_past [B,h,P,dh] refined rows (None or empty for none; a
        ``cache[:, :, :P]`` view of a contiguous cache is read in place). The config's
        local_window keeps the last W-1 rows. Returns (o [B,h,1,dh], None)."""
        if need_probs or collect is not None:
            raise NotImplementedError("attention probabilities / telemetry are not materialised on the HIP path")
        _forward_only("attend_one", None, q_r, k_self_r, v_self, K_past, V_past)   # no parameters involved
        from .engine import _row_stride
        B, h, _, dh = q_r.shape
        dt = q_r.dtype
        P = 0 if K_past is None else K_past.shape[2]
        conf = L.make_config(self.cfg, B, dt)
        q, ks, vs = (t.reshape(B, h, dh).contiguous() for t in (q_r, k_self_r, v_self))
        past_T = P
        if P:
            past_T = _row_stride(K_past, P)
            if _row_stride(V_past, P) != past_T:
                raise ValueError("K_past and V_past must have the same layout")
        o = torch.empty(B, h, dh, device=q_r.device, dtype=dt)
        import ctypes
        n = L.lib().dm_decode_workspace_bytes(ctypes.byref(conf), max(P, 1))
        ws = torch.empty(n, device=q_r.device, dtype=torch.uint8)
        L.check(L.lib().dm_attend_one(ctypes.byref(conf), L.ptr(q), L.ptr(ks), L.ptr(vs),
                                      L.ptr(K_past) if P else None, L.ptr(V_past) if P else None, P, past_T,
                                      L.ptr(o), L.ptr(ws), n, L.stream_ptr()))
        return o.reshape(B, h, 1, dh), None

    def refine_kv(self, xhat, o_cat, k_raw, v_raw, collect=None):
        """attention.py:314-434 on the HIP sweep GEMMs and their epilogues (dm_refine_kv): all
        inputs [B,t,d]; returns the UNROTATED (k'', v'') [B,t,d], as the reference (the caller
        rotates at write)."""
        if collect is not None:
            raise NotImplementedError("telemetry collection is not supported on the HIP path")
        _forward_only("refine_kv", self, xhat, o_cat, k_raw, v_raw)
        import ctypes
        B, t, d = xhat.shape
        h, dh = self.n_heads, self.head_dim
        dt, dev = xhat.dtype, xhat.device
        cell = self._hip_cell(B, t, dt)
        bufs = cell.new_bufs(t)
        # identity RoPE tables: the projection's rotated q / k rows are not used here, and the
        # refined key comes back unrotated
        one = torch.ones(t, dh // 2, device=dev, dtype=torch.float32)
        zero = torch.zeros_like(one)
        cell.layer_proj(xhat.contiguous(), bufs, one, zero, normalize=False)
        bufs.kraw.copy_(k_raw.reshape(B, t, h, dh).transpose(1, 2))
        bufs.vraw.copy_(v_raw.reshape(B, t, h, dh).transpose(1, 2))
        K = torch.empty(B, h, t, dh, device=dev, dtype=dt)
        V = torch.empty_like(K)
        conf = cell.conf
        n = L.lib().dm_refine_kv_workspace_bytes(ctypes.byref(conf), t)
        ws = torch.empty(n, device=dev, dtype=torch.uint8)
        L.check(L.lib().dm_refine_kv(ctypes.byref(conf), ctypes.byref(cell.w.struct(with_attn_norm=False)),
                                     ctypes.byref(bufs.struct()), L.ptr(o_cat.contiguous()), L.ptr(one),
                                     L.ptr(zero), L.ptr(K), L.ptr(V), L.ptr(ws), n, L.stream_ptr()))
        merge = lambda z: z.transpose(1, 2).reshape(B, t, d)   # noqa: E731
        return merge(K), merge(V)

    # ---- incremental decode (attention.py:564-588) ------------------------------
    @torch.no_grad()
    def decode_step(self, xhat_j, pos, cache, cos, sin):
        """One token at absolute position ``pos``; xhat_j [B,1,d] pre-normed.

        cache: the reference's {"K", "V"} dict. On first use a static tape of
        cfg.max_seq_len rows is attached as cache["tape"]; cache["K"]/["V"] are
        then views of its first pos+1 rows (refined, pre-rotated keys / values),
        the same tensors the reference's cat-append would hold.
        """
        from .decode import StaticTape
        B = xhat_j.shape[0]
        tape = cache.get("tape")
        if tape is None:
            tape = StaticTape(self, B, self.cfg.max_seq_len, xhat_j.device, xhat_j.dtype)
            if cache.get("K") is not None:
                P = cache["K"].shape[2]
                tape.K[:, :, :P] = cache["K"]
                tape.V[:, :, :P] = cache["V"]
            cache["tape"] = tape
        o_cat, y = tape.step(xhat_j.reshape(B, -1), pos, cos, sin, with_wo=True)
        cache["K"] = tape.K[:, :, :pos + 1]
        cache["V"] = tape.V[:, :, :pos + 1]
        return y.reshape(B, 1, -1).clone()   # the tape's output buffer is reused per step
