"""Host orchestration of the HIP cell: packed weights, layer buffers, cells.

Mirrors the reference engine's cell entry points:
  * ``HipSweepCell.pack / layer_proj / cell_forward`` — FusedSweepCell
    (engines/wavescan/cells/fused_sweep.py:1218-1553)
  * ``layer_forward`` — engines/wavescan/engine/forward.py:95-113
  * ``chunk_cell_forward`` — engines/wavescan/cells/scan_cell_fwd.py:88-116
  * ``uniform_chunks / exact_sequential`` — engines/wavescan/engine/schedule.py:58-69

All compute runs in libdm_hip.so; torch provides device memory and the stream.
"""

import ctypes

import torch

from . import _lib as L
from .lowrank import dense_params


def uniform_chunks(T, c, n_sweeps=None):
    """schedule.py:63-69 — fixed-size chunks; n_sweeps=None means K=c (exact)."""
    cells = []
    for pos in range(0, T, c):
        cc = min(c, T - pos)
        cells.append((pos, cc, cc if n_sweeps is None else min(n_sweeps, cc)))
    return cells


def exact_sequential(T):
    """schedule.py:58-60 — every position its own exact cell."""
    return [(j, 1, 1) for j in range(T)]


def check_supported(cfg):
    """The knob set the HIP path implements; anything else raises (no fallback).
    Mirrors FusedSweepCell.__init__'s asserts (fused_sweep.py:1219-1225)."""
    bad = []
    if cfg.gate_type != "convex_sigmoid":
        bad.append(f"gate_type={cfg.gate_type}")
    if getattr(cfg, "gate_type_v", "convex") != "convex":
        bad.append(f"gate_type_v={cfg.gate_type_v}")
    if cfg.gate_input != "xu":
        bad.append(f"gate_input={cfg.gate_input}")
    if not (cfg.enable_key_mod and cfg.enable_value_mod):
        bad.append("enable_key_mod/enable_value_mod must both be True")
    if not cfg.rmsnorm_on_o:
        bad.append("rmsnorm_on_o=False")
    if cfg.ctx_mod not in L.CTX_MOD:
        bad.append(f"ctx_mod={cfg.ctx_mod}")
    for knob, _, _ in L.NORM_KNOBS:
        if getattr(cfg, knob, "none") not in ("none", "rms"):
            bad.append(f"{knob}={getattr(cfg, knob)}")
    for knob in ("attn_logn_ref",):
        if getattr(cfg, knob, 0):
            bad.append(f"{knob}={getattr(cfg, knob)}")
    if cfg.head_dim not in (64, 128):
        bad.append(f"head_dim={cfg.head_dim} (64 or 128)")
    if cfg.d_model % 128:
        bad.append(f"d_model={cfg.d_model} (multiple of 128)")
    if bad:
        raise NotImplementedError("HIP DM path does not implement: " + ", ".join(bad))


class PackedWeights:
    """Device-side packed weights of one layer (dm_packed)."""

    def __init__(self, cfg, device, dtype, with_transposes=True):
        check_supported(cfg)
        d = cfg.d_model
        self.cfg, self.device, self.dtype = cfg, device, dtype
        mult = cfg.ctx_mod != "linear"
        kw = dict(device=device, dtype=dtype)
        nproj = 6 if mult else 5
        self.w_proj = torch.empty(nproj * d, d, **kw)
        self.b_proj = torch.zeros(3 * d, device=device, dtype=torch.float32)
        self.w_sweep = torch.empty(4 * d, d, **kw)
        self.w_vctx = torch.empty(d, d, **kw) if mult else None
        self.norm_ctx_w = torch.empty(d, **kw)
        self.attn_norm_w = torch.empty(d, **kw)
        self.wo = torch.empty(d, d, **kw)
        # transposed copies for the backward
        self.w_proj_t = torch.empty(d, nproj * d, **kw) if with_transposes else None
        self.w_sweep_t = torch.empty(d, 4 * d, **kw) if with_transposes else None
        self.w_vctx_t = torch.empty(d, d, **kw) if (with_transposes and mult) else None
        self.wo_t = torch.empty(d, d, **kw) if with_transposes else None
        # per-head norm gains, fp32: k_gain | ctx_gain | v_gain
        self.gains = (torch.ones(3 * cfg.n_heads, device=device, dtype=torch.float32)
                      if L.norm_bits(cfg) else None)
        self.has_attn_norm = False

    def struct(self, with_attn_norm=None):
        s = L.dm_packed()
        s.w_proj, s.b_proj, s.w_sweep = L.ptr(self.w_proj), L.ptr(self.b_proj), L.ptr(self.w_sweep)
        s.w_vctx, s.norm_ctx_w, s.wo = L.ptr(self.w_vctx), L.ptr(self.norm_ctx_w), L.ptr(self.wo)
        s.w_proj_t, s.w_sweep_t = L.ptr(self.w_proj_t), L.ptr(self.w_sweep_t)
        s.w_vctx_t, s.wo_t = L.ptr(self.w_vctx_t), L.ptr(self.wo_t)
        s.gains = L.ptr(self.gains)
        use = self.has_attn_norm if with_attn_norm is None else with_attn_norm
        s.attn_norm_w = L.ptr(self.attn_norm_w) if use else None
        return s

    @torch.no_grad()
    def pack(self, sd, attn_norm_w=None):
        """sd: mapping with the reference parameter names (attention.py:100-202) —
        a state dict or a DualModAttention's named parameters."""
        cfg = self.cfg
        keep = []
        sd = dense_params(sd)   # factored gates / ctx operators (gate_rank, ctx_rank) -> dense

        def t(name):
            x = sd[name].detach().to(device=self.device, dtype=self.dtype).contiguous()
            keep.append(x)
            return L.ptr(x)

        p = L.dm_params()
        for f, n in (("wq", "wq.weight"), ("wk", "wk.weight"), ("wv", "wv.weight"),
                     ("wo", "wo.weight"), ("w_kctx", "w_kctx.weight"), ("w_vctx", "w_vctx.weight"),
                     ("w_gk", "w_gk.weight"), ("w_gv", "w_gv.weight"), ("b_gk", "w_gk.bias"),
                     ("b_gv", "w_gv.bias"), ("norm_ctx_w", "norm_ctx.weight")):
            setattr(p, f, t(n))
        if cfg.ctx_mod == "fusion":
            p.v_pre = t("v_pre.weight")
        elif cfg.ctx_mod != "linear":
            p.v_gate, p.b_vgate, p.v_map = t("v_gate.weight"), t("v_gate.bias"), t("v_map.weight")
        for knob, _, gname in L.NORM_KNOBS:   # per-head norm gains (attention.py:113-166)
            if getattr(cfg, knob, "none") == "rms":
                setattr(p, gname, t(gname))
        if attn_norm_w is None and "attn_norm.weight" in sd:
            attn_norm_w = sd["attn_norm.weight"]
        if attn_norm_w is not None:
            a = attn_norm_w.detach().to(device=self.device, dtype=self.dtype).contiguous()
            keep.append(a)
            p.attn_norm_w = L.ptr(a)
            self.has_attn_norm = True
        out = self.struct(with_attn_norm=attn_norm_w is not None)
        c = L.make_config(cfg, 1, self.dtype)
        L.check(L.lib().dm_pack_weights(ctypes.byref(c), ctypes.byref(p), ctypes.byref(out),
                                        L.stream_ptr()))
        # sources must outlive the async copies: wait on this stream before releasing them
        torch.cuda.current_stream().synchronize()
        return self


class LayerBufs:
    """Per-layer projection buffers (dm_layer_bufs) for batch B, length T."""

    def __init__(self, cfg, B, T, device, dtype):
        d, h, dh = cfg.d_model, cfg.n_heads, cfg.head_dim
        kw = dict(device=device, dtype=dtype)
        self.B, self.T = B, T
        self.xhat = torch.empty(B, T, d, **kw)
        self.qr = torch.empty(B, h, T, dh, **kw)
        self.kraw = torch.empty(B, h, T, dh, **kw)
        self.kself = torch.empty(B, h, T, dh, **kw)
        self.vraw = torch.empty(B, h, T, dh, **kw)
        # gate inputs in the storage dtype, as the reference's LayerBufs (fused_sweep.py:1189, 1207)
        self.glogx = torch.empty(B, T, 2 * d, **kw)
        self.sig = torch.empty(B, T, d, **kw) if cfg.ctx_mod != "linear" else None
        # v_raw before the v_norm, kept for the backward
        self.vpre = torch.empty(B, h, T, dh, **kw) if getattr(cfg, "v_norm", "none") == "rms" else None

    def struct(self):
        s = L.dm_layer_bufs()
        s.T = self.T
        for n in ("xhat", "qr", "kraw", "kself", "vraw", "glogx", "sig", "vpre"):
            setattr(s, n, L.ptr(getattr(self, n)))
        return s


def _f32(t, device):
    return t.to(device=device, dtype=torch.float32).contiguous()


def _sched(schedule):
    return (ctypes.c_int32 * (3 * len(schedule)))(*[v for cell in schedule for v in cell])


class LayerGrads:
    """fp32 gradient buffers of one layer in the reference parameter layout (dm_grads).
    The backward ADDS into them (like .grad accumulation); ``zero_()`` clears."""

    def __init__(self, cfg, device):
        d = cfg.d_model
        mult = cfg.ctx_mod != "linear"
        shapes = {"wq.weight": (d, d), "wk.weight": (d, d), "wv.weight": (d, d), "wo.weight": (d, d),
                  "w_kctx.weight": (d, d), "w_vctx.weight": (d, d), "w_gk.weight": (d, 2 * d),
                  "w_gv.weight": (d, 2 * d), "w_gk.bias": (d,), "w_gv.bias": (d,),
                  "norm_ctx.weight": (d,), "attn_norm.weight": (d,)}
        if cfg.ctx_mod == "fusion":
            shapes["v_pre.weight"] = (d, 2 * d)
        elif mult:
            shapes.update({"v_gate.weight": (d, d), "v_gate.bias": (d,), "v_map.weight": (d, d)})
        for knob, _, gname in L.NORM_KNOBS:
            if getattr(cfg, knob, "none") == "rms":
                shapes[gname] = (cfg.n_heads,)
        self.t ={k: torch.zeros(v, device=device, dtype=torch.float32) for k, v in shapes.items()}

    def zero_(self):
        for v in self.t.values():
            v.zero_()
        return self

    def struct(self, with_attn_norm=True):
        g = L.dm_grads()
        for f, name in L.GRAD_FIELDS:
            if name == "attn_norm.weight" and not with_attn_norm:
                continue
            setattr(g, f, L.ptr(self.t.get(name)))
        return g

    def __getitem__(self, name):
        return self.t[name]


class HipSweepCell:
    """FusedSweepCell analogue for one DM layer on one GPU (fused_sweep.py:1218).

    Owns the packed weights and the cell workspace; callers own the layer
    buffers, K/V caches (append-only, rows [0, pos0) committed) and outputs.
    """

    def __init__(self, cfg, B, cache_T, device="cuda", dtype=torch.bfloat16, fused_attend=None):
        """fused_attend: None lets the library run sweep s + 1's attention inside sweep s's
        GEMM 2 launch when it pays (64-row cells, B*h >= 128); True / False force it."""
        check_supported(cfg)
        self.cfg, self.B, self.cache_T = cfg, B, cache_T
        self.device, self.dtype = torch.device(device), dtype
        self.w = PackedWeights(cfg, self.device, dtype)
        self.fuse_flags = {None: 0, True: L.DM_FLAG_FUSED_ATTEND, False: L.DM_FLAG_UNFUSED_ATTEND}[fused_attend]
        self.conf = L.make_config(cfg, B, dtype)
        self.conf.flags = self.fuse_flags
        nbytes = L.lib().dm_cell_workspace_bytes(ctypes.byref(self.conf), cache_T)
        if nbytes == 0:
            raise L.DMError("dm_cell_workspace_bytes rejected the configuration")
        self.workspace = torch.empty(nbytes, device=self.device, dtype=torch.uint8)

    def pack(self, sd, attn_norm_w=None):
        self.w.pack(sd, attn_norm_w)
        return self

    def new_bufs(self, T):
        return LayerBufs(self.cfg, self.B, T, self.device, self.dtype)

    def layer_proj(self, x, bufs, cos, sin, normalize=True):
        """fused_sweep.py:1403-1436 — projections for the whole layer.
        normalize=True applies attn_norm (Block input x); False takes x as xhat."""
        assert x.is_contiguous() and x.dtype == self.dtype
        cos, sin = _f32(cos, self.device), _f32(sin, self.device)
        ws = self.w.struct(with_attn_norm=normalize)
        b = bufs.struct()
        L.check(L.lib().dm_layer_proj(ctypes.byref(self.conf), ctypes.byref(ws), L.ptr(x),
                                      L.ptr(cos), L.ptr(sin), ctypes.byref(b), L.stream_ptr()))
        return bufs

    def cell_forward(self, bufs, cos, sin, K_cache, V_cache, pos0, c, n_sweeps, ocat=None,
                     o_last=None, K_rows=None, V_rows=None):
        """fused_sweep.py:1455-1553 — one chunk [pos0, pos0+c), n_sweeps Jacobi sweeps.
        Writes the chunk's final rows into K_cache/V_cache and (optionally) its
        o_cat rows into ocat [B, T, d] / the fp32 o_last [B*c, d].

        With K_rows / V_rows [B, h, >= c, dh] (chunk-local form, chunk_cell_forward's
        K_comm / V_comm): bufs, cos / sin and ocat hold only the chunk, K_cache / V_cache
        are the committed rows [0, pos0) (a [B, h, :pos0] view of a larger cache is read in
        place; None when pos0 == 0) and the chunk's rows go to K_rows / V_rows."""
        cos, sin = _f32(cos, self.device), _f32(sin, self.device)
        a = L.dm_cell_args()
        a.pos0, a.c, a.n_sweeps = pos0, c, n_sweeps
        if K_rows is not None:
            a.cache_T = _row_stride(K_cache, pos0) if K_cache is not None else 0
            if V_cache is not None and _row_stride(V_cache, pos0) != a.cache_T:
                raise ValueError("K_comm and V_comm must have the same layout")
            a.K_rows, a.V_rows = L.ptr(K_rows), L.ptr(V_rows)
            a.rows_T = _row_stride(K_rows, c)
        else:
            a.cache_T = K_cache.shape[2]
        a.K_cache, a.V_cache = L.ptr(K_cache), L.ptr(V_cache)
        a.ocat, a.o_last = L.ptr(ocat), L.ptr(o_last)
        a.workspace, a.workspace_bytes = L.ptr(self.workspace), self.workspace.numel()
        ws = self.w.struct()
        b = bufs.struct()
        L.check(L.lib().dm_cell_fwd(ctypes.byref(self.conf), ctypes.byref(ws), ctypes.byref(b),
                                    L.ptr(cos), L.ptr(sin), ctypes.byref(a), L.stream_ptr()))

    def _conf(self, residual):
        c = L.make_config(self.cfg, self.B, self.dtype)
        c.flags = (0 if residual else L.DM_FLAG_NO_RESIDUAL) | self.fuse_flags
        return c

    def tape_bytes(self, schedule):
        """Bytes of the saved cell states of one layer forward over ``schedule``."""
        n = L.lib().dm_layer_tape_bytes(ctypes.byref(self.conf), _sched(schedule), len(schedule))
        if n == 0:
            raise L.DMError("dm_layer_tape_bytes rejected the schedule")
        return n

    def new_tape(self, schedule):
        """Device buffer for ``layer_forward(..., tape=)``: every sweep state of every
        cell, so that ``layer_backward`` skips the per-cell recompute."""
        return torch.empty(self.tape_bytes(schedule), device=self.device, dtype=torch.uint8)

    def layer_forward(self, x, y, cos, sin, schedule, K_cache, V_cache, ocat, bufs, normalize=True,
                      residual=True, tape=None):
        """Attention sublayer y = x + W_O DM(attn_norm(x)) over ``schedule``
        (model.py:123-124 with forward.py:95-113's chunk loop), one C call.
        normalize=False takes x as xhat (no attn_norm); residual=False drops the +x
        (DualModAttention.forward, attention.py:438-447). ``tape`` (from new_tape)
        keeps every cell's sweep states for layer_backward."""
        sched = _sched(schedule)
        cos, sin = _f32(cos, self.device), _f32(sin, self.device)
        ws = self.w.struct(with_attn_norm=normalize)
        b = bufs.struct()
        conf = self._conf(residual)
        L.check(L.lib().dm_layer_fwd(
            ctypes.byref(conf), ctypes.byref(ws), L.ptr(x), L.ptr(y), L.ptr(cos), L.ptr(sin),
            ctypes.byref(b), sched, len(schedule), L.ptr(K_cache), L.ptr(V_cache),
            K_cache.shape[2], L.ptr(ocat), L.ptr(tape), 0 if tape is None else tape.numel(),
            L.ptr(self.workspace), self.workspace.numel(), L.stream_ptr()))
        return y

    def _bwd_workspace(self, T, cache_T, kmax):
        key = (T, cache_T, kmax)
        if getattr(self, "_bwd_key", None) != key:
            n = L.lib().dm_layer_bwd_workspace_bytes(ctypes.byref(self.conf), T, cache_T, kmax)
            if n == 0:
                raise L.DMError("dm_layer_bwd_workspace_bytes rejected the configuration")
            self._bwd_ws = torch.empty(n, device=self.device, dtype=torch.uint8)
            self._bwd_key = key
        return self._bwd_ws

    def layer_backward(self, x, dy, dx, cos, sin, schedule, K_cache, V_cache, ocat, bufs, grads,
                       normalize=True, residual=True, tape=None):
        """Reverse-scan backward of ``layer_forward`` (engines/wavescan/engine/backward.py:92-123,
        fused_sweep.py:1557-1959): writes dx and ADDS the parameter grads into
        ``grads`` (LayerGrads). With the forward's ``tape`` the cell states are read
        from it, else every cell is recomputed exactly (same values either way)."""
        sched = _sched(schedule)
        cos, sin = _f32(cos, self.device), _f32(sin, self.device)
        ws = self.w.struct(with_attn_norm=normalize)
        b = bufs.struct()
        conf = self._conf(residual)
        kmax = max(k for _, _, k in schedule)
        work = self._bwd_workspace(bufs.T, K_cache.shape[2], kmax)
        g = grads.struct(with_attn_norm=normalize)
        L.check(L.lib().dm_layer_bwd(
            ctypes.byref(conf), ctypes.byref(ws), L.ptr(x), L.ptr(dy), L.ptr(dx), L.ptr(cos),
            L.ptr(sin), ctypes.byref(b), sched, len(schedule), L.ptr(K_cache), L.ptr(V_cache),
            K_cache.shape[2], L.ptr(ocat), L.ptr(tape), 0 if tape is None else tape.numel(),
            ctypes.byref(g), L.ptr(work), work.numel(), L.stream_ptr()))
        return dx

    # ---- the backward one cell at a time (the reference engine's protocol) -----------
    # FusedSweepCell.layer_blockmlp_bwd / cell_backward / layer_close (fused_sweep.py:1557-1959)
    # with the fp32 grad cache of engines/wavescan/engine/backward.py:92-123. Call
    # layer_backward_begin, then cell_backward for every cell from the last to the first, then
    # layer_backward_end, with the same schedule, caches, tape and grads; the results equal
    # layer_backward's to fp32 rounding.

    def layer_backward_begin(self, dy, ocat, bufs, schedule, K_cache, grads, normalize=True, residual=True):
        """Zero the layer accumulators; W_O VJP (adds dW_O into ``grads``)."""
        self._bw = dict(schedule=list(schedule), sched=_sched(schedule), conf=self._conf(residual),
                        ws=self.w.struct(with_attn_norm=normalize), normalize=normalize,
                        work=self._bwd_workspace(bufs.T, K_cache.shape[2], max(k for _, _, k in schedule)))
        bw = self._bw
        b = bufs.struct()
        g = grads.struct(with_attn_norm=normalize)
        L.check(L.lib().dm_layer_bwd_begin(
            ctypes.byref(bw["conf"]), ctypes.byref(bw["ws"]), L.ptr(dy), L.ptr(ocat), ctypes.byref(b), bw["sched"],
            len(bw["schedule"]), K_cache.shape[2], ctypes.byref(g), L.ptr(bw["work"]), bw["work"].numel(),
            L.stream_ptr()))

    def cell_backward(self, bufs, cos, sin, K_cache, V_cache, cell, dK_gc, dV_gc, tape=None):
        """fused_sweep.py:1557 cell_backward: cell ``cell`` of the schedule given to
        layer_backward_begin. Its final rows' grads are dK_gc / dV_gc[:, :, pos0:pos0+c] (fp32
        [B, h, cache_T, dh], accumulated by the later cells); the grads of the committed rows it
        read are ADDED into dK_gc / dV_gc[:, :, :pos0]."""
        bw = self._bw
        cos, sin = _f32(cos, self.device), _f32(sin, self.device)
        assert dK_gc.dtype == torch.float32 and dK_gc.is_contiguous() and dV_gc.is_contiguous()
        a = L.dm_cell_bwd_args()
        a.sched, a.n_cells, a.cell, a.cache_T = bw["sched"], len(bw["schedule"]), cell, K_cache.shape[2]
        a.K_cache, a.V_cache, a.dK_gc, a.dV_gc = L.ptr(K_cache), L.ptr(V_cache), L.ptr(dK_gc), L.ptr(dV_gc)
        a.tape, a.tape_bytes = L.ptr(tape), 0 if tape is None else tape.numel()
        a.workspace, a.workspace_bytes = L.ptr(bw["work"]), bw["work"].numel()
        b = bufs.struct()
        L.check(L.lib().dm_cell_bwd(ctypes.byref(bw["conf"]), ctypes.byref(bw["ws"]), ctypes.byref(b), L.ptr(cos),
                                    L.ptr(sin), ctypes.byref(a), L.stream_ptr()))

    def layer_backward_end(self, x, dy, dx, cos, sin, bufs, K_cache, V_cache, grads, tape=None):
        """fused_sweep.py:1873-1959 layer_close: sweep weight grads, projection and attn_norm VJP;
        writes dx and adds the remaining parameter grads into ``grads``."""
        bw = self._bw
        cos, sin = _f32(cos, self.device), _f32(sin, self.device)
        b = bufs.struct()
        g = grads.struct(with_attn_norm=bw["normalize"])
        L.check(L.lib().dm_layer_bwd_end(
            ctypes.byref(bw["conf"]), ctypes.byref(bw["ws"]), L.ptr(x), L.ptr(dy), L.ptr(dx), L.ptr(cos), L.ptr(sin),
            ctypes.byref(b), bw["sched"], len(bw["schedule"]), L.ptr(K_cache), L.ptr(V_cache), K_cache.shape[2],
            L.ptr(tape), 0 if tape is None else tape.numel(), ctypes.byref(g), L.ptr(bw["work"]),
            bw["work"].numel(), L.stream_ptr()))
        self._bw = None
        return dx


def layer_backward_cells(cell, x, dy, dx, cos, sin, schedule, K_cache, V_cache, ocat, bufs, grads, tape=None,
                         normalize=True, residual=True):
    """engines/wavescan/engine/backward.py:92-123 (layer_backward) on the HIP cells: the
    reverse scan one cell at a time through a zeroed fp32 grad cache dK / dV [B, h, cache_T, dh],
    which ends up holding every cache row's grad from the later rows that read it. Returns dx
    and the grad cache."""
    dK = torch.zeros(K_cache.shape, device=K_cache.device, dtype=torch.float32)
    dV = torch.zeros_like(dK)
    cell.layer_backward_begin(dy, ocat, bufs, schedule, K_cache, grads, normalize=normalize, residual=residual)
    for ci in reversed(range(len(schedule))):
        cell.cell_backward(bufs, cos, sin, K_cache, V_cache, ci, dK, dV, tape=tape)
    cell.layer_backward_end(x, dy, dx, cos, sin, bufs, K_cache, V_cache, grads, tape=tape)
    return dx, dK, dV


def _row_stride(t, rows):
    """Rows per (b, h) block of a [B, h, rows, dh] tensor that is contiguous or a leading-rows
    view ``cache[:, :, :rows]`` of a contiguous [B, h, T, dh] cache (returns T); the kernels
    read such views in place."""
    B, h, n, dh = t.shape
    if n < rows:
        raise ValueError(f"{n} rows < {rows}")
    st = t.stride()
    if st[3] != 1 or st[2] != dh or st[1] % dh or st[0] != st[1] * h or st[1] // dh < n:
        raise ValueError("expected a [B, h, rows, dh] tensor or a leading-rows view of a contiguous cache")
    return st[1] // dh


def chunk_cell_forward(attn, xhat_c, cos_c, sin_c, K_comm, V_comm, n_sweeps, intra_mask=None):
    """scan_cell_fwd.py:88-116 signature: one chunk against a committed prefix.

    attn: a dual_mod_public_amd.attention.DualModAttention. xhat_c [B,c,d];
    cos_c/sin_c: RoPE rows of the chunk's positions; K_comm/V_comm [B,h,a,dh]
    (None or 0-length for the first chunk; a ``cache[:, :, :a]`` view of a larger
    contiguous cache is read in place). Returns (o_cat [B,c,d], K_rows [B,h,c,dh]
    rotated, V_rows [B,h,c,dh]). Only the chunk's rows are projected and the committed
    prefix is not copied: the cost is the cell's own, not O(a). ``intra_mask`` is
    accepted for signature compatibility; the kernels apply the strict-lower mask."""
    B, c, d = xhat_c.shape
    a = 0 if K_comm is None else K_comm.shape[2]
    cell = attn._hip_cell(B, max(a, c), xhat_c.dtype)
    dev, dt = xhat_c.device, xhat_c.dtype
    h, dh = attn.n_heads, attn.head_dim
    bufs = cell.new_bufs(c)
    cell.layer_proj(xhat_c.contiguous(), bufs, cos_c, sin_c, normalize=False)
    ocat = torch.empty(B, c, d, device=dev, dtype=dt)
    K_rows = torch.empty(B, h, c, dh, device=dev, dtype=dt)
    V_rows = torch.empty_like(K_rows)
    cell.cell_forward(bufs, cos_c, sin_c, K_comm if a else None, V_comm if a else None, a, c, n_sweeps,
                      ocat=ocat, K_rows=K_rows, V_rows=V_rows)
    return ocat, K_rows, V_rows


def layer_forward(attn, xhat, cos, sin, schedule, K_cache, V_cache, masks=None, o_out=None):
    """forward.py:95-113 signature: one layer's chunked scan over ``schedule``.
    K_cache/V_cache [B,h,T_max,dh] are written append-only. Returns o_cat [B,T,d]."""
    B, T, d = xhat.shape
    cell = attn._hip_cell(B, K_cache.shape[2], xhat.dtype)
    bufs = cell.new_bufs(T)
    cell.layer_proj(xhat.contiguous(), bufs, cos, sin, normalize=False)
    if o_out is None:
        o_out = torch.empty(B, T, d, device=xhat.device, dtype=xhat.dtype)
    for pos0, c, k in schedule:
        cell.cell_forward(bufs, cos, sin, K_cache, V_cache, pos0, c, k, ocat=o_out)
    return o_out
