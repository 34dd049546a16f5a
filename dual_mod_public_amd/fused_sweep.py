"""The reference engine's cell interface on the HIP path: ``FusedSweepCell`` with the call shape of
engines/wavescan/cells/fused_sweep.py:1218-1959, so an engine written against it
(engines/wavescan/engine/graphs.py: ``_proj_body`` / ``_cell_fwd_body`` / ``_blockmlp_bwd_body`` /
``_cell_bwd_body`` / ``_close_body``) drives libdm_hip.so unchanged.

Each method maps onto the library's entry points:
  pack()                    dm_pack_weights per layer (attention + attn_norm), dm_pack_mlp
  layer_proj(li, x, P)      dm_layer_proj (attn_norm + projections + RoPE + gate / v_gate hoists)
  cell_forward(li, P, ...)  dm_cell_fwd (committed accumulator + n_sweeps Jacobi sweeps; final rows
                            into the caches, o_cat rows into ocat_out and the fp32 o_buf)
  layer_blockmlp_bwd        the block's W_O + residual recomputed (dm_linear), its MLP VJP
                            (dm_mlp_fwd + dm_mlp_bwd), then dm_layer_bwd_begin (W_O VJP)
  cell_backward(li, ...)    dm_cell_bwd with the caller's fp32 grad cache dK_gc / dV_gc
                            (engines/wavescan/engine/backward.py:92-123)
  layer_close(li, ...)      dm_layer_bwd_end (sweep weight grads, projection and attn_norm VJP)
The cells run the exact recompute in the backward, as the reference's (no forward tape).

Differences of form, none of result: ``P`` is this module's ``LayerBufs`` (the library's layer
buffers; the engine constructs it with the reference's arguments); the RoPE rows, ``u_buf`` and
``scratch`` arguments are accepted and unused (the kernels index the model's RoPE tables by absolute
position and carve their own workspace); every gradient, the sweep weights' included, is added
straight into ``grads`` (the engine's GradBuffers, ``.buf[id(param)]`` fp32 views), so the
reference's staging buffers ``dW_pack_buf`` / ``dnormw_buf`` / ``dW_vctx_buf`` stay zero and its
``_bwd_epilogue_body`` adds nothing more; the layer's schedule is the sequence of cells its
forward ran (a cell's backward names it by pos0).
"""

import ctypes

import torch

from . import _lib as L
from .engine import HipSweepCell, LayerGrads
from .trunk import MlpBufs, MlpWeights


class LayerBufs:
    """Engine-owned per-layer buffers (fused_sweep.py:1179-1215's signature): the library's layer
    buffers for one layer at a time (the engine's proj pass refills them per layer)."""

    def __init__(self, B, h, T, dh, d, act, device, ctx_mod="linear"):
        self.B, self.h, self.T, self.dh, self.d = B, h, T, dh, d
        self.act, self.device, self.ctx_mod = act, torch.device(device), ctx_mod
        self.bufs = None   # engine.LayerBufs, made by the cell (it knows the config)


class GradBuffers:
    """fp32 gradient accumulators keyed by parameter identity, all views of one flat buffer
    (engines/wavescan/engine/backward.py:27-61; the tied embedding / head weight once)."""

    def __init__(self, params):
        uniq, seen = [], set()
        for p in params:
            if id(p) not in seen:
                seen.add(id(p))
                uniq.append(p)
        self.order = uniq
        self.flat = torch.zeros(sum(p.numel() for p in uniq), device=uniq[0].device, dtype=torch.float32)
        self.buf, off = {}, 0
        for p in uniq:
            self.buf[id(p)] = self.flat[off:off + p.numel()].view_as(p)
            off += p.numel()

    def zero_(self):
        self.flat.zero_()

    def add(self, param, g):
        if g is not None:
            self.buf[id(param)].add_(g.float())

    def to_param_grads(self):
        for p in self.order:
            p.grad = self.buf[id(p)].clone()


class FusedSweepCell:
    def __init__(self, model):
        cfg = model.cfg
        if cfg.gate_rank or cfg.ctx_rank:
            raise NotImplementedError("the HIP FusedSweepCell takes dense attention parameters")
        self.model, self.cfg = model, cfg
        self.dev = next(model.parameters()).device
        self.dt = model.dtype
        self._cells = {}      # (li, B, T) -> HipSweepCell
        self._mlp = {}        # li -> (MlpWeights, [MlpBufs, z, dy]) for the block VJP
        self._sched = {}      # li -> [(pos0, c, n_sweeps)] of the layer's forward
        self._kv = {}         # li -> the layer's (K_cache, V_cache) of its forward
        self._state = {}      # li -> the backward's state between blockmlp_bwd and layer_close

    # ---- helpers ---------------------------------------------------------------------------
    def _cell(self, li, B, T):
        key = (li, B, T)
        cell = self._cells.get(key)
        if cell is None:
            cell = HipSweepCell(self.cfg, B, T, device=self.dev, dtype=self.dt)
            blk = self.model.blocks[li]
            cell.pack(dict(blk.attn.named_parameters()), attn_norm_w=blk.attn_norm.weight)
            self._cells[key] = cell
        return cell

    def _grads_of(self, li, grads):
        """The layer's LayerGrads as views of the engine's GradBuffers."""
        blk = self.model.blocks[li]
        g = LayerGrads(self.cfg, self.dev)
        params = dict(blk.attn.named_parameters())
        for name in g.t:
            p = blk.attn_norm.weight if name == "attn_norm.weight" else params[name]
            g.t[name] = grads.buf[id(p)]
        return g

    def _rope(self, T):
        return (self.model.rope_cos[:T].to(self.dev, torch.float32).contiguous(),
                self.model.rope_sin[:T].to(self.dev, torch.float32).contiguous())

    # ---- fused_sweep.py:1266-1291 ------------------------------------------------------------
    @torch.no_grad()
    def pack(self):
        """Re-read every layer's parameters (the engine calls this once per step, graphs.py:232-239)."""
        for (li, _, _), cell in self._cells.items():
            blk = self.model.blocks[li]
            cell.pack(dict(blk.attn.named_parameters()), attn_norm_w=blk.attn_norm.weight)
        for li, (mw, _) in self._mlp.items():
            mw.pack(self.model.blocks[li])

    # ---- fused_sweep.py:1403-1436 ------------------------------------------------------------
    @torch.no_grad()
    def layer_proj(self, li, x_l, P, zero_grads=False):
        B, T, _ = x_l.shape
        cell = self._cell(li, B, T)
        if P.bufs is None or P.bufs.T != T:
            P.bufs = cell.new_bufs(T)
        cos, sin = self._rope(T)
        cell.layer_proj(x_l.contiguous(), P.bufs, cos, sin, normalize=True)
        if not zero_grads:   # a forward pass: the layer's schedule is recorded afresh
            self._sched[li] = []

    # ---- fused_sweep.py:1455-1553 ------------------------------------------------------------
    @torch.no_grad()
    def cell_forward(self, li, P, cos_c, sin_c, K_cache, V_cache, pos0, n_sweeps, u_buf, o_buf, ocat_out=None,
                     x_c=None):
        B, h, T, dh = K_cache.shape
        c = cos_c.shape[0]
        cell = self._cell(li, B, T)
        cos, sin = self._rope(T)
        d = self.cfg.d_model
        ocat = None
        if ocat_out is not None and ocat_out.dtype == self.dt and ocat_out.stride() == (T * d, d, 1) and \
                ocat_out.storage_offset() >= pos0 * d and \
                ocat_out.untyped_storage().nbytes() >= (ocat_out.storage_offset() - pos0 * d + B * T * d) * \
                ocat_out.element_size():
            # the [:, pos0:pos0 + c] view of the engine's [B, T, d] o_cat buffer: the kernels write its base
            ocat = torch.as_strided(ocat_out, (B, T, d), (T * d, d, 1), ocat_out.storage_offset() - pos0 * d)
        o_last = o_buf if o_buf.dtype == torch.float32 and o_buf.is_contiguous() else None
        tmp = None
        if ocat is None and (ocat_out is not None or o_last is None):
            tmp = torch.empty(B, T, d, device=self.dev, dtype=self.dt)
        cell.cell_forward(P.bufs, cos, sin, K_cache, V_cache, pos0, c, n_sweeps, ocat=ocat if tmp is None else tmp,
                          o_last=o_last)
        if tmp is not None:
            if ocat_out is not None:
                ocat_out.copy_(tmp[:, pos0:pos0 + c])
            if o_last is None:
                o_buf.copy_(tmp[:, pos0:pos0 + c])
        self._sched.setdefault(li, []).append((pos0, c, n_sweeps))
        self._kv[li] = (K_cache, V_cache)
        return o_buf

    # ---- fused_sweep.py:1854-1869 ------------------------------------------------------------
    @torch.no_grad()
    def layer_blockmlp_bwd(self, li, x_l, ocat_l, dx_next, dx_out, P, grads):
        """The block's W_O + MLP VJP over the layer's rows: dx_out = d x_l through the residual
        paths (the attention's own part is added by layer_close), the W_O / MLP / mlp_norm grads
        into ``grads``; then the attention backward's accumulators are zeroed (dm_layer_bwd_begin)."""
        blk = self.model.blocks[li]
        B, T, d = x_l.shape
        H = self.cfg.mlp_hidden
        dt = self.dt
        if li not in self._mlp:
            mw = MlpWeights(d, H, self.dev, dt)
            mw.pack(blk)
            self._mlp[li] = (mw, None)
        mw, st = self._mlp[li]
        if st is None or st[0].h.shape[:2] != (B, T):
            st = (MlpBufs(B, T, d, H, self.dev, dt), torch.empty(B, T, d, device=self.dev, dtype=dt),
                  torch.empty(B, T, d, device=self.dev, dtype=dt), torch.empty(B, T, d, device=self.dev, dtype=dt))
            self._mlp[li] = (mw, st)
        mb, y, z, dy = st
        x = x_l.to(dt).contiguous()
        oc = ocat_l.to(dt).contiguous()
        L.linear(oc.view(B * T, d), blk.attn.wo.weight.to(dt).contiguous(), residual=x.view(B * T, d),
                 out=y.view(B * T, d))                                          # x_mid = x + W_O o
        code = L.dtype_code(dt)
        L.check(L.lib().dm_mlp_fwd(code, ctypes.byref(mw.s), L.ptr(y), L.ptr(z), ctypes.byref(mb.s), B * T, d, H,
                                   float(blk.mlp_norm.eps), L.stream_ptr()))
        gm = L.dm_mlp_grads()
        gm.w1, gm.w3 = L.ptr(grads.buf[id(blk.mlp.w1.weight)]), L.ptr(grads.buf[id(blk.mlp.w3.weight)])
        gm.w2, gm.norm_w = L.ptr(grads.buf[id(blk.mlp.w2.weight)]), L.ptr(grads.buf[id(blk.mlp_norm.weight)])
        nb = L.lib().dm_mlp_workspace_bytes(code, B * T, d, H)
        ws = torch.empty(nb, device=self.dev, dtype=torch.uint8)
        dz = dx_next.to(dt).contiguous()
        L.check(L.lib().dm_mlp_bwd(code, ctypes.byref(mw.s), L.ptr(y), L.ptr(dz), L.ptr(dy), ctypes.byref(mb.s),
                                   ctypes.byref(gm), B * T, d, H, float(blk.mlp_norm.eps), L.ptr(ws), nb,
                                   L.stream_ptr()))
        dx_out.copy_(dy)
        cell = self._cell(li, B, T)
        sched = self._sched[li]
        lg = self._grads_of(li, grads)
        cell.layer_backward_begin(dy, oc, P.bufs, sched, self._kv[li][0], lg)
        self._state[li] = dict(dy=dy, lg=lg, sched=sched, pos=[p for p, _, _ in sched])

    # ---- fused_sweep.py:1557-1850 ------------------------------------------------------------
    @torch.no_grad()
    def cell_backward(self, li, P, x_c, cos_c, sin_c, K_cache, V_cache, pos0, n_sweeps, dK_rows, dV_rows, grads,
                      dK_gc, dV_gc, scratch, dW_pack_buf, dnormw_buf, dW_vctx_buf=None):
        """One cell of the reverse scan: its rows' grads are dK_gc / dV_gc[:, :, pos0:pos0 + c] (the
        later cells' contributions, fp32); the grads of the committed rows it read are ADDED into
        dK_gc / dV_gc[:, :, :pos0] (backward.py:92-123)."""
        st = self._state[li]
        B, h, T, dh = K_cache.shape
        cell = self._cell(li, B, T)
        cos, sin = self._rope(T)
        cell.cell_backward(P.bufs, cos, sin, K_cache, V_cache, st["pos"].index(pos0), dK_gc, dV_gc)

    # ---- fused_sweep.py:1873-1959 ------------------------------------------------------------
    @torch.no_grad()
    def layer_close(self, li, x_l, P, dx_add, grads):
        """The layer's all-row tail (sweep weight grads, projection and attn_norm VJP): dx_add, which
        holds d x_l through the residual paths, becomes the layer's whole input grad."""
        st = self._state.pop(li)
        B, T, d = x_l.shape
        cell = self._cell(li, B, T)
        cos, sin = self._rope(T)
        K, V = self._kv[li]
        dx = torch.empty(B, T, d, device=self.dev, dtype=self.dt)
        cell.layer_backward_end(x_l.to(self.dt).contiguous(), st["dy"], dx, cos, sin, P.bufs, K, V, st["lg"])
        dx_add.copy_(dx)
