"""One training step of the whole DualModLM on one GPU: the single-GPU part of the reference's
WaveScanEngine.train_step (engines/wavescan/engine/graphs.py:36-792).

The step runs, as the engine's bodies do:
  * the embedding (``_embed_body``, graphs.py:232-239);
  * per layer the attention sublayer ``x + W_O DM(attn_norm x)`` on the HIP path (one
    ``dm_layer_fwd`` over the chunk schedule: the cells of ``_cell_fwd_body``, graphs.py:241-265)
    and the SwiGLU MLP sublayer ``x + mlp(mlp_norm x)`` (models/dualmod/model.py:123-131);
  * the final norm, the tied head and the cross-entropy loss (``_loss_body``, graphs.py:268-275,
    with the fused chunked loss of engine/backward.py);
  * the whole backward: the head and loss (``_head_bwd_body``, graphs.py:314-341), per layer from
    the top the MLP VJP and the reverse-scan attention backward (``_blockmlp_bwd_body`` /
    ``_cell_bwd_body`` / ``_close_body``, graphs.py:373-500; here ``dm_layer_bwd``), then the
    embedding (``_emb_bwd_body``, graphs.py:502-508).
Every parameter gradient is a view of ONE flat fp32 buffer (GradBuffers, backward.py:27-61; the
tied embedding / head weight once), zeroed at the start of the backward by a fill kernel, so the
whole step can be captured as one HIP graph and replayed (graphs.py:513-576 captures per segment).

Numerics follow the reference's bf16 engine (autocast): the residual stream and every matrix
product in the compute dtype with fp32 accumulation, RMSNorm statistics, softmax and the loss in
fp32, weight gradients accumulated in fp32. The DM attention and the SwiGLU MLP sublayer run in
libdm_hip.so (dm_layer_fwd / dm_layer_bwd, dm_mlp_fwd / dm_mlp_bwd); the embedding gather, the
tied head's products (hipBLASLt through torch, the weight gradient with fp32 outputs) and the loss
in torch. With ``dtype=torch.float32`` the whole step is fp32 (the parity tests).

Layer by layer (default), each layer's forward keeps its cells' sweep states in an HBM tape while
``tape_budget`` bytes allow (the backward then skips the recompute), the remaining layers recompute
their cells exactly, as the reference does; the results are the same bits either way.
``wavefront=True`` runs the blocks layer-batched (dm_stack_fwd / dm_stack_bwd with the MLP as each
block's tail: layer l works on cell t - l at step t, each kernel of a step one launch over every
active layer, engines/wave3d/wave3d.py:1-47): the same results bit for bit; tapes for every layer
or none (``tape_budget`` decides), and a backward workspace per layer.
"""

import ctypes

import torch

from . import _lib as L
from .engine import HipSweepCell, LayerGrads, _sched, check_supported, uniform_chunks


def _rms(x, w, eps):
    """RMSNorm (attention.py:74-83): fp32 statistics, result in x's dtype; also the row scale."""
    xf = x.float()
    r = torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return (xf * r * w.float()).to(x.dtype), r


def _rms_vjp(dy, x, r, w, dw):
    """VJP of y = x r w with r = rsqrt(mean x^2 + eps): returns dx (fp32) and adds sum_rows dy x r
    into dw (fp32)."""
    xf, g = x.float(), dy.float()
    dw.add_((g * xf * r).sum(0))
    gw = g * w.float()
    return r * gw - xf * (r * r * r) * (gw * xf).mean(-1, keepdim=True)


def _mm32(a, b):
    """a @ b with fp32 output (fp32 accumulation; bf16 operands stay bf16)."""
    if a.dtype == torch.float32:
        return a @ b
    return torch.mm(a, b, out_dtype=torch.float32)


class MlpWeights:
    """One block's SwiGLU weights packed for dm_mlp_fwd / dm_mlp_bwd (dm_mlp_packed)."""

    def __init__(self, d, H, device, dtype):
        kw = dict(device=device, dtype=dtype)
        self.d, self.H, self.dtype = d, H, dtype
        self.w13 = torch.empty(2 * H, d, **kw)
        self.w2 = torch.empty(d, H, **kw)
        self.w13_t = torch.empty(d, 2 * H, **kw)
        self.w2_t = torch.empty(H, d, **kw)
        self.norm_w = torch.empty(d, **kw)
        self.s = L.dm_mlp_packed()
        for n in ("w13", "w2", "w13_t", "w2_t", "norm_w"):
            setattr(self.s, n, L.ptr(getattr(self, n)))

    @torch.no_grad()
    def pack(self, blk):
        src = [t.detach().to(self.dtype).contiguous() for t in
               (blk.mlp.w1.weight, blk.mlp.w3.weight, blk.mlp.w2.weight, blk.mlp_norm.weight)]
        L.check(L.lib().dm_pack_mlp(L.dtype_code(self.dtype), *[L.ptr(t) for t in src], self.d, self.H,
                                    ctypes.byref(self.s), L.stream_ptr()))
        torch.cuda.current_stream().synchronize()   # the sources outlive the asynchronous copies


class MlpBufs:
    """dm_mlp_bufs: the forward's saved state of one block ([B, T, .] rows) and the backward's
    intermediates (dab / dh, shared between layers when given)."""

    def __init__(self, B, T, d, H, device, dtype, dab=None, dh=None):
        kw = dict(device=device, dtype=dtype)
        self.h = torch.empty(B, T, d, **kw)
        self.ab = torch.empty(B, T, 2 * H, **kw)
        self.mid = torch.empty(B, T, H, **kw)
        self.dab = dab if dab is not None else torch.empty(B, T, 2 * H, **kw)
        self.dh = dh if dh is not None else torch.empty(B, T, d, device=device, dtype=torch.float32)
        self.s = L.dm_mlp_bufs()
        for n in ("h", "ab", "mid", "dab", "dh"):
            setattr(self.s, n, L.ptr(getattr(self, n)))


class HipTrunk:
    """Training step of a ``model.DualModLM`` (dense attention knobs, mlp_hidden a multiple of 128)
    at batch B, length T.

    schedule: the chunk schedule of every layer (default c = 64, K = 4); tape_budget: bytes of
    forward tapes to keep (layer by layer: layers 0, 1, ... while they fit; wavefront: every layer
    if all fit, else none; None: every layer; "auto": the device memory still free once everything
    else is allocated, less TAPE_RESERVE). ``refresh()`` re-reads the parameters (packs the
    attention and MLP weights, casts the embedding / head weight) and must follow every parameter
    update; ``capture()`` records one step as a HIP graph."""

    TAPE_RESERVE = 24e9   # bytes left free by tape_budget="auto" (the head's chunks, the graph pool)

    def __init__(self, model, B, T, schedule=None, tape_budget=None, loss_chunk=4096, wavefront=False):
        cfg = model.cfg
        check_supported(cfg)
        if cfg.gate_rank or cfg.ctx_rank:
            raise NotImplementedError("the trunk step takes dense attention parameters (gate_rank = ctx_rank = 0)")
        if not cfg.tie_embeddings:
            raise NotImplementedError("the trunk step ties the head to the embedding (models/dualmod/model.py:141)")
        if cfg.mlp_hidden % 128:
            raise NotImplementedError(f"mlp_hidden={cfg.mlp_hidden}: the MLP kernels take multiples of 128")
        if T > cfg.max_seq_len:
            raise ValueError(f"T={T} > max_seq_len={cfg.max_seq_len}")
        self.m, self.cfg, self.B, self.T = model, cfg, B, T
        self.dt = model.dtype
        self.dev = next(model.parameters()).device
        d, Fh, V, nl = cfg.d_model, cfg.mlp_hidden, cfg.vocab_size, cfg.n_layers
        self.H = Fh
        self.schedule = list(schedule) if schedule is not None else uniform_chunks(T, 64, 4)
        self.loss_chunk = min(loss_chunk, B * T)
        self.wavefront = wavefront
        self.eps = float(model.blocks[0].mlp_norm.eps)
        kw = dict(device=self.dev, dtype=self.dt)
        M = B * T

        # ---- one flat fp32 gradient buffer; each parameter's gradient a view of it ----
        self.names = [n for n, _ in model.named_parameters()]   # the tied weight once
        params = dict(model.named_parameters())
        sizes = [params[n].numel() for n in self.names]
        self.flat = torch.zeros(sum(sizes), device=self.dev, dtype=torch.float32)
        self.grad, off = {}, 0
        for n, sz in zip(self.names, sizes):
            self.grad[n] = self.flat[off:off + sz].view_as(params[n])
            off += sz

        # ---- attention cells: packed weights per layer; the forward and backward workspaces one per
        # layer layer-batched (the active layers' cells run concurrently), else one each ----
        self.cells = [HipSweepCell(cfg, B, T, device=self.dev, dtype=self.dt) for _ in range(nl)]
        if not wavefront:   # layer-batched, the active layers' cells run concurrently: a workspace each
            for c in self.cells[1:]:
                c.workspace = self.cells[0].workspace
        kmax = max(k for _, _, k in self.schedule)
        bws = self.cells[0]._bwd_workspace(T, T, kmax)
        for c in self.cells[1:]:
            if wavefront:
                c._bwd_workspace(T, T, kmax)
            else:
                c._bwd_ws, c._bwd_key = bws, self.cells[0]._bwd_key
        self.lgrads = []
        for l in range(nl):
            g = LayerGrads(cfg, self.dev)
            for name in g.t:
                full = f"blocks.{l}.attn_norm.weight" if name == "attn_norm.weight" else f"blocks.{l}.attn.{name}"
                g.t[name] = self.grad[full]
            self.lgrads.append(g)

        # ---- MLP sublayers: packed weights, saved state, gradient views, one workspace ----
        self.mw = [MlpWeights(d, Fh, self.dev, self.dt) for _ in range(nl)]
        shared = {} if wavefront else dict(dab=torch.empty(B, T, 2 * Fh, **kw),
                                           dh=torch.empty(B, T, d, device=self.dev, dtype=torch.float32))
        self.mb = [MlpBufs(B, T, d, Fh, self.dev, self.dt, **shared) for _ in range(nl)]
        self.mg = []
        for l in range(nl):
            g = L.dm_mlp_grads()
            for f, n in (("w1", "mlp.w1.weight"), ("w3", "mlp.w3.weight"), ("w2", "mlp.w2.weight"),
                         ("norm_w", "mlp_norm.weight")):
                setattr(g, f, L.ptr(self.grad[f"blocks.{l}.{n}"]))
            self.mg.append(g)
        nb = L.lib().dm_mlp_workspace_bytes(L.dtype_code(self.dt), M, d, Fh)
        if nb == 0:
            raise L.DMError("dm_mlp_workspace_bytes rejected the MLP shape")
        self.mlp_ws = torch.empty(nb, device=self.dev, dtype=torch.uint8)

        # ---- activations (the engine's xl ladder and the per-layer state the backward reads) ----
        self.idx = torch.zeros(B, T, dtype=torch.long, device=self.dev)
        self.targets = torch.zeros(B, T, dtype=torch.long, device=self.dev)
        self.xs = [torch.zeros(B, T, d, **kw) for _ in range(nl + 1)]    # block inputs, xs[nl] the trunk output
        self.ys = [torch.zeros(B, T, d, **kw) for _ in range(nl)]        # after the attention sublayer
        self.dxs = [torch.zeros(B, T, d, **kw) for _ in range(nl + 1)]   # grads of xs
        # grads of ys: one buffer layer by layer, one per layer layer-batched
        self.dys = [torch.zeros(B, T, d, **kw) for _ in range(nl if wavefront else 1)]
        self.bufs = [c.new_bufs(T) for c in self.cells]
        h, dh = cfg.n_heads, cfg.head_dim
        self.K = [torch.zeros(B, h, T, dh, **kw) for _ in range(nl)]
        self.V = [torch.zeros(B, h, T, dh, **kw) for _ in range(nl)]
        self.ocat = [torch.zeros(B, T, d, **kw) for _ in range(nl)]
        per_tape = self.cells[0].tape_bytes(self.schedule)
        if tape_budget == "auto":   # what is free now, less a reserve for the step's temporaries
            tape_budget = torch.cuda.mem_get_info(self.dev)[0] - self.TAPE_RESERVE
        n_tape = nl if tape_budget is None else max(0, min(nl, int(tape_budget // per_tape)))
        if wavefront and n_tape < nl:
            n_tape = 0
        self.tapes = [self.cells[l].new_tape(self.schedule) if l < n_tape else None for l in range(nl)]
        self.n_tape = n_tape
        self.loss = torch.zeros((), device=self.dev, dtype=torch.float32)
        self.cos = model.rope_cos[:T].to(self.dev, torch.float32).contiguous()
        self.sin = model.rope_sin[:T].to(self.dev, torch.float32).contiguous()
        self.w_emb = torch.zeros(V, d, **kw)   # the embedding / head weight in the compute dtype
        self._fplan = self._bplan = None
        self.graph = None
        self.timer = None   # optional per-layer attention timing (CellTimer, layer by layer only)
        self.refresh()

    @torch.no_grad()
    def refresh(self):
        """Re-read every parameter: pack each layer's attention weights (with its attn_norm) and MLP
        weights (with its mlp_norm), cast the embedding / head weight to the compute dtype. Outside
        any capture; a captured graph keeps working (the copies are rewritten in place)."""
        for cell, mw, blk in zip(self.cells, self.mw, self.m.blocks):
            cell.pack(dict(blk.attn.named_parameters()), attn_norm_w=blk.attn_norm.weight)
            mw.pack(blk)
        self.w_emb.copy_(self.m.tok_emb.weight)

    # ---- the sublayers, layer by layer ---------------------------------------------------------
    def _attn_fwd(self, l):
        self.cells[l].layer_forward(self.xs[l], self.ys[l], self.cos, self.sin, self.schedule, self.K[l], self.V[l],
                                    self.ocat[l], self.bufs[l], tape=self.tapes[l])

    def _attn_bwd(self, l):
        self.cells[l].layer_backward(self.xs[l], self.dys[0], self.dxs[l], self.cos, self.sin, self.schedule,
                                     self.K[l], self.V[l], self.ocat[l], self.bufs[l], self.lgrads[l],
                                     tape=self.tapes[l])

    def _mlp_fwd(self, l):
        L.check(L.lib().dm_mlp_fwd(L.dtype_code(self.dt), ctypes.byref(self.mw[l].s), L.ptr(self.ys[l]),
                                   L.ptr(self.xs[l + 1]), ctypes.byref(self.mb[l].s), self.B * self.T,
                                   self.cfg.d_model, self.H, self.eps, L.stream_ptr()))

    def _mlp_bwd(self, l):
        """dz = dxs[l + 1] -> dys[0] (the grad of ys[l]); the MLP weight grads added into the buffer."""
        L.check(L.lib().dm_mlp_bwd(L.dtype_code(self.dt), ctypes.byref(self.mw[l].s), L.ptr(self.ys[l]),
                                   L.ptr(self.dxs[l + 1]), L.ptr(self.dys[0]), ctypes.byref(self.mb[l].s),
                                   ctypes.byref(self.mg[l]), self.B * self.T, self.cfg.d_model, self.H, self.eps,
                                   L.ptr(self.mlp_ws), self.mlp_ws.numel(), L.stream_ptr()))

    # ---- the blocks layer-batched (dm_stack_fwd / dm_stack_bwd with the MLP tails) -------------
    def _stack_fwd(self):
        conf = self.cells[0]._conf(True)
        sched = _sched(self.schedule)
        arr = (L.dm_stack_layer * self.cfg.n_layers)()
        self._fkeep = []
        for l, cell in enumerate(self.cells):
            w, b = cell.w.struct(with_attn_norm=True), self.bufs[l].struct()
            self._fkeep += [w, b]
            a = arr[l]
            a.w, a.bufs = ctypes.addressof(w), ctypes.addressof(b)
            a.x, a.y = L.ptr(self.xs[l]), L.ptr(self.ys[l])
            a.K_cache, a.V_cache, a.ocat = L.ptr(self.K[l]), L.ptr(self.V[l]), L.ptr(self.ocat[l])
            a.tape = L.ptr(self.tapes[l])
            a.tape_bytes = 0 if self.tapes[l] is None else self.tapes[l].numel()
            a.workspace, a.workspace_bytes = L.ptr(cell.workspace), cell.workspace.numel()
            a.mlp_w, a.mlp_bufs = ctypes.addressof(self.mw[l].s), ctypes.addressof(self.mb[l].s)
            a.z, a.mlp_H = L.ptr(self.xs[l + 1]), self.H
        build = 0
        if self._fplan is None:
            n = L.lib().dm_stack_fwd_plan_bytes(ctypes.byref(conf), self.cfg.n_layers, arr, sched,
                                                len(self.schedule), self.T)
            if n == 0:
                raise L.DMError("dm_stack_fwd_plan_bytes: " + L.lib().dm_last_error().decode())
            self._fplan = torch.empty(n, device=self.dev, dtype=torch.uint8)
            build = 1
        L.check(L.lib().dm_stack_fwd(ctypes.byref(conf), self.cfg.n_layers, arr, L.ptr(self.cos), L.ptr(self.sin),
                                     sched, len(self.schedule), self.T, L.ptr(self._fplan), self._fplan.numel(), build,
                                     L.stream_ptr()))

    def _stack_bwd(self):
        conf = self.cells[0]._conf(True)
        sched = _sched(self.schedule)
        kmax = max(k for _, _, k in self.schedule)
        arr = (L.dm_stack_bwd_layer * self.cfg.n_layers)()
        self._bkeep = []
        for l, cell in enumerate(self.cells):
            w, b, g = cell.w.struct(with_attn_norm=True), self.bufs[l].struct(), self.lgrads[l].struct()
            self._bkeep += [w, b, g]
            ws = cell._bwd_workspace(self.T, self.T, kmax)
            a = arr[l]
            a.w, a.bufs, a.grads = ctypes.addressof(w), ctypes.addressof(b), ctypes.addressof(g)
            a.x, a.dy, a.dx = L.ptr(self.xs[l]), L.ptr(self.dys[l]), L.ptr(self.dxs[l])
            a.K_cache, a.V_cache, a.ocat = L.ptr(self.K[l]), L.ptr(self.V[l]), L.ptr(self.ocat[l])
            a.tape = L.ptr(self.tapes[l])
            a.tape_bytes = 0 if self.tapes[l] is None else self.tapes[l].numel()
            a.workspace, a.workspace_bytes = L.ptr(ws), ws.numel()
            a.mlp_w, a.mlp_bufs = ctypes.addressof(self.mw[l].s), ctypes.addressof(self.mb[l].s)
            a.mlp_grads = ctypes.addressof(self.mg[l])
            a.dz, a.mlp_y, a.mlp_H = L.ptr(self.dxs[l + 1]), L.ptr(self.ys[l]), self.H
            a.mlp_workspace, a.mlp_workspace_bytes = L.ptr(self.mlp_ws), self.mlp_ws.numel()
        build = 0
        if self._bplan is None:
            n = L.lib().dm_stack_bwd_plan_bytes(ctypes.byref(conf), self.cfg.n_layers, arr, sched,
                                                len(self.schedule), self.T)
            if n == 0:
                raise L.DMError("dm_stack_bwd_plan_bytes: " + L.lib().dm_last_error().decode())
            self._bplan = torch.empty(n, device=self.dev, dtype=torch.uint8)
            build = 1
        L.check(L.lib().dm_stack_bwd(ctypes.byref(conf), self.cfg.n_layers, arr, L.ptr(self.cos), L.ptr(self.sin),
                                     sched, len(self.schedule), self.T, L.ptr(self._bplan), self._bplan.numel(), build,
                                     L.stream_ptr()))

    # ---- the head, the loss and the embedding ---------------------------------------------------
    def _head(self):
        """norm_f, the tied head and the mean cross entropy (ignore_index -1, model.py:279-281), with
        its gradient: the loss's softmax gradient needs nothing but the logits, so the head's VJP runs
        with its forward, chunk by chunk of rows (the reference's loss_chunk, graphs.py:322-341)."""
        m = self.m
        M, d = self.B * self.T, self.cfg.d_model
        x = self.xs[-1].view(M, d)
        tg = self.targets.view(M)
        nvalid = (tg >= 0).sum().clamp_min(1).float()
        gw = self.grad["tok_emb.weight"]
        gnf = self.grad["norm_f.weight"]
        loss = torch.zeros((), device=self.dev, dtype=torch.float32)
        dxl = self.dxs[-1].view(M, d)
        for r0 in range(0, M, self.loss_chunk):
            r1 = min(r0 + self.loss_chunk, M)
            xc, t = x[r0:r1], tg[r0:r1]
            hf, r = _rms(xc, m.norm_f.weight, m.norm_f.eps)
            lg = (hf @ self.w_emb.t()).float()
            lse = torch.logsumexp(lg, -1)
            valid = t >= 0
            tc = t.clamp_min(0)
            loss = loss + ((lse - lg.gather(1, tc[:, None])[:, 0]) * valid).sum()
            p = torch.exp(lg - lse[:, None])
            p.scatter_add_(1, tc[:, None], -valid[:, None].float())
            dl = (p * (valid[:, None].float() / nvalid)).to(self.dt)
            gw.add_(_mm32(dl.t(), hf))
            dhf = dl @ self.w_emb
            dxl[r0:r1].copy_(_rms_vjp(dhf, xc, r, m.norm_f.weight, gnf))
        self.loss.copy_(loss / nvalid)

    def _embed_bwd(self):
        M, d = self.B * self.T, self.cfg.d_model
        g = torch.ops.aten.embedding_dense_backward(self.dxs[0].view(M, d).float(), self.idx.view(M),
                                                    self.cfg.vocab_size, -1, False)
        self.grad["tok_emb.weight"].add_(g)

    def _run(self):
        with torch.no_grad():
            torch.index_select(self.w_emb, 0, self.idx.view(-1), out=self.xs[0].view(-1, self.cfg.d_model))
            if self.wavefront:
                self._stack_fwd()
                self.flat.zero_()
                self._head()
                self._stack_bwd()
                self._embed_bwd()
                return
            tm = self.timer
            for l in range(self.cfg.n_layers):
                if tm is not None:
                    tm.start(l, 0)
                self._attn_fwd(l)
                if tm is not None:
                    tm.stop(l, 0)
                self._mlp_fwd(l)
            self.flat.zero_()
            self._head()
            for l in reversed(range(self.cfg.n_layers)):
                self._mlp_bwd(l)
                if tm is not None:
                    tm.start(l, 1)
                self._attn_bwd(l)
                if tm is not None:
                    tm.stop(l, 1)
            self._embed_bwd()

    def capture(self):
        """Record one step as a HIP graph (after an eager warm-up step on the capture stream, which
        also writes the layer-batched launch plans)."""
        s = torch.cuda.Stream(device=self.dev)
        s.wait_stream(torch.cuda.current_stream(self.dev))
        with torch.cuda.stream(s):
            self._run()
        torch.cuda.current_stream(self.dev).wait_stream(s)
        torch.cuda.synchronize(self.dev)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=s):
            self._run()
        torch.cuda.synchronize(self.dev)
        return self

    def train_step(self, idx, targets):
        """Forward + backward of the batch (idx, targets [B, T] token ids; targets -1 are ignored).
        Returns the loss (a static device scalar, overwritten by the next step); the gradients are
        the views ``grad[name]`` of the flat buffer ``flat`` (``to_param_grads`` copies them into
        the parameters' .grad)."""
        self.idx.copy_(idx)
        self.targets.copy_(targets)
        if self.graph is not None:
            self.graph.replay()
        else:
            self._run()
        return self.loss

    def to_param_grads(self):
        """param.grad = the flat buffer's view of it (GradBuffers.to_param_grads, backward.py:52-61)."""
        for n, p in self.m.named_parameters():
            p.grad = self.grad[n].clone()


class CellTimer:
    """HIP events around each layer's attention forward (slot 0) and backward (slot 1) inside a
    trunk step: the per-layer DM cell time measured in place (the reference reports its cell per
    layer inside the full step)."""

    def __init__(self, n_layers):
        self.ev = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(2)]
                   for _ in range(n_layers)]

    def start(self, l, k):
        self.ev[l][k][0].record()

    def stop(self, l, k):
        self.ev[l][k][1].record()

    def ms(self):
        """(forward ms, backward ms) per layer of the last step (after a synchronize)."""
        return [(a[0].elapsed_time(a[1]), b[0].elapsed_time(b[1])) for a, b in self.ev]
