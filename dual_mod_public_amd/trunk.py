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
fp32, weight gradients accumulated in fp32. The MLP and head products are plain library GEMMs
(hipBLASLt through torch; the weight gradients with fp32 outputs); the DM attention runs in
libdm_hip.so. With ``dtype=torch.float32`` the whole step is fp32 (the parity tests).

Each layer's forward keeps its cells' sweep states in an HBM tape while ``tape_budget`` bytes
allow (the backward then skips the recompute), the remaining layers recompute their cells
exactly, as the reference does; the results are the same bits either way.
"""

import torch
import torch.nn.functional as F

from .engine import HipSweepCell, LayerGrads, check_supported, uniform_chunks


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


class HipTrunk:
    """Training step of a ``model.DualModLM`` (dense attention knobs) at batch B, length T.

    schedule: the chunk schedule of every layer (default c = 64, K = 4); tape_budget: bytes of
    forward tapes to keep (layers 0, 1, ... while they fit; None: every layer). ``refresh()``
    re-reads the parameters (pack the attention weights, cast the MLP / embedding weights) and
    must follow every parameter update; ``capture()`` records one step as a HIP graph."""

    def __init__(self, model, B, T, schedule=None, tape_budget=None, loss_chunk=4096):
        cfg = model.cfg
        check_supported(cfg)
        if cfg.gate_rank or cfg.ctx_rank:
            raise NotImplementedError("the trunk step takes dense attention parameters (gate_rank = ctx_rank = 0)")
        if not cfg.tie_embeddings:
            raise NotImplementedError("the trunk step ties the head to the embedding (models/dualmod/model.py:141)")
        if T > cfg.max_seq_len:
            raise ValueError(f"T={T} > max_seq_len={cfg.max_seq_len}")
        self.m, self.cfg, self.B, self.T = model, cfg, B, T
        self.dt = model.dtype
        self.dev = next(model.parameters()).device
        d, Fh, V, nl = cfg.d_model, cfg.mlp_hidden, cfg.vocab_size, cfg.n_layers
        self.schedule = list(schedule) if schedule is not None else uniform_chunks(T, 64, 4)
        self.loss_chunk = min(loss_chunk, B * T)
        kw = dict(device=self.dev, dtype=self.dt)

        # ---- one flat fp32 gradient buffer; each parameter's gradient a view of it ----
        self.names = [n for n, _ in model.named_parameters()]   # the tied weight once
        params = dict(model.named_parameters())
        sizes = [params[n].numel() for n in self.names]
        self.flat = torch.zeros(sum(sizes), device=self.dev, dtype=torch.float32)
        self.grad, off = {}, 0
        for n, sz in zip(self.names, sizes):
            self.grad[n] = self.flat[off:off + sz].view_as(params[n])
            off += sz

        # ---- attention cells: packed weights per layer, one forward and one backward workspace ----
        self.cells = [HipSweepCell(cfg, B, T, device=self.dev, dtype=self.dt) for _ in range(nl)]
        for c in self.cells[1:]:
            c.workspace = self.cells[0].workspace
        kmax = max(k for _, _, k in self.schedule)
        bws = self.cells[0]._bwd_workspace(T, T, kmax)
        for c in self.cells[1:]:
            c._bwd_ws, c._bwd_key = bws, self.cells[0]._bwd_key
        self.lgrads = []
        for l in range(nl):
            g = LayerGrads(cfg, self.dev)
            for name in g.t:
                full = f"blocks.{l}.attn_norm.weight" if name == "attn_norm.weight" else f"blocks.{l}.attn.{name}"
                g.t[name] = self.grad[full]
            self.lgrads.append(g)

        # ---- activations (the engine's xl ladder and the per-layer state the backward reads) ----
        M = B * T
        self.idx = torch.zeros(B, T, dtype=torch.long, device=self.dev)
        self.targets = torch.zeros(B, T, dtype=torch.long, device=self.dev)
        self.xs = [torch.zeros(B, T, d, **kw) for _ in range(nl + 1)]    # block inputs, xs[nl] the trunk output
        self.ys = [torch.zeros(B, T, d, **kw) for _ in range(nl)]        # after the attention sublayer
        self.hm = [torch.zeros(M, d, **kw) for _ in range(nl)]           # mlp_norm(ys)
        self.rm = [torch.zeros(M, 1, device=self.dev, dtype=torch.float32) for _ in range(nl)]
        self.ga = [torch.zeros(M, Fh, **kw) for _ in range(nl)]          # w1 h (gate pre-activation)
        self.ub = [torch.zeros(M, Fh, **kw) for _ in range(nl)]          # w3 h
        self.dxs = [torch.zeros(B, T, d, **kw) for _ in range(nl + 1)]   # grads of xs
        self.dy = torch.zeros(B, T, d, **kw)                             # grad of ys (one layer at a time)
        self.bufs = [c.new_bufs(T) for c in self.cells]
        h, dh = cfg.n_heads, cfg.head_dim
        self.K = [torch.zeros(B, h, T, dh, **kw) for _ in range(nl)]
        self.V = [torch.zeros(B, h, T, dh, **kw) for _ in range(nl)]
        self.ocat = [torch.zeros(B, T, d, **kw) for _ in range(nl)]
        per_tape = self.cells[0].tape_bytes(self.schedule)
        n_tape = nl if tape_budget is None else max(0, min(nl, int(tape_budget // per_tape)))
        self.tapes = [self.cells[l].new_tape(self.schedule) if l < n_tape else None for l in range(nl)]
        self.n_tape = n_tape
        self.loss = torch.zeros((), device=self.dev, dtype=torch.float32)
        self.cos = model.rope_cos[:T].to(self.dev, torch.float32).contiguous()
        self.sin = model.rope_sin[:T].to(self.dev, torch.float32).contiguous()

        # ---- compute-dtype weight copies at fixed addresses (refresh() re-reads them) ----
        self.w_emb = torch.zeros(V, d, **kw)
        self.w_mlp = [tuple(torch.zeros_like(w, dtype=self.dt) for w in (b.mlp.w1.weight, b.mlp.w3.weight,
                                                                          b.mlp.w2.weight))
                      for b in model.blocks]
        self.graph = None
        self.timer = None   # optional per-layer attention timing (time_cells)
        self.refresh()

    @torch.no_grad()
    def refresh(self):
        """Re-read every parameter: pack each layer's attention weights (with its attn_norm), cast
        the MLP and embedding / head weights to the compute dtype. Outside any capture; a captured
        graph keeps working (the copies are rewritten in place)."""
        for cell, blk in zip(self.cells, self.m.blocks):
            cell.pack(dict(blk.attn.named_parameters()), attn_norm_w=blk.attn_norm.weight)
        for blk, ws in zip(self.m.blocks, self.w_mlp):
            for src, dst in zip((blk.mlp.w1.weight, blk.mlp.w3.weight, blk.mlp.w2.weight), ws):
                dst.copy_(src)
        self.w_emb.copy_(self.m.tok_emb.weight)

    # ---- the step ------------------------------------------------------------------------
    def _attn_fwd(self, l):
        self.cells[l].layer_forward(self.xs[l], self.ys[l], self.cos, self.sin, self.schedule, self.K[l], self.V[l],
                                    self.ocat[l], self.bufs[l], tape=self.tapes[l])

    def _attn_bwd(self, l):
        self.cells[l].layer_backward(self.xs[l], self.dy, self.dxs[l], self.cos, self.sin, self.schedule, self.K[l],
                                     self.V[l], self.ocat[l], self.bufs[l], self.lgrads[l], tape=self.tapes[l])

    def _mlp_fwd(self, l):
        blk, (w1, w3, w2) = self.m.blocks[l], self.w_mlp[l]
        M, d = self.B * self.T, self.cfg.d_model
        y = self.ys[l].view(M, d)
        hm, r = _rms(y, blk.mlp_norm.weight, blk.mlp_norm.eps)
        self.hm[l].copy_(hm)
        self.rm[l].copy_(r)
        torch.mm(hm, w1.t(), out=self.ga[l])
        torch.mm(hm, w3.t(), out=self.ub[l])
        mid = F.silu(self.ga[l]) * self.ub[l]
        torch.addmm(y, mid, w2.t(), out=self.xs[l + 1].view(M, d))

    def _mlp_bwd(self, l):
        """dz = dxs[l + 1] -> dy (the grad of ys[l]); MLP and mlp_norm weight grads into the buffer."""
        blk, (w1, w3, w2) = self.m.blocks[l], self.w_mlp[l]
        M, d = self.B * self.T, self.cfg.d_model
        pre = f"blocks.{l}."
        dz = self.dxs[l + 1].view(M, d)
        a, b, hm = self.ga[l], self.ub[l], self.hm[l]
        af = a.float()
        sg = torch.sigmoid(af)
        silu = af * sg
        mid = (silu * b.float()).to(self.dt)
        self.grad[pre + "mlp.w2.weight"].add_(_mm32(dz.t(), mid))
        dm = (dz @ w2).float()
        da = (dm * b.float() * sg * (1.0 + af * (1.0 - sg))).to(self.dt)
        db = (dm * silu).to(self.dt)
        self.grad[pre + "mlp.w1.weight"].add_(_mm32(da.t(), hm))
        self.grad[pre + "mlp.w3.weight"].add_(_mm32(db.t(), hm))
        dhm = da @ w1 + db @ w3
        dyv = _rms_vjp(dhm, self.ys[l].view(M, d), self.rm[l], blk.mlp_norm.weight, self.grad[pre + "mlp_norm.weight"])
        self.dy.view(M, d).copy_(dyv + dz.float())

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
        """Record one step as a HIP graph (after an eager warm-up step on the capture stream)."""
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
