"""A stack of DM attention sublayers trained on one GPU: the single-GPU part of the
reference's WaveScanEngine (engines/wavescan/engine/graphs.py:36-792).

Each layer is the Block's attention sublayer y = x + W_O DM(attn_norm(x))
(models/dualmod/model.py:123-124) run through its own HipSweepCell: the forward
keeps every cell's sweep states in a per-layer HBM tape, the backward reads them
(engines/wavescan/engine/backward.py:92-123 semantics). Parameter gradients of every
layer are views into ONE flat fp32 buffer (GradBuffers, backward.py:27-61), so a
multi-GPU job would reduce them with a single collective (graphs.py:768-792; this
build runs on one GPU and has no such step). The whole forward + backward step
(gradient zeroing included) can be captured once as a HIP graph and replayed
(graphs.py:513-576 captures per layer; here the step is one graph): every buffer
the step touches is allocated up front at a fixed address, and nothing in it
records a memset (the zeroing is a fill kernel). Weights live in the cells' packed
buffers, repacked in place by ``load`` (outside the graph) after an optimizer step.
"""

import torch

from .engine import HipSweepCell, LayerGrads, uniform_chunks


class HipLayerStack:
    def __init__(self, cfg, n_layers, B, T, schedule=None, device="cuda", dtype=torch.bfloat16, tape=True):
        self.cfg, self.L, self.B, self.T = cfg, n_layers, B, T
        self.device, self.dtype = torch.device(device), dtype
        d, h, dh = cfg.d_model, cfg.n_heads, cfg.head_dim
        self.schedule = list(schedule) if schedule is not None else uniform_chunks(T, 64, 4)
        kw = dict(device=self.device, dtype=dtype)
        self.cells = [HipSweepCell(cfg, B, T, device=self.device, dtype=dtype) for _ in range(n_layers)]
        # activations: xs[l] is layer l's input, xs[L] the stack's output; dxs likewise for grads
        self.xs = [torch.zeros(B, T, d, **kw) for _ in range(n_layers + 1)]
        self.dxs = [torch.zeros(B, T, d, **kw) for _ in range(n_layers + 1)]
        self.bufs = [c.new_bufs(T) for c in self.cells]
        self.K = [torch.zeros(B, h, T, dh, **kw) for _ in range(n_layers)]
        self.V = [torch.zeros(B, h, T, dh, **kw) for _ in range(n_layers)]
        self.ocat = [torch.zeros(B, T, d, **kw) for _ in range(n_layers)]
        self.tapes = [c.new_tape(self.schedule) for c in self.cells] if tape else [None] * n_layers
        # one flat fp32 gradient buffer, each layer's LayerGrads a set of views into it
        self.grads = [LayerGrads(cfg, self.device) for _ in range(n_layers)]
        names = list(self.grads[0].t)
        sizes = [self.grads[0].t[n].numel() for n in names]
        self.flat = torch.zeros(n_layers * sum(sizes), device=self.device, dtype=torch.float32)
        off = 0
        for g in self.grads:
            for n, sz in zip(names, sizes):
                g.t[n] = self.flat[off:off + sz].view_as(g.t[n])
                off += sz
        self.cos = self.sin = None
        self.graph = None

    def load(self, state_dicts, cos, sin):
        """Pack every layer's weights (reference names, incl. attn_norm.weight) and the RoPE
        tables (rows 0..T-1). Call again after an optimizer step; a captured graph keeps
        working, since the packed buffers are rewritten in place."""
        for cell, sd in zip(self.cells, state_dicts):
            cell.pack(sd)
        if self.cos is None:
            self.cos = cos[:self.T].to(self.device, torch.float32).contiguous()
            self.sin = sin[:self.T].to(self.device, torch.float32).contiguous()
        else:
            self.cos.copy_(cos[:self.T])
            self.sin.copy_(sin[:self.T])
        return self

    def _run(self):
        self.flat.zero_()
        for l, cell in enumerate(self.cells):
            cell.layer_forward(self.xs[l], self.xs[l + 1], self.cos, self.sin, self.schedule, self.K[l], self.V[l],
                               self.ocat[l], self.bufs[l], tape=self.tapes[l])
        for l in reversed(range(self.L)):
            self.cells[l].layer_backward(self.xs[l], self.dxs[l + 1], self.dxs[l], self.cos, self.sin, self.schedule,
                                         self.K[l], self.V[l], self.ocat[l], self.bufs[l], self.grads[l],
                                         tape=self.tapes[l])

    def capture(self):
        """Record one forward + backward step as a HIP graph (after one eager warm-up step on the
        capture stream, which also sizes every workspace)."""
        s = torch.cuda.Stream(device=self.device)
        s.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(s):
            self._run()
        torch.cuda.current_stream(self.device).wait_stream(s)
        torch.cuda.synchronize(self.device)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=s):
            self._run()
        torch.cuda.synchronize(self.device)
        return self

    def step(self, x, dy):
        """One forward + backward step: x [B,T,d] the stack's input, dy the gradient of its output.
        Returns (y, dx, per-layer LayerGrads); y and dx are the stack's own buffers (overwritten by
        the next step), the gradients are views of the flat buffer ``self.flat``."""
        self.xs[0].copy_(x)
        self.dxs[self.L].copy_(dy)
        if self.graph is not None:
            self.graph.replay()
        else:
            self._run()
        return self.xs[self.L], self.dxs[0], self.grads
