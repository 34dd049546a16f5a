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

import ctypes

import torch

from . import _lib as L
from .engine import HipSweepCell, LayerGrads, _sched, uniform_chunks


class HipLayerStack:
    """wavefront=True runs the forward and the backward layer-batched (dm_stack_fwd /
    dm_stack_bwd, the schedule of engines/wave3d/wave3d.py:1-47 on the chained chunk cells):
    layer l works on cell t - l at step t (the backward: the top layer first, cells last
    first) and each kernel of a step is one launch over every active layer. Same results as
    the layer-by-layer step, bit for bit; it needs a schedule of equal cells."""

    def __init__(self, cfg, n_layers, B, T, schedule=None, device="cuda", dtype=torch.bfloat16, tape=True,
                 wavefront=False):
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
        self.wavefront = wavefront
        self._plan = None
        self._bplan = None

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

    def _stack_args(self):
        """The dm_stack_layer array (and the structs it points to, kept alive here)."""
        self._keep = []
        arr = (L.dm_stack_layer * self.L)()
        for l, cell in enumerate(self.cells):
            w, b = cell.w.struct(with_attn_norm=True), self.bufs[l].struct()
            self._keep += [w, b]
            a = arr[l]
            a.w, a.bufs = ctypes.addressof(w), ctypes.addressof(b)
            a.x, a.y = L.ptr(self.xs[l]), L.ptr(self.xs[l + 1])
            a.K_cache, a.V_cache, a.ocat = L.ptr(self.K[l]), L.ptr(self.V[l]), L.ptr(self.ocat[l])
            a.tape = L.ptr(self.tapes[l])
            a.tape_bytes = 0 if self.tapes[l] is None else self.tapes[l].numel()
            a.workspace, a.workspace_bytes = L.ptr(cell.workspace), cell.workspace.numel()
        return arr

    def forward_wavefront(self):
        """The layer-batched forward over the stack's buffers (xs[0] -> xs[L]). The first call
        writes the launch plan (a blocking copy); later calls launch from it (graph-capturable)."""
        conf = self.cells[0]._conf(True)
        sched = _sched(self.schedule)
        arr = self._stack_args()
        build = 0
        if self._plan is None:
            n = L.lib().dm_stack_fwd_plan_bytes(ctypes.byref(conf), self.L, arr, sched, len(self.schedule), self.T)
            if n == 0:
                raise L.DMError("dm_stack_fwd_plan_bytes rejected the stack (equal cells of a power-of-two length "
                                "are needed)")
            self._plan = torch.empty(n, device=self.device, dtype=torch.uint8)
            build = 1
        L.check(L.lib().dm_stack_fwd(ctypes.byref(conf), self.L, arr, L.ptr(self.cos), L.ptr(self.sin), sched,
                                     len(self.schedule), self.T, L.ptr(self._plan), self._plan.numel(), build,
                                     L.stream_ptr()))

    def backward_wavefront(self):
        """The layer-batched backward over the stack's buffers (dxs[L] -> dxs[0], the gradients
        ADDED into the flat buffer); plan handling as forward_wavefront."""
        conf = self.cells[0]._conf(True)
        sched = _sched(self.schedule)
        kmax = max(k for _, _, k in self.schedule)
        self._bkeep = []
        arr = (L.dm_stack_bwd_layer * self.L)()
        for l, cell in enumerate(self.cells):
            w, b, g = cell.w.struct(with_attn_norm=True), self.bufs[l].struct(), self.grads[l].struct()
            self._bkeep += [w, b, g]
            ws = cell._bwd_workspace(self.T, self.T, kmax)
            a = arr[l]
            a.w, a.bufs, a.grads = ctypes.addressof(w), ctypes.addressof(b), ctypes.addressof(g)
            a.x, a.dy, a.dx = L.ptr(self.xs[l]), L.ptr(self.dxs[l + 1]), L.ptr(self.dxs[l])
            a.K_cache, a.V_cache, a.ocat = L.ptr(self.K[l]), L.ptr(self.V[l]), L.ptr(self.ocat[l])
            a.tape = L.ptr(self.tapes[l])
            a.tape_bytes = 0 if self.tapes[l] is None else self.tapes[l].numel()
            a.workspace, a.workspace_bytes = L.ptr(ws), ws.numel()
        build = 0
        if self._bplan is None:
            n = L.lib().dm_stack_bwd_plan_bytes(ctypes.byref(conf), self.L, arr, sched, len(self.schedule), self.T)
            if n == 0:
                raise L.DMError("dm_stack_bwd_plan_bytes rejected the stack")
            self._bplan = torch.empty(n, device=self.device, dtype=torch.uint8)
            build = 1
        L.check(L.lib().dm_stack_bwd(ctypes.byref(conf), self.L, arr, L.ptr(self.cos), L.ptr(self.sin), sched,
                                     len(self.schedule), self.T, L.ptr(self._bplan), self._bplan.numel(), build,
                                     L.stream_ptr()))

    def _run(self):
        self.flat.zero_()
        if self.wavefront:
            self.forward_wavefront()
            self.backward_wavefront()
            return
        for l, cell in enumerate(self.cells):
            cell.layer_forward(self.xs[l], self.xs[l + 1], self.cos, self.sin, self.schedule, self.K[l],
                               self.V[l], self.ocat[l], self.bufs[l], tape=self.tapes[l])
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
