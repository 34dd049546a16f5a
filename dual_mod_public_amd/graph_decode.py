"""Greedy decode of a DualModLM as one captured HIP graph per token
(lm/eval/graph_decode.py:15-125, GraphDecoder).

Same math as DualModLM.decode_step (the exact sequential scan, one position per step):
every layer's attention runs dm_decode_step on a static per-layer tape with the position
held in device memory (dm_decode_args.pos_dev), so the launches of a whole step — the
embedding gather, every layer's attention and MLP, the residual adds with their RMSNorms
(dm_residual_rmsnorm), the head, the argmax (dm_argmax_rows) and the position increment —
are recorded once and replayed per token.

The graph reads compute-dtype copies of the MLP / head weights and the attention's packed
buffers, all at fixed addresses. Every ``step()`` first compares the parameters' version
stamps (storage address and in-place version counter) with those of the last copy and
re-reads the weights when one changed (as the reference re-casts the live weights on every
replay), so an optimizer step between tokens is picked up.
"""

import torch
import torch.nn.functional as F

from . import _lib as L
from .decode import StaticTape


class GraphDecoder:
    def __init__(self, model, B, P_max, dtype=None):
        self.m = model
        cfg = model.cfg
        self.dev = next(model.parameters()).device
        if P_max > cfg.max_seq_len:
            raise ValueError(f"P_max={P_max} > max_seq_len={cfg.max_seq_len}")
        self.B, self.P = B, P_max
        self.dt = dtype or model.dtype
        self.d, self.vocab = cfg.d_model, cfg.vocab_size
        self.tapes = [StaticTape(blk.attn, B, P_max, self.dev, self.dt) for blk in model.blocks]
        self.K = [t.K for t in self.tapes]     # per-layer tapes [B, h, P_max, dh] (graph_decode.py:23-24)
        self.V = [t.V for t in self.tapes]
        self.tok = torch.zeros(B, 1, dtype=torch.long, device=self.dev)        # input token (per step)
        self.pos = torch.zeros(1, dtype=torch.int32, device=self.dev)          # absolute position
        self.logits = torch.zeros(B, 1, self.vocab, device=self.dev)          # fp32 out
        self.next = torch.zeros(B, 1, dtype=torch.long, device=self.dev)       # argmax out
        self.cos = model.rope_cos.to(self.dev, torch.float32).contiguous()
        self.sin = model.rope_sin.to(self.dev, torch.float32).contiguous()
        # compute-dtype weight copies at fixed addresses (the autocast casts, done once per version)
        self._mlp = [tuple(torch.empty_like(w, dtype=self.dt) for w in
                           (blk.mlp.w1.weight, blk.mlp.w3.weight, blk.mlp.w2.weight)) for blk in model.blocks]
        self._head = torch.empty_like(model.lm_head.weight, dtype=self.dt)
        # the MLP's intermediate and output rows (dm_swiglu_rows), at fixed addresses
        self._act = torch.empty(B, cfg.mlp_hidden, device=self.dev, dtype=self.dt)
        self._mo = torch.empty(B, 1, cfg.d_model, device=self.dev, dtype=self.dt)
        self._params = list(model.parameters())
        self._ver = None
        self.graph = None
        self._steps = 0
        self.refresh()

    def refresh(self):
        """Re-read the model's parameters into the static copies the graph uses (a no-op while
        no parameter changed)."""
        ver = tuple((p.data_ptr(), p._version) for p in self._params)
        if ver == self._ver:
            return
        with torch.no_grad():
            for blk, ws in zip(self.m.blocks, self._mlp):
                for src, dst in zip((blk.mlp.w1.weight, blk.mlp.w3.weight, blk.mlp.w2.weight), ws):
                    dst.copy_(src)
            self._head.copy_(self.m.lm_head.weight)
        for t in self.tapes:
            t._refresh()
        self._ver = ver

    # ---- one decode step on the static tapes (graph_decode.py:53-64) ----------------
    def _step(self):
        m, B, d, dt = self.m, self.B, self.d, self.dt
        x = F.embedding(self.tok, m.tok_emb.weight)                    # [B, 1, d] fp32 residual
        blocks = list(m.blocks)
        h = L.residual_rmsnorm(x, None, blocks[0].attn_norm.weight, dt, eps=blocks[0].attn_norm.eps)
        for l, (blk, tape, (w1, w3, w2)) in enumerate(zip(blocks, self.tapes, self._mlp)):
            _, y = tape.step(h.view(B, d), self.pos, self.cos, self.sin, with_wo=True)
            h = L.residual_rmsnorm(x, y, blk.mlp_norm.weight, dt, eps=blk.mlp_norm.eps)
            mo = blk.mlp.decode(h, (w1, w3, w2), act=self._act, out=self._mo)
            # the MLP's residual add fused with the next norm (the next block's attn_norm, or norm_f)
            nrm = blocks[l + 1].attn_norm if l + 1 < len(blocks) else m.norm_f
            h = L.residual_rmsnorm(x, mo, nrm.weight, dt, eps=nrm.eps)
        lg = F.linear(h, self._head)                                    # [B, 1, V]
        self.logits.copy_(lg)                                           # exact bf16 -> fp32 in one copy
        L.check(L.lib().dm_argmax_rows(L.dtype_code(self.dt), L.ptr(lg), B, self.vocab, self.vocab,
                                       L.ptr(self.next), L.stream_ptr()))
        self.pos += 1

    def _run_step(self):
        with torch.no_grad():
            self._step()

    def capture(self):
        """Warm-up steps on a side stream, then record one step (graph_decode.py:72-85)."""
        self.refresh()
        s = torch.cuda.Stream(device=self.dev)
        s.wait_stream(torch.cuda.current_stream(self.dev))
        with torch.cuda.stream(s):
            for _ in range(3):
                self._run_step()
        torch.cuda.current_stream(self.dev).wait_stream(s)
        torch.cuda.synchronize(self.dev)
        self.reset()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            self._run_step()
        torch.cuda.synchronize(self.dev)
        self.reset()
        self.graph = g
        return self

    def reset(self):
        self.pos.zero_()
        self._steps = 0
        for t in self.tapes:
            t.K.zero_()
            t.V.zero_()

    def step(self):
        """One token: the graph replay (or the eager step), after re-reading the weights if a
        parameter changed since the last step. The position lives on the device; the host
        counts the steps since reset() and refuses a step past the tape (the kernels would
        clamp the position onto the last slot)."""
        if self._steps >= self.P:
            raise ValueError(f"the tape is full: {self.P} positions since reset()")
        self.refresh()
        if self.graph is not None:
            self.graph.replay()
        else:
            self._run_step()
        self._steps += 1

    # ---- greedy generation (graph_decode.py:91-125) -----------------------------------
    @torch.no_grad()
    def generate(self, prompt, max_new, eos_id=None, stop_fn=None, check_every=16):
        """prompt [B, Lp] long on the device (equal lengths). Returns (gen [B, k] long on the
        CPU, k): greedy continuations, stopped early once every row has hit eos_id / stop_fn."""
        B, Lp = prompt.shape
        if B != self.B or Lp + max_new > self.P:
            raise ValueError(f"prompt {tuple(prompt.shape)} + {max_new} new tokens does not fit B={self.B}, "
                             f"P_max={self.P}")
        self.refresh()
        self.reset()
        for p in range(Lp):
            self.tok.copy_(prompt[:, p:p + 1])
            self.step()
        gen = torch.zeros(B, max_new, dtype=torch.long, device=self.dev)
        done = torch.zeros(B, dtype=torch.bool)
        k = 0
        while k < max_new:
            gen[:, k].copy_(self.next[:, 0])
            k += 1
            if k % check_every == 0 or k == max_new:
                g_cpu = gen[:, :k].cpu()
                if eos_id is not None:
                    done |= (g_cpu == eos_id).any(1)
                if stop_fn is not None:
                    done |= stop_fn(g_cpu)
                if bool(done.all()):
                    break
            if k < max_new:
                self.tok.copy_(self.next)
                self.step()
        return gen[:, :k].cpu(), k
