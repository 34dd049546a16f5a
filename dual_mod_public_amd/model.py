"""The LLaMA-style DM trunk around the HIP attention path: SwiGLU, Block and DualModLM with
the reference's parameter names (models/dualmod/model.py:102-134, 267-294), so a reference
state dict loads unchanged.

Numerics follow the reference's bf16 runs (autocast): parameters are fp32 masters, the
residual stream and the RMSNorm statistics are fp32, and every matrix product runs in the
compute dtype ``dtype`` (bf16 by default) with fp32 accumulation — the attention sublayer
through libdm_hip.so (DualModAttention), the MLP, embedding-tied head through torch's GEMMs
(plain library products outside the DM hot path).
"""

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib as L
from .attention import DualModAttention, RMSNorm
from .config import DualModConfig
from .rope import build_rope_cache


def _lin(x, w):
    """nn.Linear without bias in x's dtype (the autocast cast of an fp32 weight)."""
    return F.linear(x, w.to(x.dtype))


class SwiGLU(nn.Module):
    """model.py:102-112: w2(silu(w1 x) * w3 x)."""

    def __init__(self, cfg: DualModConfig):
        super().__init__()
        d, hidden = cfg.d_model, cfg.mlp_hidden
        self.w1 = nn.Linear(d, hidden, bias=False)
        self.w3 = nn.Linear(d, hidden, bias=False)
        self.w2 = nn.Linear(hidden, d, bias=False)

    def forward(self, x):
        return _lin(F.silu(_lin(x, self.w1.weight)) * _lin(x, self.w3.weight), self.w2.weight)

    def decode(self, h, w=None, act=None, out=None):
        """The MLP on a decode step's rows h [B, 1, d] (compute dtype, contiguous): dm_swiglu_rows
        where it applies (bf16, B <= 64), else the forward's torch products. w = (w1, w3, w2) in
        h's dtype (default: cast from the parameters); act / out optional static buffers."""
        if w is None:
            # the compute-dtype copies, re-cast only when a parameter changed (its storage or version)
            ps = (self.w1.weight, self.w3.weight, self.w2.weight)
            key = (h.dtype,) + tuple((p.data_ptr(), p._version) for p in ps)
            cached = getattr(self, "_decode_w", None)
            if cached is None or cached[0] != key:
                cached = (key, tuple(p.detach().to(h.dtype).contiguous() for p in ps))
                self._decode_w = cached
            w = cached[1]
        if L.swiglu_rows_ok(h, w[0], w[2]):
            return L.swiglu_rows(h, w[0], w[1], w[2], act=act, out=out)
        return F.linear(F.silu(F.linear(h, w[0])) * F.linear(h, w[1]), w[2]).contiguous()


class Block(nn.Module):
    """model.py:115-131: x + attn(attn_norm x), then x + mlp(mlp_norm x)."""

    def __init__(self, cfg: DualModConfig):
        super().__init__()
        self.attn_norm = RMSNorm(cfg.d_model)
        self.attn = DualModAttention(cfg)
        self.mlp_norm = RMSNorm(cfg.d_model)
        self.mlp = SwiGLU(cfg)

    def forward(self, x, cos, sin, dtype=torch.bfloat16):
        x = x + self.attn(self.attn_norm(x).to(dtype), cos, sin)
        return x + self.mlp(self.mlp_norm(x).to(dtype))

    @torch.no_grad()
    def decode_step(self, x_j, pos, cache, cos, sin, dtype=torch.bfloat16):
        """x_j [B, 1, d] (fp32 residual stream) -> the block's output (a new fp32 tensor). The
        residual adds and the two RMSNorms run as dm_residual_rmsnorm passes."""
        x = x_j.float().contiguous().clone()
        h = L.residual_rmsnorm(x, None, self.attn_norm.weight, dtype, eps=self.attn_norm.eps)
        y = self.attn.decode_step(h, pos, cache, cos, sin)
        h = L.residual_rmsnorm(x, y, self.mlp_norm.weight, dtype, eps=self.mlp_norm.eps)
        L.residual_rmsnorm(x, self.mlp.decode(h), None, dtype)
        return x


class DualModLM(nn.Module):
    """model.py:134-294 (forward, decode_init / decode_step / generate). ``dtype`` is the
    compute dtype of the products (bf16 or fp32)."""

    def __init__(self, cfg: DualModConfig, dtype=torch.bfloat16):
        super().__init__()
        self.cfg, self.dtype = cfg, dtype
        self.tok_emb = nn.Embedding(cfg.vocab_size, cfg.d_model)
        self.blocks = nn.ModuleList(Block(cfg) for _ in range(cfg.n_layers))
        self.norm_f = RMSNorm(cfg.d_model)
        self.lm_head = nn.Linear(cfg.d_model, cfg.vocab_size, bias=False)
        if cfg.tie_embeddings:
            self.lm_head.weight = self.tok_emb.weight
        cos, sin = build_rope_cache(cfg.max_seq_len, cfg.head_dim, cfg.rope_theta, use_rope=cfg.use_rope)
        self.register_buffer("rope_cos", cos, persistent=False)
        self.register_buffer("rope_sin", sin, persistent=False)

    def head(self, x):
        """Final norm + head: logits in the compute dtype."""
        return _lin(self.norm_f(x).to(self.dtype), self.lm_head.weight)

    # ---- teacher-forced forward (model.py:267-281) ---------------------------------
    def forward(self, idx, targets=None):
        x = self.tok_emb(idx)
        T = x.shape[1]
        assert T <= self.cfg.max_seq_len
        cos, sin = self.rope_cos[:T], self.rope_sin[:T]
        for blk in self.blocks:
            x = blk(x, cos, sin, self.dtype)
        logits = self.head(x)
        loss = None
        if targets is not None:
            loss = F.cross_entropy(logits.float().view(-1, logits.shape[-1]), targets.reshape(-1), ignore_index=-1)
        return logits, loss

    # ---- incremental decode (model.py:285-313) --------------------------------------
    def decode_init(self):
        return [{"K": None, "V": None} for _ in self.blocks]

    @torch.no_grad()
    def decode_step(self, idx_j, pos, caches):
        """idx_j [B, 1] token ids at absolute position pos; returns logits [B, 1, V]."""
        x = self.tok_emb(idx_j)
        for blk, cache in zip(self.blocks, caches):
            x = blk.decode_step(x, pos, cache, self.rope_cos, self.rope_sin, self.dtype)
        h = L.residual_rmsnorm(x, None, self.norm_f.weight, self.dtype, eps=self.norm_f.eps)
        return _lin(h, self.lm_head.weight)

    @torch.no_grad()
    def generate(self, idx, max_new_tokens, temperature=1.0, top_k=None):
        caches = self.decode_init()
        logits = None
        for t in range(idx.shape[1]):
            logits = self.decode_step(idx[:, t:t + 1], t, caches)
        out = idx
        for _ in range(max_new_tokens):
            pos = out.shape[1] - 1
            if pos + 1 >= self.cfg.max_seq_len:
                break
            lg = logits[:, -1, :].float() / max(temperature, 1e-6)
            if top_k is not None:
                kth = torch.topk(lg, top_k, dim=-1).values[:, -1:]
                lg = lg.masked_fill(lg < kth, float("-inf"))
            nxt = torch.multinomial(torch.softmax(lg, dim=-1), 1)
            out = torch.cat([out, nxt], dim=1)
            logits = self.decode_step(nxt, pos + 1, caches)
        return out
