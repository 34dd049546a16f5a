"""GPU test of the reference-shaped engine adapter (fused_sweep.FusedSweepCell): a training step
driven exactly as the reference's WaveScanEngine drives its FusedSweepCell — the embedding, per
layer ``layer_proj`` then per cell ``cell_forward`` followed by ``x + wo(o) + mlp(mlp_norm(.))`` on
the chunk (engines/wavescan/engine/graphs.py:241-265), the head and loss under autograd
(graphs.py:314-341), then per layer from the top ``layer_proj(zero_grads=True)``,
``layer_blockmlp_bwd``, ``cell_backward`` for the cells last first with the fp32 grad caches dK / dV,
``layer_close`` (graphs.py:373-389, 466-500), and the embedding backward (graphs.py:502-508) — checked
against autograd through the oracle's fp64 LM: the loss and every parameter gradient within 1e-5
(fp32), K < c and K = c."""

import pytest
import torch
import torch.nn.functional as F

import oracle as O
from dual_mod_public_amd import _lib as L
from dual_mod_public_amd.config import DualModConfig
from dual_mod_public_amd.engine import uniform_chunks
from dual_mod_public_amd.fused_sweep import FusedSweepCell, GradBuffers, LayerBufs
from dual_mod_public_amd.model import DualModLM
from dual_mod_public_amd.synthetic import make_lm_state_dict
from tests.hip_helpers import DEV, record, relerr, say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    L.load()
    torch.backends.cuda.matmul.allow_tf32 = False


def _engine_step(m, fs, idx, tg, sched):
    """The reference engine's layer-major fused forward + backward (graphs.py), on the adapter."""
    cfg = m.cfg
    B, T = idx.shape
    d, h, dh, nl = cfg.d_model, cfg.n_heads, cfg.head_dim, cfg.n_layers
    f32 = dict(device=DEV, dtype=torch.float32)
    xl = [torch.zeros(B, T, d, **f32) for _ in range(nl + 1)]
    K = [torch.zeros(B, h, T, dh, **f32) for _ in range(nl)]
    V = [torch.zeros(B, h, T, dh, **f32) for _ in range(nl)]
    ocat = [torch.zeros(B, T, d, **f32) for _ in range(nl)]
    dK = [torch.zeros(B, h, T, dh, **f32) for _ in range(nl)]
    dV = [torch.zeros(B, h, T, dh, **f32) for _ in range(nl)]
    dx = [torch.zeros(B, T, d, **f32) for _ in range(nl + 1)]
    P = LayerBufs(B, h, T, dh, d, torch.float32, DEV, ctx_mod=cfg.ctx_mod)
    grads = GradBuffers(list(m.parameters()))
    fs.pack()
    with torch.no_grad():
        xl[0].copy_(m.tok_emb(idx))                                            # _embed_body
        for li, blk in enumerate(m.blocks):
            fs.layer_proj(li, xl[li], P)                                       # _proj_body
            for pos0, c, k in sched:                                           # _cell_fwd_body
                cos, sin = m.rope_cos[pos0:pos0 + c], m.rope_sin[pos0:pos0 + c]
                u_buf = torch.zeros(B, c, d, **f32)
                o_buf = torch.zeros(B, c, d, **f32)
                x_c = xl[li][:, pos0:pos0 + c]
                o = fs.cell_forward(li, P, cos, sin, K[li], V[li], pos0, k, u_buf, o_buf,
                                    ocat_out=ocat[li][:, pos0:pos0 + c], x_c=x_c)
                x_mid = x_c + blk.attn.wo(o.to(x_c.dtype))
                xl[li + 1][:, pos0:pos0 + c] = x_mid + blk.mlp(blk.mlp_norm(x_mid))
    # _loss_body + _head_bwd_body: the head and the loss under autograd
    head = [m.norm_f.weight, m.lm_head.weight]
    x_fin = xl[nl].detach().requires_grad_(True)
    logits = m.lm_head(m.norm_f(x_fin))
    loss = F.cross_entropy(logits.float().reshape(-1, cfg.vocab_size), tg.reshape(-1), ignore_index=-1)
    gs = torch.autograd.grad([loss], [x_fin] + head)
    dx[nl].copy_(gs[0])
    for p, g in zip(head, gs[1:]):
        grads.add(p, g)
    with torch.no_grad():
        for li in reversed(range(nl)):
            fs.layer_proj(li, xl[li], P, zero_grads=True)                      # _proj_body(li, True)
            fs.layer_blockmlp_bwd(li, xl[li], ocat[li], dx[li + 1], dx[li], P, grads)
            for pos0, c, k in reversed(sched):                                 # _cell_bwd_body
                cos, sin = m.rope_cos[pos0:pos0 + c], m.rope_sin[pos0:pos0 + c]
                fs.cell_backward(li, P, xl[li][:, pos0:pos0 + c], cos, sin, K[li], V[li], pos0, k,
                                 dK[li][:, :, pos0:pos0 + c], dV[li][:, :, pos0:pos0 + c], grads, dK[li], dV[li],
                                 None, None, None)
            fs.layer_close(li, xl[li], P, dx[li], grads)                       # _close_body
    emb = m.tok_emb.weight                                                     # _emb_bwd_body
    leaf = emb.detach().requires_grad_(True)
    out = F.embedding(idx, leaf)
    (g,) = torch.autograd.grad([out], [leaf], [dx[0]])
    grads.add(emb, g)
    return loss.detach(), grads


@pytest.mark.parametrize("c,k", [(16, 4), (16, 16)])
def test_engine_loop_on_the_adapter_matches_oracle(c, k):
    say(f"reference engine loop on FusedSweepCell, fp32, c={c} K={k}")
    cfg = DualModConfig(d_model=256, n_heads=4, n_layers=2, vocab_size=512, max_seq_len=64,
                        mlp_hidden_override=512, checkpoint_chunk=0, dtype="fp32", ctx_mod="mult_res")
    sd = make_lm_state_dict(cfg, seed=7, std=0.02)
    m = DualModLM(cfg, dtype=torch.float32).to(DEV)
    m.load_state_dict({kk: v.to(DEV) for kk, v in sd.items()})
    B, T = 2, 64
    gen = torch.Generator().manual_seed(3)
    idx = torch.randint(0, cfg.vocab_size, (B, T), generator=gen)
    tg = torch.randint(0, cfg.vocab_size, (B, T), generator=gen)
    sched = uniform_chunks(T, c, k)
    fs = FusedSweepCell(m)
    loss, grads = _engine_step(m, fs, idx.to(DEV), tg.to(DEV), sched)
    torch.cuda.synchronize()
    leaves = {kk: v.double().clone().requires_grad_(True) for kk, v in sd.items() if kk != "lm_head.weight"}
    full = dict(leaves)
    full["lm_head.weight"] = leaves["tok_emb.weight"]
    c64, s64 = O.build_rope_cache(T, cfg.head_dim, cfg.rope_theta, dtype=torch.float64)
    ref = F.cross_entropy(O.lm_forward(cfg, full, idx, c64, s64, schedule=sched).view(-1, cfg.vocab_size),
                          tg.reshape(-1), ignore_index=-1)
    ref.backward()
    errs = {"loss": relerr(loss, ref.detach())}
    params = dict(m.named_parameters())
    for kk, v in leaves.items():
        errs[kk] = relerr(grads.buf[id(params[kk])], v.grad)
    worst = max(errs, key=errs.get)
    say(f"  worst {worst} {errs[worst]:.2e}")
    record(f"engine loop on FusedSweepCell c={c} K={k}", errs, 1e-5)
    for kk, v in errs.items():
        assert v < 1e-5, f"{kk}: relerr {v:.3e}"
