"""torch.autograd glue: the DM layer forward / reverse-scan backward as one Function.

The forward runs dm_layer_fwd (projections, chunk cells, W_O) and keeps what
the backward needs (x, the projection buffers, the final K/V rows, o_cat and,
by default, the tape of every cell's sweep states); the backward runs
dm_layer_bwd, which reads the tape (or, with save_tape=False, recomputes every
cell exactly — the same values at a fraction of the memory) and returns dx
plus the gradients of the reference parameters
(engines/wavescan/engine/graphs.py:580-688 does the same per layer, with the
forward state kept in LayerBufs and caches).
"""

import torch

from .engine import LayerGrads
from .lowrank import factor_grads, is_factored


class DMLayerFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, cos, sin, cell, schedule, normalize, residual, save_tape, names, *params):
        B, T, d = x.shape
        cfg = cell.cfg
        x = x.contiguous()
        bufs = cell.new_bufs(T)
        K = torch.empty(B, cfg.n_heads, T, cfg.head_dim, device=x.device, dtype=x.dtype)
        V = torch.empty_like(K)
        ocat = torch.empty_like(x)
        y = torch.empty_like(x)
        tape = cell.new_tape(schedule) if save_tape else None
        cell.layer_forward(x, y, cos, sin, schedule, K, V, ocat, bufs, normalize=normalize,
                           residual=residual, tape=tape)
        ctx.cell, ctx.schedule, ctx.normalize, ctx.residual = cell, schedule, normalize, residual
        ctx.names = names
        ctx.params = dict(zip(names, params)) if is_factored(dict.fromkeys(names)) else None
        ctx.state = (x, cos, sin, bufs, K, V, ocat, tape)
        ctx.param_dtypes = [p.dtype for p in params]
        return y

    @staticmethod
    def backward(ctx, dy):
        x, cos, sin, bufs, K, V, ocat, tape = ctx.state
        cell = ctx.cell
        grads = LayerGrads(cell.cfg, x.device)
        dx = torch.empty_like(x)
        cell.layer_backward(x, dy.to(x.dtype).contiguous(), dx, cos, sin, ctx.schedule, K, V, ocat,
                            bufs, grads, normalize=ctx.normalize, residual=ctx.residual, tape=tape)
        g = grads.t if ctx.params is None else factor_grads(ctx.params, grads.t, ctx.names)
        pgrads = [g[n].to(dt) for n, dt in zip(ctx.names, ctx.param_dtypes)]
        ctx.state = ctx.params = None
        return (dx, None, None, None, None, None, None, None, None, *pgrads)


def dm_layer(x, cell, params, cos, sin, schedule, normalize=True, residual=True, save_tape=True):
    """Differentiable DM attention layer through the HIP path.

    params: {reference name: tensor} — the tensors ``cell`` was packed from; their
    gradients come back through autograd (factored gates / ctx operators, gate_rank /
    ctx_rank > 0, get the dense gradients chained onto their factors). normalize/residual select the Block
    sublayer y = x + W_O DM(attn_norm(x)) (default) or DualModAttention.forward's
    W_O DM(xhat). save_tape keeps every cell's sweep states from the forward
    (``cell.tape_bytes(schedule)`` of device memory) so the backward does not
    recompute them; False trades that memory for an exact recompute."""
    names = [n for n in params if normalize or n != "attn_norm.weight"]
    return DMLayerFn.apply(x, cos, sin, cell, schedule, normalize, residual, save_tape, names,
                           *[params[n] for n in names])
