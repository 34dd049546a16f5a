"""GPU parity of the per-cell backward (dm_layer_bwd_begin / dm_cell_bwd / dm_layer_bwd_end,
HipSweepCell.cell_backward): the reference engine's protocol (FusedSweepCell.cell_backward,
engines/wavescan/cells/fused_sweep.py:1557; the fp32 grad cache of
engines/wavescan/engine/backward.py:92-123) driven cell by cell, last cell first. Against
dm_layer_bwd (same values up to fp32 summation order: the committed-prefix grads are summed
through the running cache instead of per key cell) and against autograd through the oracle
(the fp32 / bf16 gradient bars of tests/test_gpu_backward.py)."""

import pytest
import torch

from dual_mod_public_amd import _lib as L
from dual_mod_public_amd.engine import HipSweepCell, LayerGrads, layer_backward_cells, uniform_chunks
from tests.hip_helpers import DEV, cfg_of, record, relerr, say, setup
from tests.test_gpu_backward import BF16_TOL, FP32_TOL, compare, hip_grads, oracle_grads

pytestmark = pytest.mark.gpu

SCHEDS = {"uniform": None, "ragged": [(0, 16, 3), (16, 16, 1), (32, 7, 2), (39, 25, 4)],
          "exact": [(0, 16, 16), (16, 16, 16), (32, 16, 16), (48, 16, 16)]}


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    L.load()


def cell_grads(cfg, sd, x, dy, cos, sin, sched, dtype, tape=False):
    B, T, d = x.shape
    cell = HipSweepCell(cfg, B, T, device=DEV, dtype=dtype)
    cell.pack({k: v.to(DEV, dtype) for k, v in sd.items()})
    bufs = cell.new_bufs(T)
    xd = x.to(DEV, dtype).contiguous()
    y = torch.empty_like(xd)
    K = torch.empty(B, cfg.n_heads, T, cfg.head_dim, device=DEV, dtype=dtype)
    V = torch.empty_like(K)
    ocat = torch.empty_like(xd)
    tp = cell.new_tape(sched) if tape else None
    cell.layer_forward(xd, y, cos, sin, sched, K, V, ocat, bufs, tape=tp)
    grads = LayerGrads(cfg, DEV)
    dx = torch.empty_like(xd)
    _, dKc, dVc = layer_backward_cells(cell, xd, dy.to(DEV, dtype).contiguous(), dx, cos, sin, sched, K, V, ocat,
                                       bufs, grads, tape=tp)
    torch.cuda.synchronize()
    return dx, grads, dKc


@pytest.mark.parametrize("ctx_mod", ["mult_res", "linear", "fusion"])
@pytest.mark.parametrize("sname", list(SCHEDS))
@pytest.mark.parametrize("tape", [False, True])
def test_cell_backward_fp32(ctx_mod, sname, tape):
    say(f"cell_backward fp32 {ctx_mod} {sname} tape={tape}")
    cfg = cfg_of(ctx_mod=ctx_mod)
    B, T = 2, 64
    sd, x, (c64, s64), (c32, s32) = setup(cfg, B, T)
    dy = torch.randn(B, T, cfg.d_model, generator=torch.Generator().manual_seed(23), dtype=torch.float64)
    sched = SCHEDS[sname] or uniform_chunks(T, 16, 4)
    dx, g, dKc = cell_grads(cfg, sd, x, dy, c32, s32, sched, torch.float32, tape=tape)
    # against the layer path (same kernels, committed grads summed the other way)
    _, dx_l, g_l = hip_grads(cfg, sd, x, dy, c32, s32, sched, torch.float32, tape=tape)
    errs = {"x": relerr(dx, dx_l)}
    errs.update({k: relerr(g[k], v) for k, v in g_l.t.items()})
    record(f"cell_backward vs layer fp32 {ctx_mod} {sname}", errs, 1e-5)
    assert max(errs.values()) < 1e-5, errs
    # the committed rows of the first cells received grads from the later rows
    assert dKc[:, :, :sched[-1][0]].abs().sum() > 0
    dx_ref, g_ref = oracle_grads(cfg, sd, x, dy, c64, s64, sched)
    compare(f"cell_backward fp32 {ctx_mod}", dx, g, dx_ref, g_ref, FP32_TOL)


def test_cell_backward_bf16_340m_shape():
    """bf16 storage at the 340M layer shape (d=1024, 16x64), c=64, K=4, T=256, tape."""
    say("cell_backward bf16 d=1024 T=256")
    cfg = cfg_of(d=1024, h=16, T=256)
    B, T = 2, 256
    sd, x, _, (c32, s32) = setup(cfg, B, T)
    dy = torch.randn(B, T, cfg.d_model, generator=torch.Generator().manual_seed(29), dtype=torch.float64)
    sched = uniform_chunks(T, 64, 4)
    dx, g, _ = cell_grads(cfg, sd, x, dy, c32, s32, sched, torch.bfloat16, tape=True)
    dx_ref, g_ref = oracle_grads(cfg, {k: v.float() for k, v in sd.items()}, x.float(), dy.float(), c32, s32, sched,
                                 dtype=torch.float32)
    compare("cell_backward bf16 340m", dx, g, dx_ref, g_ref, BF16_TOL)


def test_cell_backward_rejects_bad_cell():
    cfg = cfg_of()
    B, T = 2, 32
    sd, x, _, (c32, s32) = setup(cfg, B, T)
    cell = HipSweepCell(cfg, B, T, device=DEV, dtype=torch.float32)
    cell.pack({k: v.to(DEV, torch.float32) for k, v in sd.items()})
    bufs = cell.new_bufs(T)
    sched = uniform_chunks(T, 16, 2)
    K = torch.zeros(B, cfg.n_heads, T, cfg.head_dim, device=DEV)
    dy = torch.zeros(B, T, cfg.d_model, device=DEV)
    grads = LayerGrads(cfg, DEV)
    cell.layer_backward_begin(dy, dy, bufs, sched, K, grads)
    with pytest.raises(L.DMError, match="cell 5 of 2"):
        cell.cell_backward(bufs, c32, s32, K, K.clone(), 5, K.float(), K.float())
