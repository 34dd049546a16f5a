"""GPU tests of the local window on the chunk cells (config local_window, attention.py:291-293:
a token reads the last W - 1 rows before it and itself).

The cells window their committed prefix and, for windows no longer than the cell, their intra
rows (row p reads cell rows p - W + 1 .. p - 1): with K = c sweeps the windowed layer equals the
windowed sequential scan of the oracle (attend_one's window, pinned by brute force), with K < c
it equals the oracle's windowed Jacobi cells (whose masks are pinned to the windowed scan at
K = c in tests/test_oracle_invariants.py). The backward against autograd through the oracle, the
windowed decode against the windowed teacher-forced layer, and the layer-batched stack against
the layer-by-layer one, each with windows longer and shorter than a cell (W = 1: the self
column only).
"""

import pytest
import torch

import oracle as O
from dual_mod_public_amd import _lib as L
from dual_mod_public_amd.decode import StaticTape
from dual_mod_public_amd.engine import HipSweepCell, uniform_chunks
from tests.hip_helpers import DEV, cfg_of, record, relerr, say, setup, to_dev
from tests.test_gpu_backward import FP32_TOL, compare, hip_grads, oracle_grads

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    L.load()


def _layer(cfg, sd, x, cos, sin, sched, dtype):
    B, T, d = x.shape
    cell = HipSweepCell(cfg, B, T, device=DEV, dtype=dtype)
    cell.pack({k: v.to(DEV, dtype) for k, v in sd.items()})
    bufs = cell.new_bufs(T)
    xd = x.to(DEV, dtype).contiguous()
    y = torch.empty_like(xd)
    K = torch.empty(B, cfg.n_heads, T, cfg.head_dim, device=DEV, dtype=dtype)
    V = torch.empty_like(K)
    ocat = torch.empty_like(xd)
    cell.layer_forward(xd, y, cos, sin, sched, K, V, ocat, bufs, normalize=False, residual=False)
    torch.cuda.synchronize()
    return ocat, K, V


@pytest.mark.parametrize("W,T", [(1, 192), (17, 256), (64, 256), (65, 256), (100, 256), (300, 512), (2048, 256)])
def test_windowed_exact_cells_equal_windowed_scan_fp32(W, T):
    say(f"windowed cells K=c vs windowed sequential scan, W={W} T={T}")
    cfg = cfg_of(T=T, local_window=W)
    B = 2
    sd, x, (c64, s64), (c32, s32) = setup(cfg, B, T)
    o, K, V = _layer(cfg, sd, x, c32, s32, uniform_chunks(T, 64), torch.float32)
    o_ref, K_ref, V_ref = O.sequential_scan(cfg, sd, x, c64, s64, return_cache=True)
    errs = {"o": relerr(o, o_ref), "K": relerr(K, K_ref), "V": relerr(V, V_ref)}
    record(f"window W={W} T={T} K=c", errs, 1e-5)
    say(f"  {errs}")
    assert max(errs.values()) < 1e-5


@pytest.mark.parametrize("W", [150, 40])
@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.bfloat16, 2e-2)])
def test_windowed_jacobi_cells_equal_oracle(dtype, tol, W):
    say(f"windowed Jacobi cells K=3 W={W} vs the oracle, {dtype}")
    T = 320
    cfg = cfg_of(T=T, local_window=W)
    B = 2
    sd, x, (c64, s64), (c32, s32) = setup(cfg, B, T)
    sched = uniform_chunks(T, 64, 3)
    o, K, V = _layer(cfg, sd, x, c32, s32, sched, dtype)
    o_ref, K_ref, V_ref = O.layer_forward(cfg, sd, x, c64, s64, sched)
    errs = {"o": relerr(o, o_ref), "K": relerr(K, K_ref), "V": relerr(V, V_ref)}
    record(f"window Jacobi W={W} {dtype}", errs, tol)
    assert max(errs.values()) < tol, errs


@pytest.mark.parametrize("K,W", [(4, 90), (64, 130), (4, 40), (64, 23), (3, 1)])
def test_windowed_backward_fp32(K, W):
    say(f"windowed backward K={K} W={W} vs autograd through the oracle")
    T = 192
    cfg = cfg_of(T=T, local_window=W)
    B = 2
    sd, x, (c64, s64), (c32, s32) = setup(cfg, B, T)
    dy = torch.randn(B, T, cfg.d_model, generator=torch.Generator().manual_seed(3), dtype=torch.float64)
    sched = uniform_chunks(T, 64, K)
    dx_ref, g_ref = oracle_grads(cfg, sd, x, dy, c64, s64, sched)
    for tape in (False, True):
        _, dx, grads = hip_grads(cfg, sd, x, dy, c32, s32, sched, torch.float32, tape=tape)
        compare(f"window bwd K={K} W={W} tape={tape}", dx, grads, dx_ref, g_ref, FP32_TOL)


@pytest.mark.parametrize("W", [70, 20])
def test_windowed_decode_equals_teacher_forced(W):
    """Two independent paths of the same windowed operator: token-by-token decode on the static
    tape and the K = c windowed layer forward."""
    say(f"windowed decode vs windowed teacher-forced layer, W={W}")
    T, B = 160, 2
    cfg = cfg_of(T=T, local_window=W)
    sd, x, _, (c32, s32) = setup(cfg, B, T)
    o_f, K_f, V_f = _layer(cfg, sd, x, c32, s32, uniform_chunks(T, 64), torch.float32)
    tape = StaticTape(cfg, B, T, DEV, torch.float32, sd=to_dev(sd, torch.float32))
    xd = x.float().to(DEV)
    outs = [tape.step(xd[:, t].contiguous(), t, c32, s32)[0].clone() for t in range(T)]
    torch.cuda.synchronize()
    errs = {"o": relerr(torch.stack(outs, 1), o_f), "K": relerr(tape.K, K_f), "V": relerr(tape.V, V_f)}
    record(f"window decode vs layer W={W}", errs, 1e-5)
    assert max(errs.values()) < 1e-5, errs


@pytest.mark.parametrize("W", [100, 30])
def test_windowed_stack_wavefront_equals_layer_by_layer(W):
    from dual_mod_public_amd.stack import HipLayerStack
    from dual_mod_public_amd.synthetic import make_state_dict
    say(f"windowed stack W={W}: layer-batched vs layer by layer")
    T, B, n = 256, 2, 3
    cfg = cfg_of(T=T, local_window=W)
    sds = [{k: v.to(DEV) for k, v in make_state_dict(cfg, seed=90 + i).items()} for i in range(n)]
    cos, sin = O.build_rope_cache(T, cfg.head_dim, cfg.rope_theta)
    sts = []
    for wf in (True, False):
        st = HipLayerStack(cfg, n, B, T, schedule=uniform_chunks(T, 64, 4), device=DEV, dtype=torch.bfloat16,
                           wavefront=wf)
        sts.append(st.load(sds, cos, sin))
    g = torch.Generator(device=DEV).manual_seed(5)
    x = torch.randn(B, T, cfg.d_model, generator=g, device=DEV).bfloat16()
    dy = torch.randn(B, T, cfg.d_model, generator=g, device=DEV).bfloat16()
    y1, dx1, _ = sts[0].step(x, dy)
    torch.cuda.synchronize()
    y1, dx1 = y1.clone(), dx1.clone()
    y2, dx2, _ = sts[1].step(x, dy)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2) and torch.equal(dx1, dx2) and torch.equal(sts[0].flat, sts[1].flat)


@pytest.mark.parametrize("W", [40, 150])
def test_windowed_backward_340m_shape_bf16(W):
    """bf16 storage at the 340M layer shape (d=1024, 16x64, c=64, K=4, T=256), forward tape,
    windows shorter and longer than the cell: gradients and the forward against autograd through
    the oracle's windowed chunked-Jacobi layer at the same K, run in fp32 torch on the GPU."""
    from tests.test_gpu_backward import BF16_TOL
    say(f"windowed bwd bf16 d=1024 T=256 K=4 W={W} vs fp32 oracle on the GPU")
    torch.backends.cuda.matmul.allow_tf32 = False
    T = 256
    cfg = cfg_of(d=1024, h=16, T=T, local_window=W)
    B = 2
    sd, x, _, (c32, s32) = setup(cfg, B, T)
    dy = torch.randn(B, T, cfg.d_model, generator=torch.Generator().manual_seed(17), dtype=torch.float32)
    sched = uniform_chunks(T, 64, 4)
    _, dx, g, (K, V, ocat) = hip_grads(cfg, sd, x, dy, c32, s32, sched, torch.bfloat16, tape=True, full=True)
    dx_ref, g_ref, (o_ref, K_ref, V_ref) = oracle_grads(
        cfg, {k: v.float() for k, v in sd.items()}, x.float(), dy, c32, s32, sched, dtype=torch.float32,
        device=DEV, with_forward=True)
    fwd = {"o_cat": relerr(ocat, o_ref), "K": relerr(K, K_ref), "V": relerr(V, V_ref)}
    record(f"window bf16 W={W} forward", fwd, BF16_TOL)
    assert max(fwd.values()) < BF16_TOL, fwd
    compare(f"window bwd bf16 W={W}", dx, g, dx_ref, g_ref, BF16_TOL)


@pytest.mark.parametrize("W", [1, 30, 100])
def test_windowed_head_dim_128_fp32(W):
    """head_dim 128 (d=256, 2 heads), windows shorter and longer than the 64-row cell, K = 3:
    forward against the oracle's windowed cells and gradients against autograd through it."""
    say(f"windowed dh=128 fp32 W={W}")
    T = 192
    cfg = cfg_of(d=256, h=2, T=T, local_window=W)
    assert cfg.head_dim == 128
    B = 2
    sd, x, (c64, s64), (c32, s32) = setup(cfg, B, T)
    sched = uniform_chunks(T, 64, 3)
    o, K, V = _layer(cfg, sd, x, c32, s32, sched, torch.float32)
    o_ref, K_ref, V_ref = O.layer_forward(cfg, sd, x, c64, s64, sched)
    errs = {"o": relerr(o, o_ref), "K": relerr(K, K_ref), "V": relerr(V, V_ref)}
    record(f"window dh128 W={W} forward", errs, 1e-5)
    assert max(errs.values()) < 1e-5, errs
    dy = torch.randn(B, T, cfg.d_model, generator=torch.Generator().manual_seed(19), dtype=torch.float64)
    dx_ref, g_ref = oracle_grads(cfg, sd, x, dy, c64, s64, sched)
    _, dx, grads = hip_grads(cfg, sd, x, dy, c32, s32, sched, torch.float32, tape=True)
    compare(f"window bwd dh128 W={W}", dx, grads, dx_ref, g_ref, FP32_TOL)


def test_window_one_equals_no_window_on_the_gpu():
    """W = 1 is read as no window (attend_one's K_past[:, :, -0:] is the whole past): the layer at
    W = 1 and at W = 0 give the same bits, and the decode step too."""
    say("W=1 layer and decode == no window")
    T, B = 128, 2
    outs = []
    for W in (0, 1):
        cfg = cfg_of(T=T, local_window=W)
        sd, x, _, (c32, s32) = setup(cfg, B, T)
        o, K, V = _layer(cfg, sd, x, c32, s32, uniform_chunks(T, 64, 3), torch.float32)
        tape = StaticTape(cfg, B, T, DEV, torch.float32, sd=to_dev(sd, torch.float32))
        xd = x.float().to(DEV)
        dec = torch.stack([tape.step(xd[:, t].contiguous(), t, c32, s32)[0].clone() for t in range(T)], 1)
        torch.cuda.synchronize()
        outs.append((o, K, V, dec))
    for a, b in zip(*outs):
        assert torch.equal(a, b)


@pytest.mark.parametrize("W", [20, 90])
def test_windowed_module_autograd_matches_oracle(W):
    """DualModAttention (reference signature) with local_window W, forward + loss.backward()
    through the HIP path, against autograd through the oracle's windowed cells (W = 20 inside a
    64-row chunk, W = 90 across chunks)."""
    from dual_mod_public_amd.attention import DualModAttention
    say(f"DualModAttention autograd fp32, W={W}")
    T, B = 128, 2
    cfg = cfg_of(T=T, local_window=W)
    sd, x, (c64, s64), (c32, s32) = setup(cfg, B, T)
    attn = DualModAttention(cfg).to(DEV)
    attn.load_state_dict({k: v.float() for k, v in sd.items() if k != "attn_norm.weight"})
    xd = x.float().to(DEV).requires_grad_(True)
    dy = torch.randn(B, T, cfg.d_model, generator=torch.Generator().manual_seed(23), dtype=torch.float64)
    y = attn(xd, c32.to(DEV), s32.to(DEV), n_sweeps=4)
    (y * dy.float().to(DEV)).sum().backward()
    torch.cuda.synchronize()
    sched = uniform_chunks(T, attn.CHUNK, 4)
    dx_ref, g_ref = oracle_grads(cfg, sd, x, dy, c64, s64, sched, normalize=False, residual=False)
    got = {n: p.grad for n, p in attn.named_parameters()}
    compare(f"module W={W}", xd.grad, got, dx_ref, g_ref, FP32_TOL, skip=("attn_norm.weight",))
