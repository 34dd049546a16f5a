"""GPU parity at head_dim 128 (the config-4 trunk's head size: d=2048, 16 x 128).

Every kernel is instantiated per head size; these tests run the head_dim-128
instances against the CPU oracle with the same bars as the head_dim-64 tests:
fp32 forward / decode within 1e-5 relative, bf16 forward within 2e-2, fp32
gradients within 1e-5 and bf16 gradients within 2e-2 of the fp64 oracle.
"""

import pytest
import torch

import oracle as O
from dual_mod_public_amd import _lib as L
from dual_mod_public_amd.decode import StaticTape
from dual_mod_public_amd.engine import HipSweepCell, LayerGrads, uniform_chunks
from tests.hip_helpers import DEV, cfg_of, record, relerr, say, setup, to_dev
from tests.test_gpu_backward import compare, hip_grads, oracle_grads
from tests.test_gpu_forward import _cell, _hip_layer

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-5
BF16_TOL = 2e-2
BF16_GRAD_TOL = 2e-2
FP32_GRAD_TOL = 1e-5


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    L.load()


def cfg128(ctx_mod="mult_res", d=256, T=64, **kw):
    return cfg_of(d=d, h=d // 128, ctx_mod=ctx_mod, T=T, **kw)


def test_layer_proj_dh128_fp32():
    say("layer_proj fp32 dh=128")
    cfg = cfg128()
    assert cfg.head_dim == 128
    B, T = 2, 64
    sd, x, (c64, s64), (c32, s32) = setup(cfg, B, T)
    cell = _cell(cfg, B, T, sd, torch.float32)
    bufs = cell.new_bufs(T)
    cell.layer_proj(x.float().to(DEV), bufs, c32, s32, normalize=True)
    torch.cuda.synchronize()
    xhat = O.rms_norm(x, sd["attn_norm.weight"])
    q_r, k, k_self_r, v = O.dm_oracle._projections(cfg, sd, xhat, c64, s64)
    for got, ref in ((bufs.qr, q_r), (bufs.kraw, k), (bufs.kself, k_self_r), (bufs.vraw, v)):
        assert relerr(got, ref) < 1e-6


@pytest.mark.parametrize("ctx_mod", ["mult_res", "linear", "mult"])
@pytest.mark.parametrize("c", [16, 64])
def test_cell_exact_equals_scan_dh128_fp32(ctx_mod, c):
    say(f"cell K=c fp32 dh=128 ctx_mod={ctx_mod} c={c}")
    cfg = cfg128(ctx_mod)
    B, T = 2, 64
    sd, x, (c64, s64), (c32, s32) = setup(cfg, B, T)
    ocat, K, V = _hip_layer(cfg, sd, x, c32, s32, uniform_chunks(T, c), torch.float32)
    o_ref, K_ref, V_ref = O.sequential_scan(cfg, sd, x, c64, s64, return_cache=True)
    assert relerr(ocat, o_ref) < FP32_TOL
    assert relerr(K, K_ref) < FP32_TOL
    assert relerr(V, V_ref) < FP32_TOL


@pytest.mark.parametrize("c,k", [(16, 4), (64, 2), (8, 3)])
def test_cell_jacobi_dh128_fp32(c, k):
    say(f"cell Jacobi fp32 dh=128 c={c} K={k}")
    cfg = cfg128()
    B, T = 2, 64
    sd, x, (c64, s64), (c32, s32) = setup(cfg, B, T)
    sched = uniform_chunks(T, c, k)
    ocat, K, V = _hip_layer(cfg, sd, x, c32, s32, sched, torch.float32)
    o_ref, K_ref, V_ref = O.layer_forward(cfg, sd, x, c64, s64, sched)
    assert relerr(ocat, o_ref) < FP32_TOL
    assert relerr(K, K_ref) < FP32_TOL
    assert relerr(V, V_ref) < FP32_TOL


def test_bf16_config4_shape_dh128():
    """bf16 at the config-4 layer shape (d=2048, 16 x 128), c=64, K=4, T=256."""
    say("bf16 d=2048 16x128 T=256 c=64 K=4")
    cfg = cfg_of(d=2048, h=16, T=256)
    B, T = 1, 256
    sd, x, (c64, s64), (c32, s32) = setup(cfg, B, T)
    sched = uniform_chunks(T, 64, 4)
    ocat, K, V = _hip_layer(cfg, sd, x, c32, s32, sched, torch.bfloat16)
    o_ref, K_ref, V_ref = O.layer_forward(cfg, sd, x.float(), c32, s32, sched)
    e = (relerr(ocat, o_ref), relerr(K, K_ref), relerr(V, V_ref))
    say(f"  bf16 relerr o={e[0]:.2e} K={e[1]:.2e} V={e[2]:.2e}")
    assert max(e) < BF16_TOL


@pytest.mark.parametrize("ctx_mod", ["mult_res", "linear"])
def test_decode_teacher_forced_dh128_fp32(ctx_mod):
    say(f"decode fp32 dh=128 ctx_mod={ctx_mod}")
    cfg = cfg128(ctx_mod)
    B, T = 2, 48
    sd, x, (c64, s64), (c32, s32) = setup(cfg, B, T)
    tape = StaticTape(cfg, B, T, DEV, torch.float32, sd=to_dev(sd, torch.float32))
    xd = x.float().to(DEV)
    outs = []
    for t in range(T):
        o, _ = tape.step(xd[:, t].contiguous(), t, c32, s32)
        outs.append(o.clone())
    torch.cuda.synchronize()
    o_ref, K_ref, V_ref = O.sequential_scan(cfg, sd, x, c64, s64, return_cache=True)
    assert relerr(torch.stack(outs, 1), o_ref) < FP32_TOL
    assert relerr(tape.K, K_ref) < FP32_TOL
    assert relerr(tape.V, V_ref) < FP32_TOL


@pytest.mark.parametrize("ctx_mod", ["mult_res", "linear", "mult"])
@pytest.mark.parametrize("tape", [False, True])
def test_layer_grads_dh128_bf16(ctx_mod, tape):
    say(f"bwd bf16 dh=128 ctx_mod={ctx_mod} tape={tape}")
    cfg = cfg128(ctx_mod)
    B, T = 2, 64
    sd, x, (c64, s64), (c32, s32) = setup(cfg, B, T)
    dy = torch.randn(B, T, cfg.d_model, generator=torch.Generator().manual_seed(31), dtype=torch.float64)
    sched = uniform_chunks(T, 16, 3)
    _, dx, g = hip_grads(cfg, sd, x, dy, c32, s32, sched, torch.bfloat16, tape=tape)
    dx_ref, g_ref = oracle_grads(cfg, sd, x, dy, c64, s64, sched)
    compare("bf16 dh128", dx, g, dx_ref, g_ref, BF16_GRAD_TOL)


def test_tape_equals_recompute_dh128_bf16():
    say("tape == recompute bf16 dh=128")
    cfg = cfg128()
    B, T = 2, 64
    sd, x, _, (c32, s32) = setup(cfg, B, T)
    dy = torch.randn(B, T, cfg.d_model, generator=torch.Generator().manual_seed(32), dtype=torch.float64)
    sched = [(0, 24, 2), (24, 40, 3)]
    y0, dx0, g0 = hip_grads(cfg, sd, x, dy, c32, s32, sched, torch.bfloat16)
    y1, dx1, g1 = hip_grads(cfg, sd, x, dy, c32, s32, sched, torch.bfloat16, tape=True)
    assert torch.equal(y0, y1) and torch.equal(dx0, dx1)
    for name, t in g0.t.items():
        assert torch.equal(t, g1[name]), name


@pytest.mark.parametrize("ctx_mod", ["mult_res", "linear"])
@pytest.mark.parametrize("tape", [False, True])
def test_layer_grads_dh128_fp32(ctx_mod, tape):
    """fp32 gradients at head_dim 128 against the fp64 oracle (the fp32 bar of the head_dim-64 tests)."""
    say(f"bwd fp32 dh=128 ctx_mod={ctx_mod} tape={tape}")
    cfg = cfg128(ctx_mod)
    B, T = 2, 64
    sd, x, (c64, s64), (c32, s32) = setup(cfg, B, T)
    dy = torch.randn(B, T, cfg.d_model, generator=torch.Generator().manual_seed(33), dtype=torch.float64)
    sched = [(0, 24, 2), (24, 16, 3), (40, 24, 1)]
    _, dx, g = hip_grads(cfg, sd, x, dy, c32, s32, sched, torch.float32, tape=tape)
    dx_ref, g_ref = oracle_grads(cfg, sd, x, dy, c64, s64, sched)
    compare("fp32 dh128", dx, g, dx_ref, g_ref, FP32_GRAD_TOL)


@pytest.mark.parametrize("k", [1, 2, 4, 8])
def test_layer_grads_config4_shape_bf16(k):
    """Config 4's layer shape (d=2048, 16 x 128), c=64, the ladder's K = 1 / 2 / 4 / 8, T=256, bf16 storage,
    forward tape: gradients and the forward against autograd through the oracle's
    chunked-Jacobi layer at the same K, run in fp32 torch on the GPU."""
    say(f"bwd bf16 d=2048 16x128 T=256 c=64 K={k} vs fp32 oracle on the GPU")
    torch.backends.cuda.matmul.allow_tf32 = False
    cfg = cfg_of(d=2048, h=16, T=256)
    B, T = 2, 256
    sd, x, _, (c32, s32) = setup(cfg, B, T)
    dy = torch.randn(B, T, cfg.d_model, generator=torch.Generator().manual_seed(41), dtype=torch.float32)
    sched = uniform_chunks(T, 64, k)
    _, dx, g, (K, V, ocat) = hip_grads(cfg, sd, x, dy, c32, s32, sched, torch.bfloat16, tape=True, full=True)
    dx_ref, g_ref, (o_ref, K_ref, V_ref) = oracle_grads(
        cfg, {k: v.float() for k, v in sd.items()}, x.float(), dy, c32, s32, sched, dtype=torch.float32,
        device=DEV, with_forward=True)
    fwd = {"o_cat": relerr(ocat, o_ref), "K": relerr(K, K_ref), "V": relerr(V, V_ref)}
    say("  forward relerr " + " ".join(f"{k}={v:.2e}" for k, v in fwd.items()))
    record(f"bf16 C4 shape T=256 K={k} forward", fwd, BF16_TOL)
    assert max(fwd.values()) < BF16_TOL, fwd
    compare(f"bf16 C4 shape T=256 K={k}", dx, g, dx_ref, g_ref, BF16_GRAD_TOL)
