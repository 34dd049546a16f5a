"""GPU parity of the per-head RMS norms (models/dualmod/attention.py:218-269):
k_ctx_norm (norm_kctx, gain k_gain), v_ctx_norm (norm_vctx, gain ctx_gain) and v_norm
(project_v, gain v_gain), each y = gain x rsqrt(mean x^2 + 1e-6) per (row, head).

Forward, gradients (the gains' included) and decode against the oracle, which the
reference's golden knob case pins for k_ctx_norm and v_ctx_norm (tests/golden,
knobs_mult_res) and closed forms pin for all three (tests/test_oracle_invariants.py).
The gains are drawn away from 1 so a dropped gain or a wrong head index fails.
fp32 bars as the dense tests: 1e-5 forward / decode, 1e-5 gradients; bf16 as
tests/test_gpu_backward.py."""

import pytest
import torch

import oracle as O
from dual_mod_public_amd import _lib as L
from dual_mod_public_amd.engine import HipSweepCell, uniform_chunks
from tests.hip_helpers import DEV, cfg_of, relerr, say, setup
from tests.test_gpu_backward import BF16_FWD_TOL, BF16_TOL, FP32_TOL, compare, hip_grads, oracle_grads

pytestmark = pytest.mark.gpu

NORMS = {"k": dict(k_ctx_norm="rms"), "vctx": dict(v_ctx_norm="rms"), "v": dict(v_norm="rms"),
         "all": dict(k_ctx_norm="rms", v_ctx_norm="rms", v_norm="rms")}


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    L.load()


def norm_setup(cfg, B, T, seed=5):
    """setup() with the present gains drawn from N(1.3, 0.4) (k_gain around its 1.75 init)."""
    sd, x, r64, r32 = setup(cfg, B, T)
    g = torch.Generator().manual_seed(seed)
    for name, mean in (("k_gain", 1.75), ("ctx_gain", 1.3), ("v_gain", 1.3)):
        if name in sd:
            sd[name] = (mean + 0.4 * torch.randn(cfg.n_heads, generator=g)).double()
    return sd, x, r64, r32


def oracle_y(cfg, sd, x, c64, s64, sched):
    with torch.no_grad():
        xh = O.rms_norm(x, sd["attn_norm.weight"], 1e-5)
        o = O.layer_forward(cfg, sd, xh, c64, s64, sched)[0]
        return O.dm_oracle._lin(o, sd, "wo") + x


@pytest.mark.parametrize("norm", list(NORMS))
@pytest.mark.parametrize("ctx_mod", ["mult_res", "linear"])
@pytest.mark.parametrize("h", [4, 2], ids=["dh64", "dh128"])
def test_norm_layer_fp32(norm, ctx_mod, h):
    say(f"norms {norm} {ctx_mod} h={h}")
    cfg = cfg_of(h=h, ctx_mod=ctx_mod, **NORMS[norm])
    B, T = 2, 64
    sd, x, (c64, s64), (c32, s32) = norm_setup(cfg, B, T)
    dy = torch.randn(B, T, cfg.d_model, generator=torch.Generator().manual_seed(17), dtype=torch.float64)
    sched = uniform_chunks(T, 16, 4)
    tape = h == 4
    y, dx, g = hip_grads(cfg, sd, x, dy, c32, s32, sched, torch.float32, tape=tape)
    err = relerr(y, oracle_y(cfg, sd, x, c64, s64, sched))
    say(f"  forward relerr {err:.2e}")
    assert err < 1e-5
    dx_ref, g_ref = oracle_grads(cfg, sd, x, dy, c64, s64, sched)
    for name in ("k_gain", "ctx_gain", "v_gain"):
        assert (name in g_ref) == (name in sd)
    compare(f"norm-{norm}", dx, g, dx_ref, g_ref, FP32_TOL)


@pytest.mark.parametrize("ctx_mod", ["mult_res", "fusion"])
@pytest.mark.parametrize("fused", [True, False])
def test_norm_64row_cells_with_kmod_and_clamp(ctx_mod, fused):
    """64-row cells: GEMM 2 fused with the next sweep's attention (fused=True) or the
    64 x dh head-tile GEMM 2 (fused=False), each holding the v_ctx norm, the gated_norm
    kmod heads' zeroing after it and the v'' clamp."""
    say(f"norm 64-row cells {ctx_mod} fused={fused}")
    cfg = cfg_of(ctx_mod=ctx_mod, k_ctx_norm="rms", v_ctx_norm="rms", v_norm="rms", kmod_vraw_heads=1,
                 kmod_mode="gated_norm", v_clamp_tau=8.0)
    B, T = 2, 128
    sd, x, (c64, s64), (c32, s32) = norm_setup(cfg, B, T, seed=9)
    sched = uniform_chunks(T, 64, 3)
    cell = HipSweepCell(cfg, B, T, device=DEV, dtype=torch.float32, fused_attend=fused)
    cell.pack({k: v.to(DEV, torch.float32) for k, v in sd.items()})
    bufs = cell.new_bufs(T)
    xd = x.to(DEV, torch.float32).contiguous()
    y = torch.empty_like(xd)
    K = torch.empty(B, cfg.n_heads, T, cfg.head_dim, device=DEV)
    V = torch.empty_like(K)
    ocat = torch.empty_like(xd)
    cell.layer_forward(xd, y, c32, s32, sched, K, V, ocat, bufs)
    torch.cuda.synchronize()
    err = relerr(y, oracle_y(cfg, sd, x, c64, s64, sched))
    say(f"  forward relerr {err:.2e}")
    assert err < 1e-5


def test_norm_decode_fp32():
    from dual_mod_public_amd.decode import StaticTape
    cfg = cfg_of(ctx_mod="mult_res", **NORMS["all"])
    B, T = 2, 16
    sd, x, (c64, s64), (c32, s32) = norm_setup(cfg, B, T)
    tape = StaticTape(cfg, B, T, DEV, torch.float32, sd={k: v.float().to(DEV) for k, v in sd.items()})
    cache = {"K": None, "V": None}
    xd = x.float().to(DEV)
    worst = 0.0
    for t in range(T):
        o, _ = tape.step(xd[:, t].contiguous(), t, c32.to(DEV), s32.to(DEV))
        o_ref, _ = O.decode_step(cfg, sd, x[:, t:t + 1], t, cache, c64, s64)
        worst = max(worst, relerr(o, o_ref[:, 0]))
    say(f"norm decode worst relerr {worst:.2e}")
    assert worst < 1e-5


@pytest.mark.parametrize("ctx_mod", ["mult_res", "linear"])
def test_norm_grads_bf16_340m_shape(ctx_mod):
    """d=1024, h=16 (the 340M layer shape), bf16 storage, every norm on."""
    say(f"norms bf16 340M shape {ctx_mod}")
    cfg = cfg_of(d=1024, h=16, T=128, ctx_mod=ctx_mod, **NORMS["all"])
    B, T = 2, 128
    sd, x, (c64, s64), (c32, s32) = norm_setup(cfg, B, T)
    dy = torch.randn(B, T, cfg.d_model, generator=torch.Generator().manual_seed(3), dtype=torch.float64)
    sched = uniform_chunks(T, 64, 4)
    y, dx, g = hip_grads(cfg, sd, x, dy, c32, s32, sched, torch.bfloat16, tape=True)
    err = relerr(y, oracle_y(cfg, sd, x, c64, s64, sched))
    say(f"  forward relerr {err:.2e}")
    assert err < BF16_FWD_TOL
    dx_ref, g_ref = oracle_grads(cfg, sd, x, dy, c64, s64, sched)
    compare("norm-bf16", dx, g, dx_ref, g_ref, BF16_TOL)


def test_norm_cell_backward_matches_layer_path():
    """The per-cell backward (reference grad-cache protocol) with every norm on: gains'
    grads accumulate across the cells the same way as the layer path's."""
    from tests.test_gpu_cell_bwd import cell_grads
    cfg = cfg_of(ctx_mod="mult_res", **NORMS["all"])
    B, T = 2, 64
    sd, x, (c64, s64), (c32, s32) = norm_setup(cfg, B, T)
    dy = torch.randn(B, T, cfg.d_model, generator=torch.Generator().manual_seed(29), dtype=torch.float64)
    sched = [(0, 16, 3), (16, 16, 1), (32, 7, 2), (39, 25, 4)]
    dx, g, _ = cell_grads(cfg, sd, x, dy, c32, s32, sched, torch.float32, tape=True)
    dx_ref, g_ref = oracle_grads(cfg, sd, x, dy, c64, s64, sched)
    compare("norm-cells", dx, g, dx_ref, g_ref, FP32_TOL)
