"""GPU parity of the v'' entry-norm clamp (config.py v_clamp_tau; models/dualmod/
attention.py:389-402): v'' <- v'' min(1, tau / ||v''||) per (position, head) after the
value blend, in every sweep and in decode. Forward, gradients (autograd through the
oracle) and decode; tau is chosen so that a good share of the rows is clamped (checked),
alone and with kmod heads. fp32 tolerances as the dense tests."""

import pytest
import torch

import oracle as O
from dual_mod_public_amd import _lib as L
from dual_mod_public_amd.engine import uniform_chunks
from tests.hip_helpers import DEV, cfg_of, relerr, say, setup
from tests.test_gpu_backward import FP32_TOL, compare, hip_grads, oracle_grads

pytestmark = pytest.mark.gpu

TAU = 1.8


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    L.load()


def clamped_share(V, tau):
    n = V.double().norm(dim=-1)
    return ((n - tau).abs() < 1e-4 * tau).double().mean().item()


@pytest.mark.parametrize("ctx_mod,kw", [("mult_res", {}), ("linear", {}), ("fusion", {}),
                                        ("mult_res", dict(kmod_vraw_heads=1))],
                         ids=["mult_res", "linear", "fusion", "mult_res_kmod"])
@pytest.mark.parametrize("tape", [True, False], ids=["tape", "recompute"])
def test_clamp_layer_matches_oracle(ctx_mod, kw, tape):
    say(f"clamp tau={TAU} {ctx_mod} {kw} tape={tape}")
    cfg = cfg_of(ctx_mod=ctx_mod, v_clamp_tau=TAU, **kw)
    B, T = 2, 64
    sd, x, (c64, s64), (c32, s32) = setup(cfg, B, T)
    dy = torch.randn(B, T, cfg.d_model, generator=torch.Generator().manual_seed(9), dtype=torch.float64)
    sched = uniform_chunks(T, 16, 4)
    y, dx, g, (K, V, _) = hip_grads(cfg, sd, x, dy, c32, s32, sched, torch.float32, tape=tape, full=True)
    with torch.no_grad():
        xh = O.rms_norm(x, sd["attn_norm.weight"], 1e-5)
        o, K_ref, V_ref = O.layer_forward(cfg, sd, xh, c64, s64, sched)
        y_ref = O.dm_oracle._lin(o, sd, "wo") + x
    share = clamped_share(V_ref, TAU)
    say(f"  clamped share {share:.2f}")
    assert 0.1 < share < 0.9, share
    errs = (relerr(y, y_ref), relerr(V, V_ref))
    say(f"  forward relerr y {errs[0]:.2e} V {errs[1]:.2e}")
    assert max(errs) < 1e-5
    dx_ref, g_ref = oracle_grads(cfg, sd, x, dy, c64, s64, sched)
    compare("clamp", dx, g, dx_ref, g_ref, FP32_TOL)


def test_clamp_decode_matches_oracle():
    from dual_mod_public_amd.decode import StaticTape
    cfg = cfg_of(v_clamp_tau=TAU)
    B, T = 2, 16
    sd, x, (c64, s64), (c32, s32) = setup(cfg, B, T)
    tape = StaticTape(cfg, B, T, DEV, torch.float32, sd={k: v.float().to(DEV) for k, v in sd.items()})
    cache = {"K": None, "V": None}
    xd = x.float().to(DEV)
    worst = 0.0
    for t in range(T):
        o, _ = tape.step(xd[:, t].contiguous(), t, c32.to(DEV), s32.to(DEV))
        o_ref, _ = O.decode_step(cfg, sd, x[:, t:t + 1], t, cache, c64, s64)
        worst = max(worst, relerr(o, o_ref[:, 0]))
    share = clamped_share(cache["V"], TAU)
    say(f"clamp decode worst relerr {worst:.2e}, clamped share {share:.2f}")
    assert 0.1 < share < 0.9
    assert worst < 1e-5
    assert relerr(tape.V[:, :, :T], cache["V"]) < 1e-5
