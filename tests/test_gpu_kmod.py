"""GPU parity of the kmod heads knob (config.py kmod_vraw_heads / kmod_mode /
kmod_vraw_bound; models/dualmod/attention.py:362-384): the first n heads keep their
raw value (raw, optionally tanh-bounded) or blend it with a zeroed v_ctx
(gated_norm). Forward, gradients (autograd through the oracle) and decode. The
oracle's kmod branches are pinned by closed forms (tests/test_oracle_invariants.py:
gated_norm heads' v'' == sigmoid(gate) v_raw, raw heads' v'' == v_raw or tanh(v_raw));
the reference's golden knob case covers raw mode without the tanh bound. fp32
tolerances as the dense tests: 1e-5 forward / decode, 1e-5 grads."""

import pytest
import torch

import oracle as O
from dual_mod_public_amd import _lib as L
from dual_mod_public_amd.engine import uniform_chunks
from tests.hip_helpers import DEV, cfg_of, relerr, say, setup
from tests.test_gpu_backward import FP32_TOL, compare, hip_grads, oracle_grads

pytestmark = pytest.mark.gpu

MODES = [dict(kmod_vraw_heads=1), dict(kmod_vraw_heads=2, kmod_vraw_bound="tanh"),
         dict(kmod_vraw_heads=1, kmod_mode="gated_norm")]


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    L.load()


@pytest.mark.parametrize("ctx_mod", ["mult_res", "linear"])
@pytest.mark.parametrize("kw", MODES, ids=["raw", "raw_tanh", "gated_norm"])
def test_kmod_layer_matches_oracle(kw, ctx_mod):
    say(f"kmod {kw} {ctx_mod}")
    cfg = cfg_of(ctx_mod=ctx_mod, **kw)
    B, T = 2, 64
    sd, x, (c64, s64), (c32, s32) = setup(cfg, B, T)
    dy = torch.randn(B, T, cfg.d_model, generator=torch.Generator().manual_seed(8), dtype=torch.float64)
    sched = uniform_chunks(T, 16, 4)
    y, dx, g = hip_grads(cfg, sd, x, dy, c32, s32, sched, torch.float32, tape=True)
    with torch.no_grad():
        xh = O.rms_norm(x, sd["attn_norm.weight"], 1e-5)
        o = O.layer_forward(cfg, sd, xh, c64, s64, sched)[0]
        y_ref = O.dm_oracle._lin(o, sd, "wo") + x
    err = relerr(y, y_ref)
    say(f"  forward relerr {err:.2e}")
    assert err < 1e-5
    dx_ref, g_ref = oracle_grads(cfg, sd, x, dy, c64, s64, sched)
    compare("kmod", dx, g, dx_ref, g_ref, FP32_TOL)


@pytest.mark.parametrize("kw", MODES, ids=["raw", "raw_tanh", "gated_norm"])
def test_kmod_decode_matches_oracle(kw):
    from dual_mod_public_amd.decode import StaticTape
    cfg = cfg_of(**kw)
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
    say(f"kmod decode {kw} worst relerr {worst:.2e}")
    assert worst < 1e-5
