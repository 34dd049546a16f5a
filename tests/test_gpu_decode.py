"""GPU parity of the HIP decode step (dm_decode_step) against the CPU oracle.

T3 analogue (tests/test_dualmod_equivalence.py:98-112): decoding token by token
through the static tape reproduces the teacher-forced sequential scan; plus a
pre-written random bf16 tape (BASELINE config 5 shape, scaled down) checked
against the oracle's static-tape decode (lm/eval/graph_decode.py:33-51).
"""

import pytest
import torch

import oracle as O
from dual_mod_public_amd import _lib as L
from dual_mod_public_amd.decode import StaticTape
from tests.hip_helpers import DEV, cfg_of, record, relerr, say, setup, to_dev

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    L.load()


@pytest.mark.parametrize("ctx_mod", ["mult_res", "linear", "fusion"])
def test_decode_equals_teacher_forced_fp32(ctx_mod):
    say(f"decode fp32 teacher-forced ctx_mod={ctx_mod}")
    cfg = cfg_of(ctx_mod=ctx_mod)
    B, T = 2, 64
    sd, x, (c64, s64), (c32, s32) = setup(cfg, B, T)
    tape = StaticTape(cfg, B, T, DEV, torch.float32, sd=to_dev(sd, torch.float32))
    xd = x.float().to(DEV)
    outs = []
    for t in range(T):
        o, _ = tape.step(xd[:, t].contiguous(), t, c32, s32)
        outs.append(o.clone())
    torch.cuda.synchronize()
    o_ref, K_ref, V_ref = O.sequential_scan(cfg, sd, x, c64, s64, return_cache=True)
    assert relerr(torch.stack(outs, 1), o_ref) < 1e-5
    assert relerr(tape.K, K_ref) < 1e-5
    assert relerr(tape.V, V_ref) < 1e-5


def test_decode_local_window_fp32():
    say("decode fp32 local_window=8")
    cfg = cfg_of(local_window=8, T=24)
    B, T = 2, 24
    sd, x, (c64, s64), (c32, s32) = setup(cfg, B, T)
    tape = StaticTape(cfg, B, T, DEV, torch.float32, sd=to_dev(sd, torch.float32))
    xd = x.float().to(DEV)
    cache = {"K": None, "V": None}
    for t in range(T):
        o, _ = tape.step(xd[:, t].contiguous(), t, c32, s32)
        o_ref, _ = O.decode_step(cfg, sd, x[:, t:t + 1], t, cache, c64, s64)
        assert relerr(o, o_ref[:, 0]) < 1e-5, t
    assert relerr(tape.K, cache["K"]) < 1e-5


@pytest.mark.parametrize("P0", [0, 1, 511, 1500])
def test_decode_on_random_bf16_tape(P0):
    """Pre-written N(0,1) bf16 tape of P0 rows (multi-split when P0 > 512), d=1024
    16x64, 4 steps; vs the oracle static-tape decode in fp32 on the same tape."""
    say(f"decode bf16 random tape P0={P0}")
    cfg = cfg_of(d=1024, h=16, T=P0 + 8)
    B, steps = 4, 4
    P = P0 + steps
    sd, x, _, (c32, s32) = setup(cfg, B, P)
    g = torch.Generator().manual_seed(5)
    K0 = torch.randn(B, 16, P, 64, generator=g).bfloat16()
    V0 = torch.randn(B, 16, P, 64, generator=g).bfloat16()
    tape = StaticTape(cfg, B, P, DEV, torch.bfloat16, sd=to_dev(sd, torch.bfloat16))
    tape.K.copy_(K0.to(DEV))
    tape.V.copy_(V0.to(DEV))
    Kb, Vb = K0.float(), V0.float()
    sdf = {k: v.float() for k, v in sd.items()}
    xb = x.bfloat16()
    for t in range(P0, P):
        o, _ = tape.step(xb[:, t].to(DEV).contiguous(), t, c32, s32)
        o_ref = O.static_decode_step(cfg, sdf, xb[:, t:t + 1].float(), t, Kb, Vb, c32, s32)
        torch.cuda.synchronize()
        e = relerr(o, o_ref[:, 0])
        say(f"  step {t}: relerr o={e:.2e}")
        assert e < 2e-2
    assert relerr(tape.K[:, :, P0:P], Kb[:, :, P0:P]) < 2e-2
    assert relerr(tape.V[:, :, P0:P], Vb[:, :, P0:P]) < 2e-2
    assert torch.equal(tape.K[:, :, :P0].cpu(), K0[:, :, :P0])   # append-only


def test_attention_module_decode_matches_scan():
    from dual_mod_public_amd.attention import DualModAttention
    say("DualModAttention.decode_step fp32")
    cfg = cfg_of(T=32)
    B, T = 2, 32
    sd, x, (c64, s64), (c32, s32) = setup(cfg, B, T)
    attn = DualModAttention(cfg).to(DEV)
    attn.load_state_dict({k: v.float() for k, v in sd.items() if k != "attn_norm.weight"})
    cache = {"K": None, "V": None}
    xd = x.float().to(DEV)
    ys = [attn.decode_step(xd[:, t:t + 1], t, cache, c32.to(DEV), s32.to(DEV)) for t in range(T)]
    torch.cuda.synchronize()
    o_ref, K_ref, _ = O.sequential_scan(cfg, sd, x, c64, s64, return_cache=True)
    y_ref = O.dm_oracle._lin(o_ref, sd, "wo")
    assert relerr(torch.cat(ys, 1), y_ref) < 1e-5
    assert relerr(cache["K"], K_ref) < 1e-5


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("W", [0, 3001])
def test_decode_many_splits(dtype, W):
    """A pre-written N(0,1) tape of 4700 rows: 10 splits of the split-P read (more than
    any smaller test) merged by k_decode_merge, with and without a window whose first row
    falls inside a split (W = 3001: rows [pos - 3000, pos) + self). Against the oracle's
    decode_step (attend_one applies the window, attention.py:291-293) in fp64.
    fp32 bar: 1e-5, or four times the fp32 oracle's own error on the same inputs where that
    is larger. o sums ~4700 N(0,1) value rows with random signs, so its fp32 rounding error
    in any summation order is ~sqrt(P) eps relative to |o|; the oracle run in fp32 (same
    inputs, torch's summation order) measures it and both errors are recorded. A dropped or
    doubled split, or a window offset off by a row, is an error of 1e-3 or more."""
    say(f"decode many splits {dtype} W={W}")
    cfg = cfg_of(d=256, h=4, T=4708, local_window=W)
    B, P0, steps = 2, 4700, 3
    P = P0 + steps
    sd, x, (c64, s64), (c32, s32) = setup(cfg, B, P)
    g = torch.Generator().manual_seed(21)
    K0 = torch.randn(B, 4, P, 64, generator=g).to(dtype)
    V0 = torch.randn(B, 4, P, 64, generator=g).to(dtype)
    tape = StaticTape(cfg, B, P, DEV, dtype, sd=to_dev(sd, dtype))
    tape.K.copy_(K0.to(DEV))
    tape.V.copy_(V0.to(DEV))
    cache = {"K": K0[:, :, :P0].double(), "V": V0[:, :, :P0].double()}
    xs = x.to(dtype)
    fp32 = dtype == torch.float32
    # the same steps through the oracle in fp32: its own rounding error at this length
    cache32 = {"K": K0[:, :, :P0].float(), "V": V0[:, :, :P0].float()}
    sd32 = {k: v.float() for k, v in sd.items()}
    errs, own = {}, {}
    for t in range(P0, P):
        o, _ = tape.step(xs[:, t].to(DEV).contiguous(), t, c32, s32)
        o_ref, _ = O.decode_step(cfg, sd, xs[:, t:t + 1].double(), t, cache, c64, s64)
        if fp32:
            o32, _ = O.decode_step(cfg, sd32, xs[:, t:t + 1].float(), t, cache32, c32, s32)
            own[f"o@{t}"] = relerr(o32[:, 0], o_ref[:, 0])
        torch.cuda.synchronize()
        errs[f"o@{t}"] = relerr(o, o_ref[:, 0])
    errs["K rows"] = relerr(tape.K[:, :, P0:P], cache["K"][:, :, P0:P])
    errs["V rows"] = relerr(tape.V[:, :, P0:P], cache["V"][:, :, P0:P])
    if fp32:
        own["K rows"] = relerr(cache32["K"][:, :, P0:P], cache["K"][:, :, P0:P])
        own["V rows"] = relerr(cache32["V"][:, :, P0:P], cache["V"][:, :, P0:P])
        tol = max(1e-5, 4 * max(own.values()))
        say("  fp32 oracle's own error: " + " ".join(f"{k}={v:.2e}" for k, v in own.items()))
        record(f"decode 10 splits fp32 oracle's own error W={W}", own, tol)
    else:
        tol = 2e-2
    say("  " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()))
    record(f"decode 10 splits {dtype} W={W}", errs, tol)
    assert max(errs.values()) < tol, errs


def test_decode_config5_shape():
    """BASELINE config 5 itself: B=64, d=1024 16x64, a pre-written N(0,1) bf16 tape of 32768
    rows (64 splits per (b, h) merged by k_decode_merge), 3 steps; against the oracle's
    static-tape decode (lm/eval/graph_decode.py:33-51) run in fp32 torch on the GPU."""
    say("decode C5 shape: B=64 P0=32768 bf16 vs fp32 oracle on the GPU")
    torch.backends.cuda.matmul.allow_tf32 = False
    cfg = cfg_of(d=1024, h=16, T=32776)
    B, P0, steps = 64, 32768, 3
    P = P0 + steps
    sd = {k: v.float() for k, v in setup(cfg, 1, 8)[0].items()}
    g = torch.Generator(device=DEV).manual_seed(5)
    tape = StaticTape(cfg, B, P, DEV, torch.bfloat16, sd=to_dev(sd, torch.bfloat16))
    tape.K.normal_(generator=g)
    tape.V.normal_(generator=g)
    x = torch.randn(B, steps, 1024, generator=g, device=DEV).to(torch.bfloat16)
    cos, sin = O.build_rope_cache(P, 64, 10000.0)
    cos, sin = cos.to(DEV), sin.to(DEV)
    Kb, Vb = tape.K.float(), tape.V.float()
    sdd = to_dev(sd, torch.float32)
    errs = {}
    for t in range(P0, P):
        o, _ = tape.step(x[:, t - P0].contiguous(), t, cos, sin)
        o_ref = O.static_decode_step(cfg, sdd, x[:, t - P0:t - P0 + 1].float(), t, Kb, Vb, cos, sin)
        torch.cuda.synchronize()
        errs[f"o@{t}"] = relerr(o, o_ref[:, 0])
    errs["K rows"] = relerr(tape.K[:, :, P0:P], Kb[:, :, P0:P])
    errs["V rows"] = relerr(tape.V[:, :, P0:P], Vb[:, :, P0:P])
    say("  " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()))
    record("decode C5 shape bf16", errs, 2e-2)
    assert max(errs.values()) < 2e-2, errs
    del Kb, Vb
