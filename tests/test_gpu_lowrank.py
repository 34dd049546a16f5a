"""GPU parity of the factored knobs (gate_rank, ctx_rank > 0) through the HIP path.

DualModAttention with factored gates and context operators (the reference's LoRAGate /
LoRALinear parameters, models/dualmod/attention.py:24-75) runs its forward and backward
on libdm_hip.so with the dense products packed; the factor gradients come from the
dense ones by the chain rule (fused_sweep.py:43-56, :1882-1936). The oracle side builds
the dense weights from the factor leaves inside torch autograd (fp64, CPU), so the
chain rule is computed independently. fp32 tolerance 1e-5 relative (the dense tests' bar)."""

import pytest
import torch

import oracle as O
from dual_mod_public_amd import _lib as L
from dual_mod_public_amd.engine import uniform_chunks
from tests.hip_helpers import DEV, cfg_of, record, relerr, say, setup

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-5


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    L.load()


def dense_graph(leaves):
    """Dense reference-named weights as differentiable products of the factor leaves."""
    dense = dict(leaves)
    for n in ("w_kctx", "w_vctx", "v_gate", "v_map"):
        if f"{n}.down.weight" in leaves:
            dense[f"{n}.weight"] = leaves[f"{n}.up.weight"] @ leaves[f"{n}.down.weight"]
            if f"{n}.up.bias" in leaves:
                dense[f"{n}.bias"] = leaves[f"{n}.up.bias"]
    for n in ("w_gk", "w_gv"):
        if f"{n}.a.weight" in leaves:
            dense[f"{n}.weight"] = leaves[f"{n}.b.weight"] @ leaves[f"{n}.a.weight"]
            dense[f"{n}.bias"] = leaves[f"{n}.b.bias"]
    return dense


@pytest.mark.parametrize("gate_rank,ctx_rank,ctx_mod", [(8, 16, "mult_res"), (16, 0, "linear"), (0, 32, "mult")])
def test_factored_module_matches_oracle(gate_rank, ctx_rank, ctx_mod):
    from dual_mod_public_amd.attention import DualModAttention
    say(f"factored gate_rank={gate_rank} ctx_rank={ctx_rank} {ctx_mod}")
    cfg = cfg_of(ctx_mod=ctx_mod, gate_rank=gate_rank, ctx_rank=ctx_rank)
    B, T = 2, 64
    sd, x, (c64, s64), (c32, s32) = setup(cfg, B, T)
    sd = {k: v for k, v in sd.items() if k != "attn_norm.weight"}
    attn = DualModAttention(cfg).to(DEV)
    attn.load_state_dict({k: v.float() for k, v in sd.items()})
    xd = x.float().to(DEV).requires_grad_(True)
    dy = torch.randn(B, T, cfg.d_model, generator=torch.Generator().manual_seed(7), dtype=torch.float64)
    y = attn(xd, c32.to(DEV), s32.to(DEV), n_sweeps=4)
    (y * dy.float().to(DEV)).sum().backward()
    torch.cuda.synchronize()

    leaves = {k: v.clone().requires_grad_(True) for k, v in sd.items()}
    xr = x.clone().requires_grad_(True)
    with torch.enable_grad():
        dense = dense_graph(leaves)
        o = O.layer_forward(cfg, dense, xr, c64, s64, uniform_chunks(T, attn.CHUNK, 4))[0]
        y_ref = O.dm_oracle._lin(o, dense, "wo")
        (y_ref * dy).sum().backward()
    errs = {"y": relerr(y.detach(), y_ref.detach()), "x": relerr(xd.grad, xr.grad)}
    for n, p in attn.named_parameters():
        errs[n] = relerr(p.grad, leaves[n].grad)
    worst = max(errs, key=errs.get)
    say(f"  worst {worst} {errs[worst]:.2e}")
    record(f"factored gate_rank={gate_rank} ctx_rank={ctx_rank} {ctx_mod}", errs, FP32_TOL)
    for k, v in errs.items():
        assert v < FP32_TOL, f"{k}: relerr {v:.3e}"


def test_factored_decode_matches_oracle():
    """Decode with a factored state dict: the static tape packs the dense products."""
    from dual_mod_public_amd.decode import StaticTape
    cfg = cfg_of(gate_rank=8, ctx_rank=16)
    B, T = 2, 16
    sd, x, (c64, s64), (c32, s32) = setup(cfg, B, T)
    tape = StaticTape(cfg, B, T, DEV, torch.float32, sd={k: v.float().to(DEV) for k, v in sd.items()})
    dense = {k: v.detach() for k, v in dense_graph(sd).items()}
    cache = {"K": None, "V": None}
    xd = x.float().to(DEV)
    for t in range(T):
        o, _ = tape.step(xd[:, t].contiguous(), t, c32.to(DEV), s32.to(DEV))
        o_ref, _ = O.decode_step(cfg, dense, x[:, t:t + 1], t, cache, c64, s64)
    torch.cuda.synchronize()
    err = relerr(o, o_ref[:, 0])
    say(f"factored decode relerr {err:.2e}")
    record("factored decode", {"o": err}, 1e-5)
    assert err < 1e-5
