"""Factored gates / context operators (gate_rank, ctx_rank > 0) on the host side of the
boundary: dense materialisation before packing and the chain rule of the dense weight
gradients onto the factors (fused_sweep.py:43-56, :1882-1936 do the same). CPU only;
the kernels see dense weights, so their parity is the dense tests' (the GPU check of
the whole path is tests/test_gpu_lowrank.py).

Pinned by torch autograd through the products W = up @ down and W = b @ a (an
independent computation of the same chain rule) and by the reference's parameter
names (models/dualmod/attention.py:24-75, 125-152, 182-183)."""

import torch

from dual_mod_public_amd.config import DualModConfig
from dual_mod_public_amd.engine import check_supported
from dual_mod_public_amd.lowrank import dense_params, factor_grads, is_factored
from dual_mod_public_amd.synthetic import make_state_dict


def cfg_r(gate_rank=8, ctx_rank=16, ctx_mod="mult_res"):
    return DualModConfig(d_model=256, n_heads=4, n_layers=1, max_seq_len=64, ctx_mod=ctx_mod,
                         gate_rank=gate_rank, ctx_rank=ctx_rank, dtype="fp32")


def test_reference_parameter_names():
    """The factored module's parameters carry the reference's names and shapes."""
    from dual_mod_public_amd.attention import DualModAttention
    cfg = cfg_r()
    m = DualModAttention(cfg)
    shapes = {n: tuple(p.shape) for n, p in m.named_parameters()}
    d, rg, rc = 256, 8, 16
    for n in ("w_kctx", "w_vctx", "v_gate", "v_map"):
        assert shapes[f"{n}.down.weight"] == (rc, d) and shapes[f"{n}.up.weight"] == (d, rc)
        assert f"{n}.weight" not in shapes
    assert shapes["v_gate.up.bias"] == (d,)
    for n in ("w_gk", "w_gv"):
        assert shapes[f"{n}.a.weight"] == (rg, 2 * d) and shapes[f"{n}.b.weight"] == (d, rg)
        assert shapes[f"{n}.b.bias"] == (d,)
    sd = make_state_dict(cfg, seed=3, with_attn_norm=False)
    assert set(sd) == set(shapes)
    m.load_state_dict(sd)   # a synthetic factored state dict loads into the module
    check_supported(cfg)


def test_dense_products():
    cfg = cfg_r()
    sd = make_state_dict(cfg, seed=4, dtype=torch.float64)
    assert is_factored(sd)
    dn = dense_params(sd)
    for n in ("w_kctx", "w_vctx", "v_gate", "v_map"):
        ref = sd[f"{n}.up.weight"] @ sd[f"{n}.down.weight"]
        assert torch.allclose(dn[f"{n}.weight"], ref, rtol=1e-6, atol=1e-9)
    for n in ("w_gk", "w_gv"):
        ref = sd[f"{n}.b.weight"] @ sd[f"{n}.a.weight"]
        assert torch.allclose(dn[f"{n}.weight"], ref, rtol=1e-6, atol=1e-9)
        assert dn[f"{n}.bias"] is sd[f"{n}.b.bias"]
    assert dn["v_gate.bias"] is sd["v_gate.up.bias"]
    # the products carry the dense weights' scale (factor std sqrt(0.02 / sqrt(r)))
    assert 0.01 < dn["w_kctx.weight"].std().item() < 0.04
    # a dense state dict passes through untouched
    plain = make_state_dict(cfg_r(0, 0), seed=4)
    assert not is_factored(plain) and dense_params(plain) is plain


def test_factor_grads_match_autograd():
    """Chain rule onto the factors == autograd through the products, for a loss whose dense
    gradients are arbitrary (L = sum_n <W_n, G_n> + <bias_n, g_n>)."""
    cfg = cfg_r()
    sd = {k: v.clone().requires_grad_(True) for k, v in make_state_dict(cfg, seed=5, dtype=torch.float64).items()}
    gen = torch.Generator().manual_seed(6)
    dense_grads = {}
    loss = 0.0
    with torch.enable_grad():
        for n in ("w_kctx", "w_vctx", "v_gate", "v_map"):
            W = sd[f"{n}.up.weight"] @ sd[f"{n}.down.weight"]
            G = torch.randn(W.shape, generator=gen, dtype=torch.float64)
            dense_grads[f"{n}.weight"] = G
            loss = loss + (W * G).sum()
        gb = torch.randn(256, generator=gen, dtype=torch.float64)
        dense_grads["v_gate.bias"] = gb
        loss = loss + (sd["v_gate.up.bias"] * gb).sum()
        for n in ("w_gk", "w_gv"):
            W = sd[f"{n}.b.weight"] @ sd[f"{n}.a.weight"]
            G = torch.randn(W.shape, generator=gen, dtype=torch.float64)
            gbias = torch.randn(256, generator=gen, dtype=torch.float64)
            dense_grads[f"{n}.weight"], dense_grads[f"{n}.bias"] = G, gbias
            loss = loss + (W * G).sum() + (sd[f"{n}.b.bias"] * gbias).sum()
        loss.backward()
    names = [n for n in sd if sd[n].grad is not None]
    got = factor_grads(sd, dense_grads, names)
    for n in names:
        assert torch.allclose(got[n].double(), sd[n].grad, rtol=1e-5, atol=1e-9), n
