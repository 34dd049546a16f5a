"""Seeded synthetic weights and inputs for the benchmark configurations.

Weights use the reference's parameter names (models/dualmod/attention.py:100-202,
models/dualmod/model.py:118-121) so a state dict made here loads into either
implementation. Every draw comes from ``numpy.random.default_rng(seed)`` in the
fixed order of ``param_specs`` — platform-independent, so the CPU oracle, the
golden-vector script and the GPU run all see identical numbers.

Distribution (all configs): every matrix N(0, std=0.02), including w_kctx,
w_vctx and v_map so the mult_res branch is live; gate biases and the v_gate
bias N(0, 0.02) (gates open, sigma ~ 0.5); RMSNorm weights 1; per-head gains 1.
Factored operators (gate_rank / ctx_rank > 0, attention.py:24-75) draw both factors
N(0, sqrt(std / sqrt(r))), so their product has the dense weights' scale.
"""

from collections import OrderedDict

import numpy as np
import torch


def param_specs(cfg, with_attn_norm=True):
    """Ordered (name, shape, kind) of one DM attention layer's parameters."""
    d = cfg.d_model
    h = cfg.n_heads
    mod = getattr(cfg, "ctx_mod", "linear")
    specs = [("wq.weight", (d, d), "w"), ("wk.weight", (d, d), "w"),
             ("wv.weight", (d, d), "w"), ("wo.weight", (d, d), "w")]
    if getattr(cfg, "v_norm", "none") == "rms":
        specs.append(("v_gain", (h,), "one"))
    rc, rg = getattr(cfg, "ctx_rank", 0), getattr(cfg, "gate_rank", 0)

    def ctx(name, bias=False):
        if rc > 0:
            out = [(f"{name}.down.weight", (rc, d), "f"), (f"{name}.up.weight", (d, rc), "f")]
            return out + ([(f"{name}.up.bias", (d,), "b")] if bias else [])
        return [(f"{name}.weight", (d, d), "w")] + ([(f"{name}.bias", (d,), "b")] if bias else [])

    def gate(name):
        if rg > 0:
            return [(f"{name}.a.weight", (rg, 2 * d), "f"), (f"{name}.b.weight", (d, rg), "f"),
                    (f"{name}.b.bias", (d,), "b")]
        return [(f"{name}.weight", (d, 2 * d), "w"), (f"{name}.bias", (d,), "b")]

    if cfg.enable_key_mod:
        specs += ctx("w_kctx") + gate("w_gk")
        if getattr(cfg, "k_ctx_norm", "none") == "rms":
            specs.append(("k_gain", (h,), "one"))
    if cfg.enable_value_mod:
        specs += ctx("w_vctx") + gate("w_gv")
        if getattr(cfg, "v_ctx_norm", "none") == "rms":
            specs.append(("ctx_gain", (h,), "one"))
    if mod in ("mult", "mult_res"):
        specs += ctx("v_gate", bias=True) + ctx("v_map")
    elif mod == "fusion":
        specs.append(("v_pre.weight", (d, 2 * d), "w"))
    if cfg.enable_key_mod or cfg.enable_value_mod:
        specs.append(("norm_ctx.weight", (d,), "one"))
    if with_attn_norm:
        specs.append(("attn_norm.weight", (d,), "one"))
    return specs


def make_state_dict(cfg, seed=0, std=0.02, dtype=torch.float32, with_attn_norm=True):
    rng = np.random.default_rng(seed)
    sd = OrderedDict()
    for name, shape, kind in param_specs(cfg, with_attn_norm):
        if kind == "one":
            a = np.ones(shape, dtype=np.float64)
        elif kind == "f":   # one factor of a rank-r product: r is the smaller dimension
            a = rng.normal(0.0, (std / min(shape) ** 0.5) ** 0.5, size=shape)
        else:
            a = rng.normal(0.0, std, size=shape)
        sd[name] = torch.from_numpy(a).to(dtype)
    return sd


def make_lm_state_dict(cfg, seed=0, std=0.02, dtype=torch.float32):
    """A DualModLM state dict (models/dualmod/model.py:134-150 names): token embedding
    N(0, std) (tied head: ``lm_head.weight`` is the same tensor), per layer the attention
    parameters of ``make_state_dict`` (seed 1000 * seed + layer), SwiGLU matrices N(0, std),
    RMSNorm weights 1."""
    rng = np.random.default_rng(seed)
    d, hid = cfg.d_model, cfg.mlp_hidden
    t = lambda *shape: torch.from_numpy(rng.normal(0.0, std, size=shape)).to(dtype)   # noqa: E731
    sd = OrderedDict()
    sd["tok_emb.weight"] = t(cfg.vocab_size, d)
    for l in range(cfg.n_layers):
        pre = f"blocks.{l}."
        sd[pre + "attn_norm.weight"] = torch.ones(d, dtype=dtype)
        for k, v in make_state_dict(cfg, seed=1000 * seed + l, std=std, dtype=dtype, with_attn_norm=False).items():
            sd[pre + "attn." + k] = v
        sd[pre + "mlp_norm.weight"] = torch.ones(d, dtype=dtype)
        sd[pre + "mlp.w1.weight"] = t(hid, d)
        sd[pre + "mlp.w3.weight"] = t(hid, d)
        sd[pre + "mlp.w2.weight"] = t(d, hid)
    sd["norm_f.weight"] = torch.ones(d, dtype=dtype)
    sd["lm_head.weight"] = sd["tok_emb.weight"] if cfg.tie_embeddings else t(cfg.vocab_size, d)
    return sd


def make_input(shape, seed=1, dtype=torch.float32, scale=1.0):
    """x ~ N(0, scale^2) of the given shape (float64 draw, cast)."""
    rng = np.random.default_rng(seed)
    return torch.from_numpy(rng.normal(0.0, scale, size=shape)).to(dtype)
