"""Invariants that pin the oracle independently of the golden vectors.

Re-states the reference's relational tests on the CPU restatement:
T1/T2 (tests/test_dualmod_equivalence.py:57-93) reduce to torch's SDPA,
T3 decode == teacher forcing (:98-112), T5 causality (:153-164),
T-K2 chunked == exact for K=c (engines/wavescan/tests/test_k1_k9.py:87-109),
T-K3 nilpotency + frontier (:114-137), T-K9 RoPE pairing (:142-152), and the
special case v_map = 0, lambda = 1 (mult_res reduces to linear).
"""

import math

import pytest
import torch

import oracle as O
from dual_mod_public_amd.config import DualModConfig
from dual_mod_public_amd.synthetic import make_input, make_state_dict
from tests.conftest import relerr

D = torch.float64
TOL = 1e-10       # fp64: relations hold to rounding


def _cfg(**kw):
    base = dict(d_model=64, n_layers=1, n_heads=4, max_seq_len=48, checkpoint_chunk=0,
                dtype="fp32", ctx_mod="mult_res")
    base.update(kw)
    return DualModConfig(**base)


def _setup(cfg, B=2, T=24, seed=5):
    sd = {k: v.to(D) for k, v in make_state_dict(cfg, seed=seed, std=0.05).items()}
    cos, sin = O.build_rope_cache(cfg.max_seq_len, cfg.head_dim, cfg.rope_theta, dtype=D)
    x = make_input((B, T, cfg.d_model), seed=seed + 1, dtype=D)
    return sd, cos[:T], sin[:T], x


def test_t1_mods_off_is_vanilla():
    cfg = _cfg(enable_key_mod=False, enable_value_mod=False)
    sd, cos, sin, x = _setup(cfg)
    with torch.no_grad():
        a = O.sequential_scan(cfg, sd, x, cos, sin)
        b = O.vanilla_attention(cfg, sd, x, cos, sin)
    assert relerr(a, b) < TOL


@pytest.mark.parametrize("mod", ["linear", "mult_res"])
def test_t2_gates_closed_is_vanilla(mod):
    cfg = _cfg(ctx_mod=mod)
    sd, cos, sin, x = _setup(cfg)
    for g in ("w_gk", "w_gv"):
        sd[g + ".bias"].fill_(40.0)
        sd[g + ".weight"].zero_()
    sd["w_kctx.weight"].normal_(0, 0.5)
    sd["w_vctx.weight"].normal_(0, 0.5)
    with torch.no_grad():
        a = O.sequential_scan(cfg, sd, x, cos, sin)
        b = O.vanilla_attention(cfg, sd, x, cos, sin)
    assert relerr(a, b) < TOL


def test_t2_gates_open_is_not_vanilla():
    cfg = _cfg()
    sd, cos, sin, x = _setup(cfg)
    with torch.no_grad():
        a = O.sequential_scan(cfg, sd, x, cos, sin)
        b = O.vanilla_attention(cfg, sd, x, cos, sin)
    assert relerr(a, b) > 1e-3


@pytest.mark.parametrize("mod", ["linear", "mult_res"])
def test_t3_decode_is_teacher_forced(mod):
    cfg = _cfg(ctx_mod=mod)
    sd, cos, sin, x = _setup(cfg)
    T = x.shape[1]
    with torch.no_grad():
        o_tf, K_tf, V_tf = O.sequential_scan(cfg, sd, x, cos, sin, return_cache=True)
        cache = {"K": None, "V": None}
        o_dec = torch.cat([O.decode_step(cfg, sd, x[:, t:t + 1], t, cache, cos, sin)[0]
                           for t in range(T)], 1)
        Kb = torch.zeros(x.shape[0], cfg.n_heads, T, cfg.head_dim, dtype=D)
        Vb = torch.zeros_like(Kb)
        o_st = torch.cat([O.static_decode_step(cfg, sd, x[:, t:t + 1], t, Kb, Vb, cos, sin)
                          for t in range(T)], 1)
    assert relerr(o_dec, o_tf) < TOL
    assert relerr(cache["K"], K_tf) < TOL and relerr(cache["V"], V_tf) < TOL
    assert relerr(o_st, o_tf) < TOL
    assert relerr(Kb, K_tf) < TOL and relerr(Vb, V_tf) < TOL


def test_t5_causality():
    cfg = _cfg()
    sd, cos, sin, x = _setup(cfg, T=16)
    x = x.clone().requires_grad_(True)
    t = 7
    y = O.dm_layer(cfg, sd, x, cos, sin)
    (g,) = torch.autograd.grad(y[:, t].sum(), x)
    assert g[:, t + 1:].abs().max().item() == 0.0
    assert g[:, :t + 1].abs().max().item() > 0.0


@pytest.mark.parametrize("sched_fn", [
    lambda T: O.exact_sequential(T),
    lambda T: O.uniform_chunks(T, 4),
    lambda T: O.uniform_chunks(T, 8),
    lambda T: [(0, 3, 3)] + [(p + 3, c, c) for p, c, _ in O.uniform_chunks(T - 3, 8)],
])
def test_k2_chunked_exact_equals_scan(sched_fn):
    cfg = _cfg()
    sd, cos, sin, x = _setup(cfg, T=40)
    sched = sched_fn(40)
    assert sum(c for _, c, _ in sched) == 40
    with torch.no_grad():
        o, K, V = O.layer_forward(cfg, sd, x, cos, sin, sched)
        o_ref, K_ref, V_ref = O.sequential_scan(cfg, sd, x, cos, sin, return_cache=True)
    assert relerr(o, o_ref) < TOL
    assert relerr(K, K_ref) < TOL and relerr(V, V_ref) < TOL


@pytest.mark.parametrize("c", [4, 8, 16])
def test_k3_nilpotency_and_frontier(c):
    cfg = _cfg()
    a = 12
    sd, cos, sin, x = _setup(cfg, T=a + c, seed=9)
    with torch.no_grad():
        _, K_all, V_all = O.sequential_scan(cfg, sd, x, cos, sin, return_cache=True)
        o_all = O.sequential_scan(cfg, sd, x, cos, sin)
        K_comm, V_comm = K_all[:, :, :a], V_all[:, :, :a]
        for s in range(1, c + 1):
            o_s, K_s, V_s = O.chunk_cell_forward(cfg, sd, x[:, a:], cos[a:], sin[a:],
                                                 K_comm, V_comm, s)
            assert relerr(o_s[:, :s], o_all[:, a:a + s]) < TOL
            assert relerr(K_s[:, :, :s], K_all[:, :, a:a + s]) < TOL
            if s <= c // 4:   # rows beyond the early frontier are still approximate
                assert relerr(o_s[:, s:], o_all[:, a + s:]) > 1e-12
    assert relerr(o_s, o_all[:, a:]) < TOL
    assert relerr(V_s, V_all[:, :, a:]) < TOL


def test_k9_rope_pairing():
    dh = 16
    cos, sin = O.build_rope_cache(8, dh, 10000.0)
    for i in range(dh // 2):
        e = torch.zeros(1, 1, 1, dh)
        e[..., i] = 1.0
        r = O.apply_rope(e, cos[3:4], sin[3:4])
        moved = set((r[0, 0, 0] != 0).nonzero().flatten().tolist())
        assert moved <= {i, i + dh // 2}
        # rotation preserves the norm
        assert abs(r.norm().item() - 1.0) < 1e-6


def test_rope_closed_form():
    # position p, pair i: angle p * theta^(-2i/dh)
    cos, sin = O.build_rope_cache(10, 8, 10000.0, dtype=D)
    for p in (0, 1, 9):
        for i in range(4):
            ang = p * 10000.0 ** (-2 * i / 8)
            assert abs(cos[p, i].item() - torch.cos(torch.tensor(ang, dtype=D)).item()) < 1e-12
            assert abs(sin[p, i].item() - torch.sin(torch.tensor(ang, dtype=D)).item()) < 1e-12


def test_rms_norm_closed_form():
    x = torch.tensor([[3.0, 4.0]], dtype=D)
    w = torch.tensor([1.0, 2.0], dtype=D)
    y = O.rms_norm(x, w, eps=0.0)
    r = (12.5) ** -0.5
    assert torch.allclose(y, torch.tensor([[3 * r, 8 * r]], dtype=D))


def test_mult_res_with_zero_map_is_linear():
    """v_map = 0 => tanh(0) = 0 => v_in = lambda*u; lambda = 1 => linear."""
    cfg_m = _cfg(ctx_mod="mult_res")
    cfg_l = _cfg(ctx_mod="linear")
    sd, cos, sin, x = _setup(cfg_m)
    sd["v_map.weight"].zero_()
    sd_l = {k: v for k, v in sd.items() if not k.startswith(("v_map", "v_gate"))}
    with torch.no_grad():
        a = O.sequential_scan(cfg_m, sd, x, cos, sin)
        b = O.sequential_scan(cfg_l, sd_l, x, cos, sin)
    assert relerr(a, b) < TOL


def test_attend_one_brute_force():
    """attend_one against a scalar softmax written out per key (tiny)."""
    cfg = _cfg()
    g = torch.Generator().manual_seed(3)
    q = torch.randn(1, 1, 1, 4, generator=g, dtype=D)
    ks = torch.randn(1, 1, 1, 4, generator=g, dtype=D)
    vs = torch.randn(1, 1, 1, 4, generator=g, dtype=D)
    K = torch.randn(1, 1, 3, 4, generator=g, dtype=D)
    V = torch.randn(1, 1, 3, 4, generator=g, dtype=D)
    o = O.attend_one(cfg, q, ks, vs, K, V)[0, 0, 0]
    keys = [K[0, 0, i] for i in range(3)] + [ks[0, 0, 0]]
    vals = [V[0, 0, i] for i in range(3)] + [vs[0, 0, 0]]
    sc = [float((q[0, 0, 0] * k).sum()) / 2.0 for k in keys]
    import math
    e = [math.exp(s - max(sc)) for s in sc]
    ref = sum(ei * v for ei, v in zip(e, vals)) / sum(e)
    assert torch.allclose(o, ref, atol=1e-12)


# ---------------------------------------------------------------------------
# pins of the knob branches that no golden vector covers (attention.py:291-293,
# 338-384): each check is a closed form the reference's formulas fix, computed here
# from the raw projections rather than by calling the branch under test
# ---------------------------------------------------------------------------

def _refine_inputs(cfg, seed=9, T=5):
    sd, _, _, x = _setup(cfg, T=T, seed=seed)
    g = torch.Generator().manual_seed(seed + 1)
    o_cat = torch.randn(x.shape, generator=g, dtype=D)
    k_raw = torch.randn(x.shape, generator=g, dtype=D)
    v_raw = torch.randn(x.shape, generator=g, dtype=D)
    return sd, x, o_cat, k_raw, v_raw


def test_mult_equals_mult_res_at_zero_lambda():
    """attention.py:347-353: mult's v_in = sigmoid(v_gate x) tanh(v_map u) is mult_res's with
    lambda = 0. A dropped sigmoid / tanh or swapped v_gate, v_map in the mult branch fails."""
    cfg_m = _cfg(ctx_mod="mult")
    cfg_r = _cfg(ctx_mod="mult_res", mult_res_lambda=0.0)
    sd, x, o_cat, k_raw, v_raw = _refine_inputs(cfg_m)
    km, vm = O.refine_kv(cfg_m, sd, x, o_cat, k_raw, v_raw)
    kr, vr = O.refine_kv(cfg_r, sd, x, o_cat, k_raw, v_raw)
    assert torch.equal(km, kr) and relerr(vm, vr) < TOL
    # and lambda matters: mult_res at lambda = 1 differs by (1 - g_v) w_vctx(u)
    cfg_1 = _cfg(ctx_mod="mult_res", mult_res_lambda=1.0)
    _, v1 = O.refine_kv(cfg_1, sd, x, o_cat, k_raw, v_raw)
    u = O.rms_norm(o_cat, sd["norm_ctx.weight"], 1e-5)
    gv = torch.sigmoid(torch.nn.functional.linear(torch.cat([x, u], -1), sd["w_gv.weight"], sd["w_gv.bias"]))
    assert relerr(v1 - vm, (1 - gv) * torch.nn.functional.linear(u, sd["w_vctx.weight"])) < TOL


def _value_gate(sd, x, o_cat):
    u = O.rms_norm(o_cat, sd["norm_ctx.weight"], 1e-5)
    return torch.sigmoid(torch.nn.functional.linear(torch.cat([x, u], -1), sd["w_gv.weight"], sd["w_gv.bias"]))


@pytest.mark.parametrize("mod", ["mult_res", "linear"])
def test_kmod_gated_norm_closed_form(mod):
    """attention.py:364-372 (kmod_mode gated_norm): the kmod heads' v_ctx is zeroed before
    the blend, so their v'' = g_v v_raw exactly; the other heads and k'' are untouched."""
    nvr = 2
    cfg = _cfg(ctx_mod=mod, kmod_vraw_heads=nvr, kmod_mode="gated_norm")
    base = _cfg(ctx_mod=mod)
    sd, x, o_cat, k_raw, v_raw = _refine_inputs(cfg)
    k, v = O.refine_kv(cfg, sd, x, o_cat, k_raw, v_raw)
    k0, v0 = O.refine_kv(base, sd, x, o_cat, k_raw, v_raw)
    cut = nvr * cfg.head_dim
    gv = _value_gate(sd, x, o_cat)
    assert relerr(v[..., :cut], (gv * v_raw)[..., :cut]) < TOL
    assert torch.equal(v[..., cut:], v0[..., cut:]) and torch.equal(k, k0)


@pytest.mark.parametrize("bound", ["none", "tanh"])
def test_kmod_raw_closed_form(bound):
    """attention.py:373-383 (kmod_mode raw): the kmod heads keep v_raw (tanh(v_raw) with
    kmod_vraw_bound tanh), no gate and no ctx term; the other heads are untouched."""
    nvr = 1
    cfg = _cfg(kmod_vraw_heads=nvr, kmod_vraw_bound=bound)
    base = _cfg()
    sd, x, o_cat, k_raw, v_raw = _refine_inputs(cfg)
    v_raw = 3.0 * v_raw   # beyond tanh's linear range
    _, v = O.refine_kv(cfg, sd, x, o_cat, k_raw, v_raw)
    _, v0 = O.refine_kv(base, sd, x, o_cat, k_raw, v_raw)
    cut = nvr * cfg.head_dim
    want = torch.tanh(v_raw[..., :cut]) if bound == "tanh" else v_raw[..., :cut]
    assert torch.equal(v[..., :cut], want)
    assert torch.equal(v[..., cut:], v0[..., cut:])


@pytest.mark.parametrize("W,P", [(3, 7), (5, 4), (8, 8)])
def test_attend_one_local_window_brute_force(W, P):
    """attention.py:291-293: with local_window W the read keeps the last W - 1 tape rows
    plus the raw self column; written out as a scalar softmax per key."""
    cfg = _cfg(local_window=W)
    g = torch.Generator().manual_seed(W * 10 + P)
    dh = 4
    q = torch.randn(1, 1, 1, dh, generator=g, dtype=D)
    ks = torch.randn(1, 1, 1, dh, generator=g, dtype=D)
    vs = torch.randn(1, 1, 1, dh, generator=g, dtype=D)
    K = torch.randn(1, 1, P, dh, generator=g, dtype=D)
    V = torch.randn(1, 1, P, dh, generator=g, dtype=D)
    o = O.attend_one(cfg, q, ks, vs, K, V)[0, 0, 0]
    lo = max(0, P - (W - 1))
    keys = [K[0, 0, i] for i in range(lo, P)] + [ks[0, 0, 0]]
    vals = [V[0, 0, i] for i in range(lo, P)] + [vs[0, 0, 0]]
    sc = [float((q[0, 0, 0] * k).sum()) / math.sqrt(dh) for k in keys]
    e = [math.exp(s - max(sc)) for s in sc]
    ref = sum(ei * v for ei, v in zip(e, vals)) / sum(e)
    assert torch.allclose(o, ref, atol=1e-12)


def _head_rms_ref(y, gain, h, eps=1e-6):
    """Per-head RMS norm written element by element (attention.py:227-269)."""
    out = torch.empty_like(y)
    dh = y.shape[-1] // h
    for idx in range(y.shape[0] * y.shape[1]):
        b, t = divmod(idx, y.shape[1])
        for hd in range(h):
            seg = y[b, t, hd * dh:(hd + 1) * dh]
            r = 1.0 / math.sqrt(float((seg * seg).sum()) / dh + eps)
            out[b, t, hd * dh:(hd + 1) * dh] = seg * r * float(gain[hd])
    return out



def test_k_ctx_norm_closed_form():
    """attention.py:257-269 (k_ctx_norm rms): k'' = g k_raw + (1 - g) N(w_kctx u) with N the
    per-head RMS norm (eps 1e-6) times k_gain."""
    cfg = _cfg(k_ctx_norm="rms")
    sd, x, o_cat, k_raw, v_raw = _refine_inputs(cfg)
    sd["k_gain"] = torch.tensor([1.75, 0.5, 2.0, 1.0], dtype=D)
    k, _ = O.refine_kv(cfg, sd, x, o_cat, k_raw, v_raw)
    u = O.rms_norm(o_cat, sd["norm_ctx.weight"], 1e-5)
    kc = _head_rms_ref(torch.nn.functional.linear(u, sd["w_kctx.weight"]), sd["k_gain"], 4)
    gk = torch.sigmoid(torch.nn.functional.linear(torch.cat([x, u], -1), sd["w_gk.weight"], sd["w_gk.bias"]))
    assert relerr(k, gk * k_raw + (1 - gk) * kc) < TOL


def test_v_ctx_norm_closed_form():
    """attention.py:238-255 (v_ctx_norm rms): v_ctx = N(w_vctx v_in), per-head RMS x ctx_gain."""
    cfg = _cfg(v_ctx_norm="rms", ctx_mod="linear")
    sd, x, o_cat, k_raw, v_raw = _refine_inputs(cfg)
    sd["ctx_gain"] = torch.tensor([0.5, 1.0, 1.5, 2.0], dtype=D)
    _, v = O.refine_kv(cfg, sd, x, o_cat, k_raw, v_raw)
    u = O.rms_norm(o_cat, sd["norm_ctx.weight"], 1e-5)
    vc = _head_rms_ref(torch.nn.functional.linear(u, sd["w_vctx.weight"]), sd["ctx_gain"], 4)
    gv = _value_gate(sd, x, o_cat)
    assert relerr(v, gv * v_raw + (1 - gv) * vc) < TOL


def test_v_norm_closed_form():
    """attention.py:218-234 (v_norm rms): v_raw = N(wv x), per-head RMS x v_gain."""
    cfg = _cfg(v_norm="rms")
    sd, _, _, x = _setup(cfg, T=3)
    sd["v_gain"] = torch.tensor([2.0, 1.0, 0.25, 1.0], dtype=D)
    v = O.project_v(cfg, sd, x)
    assert relerr(v, _head_rms_ref(torch.nn.functional.linear(x, sd["wv.weight"]), sd["v_gain"], 4)) < TOL


# ---- the trunk around the attention (models/dualmod/model.py:102-131, 267-291) -----------

def _lm_cfg(**kw):
    return _cfg(n_layers=2, vocab_size=40, mlp_hidden_override=96, **kw)


def _lm_sd(cfg, seed=3):
    from dual_mod_public_amd.synthetic import make_lm_state_dict
    return {k: v.to(D) for k, v in make_lm_state_dict(cfg, seed=seed, std=0.05).items()}


def test_swiglu_gate_and_linear_paths():
    """silu gates the w1 path only: the output is linear in w3 and in w2 (scaling either by a
    scales it by a) and not in w1 — a swap of w1 / w3 or a silu on the wrong product fails."""
    g = torch.Generator().manual_seed(9)
    sd = {f"mlp.{n}.weight": torch.randn(*s, generator=g, dtype=D)
          for n, s in (("w1", (6, 4)), ("w3", (6, 4)), ("w2", (4, 6)))}
    x = torch.randn(3, 4, generator=g, dtype=D)
    y = O.swiglu(sd, x)
    for n in ("w3", "w2"):
        s2 = dict(sd)
        s2[f"mlp.{n}.weight"] = 2.5 * sd[f"mlp.{n}.weight"]
        assert relerr(O.swiglu(s2, x), 2.5 * y) < TOL
    s2 = dict(sd)
    s2["mlp.w1.weight"] = 2.5 * sd["mlp.w1.weight"]
    assert relerr(O.swiglu(s2, x), 2.5 * y) > 1e-2
    # w1 -> +inf-like scale: silu(z) -> z for z > 0, 0 for z < 0 (a ReLU gate)
    s2 = dict(sd)
    s2["mlp.w1.weight"] = 1e3 * sd["mlp.w1.weight"]
    a, b = x @ s2["mlp.w1.weight"].t(), x @ sd["mlp.w3.weight"].t()
    assert relerr(O.swiglu(s2, x), (a.clamp(min=0) * b) @ sd["mlp.w2.weight"].t()) < 1e-6


def test_lm_identity_blocks_give_tied_head_of_normed_embedding():
    """With every block's output projections zero (wo = w2 = 0) the blocks are the identity and
    logits = rmsnorm(E[idx]) . E^T (tied head): pins the embedding gather, the final norm and
    the head's operand."""
    cfg = _lm_cfg()
    sd = _lm_sd(cfg)
    for l in range(cfg.n_layers):
        sd[f"blocks.{l}.attn.wo.weight"] = torch.zeros_like(sd[f"blocks.{l}.attn.wo.weight"])
        sd[f"blocks.{l}.mlp.w2.weight"] = torch.zeros_like(sd[f"blocks.{l}.mlp.w2.weight"])
    E = sd["tok_emb.weight"]
    idx = torch.tensor([[1, 7, 39, 0], [5, 5, 2, 11]])
    cos, sin = O.build_rope_cache(4, cfg.head_dim, cfg.rope_theta, dtype=D)
    e = E[idx]
    ref = (e / e.pow(2).mean(-1, keepdim=True).add(1e-5).sqrt()) @ E.t()
    assert relerr(O.lm_forward(cfg, sd, idx, cos, sin), ref) < TOL


def test_lm_decode_is_teacher_forced():
    """T3 at the model level (model.py:285-291 vs :267-281): decoding token by token through
    the per-layer caches reproduces the teacher-forced forward (exact sequential scan)."""
    cfg = _lm_cfg()
    sd = _lm_sd(cfg)
    B, T = 2, 12
    idx = torch.randint(0, cfg.vocab_size, (B, T), generator=torch.Generator().manual_seed(2))
    cos, sin = O.build_rope_cache(T, cfg.head_dim, cfg.rope_theta, dtype=D)
    ref = O.lm_forward(cfg, sd, idx, cos, sin)
    caches = [{"K": None, "V": None} for _ in range(cfg.n_layers)]
    out = torch.cat([O.lm_decode_step(cfg, sd, idx[:, t:t + 1], t, caches, cos, sin) for t in range(T)], 1)
    assert relerr(out, ref) < TOL


def test_lm_chunked_schedule_exact_equals_scan_and_differs_below_c():
    """lm_forward with a chunk schedule (the trunk step's oracle): K = c cells per layer give the
    sequential-scan model (nilpotency, scan_cell_fwd.py:1-10), K < c a different one."""
    cfg = _lm_cfg()
    sd = _lm_sd(cfg)
    B, T = 2, 16
    idx = torch.randint(0, cfg.vocab_size, (B, T), generator=torch.Generator().manual_seed(4))
    cos, sin = O.build_rope_cache(T, cfg.head_dim, cfg.rope_theta, dtype=D)
    ref = O.lm_forward(cfg, sd, idx, cos, sin)
    assert relerr(O.lm_forward(cfg, sd, idx, cos, sin, schedule=O.uniform_chunks(T, 8)), ref) < TOL
    assert relerr(O.lm_forward(cfg, sd, idx, cos, sin, schedule=O.uniform_chunks(T, 8, 2)), ref) > 1e-6


@pytest.mark.parametrize("W,c", [(5, 8), (9, 8), (20, 8), (3, 4), (2, 8), (1, 8)])
def test_windowed_cells_equal_windowed_scan(W, c):
    """The local window on the chunk cells (chunk_attend's window masks) with K = c sweeps
    reproduces the windowed sequential scan (scan.py over attend_one, whose window is pinned by
    the brute-force test above) — windows shorter and longer than the chunk, and W = 1, which
    attend_one reads as no window (its K_past[:, :, -(W - 1):] slices -0:, the whole past)."""
    cfg = _cfg(local_window=W)
    sd, cos, sin, x = _setup(cfg, T=24)
    ref = O.sequential_scan(cfg, sd, x, cos, sin)
    out = O.layer_forward(cfg, sd, x, cos, sin, O.uniform_chunks(24, c))[0]
    assert relerr(out, ref) < TOL


def test_window_one_reads_the_whole_past():
    """attention.py:292-293 at W = 1: the slice -(W - 1): is -0:, so attend_one keeps every past
    row; the windowed scan then equals the unwindowed one (and W = 2 does not)."""
    sd, cos, sin, x = _setup(_cfg(), T=12)
    ref = O.sequential_scan(_cfg(), sd, x, cos, sin)
    assert relerr(O.sequential_scan(_cfg(local_window=1), sd, x, cos, sin), ref) < TOL
    assert relerr(O.sequential_scan(_cfg(local_window=2), sd, x, cos, sin), ref) > 1e-3


def test_window_changes_the_cells():
    cfg_w = _cfg(local_window=6)
    sd, cos, sin, x = _setup(cfg_w, T=24)
    a = O.layer_forward(cfg_w, sd, x, cos, sin, O.uniform_chunks(24, 8, 3))[0]
    b = O.layer_forward(_cfg(), sd, x, cos, sin, O.uniform_chunks(24, 8, 3))[0]
    assert relerr(a[:, 6:], b[:, 6:]) > 1e-3 and relerr(a[:, :5], b[:, :5]) < TOL
