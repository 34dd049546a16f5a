"""CPU restatement of the reference Dual-Mod attention path (test oracle).

TEST INFRASTRUCTURE: imported only by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg. Never part of the product path.

Every function cites the reference file:line it restates (paths relative to
the reference repository root). Weights are passed as a plain state dict with
the reference's parameter names (``wq.weight``, ``w_gk.bias`` ...), so one
random state dict drives both this oracle and the HIP path.

Precision model. The reference computes softmax, sigmoid, RMS and RoPE in
fp32 "islands" (``.float()`` calls) inside bf16 storage. Here every island is
"at least fp32": in fp64 mode the whole computation stays fp64 (the most
accurate restatement), in fp32 mode it is the reference's fp32 computation,
and in bf16 mode the storage roundings happen where the reference's do.
"""

import math

import torch
import torch.nn.functional as F

__all__ = [
    "build_rope_cache", "apply_rope", "rms_norm", "split_heads", "merge_heads",
    "attend_one", "refine_kv", "project_v", "sequential_scan",
    "make_intra_mask", "chunk_attend", "chunk_cell_forward", "layer_forward",
    "uniform_chunks", "exact_sequential", "decode_step", "static_decode_step",
    "vanilla_attention", "dm_layer", "cfg_get", "swiglu", "lm_forward", "lm_decode_step",
]


def _hi(x):
    """The reference's ``.float()`` island: upcast to at least fp32."""
    return x.to(torch.promote_types(x.dtype, torch.float32))


def cfg_get(cfg, name, default):
    return getattr(cfg, name, default)


# ---------------------------------------------------------------------------
# RoPE — models/dualmod/rope.py
# ---------------------------------------------------------------------------

def build_rope_cache(max_seq_len, head_dim, theta, dtype=torch.float32):
    """rope.py:13-19 — inv_freq = theta^(-2i/dh), cos/sin [T, dh/2].
    The reference builds these in fp32; ``dtype=float64`` gives the exact
    table (used by fp64 oracle runs)."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=dtype) / head_dim))
    t = torch.arange(max_seq_len, dtype=dtype)
    freqs = torch.outer(t, inv_freq)
    return freqs.cos(), freqs.sin()


def apply_rope(x, cos, sin):
    """rope.py:22-33 — half-split pairs (i, i+dh/2), math in >=fp32, cast back."""
    xf = _hi(x)
    x1, x2 = xf.chunk(2, dim=-1)
    c, s = cos.to(xf.dtype), sin.to(xf.dtype)
    out = torch.cat([x1 * c - x2 * s, x2 * c + x1 * s], dim=-1)
    return out.to(x.dtype)


# ---------------------------------------------------------------------------
# norms — models/dualmod/attention.py
# ---------------------------------------------------------------------------

def rms_norm(x, w, eps=1e-5):
    """attention.py:74-83 — x*rsqrt(mean(x^2)+eps)*w in >=fp32, cast back."""
    xf = _hi(x)
    out = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return (out * w.to(xf.dtype)).to(x.dtype)


def _head_rms(y, gain, n_heads, head_dim, eps=1e-6):
    """attention.py:238-269 (norm_vctx / norm_kctx) and :227-234 (v_norm):
    per-head RMS in >=fp32 with a per-head gain."""
    shp = y.shape
    yh = _hi(y.reshape(*shp[:-1], n_heads, head_dim))
    yh = yh * torch.rsqrt(yh.pow(2).mean(-1, keepdim=True) + eps)
    yh = yh * gain.to(yh.dtype).unsqueeze(-1)
    return yh.to(y.dtype).reshape(shp)


def split_heads(x, h):
    """attention.py:206-209 — [B,T,d] -> [B,h,T,dh]."""
    B, T, d = x.shape
    return x.view(B, T, h, d // h).transpose(1, 2)


def merge_heads(x):
    """attention.py:211-214 — [B,h,T,dh] -> [B,T,d]."""
    B, h, T, dh = x.shape
    return x.transpose(1, 2).reshape(B, T, h * dh)


def _lin(x, sd, name, bias=False):
    w = sd[name + ".weight"].to(x.dtype)
    b = sd[name + ".bias"].to(x.dtype) if bias else None
    return F.linear(x, w, b)


def project_v(cfg, sd, xhat):
    """attention.py:218-234 — wv(x); optional per-head RMS (v_norm='rms')."""
    v = _lin(xhat, sd, "wv")
    if cfg_get(cfg, "v_norm", "none") != "rms":
        return v
    h = cfg.n_heads
    return _head_rms(v, sd["v_gain"], h, v.shape[-1] // h)


# ---------------------------------------------------------------------------
# the per-position step — attention.py:283-434
# ---------------------------------------------------------------------------

def attend_one(cfg, q_r, k_self_r, v_self, K_past, V_past):
    """attention.py:283-312 — read over [refined tape ; raw self].

    q_r, k_self_r, v_self: [B,h,1,dh]; K_past/V_past [B,h,P,dh] or None.
    Scores and softmax in >=fp32, probabilities cast to the value dtype
    before the PV product (attention.py:310-311).
    """
    dh = q_r.shape[-1]
    scale = 1.0 / math.sqrt(dh)
    W = cfg_get(cfg, "local_window", 0) or 0
    if W and K_past is not None and K_past.shape[2] > W - 1:          # :291-293
        K_past, V_past = K_past[:, :, -(W - 1):], V_past[:, :, -(W - 1):]
    if K_past is None or K_past.shape[2] == 0:
        k_all, v_all = k_self_r, v_self
    else:
        k_all = torch.cat([K_past, k_self_r], dim=2)
        v_all = torch.cat([V_past, v_self], dim=2)
    s = (q_r @ k_all.transpose(-1, -2)) * scale
    a = torch.softmax(_hi(s), dim=-1)
    return a.to(v_all.dtype) @ v_all


def _blend(logits, raw, ctx):
    """attention.py:404-418 (convex_sigmoid): g = sigmoid(logits) in >=fp32,
    cast to the raw dtype, out = g*raw + (1-g)*ctx."""
    g = torch.sigmoid(_hi(logits)).to(raw.dtype)
    return g * raw + (1.0 - g) * ctx


def refine_kv(cfg, sd, xhat, o_cat, k_raw, v_raw):
    """attention.py:314-387 — ctx norm, ctx projections, gates, convex blend.

    All inputs [B,t,d]. Returns (k'', v'') UNROTATED. Supports the knob set
    the HIP path honours: ctx_mod in {linear, mult, mult_res, fusion}, mult_res_lambda,
    k_ctx_norm, v_ctx_norm, kmod_vraw_heads (raw / gated_norm), v_clamp_tau.
    """
    if not (cfg_get(cfg, "enable_key_mod", True) or cfg_get(cfg, "enable_value_mod", True)):
        return k_raw, v_raw                                            # :321-322
    h = cfg.n_heads
    d = xhat.shape[-1]
    dh = d // h
    u = rms_norm(o_cat, sd["norm_ctx.weight"], 1e-5)                   # :323
    g_in = torch.cat([xhat, u], dim=-1)                                # :324-325
    kpp, vpp = k_raw, v_raw
    mod = cfg_get(cfg, "ctx_mod", "linear")
    if cfg_get(cfg, "enable_key_mod", True):                          # :332-337
        k_ctx = _lin(u, sd, "w_kctx")
        if cfg_get(cfg, "k_ctx_norm", "none") == "rms":
            k_ctx = _head_rms(k_ctx, sd["k_gain"], h, dh)
        kpp = _blend(_lin(g_in, sd, "w_gk", bias=True), k_raw, k_ctx)
    if cfg_get(cfg, "enable_value_mod", True):                        # :338-384
        if mod == "mult":                                              # :347-349
            v_in = torch.sigmoid(_hi(_lin(xhat, sd, "v_gate", bias=True))).to(u.dtype) \
                * torch.tanh(_lin(u, sd, "v_map"))
        elif mod == "mult_res":                                        # :350-353
            lam = cfg_get(cfg, "mult_res_lambda", 1.0)
            v_in = lam * u + torch.sigmoid(_hi(_lin(xhat, sd, "v_gate", bias=True))).to(u.dtype) \
                * torch.tanh(_lin(u, sd, "v_map"))
        elif mod == "fusion":                                          # :341-342
            v_in = u + F.silu(_lin(g_in, sd, "v_pre"))
        elif mod == "linear":
            v_in = u                                                   # :359-360
        else:
            raise NotImplementedError(f"ctx_mod={mod!r}")
        v_ctx = _lin(v_in, sd, "w_vctx")                               # :361
        if cfg_get(cfg, "v_ctx_norm", "none") == "rms":
            v_ctx = _head_rms(v_ctx, sd["ctx_gain"], h, dh)
        nvr = cfg_get(cfg, "kmod_vraw_heads", 0)
        kmode = cfg_get(cfg, "kmod_mode", "raw")
        if nvr > 0 and kmode == "gated_norm":                          # :364-371
            dcut = nvr * dh
            v_ctx = torch.cat([torch.zeros_like(v_ctx[..., :dcut]), v_ctx[..., dcut:]], dim=-1)
        vpp = _blend(_lin(g_in, sd, "w_gv", bias=True), v_raw, v_ctx)  # :372
        if nvr > 0 and kmode == "raw":                                 # :373-383
            dcut = nvr * dh
            raw = v_raw[..., :dcut]
            if cfg_get(cfg, "kmod_vraw_bound", "none") == "tanh":
                raw = torch.tanh(_hi(raw)).to(raw.dtype)
            vpp = torch.cat([raw, vpp[..., dcut:]], dim=-1)
        tau = cfg_get(cfg, "v_clamp_tau", 0.0)                        # :389-402
        if tau and tau > 0:
            shp = vpp.shape
            vh = _hi(vpp.reshape(*shp[:-1], h, dh))
            n = vh.norm(dim=-1, keepdim=True)
            vpp = (vh * (tau / n.clamp_min(1e-20)).clamp(max=1.0)).to(vpp.dtype).reshape(shp)
    return kpp, vpp


# ---------------------------------------------------------------------------
# exact sequential scan — models/dualmod/scan.py
# ---------------------------------------------------------------------------

def _projections(cfg, sd, xhat, cos, sin):
    """scan.py:66-69 — q_r, k (unrotated), k_self_r, v, per head."""
    h = cfg.n_heads
    q_r = apply_rope(split_heads(_lin(xhat, sd, "wq"), h), cos, sin)
    k = split_heads(_lin(xhat, sd, "wk"), h)
    k_self_r = apply_rope(k, cos, sin)
    v = split_heads(project_v(cfg, sd, xhat), h)
    return q_r, k, k_self_r, v


def _scan_chunk(cfg, sd, xhat_c, q_r_c, k_c, k_self_r_c, v_c, cos_c, sin_c,
                K_past, V_past):
    """scan.py:19-57 — per-position loop over one chunk."""
    Tc = xhat_c.shape[1]
    new_K, new_V, o_list = [], [], []
    for j in range(Tc):
        K_cur = torch.cat([K_past] + new_K, dim=2) if new_K else K_past
        V_cur = torch.cat([V_past] + new_V, dim=2) if new_V else V_past
        o_j = attend_one(cfg, q_r_c[:, :, j:j + 1], k_self_r_c[:, :, j:j + 1],
                         v_c[:, :, j:j + 1], K_cur, V_cur)
        o_cat = merge_heads(o_j)
        kpp, vpp = refine_kv(cfg, sd, xhat_c[:, j:j + 1], o_cat,
                             merge_heads(k_c[:, :, j:j + 1]), merge_heads(v_c[:, :, j:j + 1]))
        new_K.append(apply_rope(split_heads(kpp, cfg.n_heads), cos_c[j:j + 1], sin_c[j:j + 1]))
        new_V.append(split_heads(vpp, cfg.n_heads))
        o_list.append(o_j)
    return torch.cat(o_list, dim=2), torch.cat(new_K, dim=2), torch.cat(new_V, dim=2)


def sequential_scan(cfg, sd, xhat, cos, sin, return_cache=False):
    """scan.py:60-95 — exact scan. Returns o_cat [B,T,d] (pre-W_O); with
    ``return_cache`` also the refined, rotated K and V rows [B,h,T,dh]."""
    B, T, d = xhat.shape
    h = cfg.n_heads
    q_r, k, k_self_r, v = _projections(cfg, sd, xhat, cos[:T], sin[:T])
    K_past = q_r.new_zeros(B, h, 0, d // h)
    V_past = v.new_zeros(B, h, 0, d // h)
    o, K_new, V_new = _scan_chunk(cfg, sd, xhat, q_r, k, k_self_r, v,
                                  cos[:T], sin[:T], K_past, V_past)
    o_cat = merge_heads(o)
    return (o_cat, K_new, V_new) if return_cache else o_cat


# ---------------------------------------------------------------------------
# chunked Jacobi cell — engines/wavescan/cells/scan_cell_fwd.py
# ---------------------------------------------------------------------------

def make_intra_mask(c, dtype=torch.float32):
    """scan_cell_fwd.py:56-60 — [c,c] additive mask, diagonal and above blocked."""
    m = torch.full((c, c), torch.finfo(torch.float32).min, dtype=dtype)
    return m.triu(0)


def _window_masks(c, P, W, device, dtype):
    """attend_one's window (attention.py:291-293: the last W-1 rows before a token, plus
    itself) on a cell's reads: chunk row p (position P + p) keeps committed key j iff
    j >= P + p - W + 1 and intra row j' iff p - j' <= W - 1. Additive masks [c, P], [c, c]."""
    neg = torch.finfo(torch.float32).min
    p = torch.arange(c, device=device)[:, None]
    mc = torch.zeros(c, P, device=device, dtype=dtype)
    mc = mc.masked_fill(torch.arange(P, device=device)[None, :] < P + p - W + 1, neg)
    mi = torch.zeros(c, c, device=device, dtype=dtype)
    mi = mi.masked_fill(p - torch.arange(c, device=device)[None, :] > W - 1, neg)
    return mc, mi


def chunk_attend(q_r, k_self_r, v_raw, K_comm, V_comm, K_intra, V_intra,
                 intra_mask, scale, window=0):
    """scan_cell_fwd.py:63-85 — [committed | intra (strict lower) | raw self]. window > 1:
    attend_one's local window on the committed and intra reads (_window_masks); with K = c
    sweeps the cell then equals the windowed sequential scan (scan.py over attend_one).
    window = 1 reads like no window, as attend_one does: its K_past[:, :, -(W - 1):] is
    K_past[:, :, -0:], the whole past (attention.py:292-293)."""
    c = q_r.shape[2]
    P = 0 if K_comm is None else K_comm.shape[2]
    s_intra = _hi(q_r @ K_intra.transpose(-1, -2) * scale)
    s_intra = s_intra + intra_mask.to(device=s_intra.device, dtype=s_intra.dtype)
    if window > 1:
        mc, mi = _window_masks(c, P, window, s_intra.device, s_intra.dtype)
        s_intra = s_intra + mi
    s_self = _hi((q_r * k_self_r).sum(-1, keepdim=True)) * scale
    if K_comm is not None and K_comm.shape[2] > 0:
        s_comm = _hi(q_r @ K_comm.transpose(-1, -2) * scale)
        if window > 1:
            s_comm = s_comm + mc
        scores = torch.cat([s_comm, s_intra, s_self], dim=-1)
    else:
        scores = torch.cat([s_intra, s_self], dim=-1)
    p = torch.softmax(scores, dim=-1).to(v_raw.dtype)
    p_rows, p_self = p[..., :-1], p[..., -1:]
    if V_comm is not None and V_comm.shape[2] > 0:
        v_all = torch.cat([V_comm, V_intra], dim=2)
    else:
        v_all = V_intra
    return p_rows @ v_all + p_self * v_raw


def chunk_cell_forward(cfg, sd, xhat_c, cos_c, sin_c, K_comm, V_comm, n_sweeps):
    """scan_cell_fwd.py:88-116 — K Jacobi sweeps over one chunk.

    Sweep 0 reads the chunk's RAW intra rows; every sweep reads committed +
    previous-sweep intra rows + the raw self column. Returns (o_cat [B,c,d],
    K_rows [B,h,c,dh] rotated, V_rows [B,h,c,dh])."""
    c = xhat_c.shape[1]
    h = cfg.n_heads
    dh = xhat_c.shape[-1] // h
    mask = make_intra_mask(c)
    q_r = apply_rope(split_heads(_lin(xhat_c, sd, "wq"), h), cos_c, sin_c)
    k_flat = _lin(xhat_c, sd, "wk")
    v_flat = project_v(cfg, sd, xhat_c)
    k_self_r = apply_rope(split_heads(k_flat, h), cos_c, sin_c)
    v_raw = split_heads(v_flat, h)
    K_intra, V_intra = k_self_r, v_raw
    o_cat = None
    W = cfg_get(cfg, "local_window", 0) or 0
    for _ in range(n_sweeps):
        o = chunk_attend(q_r, k_self_r, v_raw, K_comm, V_comm, K_intra, V_intra,
                         mask, 1.0 / math.sqrt(dh), window=W)
        o_cat = merge_heads(o)
        kpp, vpp = refine_kv(cfg, sd, xhat_c, o_cat, k_flat, v_flat)
        K_intra = apply_rope(split_heads(kpp, h), cos_c, sin_c)
        V_intra = split_heads(vpp, h)
    return o_cat, K_intra, V_intra


def uniform_chunks(T, c, n_sweeps=None):
    """engines/wavescan/engine/schedule.py:63-69."""
    cells = []
    for pos in range(0, T, c):
        cc = min(c, T - pos)
        cells.append((pos, cc, cc if n_sweeps is None else min(n_sweeps, cc)))
    return cells


def exact_sequential(T):
    """engines/wavescan/engine/schedule.py:58-60."""
    return [(j, 1, 1) for j in range(T)]


def layer_forward(cfg, sd, xhat, cos, sin, schedule):
    """engines/wavescan/engine/forward.py:95-113, written functionally
    (cat-grown cache, no in-place) so autograd runs through it — the same
    construction the reference uses as the K<c gradient oracle
    (engines/wavescan/tests/test_k1_k9.py:253-270).
    Returns (o_cat [B,T,d], K [B,h,T,dh], V [B,h,T,dh])."""
    B, T, d = xhat.shape
    h = cfg.n_heads
    K = xhat.new_zeros(B, h, 0, d // h)
    V = xhat.new_zeros(B, h, 0, d // h)
    outs = []
    for pos0, c, n_sweeps in schedule:
        o_cat, K_rows, V_rows = chunk_cell_forward(
            cfg, sd, xhat[:, pos0:pos0 + c], cos[pos0:pos0 + c], sin[pos0:pos0 + c],
            K, V, n_sweeps)
        K = torch.cat([K, K_rows], dim=2)
        V = torch.cat([V, V_rows], dim=2)
        outs.append(o_cat)
    return torch.cat(outs, dim=1), K, V


def dm_layer(cfg, sd, x, cos, sin, schedule=None, attn_norm_w=None):
    """The attention sublayer of Block.forward (models/dualmod/model.py:123-124):
    y = x + wo(DM(attn_norm(x))). ``schedule=None`` runs the exact sequential
    scan (scan.py), else the chunked Jacobi layer."""
    w = attn_norm_w if attn_norm_w is not None else sd["attn_norm.weight"]
    xhat = rms_norm(x, w, 1e-5)
    if schedule is None:
        o_cat = sequential_scan(cfg, sd, xhat, cos, sin)
    else:
        o_cat = layer_forward(cfg, sd, xhat, cos, sin, schedule)[0]
    return x + _lin(o_cat, sd, "wo")


# ---------------------------------------------------------------------------
# decode — attention.py:564-588 and lm/eval/graph_decode.py:33-51
# ---------------------------------------------------------------------------

def decode_step(cfg, sd, xhat_j, pos, cache, cos, sin):
    """attention.py:564-588 — one token at absolute position ``pos``.

    cache: {"K": [B,h,P,dh] | None, "V": ...}, appended in place (cat).
    Returns (o_cat [B,1,d], wo(o_cat) [B,1,d])."""
    h = cfg.n_heads
    q = split_heads(_lin(xhat_j, sd, "wq"), h)
    k = split_heads(_lin(xhat_j, sd, "wk"), h)
    v = split_heads(project_v(cfg, sd, xhat_j), h)
    cj, sj = cos[pos:pos + 1], sin[pos:pos + 1]
    q_r = apply_rope(q, cj, sj)
    k_self_r = apply_rope(k, cj, sj)
    o_j = attend_one(cfg, q_r, k_self_r, v, cache["K"], cache["V"])
    o_cat = merge_heads(o_j)
    kpp, vpp = refine_kv(cfg, sd, xhat_j, o_cat, merge_heads(k), merge_heads(v))
    kpp_r = apply_rope(split_heads(kpp, h), cj, sj)
    vpp_h = split_heads(vpp, h)
    if cache["K"] is None:
        cache["K"], cache["V"] = kpp_r, vpp_h
    else:
        cache["K"] = torch.cat([cache["K"], kpp_r], dim=2)
        cache["V"] = torch.cat([cache["V"], vpp_h], dim=2)
    return o_cat, _lin(o_cat, sd, "wo")


def static_decode_step(cfg, sd, xhat_j, pos, Kb, Vb, cos, sin):
    """lm/eval/graph_decode.py:33-51 — static-tape twin of decode_step:
    raw self pair into slot ``pos``, masked read over slots <= pos, refined
    pair overwrites slot ``pos``. Kb/Vb [B,h,P_max,dh] are updated in place.
    Returns o_cat [B,1,d]."""
    h = cfg.n_heads
    q = split_heads(_lin(xhat_j, sd, "wq"), h)
    k = split_heads(_lin(xhat_j, sd, "wk"), h)
    v = split_heads(project_v(cfg, sd, xhat_j), h)
    cj, sj = cos[pos:pos + 1], sin[pos:pos + 1]
    q_r = apply_rope(q, cj, sj)
    k_r = apply_rope(k, cj, sj)
    Kb[:, :, pos:pos + 1] = k_r.to(Kb.dtype)
    Vb[:, :, pos:pos + 1] = v.to(Vb.dtype)
    dh = q.shape[-1]
    s = (q_r.to(Kb.dtype) @ Kb[:, :, :pos + 1].transpose(-1, -2)) * (1.0 / math.sqrt(dh))
    a = torch.softmax(_hi(s), dim=-1)
    o = a.to(Vb.dtype) @ Vb[:, :, :pos + 1]
    o_cat = merge_heads(o).to(xhat_j.dtype)
    kpp, vpp = refine_kv(cfg, sd, xhat_j, o_cat, merge_heads(k), merge_heads(v))
    Kb[:, :, pos:pos + 1] = apply_rope(split_heads(kpp, h), cj, sj).to(Kb.dtype)
    Vb[:, :, pos:pos + 1] = split_heads(vpp, h).to(Vb.dtype)
    return o_cat


# ---------------------------------------------------------------------------
# the LLaMA-style trunk — models/dualmod/model.py:102-131, 267-291
# ---------------------------------------------------------------------------

def swiglu(sd, x, prefix="mlp."):
    """model.py:111-112: w2(silu(w1 x) * w3 x)."""
    def lin(t, n):
        w = sd[prefix + n + ".weight"]
        return t.to(w.dtype) @ w.t()
    return lin(F.silu(lin(x, "w1")) * lin(x, "w3"), "w2")


def _block_sd(sd, l):
    pre = f"blocks.{l}."
    return {k[len(pre):]: v for k, v in sd.items() if k.startswith(pre)}


def _attn_sd(bsd):
    return {k[len("attn."):]: v for k, v in bsd.items() if k.startswith("attn.")}


def lm_forward(cfg, sd, idx, cos, sin, schedule=None):
    """model.py:267-281 with the exact sequential scan per layer (Block.forward,
    model.py:123-125): logits [B, T, V]. ``sd`` holds the LM's parameter names
    (tok_emb.weight, blocks.{l}.attn.*, blocks.{l}.mlp.w1..., norm_f.weight, lm_head.weight).
    ``schedule`` runs each layer's attention as the chunked Jacobi layer instead (the
    engine's forward, engines/wavescan/engine/forward.py:95-113)."""
    x = sd["tok_emb.weight"][idx]
    for l in range(cfg.n_layers):
        b = _block_sd(sd, l)
        xhat = rms_norm(x, b["attn_norm.weight"], 1e-5)
        if schedule is None:
            o = sequential_scan(cfg, _attn_sd(b), xhat, cos, sin)
        else:
            o = layer_forward(cfg, _attn_sd(b), xhat, cos, sin, schedule)[0]
        x = x + _lin(o, _attn_sd(b), "wo")
        x = x + swiglu(b, rms_norm(x, b["mlp_norm.weight"], 1e-5))
    w = sd.get("lm_head.weight", sd["tok_emb.weight"])
    return rms_norm(x, sd["norm_f.weight"], 1e-5) @ w.t()


def lm_decode_step(cfg, sd, idx_j, pos, caches, cos, sin):
    """model.py:285-291 with Block.decode_step (model.py:127-130): one token per row at
    position ``pos``; caches: one {"K", "V"} dict per layer (decode_step's cat cache).
    Returns logits [B, 1, V]."""
    x = sd["tok_emb.weight"][idx_j]
    for l in range(cfg.n_layers):
        b = _block_sd(sd, l)
        xhat = rms_norm(x, b["attn_norm.weight"], 1e-5)
        x = x + decode_step(cfg, _attn_sd(b), xhat, pos, caches[l], cos, sin)[1]
        x = x + swiglu(b, rms_norm(x, b["mlp_norm.weight"], 1e-5))
    w = sd.get("lm_head.weight", sd["tok_emb.weight"])
    return rms_norm(x, sd["norm_f.weight"], 1e-5) @ w.t()


# ---------------------------------------------------------------------------
# vanilla causal attention — attention.py:452-483 (T1/T2 oracle)
# ---------------------------------------------------------------------------

def vanilla_attention(cfg, sd, xhat, cos, sin):
    """attention.py:452-483 (no window, no logn): SDPA over raw rotated keys.
    Returns o_cat [B,T,d] (pre-W_O)."""
    h = cfg.n_heads
    q = apply_rope(split_heads(_lin(xhat, sd, "wq"), h), cos, sin)
    k = apply_rope(split_heads(_lin(xhat, sd, "wk"), h), cos, sin)
    v = split_heads(project_v(cfg, sd, xhat), h)
    o = F.scaled_dot_product_attention(q, k, v, is_causal=True)
    return merge_heads(o)
