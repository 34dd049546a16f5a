"""CPU checks of the C ABI: the library loads, exports every symbol declared in
include/dm_abi.h, and rejects bad arguments before touching a device."""

import ctypes
import os
import re

import pytest
import torch

from dual_mod_public_amd import _lib as L
from dual_mod_public_amd.config import DualModConfig

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    src = open(os.path.join(REPO, "include", "dm_abi.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(dm_[a-z0-9_]+)\s*\(", src)))


def test_every_declared_symbol_is_exported_and_bound():
    lib = L.load()
    names = declared_symbols()
    assert len(names) >= 10
    for n in names:
        assert hasattr(lib, n), n
        assert n in L.SIGNATURES, f"{n} has no ctypes signature"
    assert set(L.SIGNATURES) == set(names)


def test_abi_version():
    assert L.load().dm_abi_version() == 7


def _conf(**kw):
    cfg = DualModConfig(d_model=256, n_heads=4, ctx_mod="mult_res")
    import torch
    c = L.make_config(cfg, 2, torch.float32)
    for k, v in kw.items():
        setattr(c, k, v)
    return c


def test_rejects_bad_config_without_device():
    lib = L.load()
    c = _conf(dh=32, h=8)           # d == h*dh but head_dim 32 unsupported
    assert lib.dm_cell_workspace_bytes(ctypes.byref(c), 64) == 0
    c = _conf(d=250)
    rc = lib.dm_layer_proj(ctypes.byref(c), None, None, None, None, None, None)
    assert rc == -1
    assert b"d=250" in lib.dm_last_error()


def test_rejects_null_and_bad_shapes():
    lib = L.load()
    c = _conf()
    a = L.dm_cell_args()
    a.c = 65
    rc = lib.dm_cell_fwd(ctypes.byref(c), None, None, None, None, ctypes.byref(a), None)
    assert rc == -1 and b"null packed" in lib.dm_last_error()
    assert lib.dm_gemm(0, 0, 0, None, None, None, 128, 128, 64, 0, None) == -1
    assert lib.dm_linear(0, 1, 1, None, 1, 64, 100, 64, None) == -1
    # dm_swiglu_rows: null operands, more than 64 rows, d not a multiple of 128, fp32 (unsupported)
    assert lib.dm_swiglu_rows(1, None, 16, 16, 16, 16, 16, 8, 1024, 2816, None) == -1
    assert lib.dm_swiglu_rows(1, 16, 16, 16, 16, 16, 16, 65, 1024, 2816, None) == -1
    assert lib.dm_swiglu_rows(1, 16, 16, 16, 16, 16, 16, 8, 1000, 2816, None) == -1
    assert lib.dm_swiglu_rows(0, 16, 16, 16, 16, 16, 16, 8, 1024, 2816, None) == -2


def test_workspace_query():
    lib = L.load()
    c = _conf()
    n1 = lib.dm_cell_workspace_bytes(ctypes.byref(c), 64)
    n2 = lib.dm_cell_workspace_bytes(ctypes.byref(c), 4096)
    assert 0 < n1 < n2
    assert lib.dm_decode_workspace_bytes(ctypes.byref(c), 32768) > 0


def test_unsupported_knobs_raise():
    from dual_mod_public_amd.engine import check_supported
    for kw in (dict(gate_type_v="independent"), dict(ctx_mod="vmlp"), dict(attn_logn_ref=64)):
        cfg = DualModConfig(d_model=256, n_heads=4, **kw)
        with pytest.raises(NotImplementedError):
            check_supported(cfg)
    check_supported(DualModConfig(d_model=256, n_heads=4, ctx_mod="mult_res"))
    # implemented knobs: kmod heads (every mode), factored gates / ctx operators
    for kw in (dict(kmod_vraw_heads=1), dict(kmod_vraw_heads=2, kmod_vraw_bound="tanh"),
               dict(kmod_vraw_heads=1, kmod_mode="gated_norm"), dict(gate_rank=8, ctx_rank=16)):
        check_supported(DualModConfig(d_model=256, n_heads=4, ctx_mod="mult_res", **kw))
    check_supported(DualModConfig(d_model=256, n_heads=4, ctx_mod="fusion"))
    check_supported(DualModConfig(d_model=256, n_heads=4, ctx_mod="mult_res", v_clamp_tau=1.0))
    # per-head RMS norms (attention.py:218-269)
    for kw in (dict(k_ctx_norm="rms"), dict(v_norm="rms"), dict(v_ctx_norm="rms")):
        check_supported(DualModConfig(d_model=256, n_heads=4, ctx_mod="mult_res", **kw))


def test_norm_config_bits():
    """The head-norm knobs reach dm_config.norms; the library rejects unknown bits."""
    import torch
    cfg = DualModConfig(d_model=256, n_heads=4, k_ctx_norm="rms", v_norm="rms")
    c = L.make_config(cfg, 2, torch.float32)
    assert c.norms == L.DM_NORM_K_CTX | L.DM_NORM_V
    assert L.make_config(DualModConfig(d_model=256, n_heads=4), 2, torch.float32).norms == 0
    lib = L.load()
    assert lib.dm_cell_workspace_bytes(ctypes.byref(c), 64) > 0
    c.norms = 8
    assert lib.dm_cell_workspace_bytes(ctypes.byref(c), 64) == 0


def test_kmod_config_fields():
    """The kmod knob reaches dm_config (and is validated by the library)."""
    c = L.make_config(DualModConfig(d_model=256, n_heads=4, kmod_vraw_heads=2, kmod_mode="gated_norm"), 2,
                      __import__("torch").float32)
    assert (c.kmod_vraw_heads, c.kmod_mode) == (2, 2)
    c = L.make_config(DualModConfig(d_model=256, n_heads=4, kmod_vraw_heads=1, kmod_vraw_bound="tanh"), 2,
                      __import__("torch").float32)
    assert (c.kmod_vraw_heads, c.kmod_mode) == (1, 1)
    c.kmod_vraw_heads = 5   # more kmod heads than heads: rejected by the library
    assert L.load().dm_cell_workspace_bytes(c, 64) == 0


def test_training_entry_points_reject_a_negative_window():
    """dm_layer_fwd (tape and recompute forms) and dm_layer_bwd reject local_window < 0 with
    DM_ERR_INVALID before any launch (the checks run on the host; the placeholder pointers below
    are never dereferenced)."""
    lib = L.load()
    c = _conf(local_window=-1)
    fake = ctypes.c_void_p(1 << 20)   # non-null, 16-byte aligned, never dereferenced
    w = L.dm_packed()
    for f in ("w_proj", "b_proj", "w_sweep", "w_vctx", "norm_ctx_w", "attn_norm_w", "wo", "w_proj_t",
              "w_sweep_t", "w_vctx_t", "wo_t"):
        setattr(w, f, fake.value)
    b = L.dm_layer_bufs()
    b.T = 64
    for f in ("xhat", "qr", "kraw", "kself", "vraw", "glogx", "sig"):
        setattr(b, f, fake.value)
    sched = (ctypes.c_int32 * 3)(0, 64, 4)
    g = L.dm_grads()
    for f, _ in L.GRAD_FIELDS:
        setattr(g, f, fake.value)
    for tape in (None, fake):
        rc = lib.dm_layer_fwd(ctypes.byref(c), ctypes.byref(w), fake, fake, fake, fake, ctypes.byref(b), sched, 1,
                              fake, fake, 64, fake, tape, 1 << 30, fake, 1 << 30, None)
        assert rc == -1 and b"local_window" in lib.dm_last_error()
    rc = lib.dm_layer_bwd(ctypes.byref(c), ctypes.byref(w), fake, fake, fake, fake, fake, ctypes.byref(b), sched, 1,
                          fake, fake, 64, fake, None, 0, ctypes.byref(g), fake, 1 << 30, None)
    assert rc == -1 and b"local_window" in lib.dm_last_error()


def test_training_windows_pass_host_checks():
    """Any W >= 1 is a training configuration (the committed-prefix and intra-cell attention mask
    keys below i - W + 1): the layer-batched forward's plan query, which runs every host check of
    the training entry points and launches nothing, accepts W = 1, 8 and 100 with 64-row cells and
    refuses W = -1 (the placeholder pointers are never dereferenced)."""
    lib = L.load()
    fake = ctypes.c_void_p(1 << 20)
    w = L.dm_packed()
    for f in ("w_proj", "b_proj", "w_sweep", "w_vctx", "norm_ctx_w", "attn_norm_w", "wo", "w_proj_t",
              "w_sweep_t", "w_vctx_t", "wo_t"):
        setattr(w, f, fake.value)
    b = L.dm_layer_bufs()
    b.T = 256
    for f in ("xhat", "qr", "kraw", "kself", "vraw", "glogx", "sig"):
        setattr(b, f, fake.value)
    ly = (L.dm_stack_layer * 1)()
    ly[0].w, ly[0].bufs = ctypes.addressof(w), ctypes.addressof(b)
    for f in ("x", "y", "K_cache", "V_cache", "ocat", "workspace"):
        setattr(ly[0], f, fake.value)
    ly[0].workspace_bytes = 1 << 34
    sched = (ctypes.c_int32 * 12)(0, 64, 4, 64, 64, 4, 128, 64, 4, 192, 64, 4)
    for W in (1, 8, 100):
        ok = _conf(local_window=W)
        assert lib.dm_stack_fwd_plan_bytes(ctypes.byref(ok), 1, ly, sched, 4, 256) > 0, lib.dm_last_error()
    bad = _conf(local_window=-1)
    assert lib.dm_stack_fwd_plan_bytes(ctypes.byref(bad), 1, ly, sched, 4, 256) == 0
    assert b"local_window" in lib.dm_last_error()


def test_attend_one_refine_kv_refuse_autograd():
    """The HIP attend_one / refine_kv build no autograd graph: a call that would need gradients
    raises (before any library call) instead of returning a result without them."""
    import torch
    from dual_mod_public_amd.attention import DualModAttention
    cfg = DualModConfig(d_model=256, n_heads=4, ctx_mod="mult_res")
    attn = DualModAttention(cfg)
    q = torch.zeros(1, 4, 1, 64, requires_grad=True)
    with pytest.raises(NotImplementedError, match="forward-only"):
        attn.attend_one(q, q, q, None, None)
    x = torch.zeros(1, 2, 256)
    with pytest.raises(NotImplementedError, match="forward-only"):   # the module's parameters need grads
        attn.refine_kv(x, x, x, x)


def test_lm_state_dict_loads_into_model():
    """DualModLM carries the reference's parameter names (models/dualmod/model.py:134-150):
    a synthetic LM state dict loads strictly, the head is tied to the embedding, and every
    attention parameter sits where DualModAttention reads it."""
    from dual_mod_public_amd.model import DualModLM
    from dual_mod_public_amd.synthetic import make_lm_state_dict
    cfg = DualModConfig(d_model=128, n_heads=2, n_layers=2, vocab_size=64, max_seq_len=32,
                        mlp_hidden_override=192, ctx_mod="mult_res", v_norm="rms")
    sd = make_lm_state_dict(cfg, seed=1)
    m = DualModLM(cfg)
    m.load_state_dict(sd, strict=True)
    assert m.lm_head.weight is m.tok_emb.weight
    assert torch.equal(m.blocks[1].attn.w_gk.bias, sd["blocks.1.attn.w_gk.bias"])
    assert torch.equal(m.blocks[0].mlp.w2.weight, sd["blocks.0.mlp.w2.weight"])
    assert set(m.state_dict()) == set(sd)
