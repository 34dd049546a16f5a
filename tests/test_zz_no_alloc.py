"""dm_decode_step_noalloc (the decode step that allocates nothing: workspace in the
library's static device scratch) against dm_decode_step with a caller workspace, called
through the C ABI: two calls in a row, the second with a smaller input (fewer batch rows,
shorter tape), each compared bit for bit (the same kernels on the same inputs), plus the
rejection of a step whose scratch would exceed the static array."""

import ctypes

import pytest
import torch

from dual_mod_public_amd import _lib as L
from dual_mod_public_amd.config import DualModConfig
from dual_mod_public_amd.engine import PackedWeights
from dual_mod_public_amd.rope import build_rope_cache
from dual_mod_public_amd.synthetic import make_state_dict

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    L.load()


def _args(pos, tape_T, xhat, K, V, o_cat, y, ws=None):
    a = L.dm_decode_args()
    a.pos, a.tape_T = pos, tape_T
    a.xhat, a.K_tape, a.V_tape = L.ptr(xhat), L.ptr(K), L.ptr(V)
    a.o_cat, a.y = L.ptr(o_cat), L.ptr(y)
    if ws is not None:
        a.workspace, a.workspace_bytes = L.ptr(ws), ws.numel()
    return a


def _one(cfg, B, tape_T, pos, seed):
    """One decode step both ways on identical copies of a random tape; returns both results."""
    dt = torch.bfloat16
    d, h, dh = cfg.d_model, cfg.n_heads, cfg.head_dim
    sd = make_state_dict(cfg, seed=seed, with_attn_norm=False)
    w = PackedWeights(cfg, torch.device(DEV), dt, with_transposes=False).pack({k: v.to(DEV) for k, v in sd.items()})
    g = torch.Generator(device=DEV).manual_seed(seed)
    K = torch.randn(B, h, tape_T, dh, generator=g, device=DEV).to(dt)
    V = torch.randn(B, h, tape_T, dh, generator=g, device=DEV).to(dt)
    xhat = torch.randn(B, d, generator=g, device=DEV).to(dt)
    cos, sin = build_rope_cache(tape_T, dh, cfg.rope_theta, device=DEV)
    cos, sin = cos.contiguous(), sin.contiguous()
    conf = L.make_config(cfg, B, dt)
    ws_bytes = L.lib().dm_decode_workspace_bytes(ctypes.byref(conf), tape_T)
    assert 0 < ws_bytes <= L.DM_DECODE_SCRATCH_MAX
    out = []
    for noalloc in (False, True):
        Kc, Vc = K.clone(), V.clone()
        o_cat, y = torch.empty(B, d, device=DEV, dtype=dt), torch.empty(B, d, device=DEV, dtype=dt)
        ws = None if noalloc else torch.empty(ws_bytes, device=DEV, dtype=torch.uint8)
        a = _args(pos, tape_T, xhat, Kc, Vc, o_cat, y, ws)
        fn = L.lib().dm_decode_step_noalloc if noalloc else L.lib().dm_decode_step
        L.check(fn(ctypes.byref(conf), ctypes.byref(w.struct(with_attn_norm=False)), L.ptr(cos), L.ptr(sin),
                   ctypes.byref(a), L.stream_ptr()))
        torch.cuda.synchronize()
        out.append((o_cat, y, Kc[:, :, pos].clone(), Vc[:, :, pos].clone()))
    return out


def test_noalloc_decode_equals_workspace_decode():
    cfg = DualModConfig(d_model=1024, n_heads=16, ctx_mod="mult_res", max_seq_len=8, dtype="bf16")
    # BASELINE config 5's step (64 rows over a 32768-row tape: 64 split partials), then a
    # smaller one (4 rows, 1000-row tape) that reuses the same scratch
    for B, tape_T, pos, seed in ((64, 32776, 32768, 3), (4, 1024, 1000, 4)):
        (o0, y0, k0, v0), (o1, y1, k1, v1) = _one(cfg, B, tape_T, pos, seed)
        assert torch.isfinite(o0.float()).all() and torch.isfinite(y0.float()).all()
        assert torch.equal(o0, o1), (B, tape_T)
        assert torch.equal(y0, y1), (B, tape_T)
        assert torch.equal(k0, k1) and torch.equal(v0, v1), (B, tape_T)


def test_noalloc_decode_rejects_oversized_step():
    cfg = DualModConfig(d_model=1024, n_heads=16, ctx_mod="mult_res", max_seq_len=8, dtype="bf16")
    conf = L.make_config(cfg, 64, torch.bfloat16)
    tape_T = 1 << 17   # 256 splits x 64 x 16 (b, h) partials: beyond the static scratch
    assert L.lib().dm_decode_workspace_bytes(ctypes.byref(conf), tape_T) > L.DM_DECODE_SCRATCH_MAX
    a = L.dm_decode_args()
    a.pos, a.tape_T = 5, tape_T
    rc = L.lib().dm_decode_step_noalloc(ctypes.byref(conf), None, None, None, ctypes.byref(a), None)
    assert rc == -3 and b"static scratch" in L.lib().dm_last_error()
