"""GPU parity of the reference-shaped callables on the HIP kernels:
DualModAttention.attend_one / refine_kv (models/dualmod/attention.py:283-434, via
dm_attend_one / dm_refine_kv) and engine.chunk_cell_forward
(engines/wavescan/cells/scan_cell_fwd.py:88-116, chunk-local dm_cell_fwd: only the chunk
is projected and the committed prefix is read in place), each against the oracle in fp64;
and the exact scan written as the reference's own per-position loop over attend_one +
refine_kv (models/dualmod/scan.py:19-57). fp32 bar 1e-5 relative."""

import pytest
import torch

import oracle as O
from dual_mod_public_amd import _lib as L
from dual_mod_public_amd.attention import DualModAttention
from dual_mod_public_amd.engine import chunk_cell_forward
from tests.hip_helpers import DEV, cfg_of, record, relerr, say, setup

pytestmark = pytest.mark.gpu
TOL = 1e-5


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    L.load()


def _module(cfg, sd):
    attn = DualModAttention(cfg).to(DEV)
    attn.load_state_dict({k: v.float() for k, v in sd.items() if k != "attn_norm.weight"})
    return attn


@pytest.mark.parametrize("P", [0, 1, 100, 1500])
@pytest.mark.parametrize("W", [0, 37])
def test_attend_one(P, W):
    say(f"attend_one P={P} W={W}")
    cfg = cfg_of(local_window=W)
    sd, _, _, _ = setup(cfg, 1, 8)
    attn = _module(cfg, sd)
    g = torch.Generator().manual_seed(P + W)
    B, h, dh, T = 2, 4, 64, 1600
    q, ks, vs = (torch.randn(B, h, 1, dh, generator=g, dtype=torch.float64) for _ in range(3))
    cache = torch.randn(2, B, h, T, dh, generator=g, dtype=torch.float64)
    Kd, Vd = cache[0].float().to(DEV), cache[1].float().to(DEV)
    with torch.no_grad():
        o, probs = attn.attend_one(q.float().to(DEV), ks.float().to(DEV), vs.float().to(DEV),
                                   Kd[:, :, :P] if P else None, Vd[:, :, :P] if P else None)
    torch.cuda.synchronize()
    assert probs is None
    ref = O.attend_one(cfg, q, ks, vs, cache[0][:, :, :P] if P else None, cache[1][:, :, :P] if P else None)
    e = relerr(o, ref)
    record(f"attend_one P={P} W={W}", {"o": e}, TOL)
    assert e < TOL


@pytest.mark.parametrize("ctx_mod,kw", [("mult_res", {}), ("linear", {}), ("fusion", {}), ("mult", {}),
                                        ("mult_res", dict(kmod_vraw_heads=1, kmod_vraw_bound="tanh")),
                                        ("linear", dict(kmod_vraw_heads=2, kmod_mode="gated_norm")),
                                        ("mult_res", dict(v_clamp_tau=0.5))])
@pytest.mark.parametrize("t", [1, 5, 64, 100])
def test_refine_kv(ctx_mod, kw, t):
    say(f"refine_kv {ctx_mod} {kw} t={t}")
    cfg = cfg_of(ctx_mod=ctx_mod, **kw)
    sd, x, _, _ = setup(cfg, 2, t)
    attn = _module(cfg, sd)
    g = torch.Generator().manual_seed(t)
    o_cat, k_raw, v_raw = (torch.randn(2, t, cfg.d_model, generator=g, dtype=torch.float64) for _ in range(3))
    with torch.no_grad():
        k, v = attn.refine_kv(*(z.float().to(DEV) for z in (x, o_cat, k_raw, v_raw)))
    torch.cuda.synchronize()
    k_ref, v_ref = O.refine_kv(cfg, sd, x, o_cat, k_raw, v_raw)
    errs = {"k": relerr(k, k_ref), "v": relerr(v, v_ref)}
    record(f"refine_kv {ctx_mod} {kw} t={t}", errs, TOL)
    assert max(errs.values()) < TOL, errs


@pytest.mark.parametrize("a,c,k", [(0, 16, 16), (64, 16, 4), (100, 64, 3), (37, 27, 27)])
def test_chunk_cell_forward_reads_prefix_in_place(a, c, k):
    say(f"chunk_cell_forward a={a} c={c} K={k}")
    cfg = cfg_of(T=a + c + 8)
    sd, x, (c64, s64), (c32, s32) = setup(cfg, 2, a + c)
    attn = _module(cfg, sd)
    g = torch.Generator().manual_seed(a + c)
    h, dh = 4, 64
    # the committed prefix: the first a rows of a larger cache (read through the view, not copied)
    cache = torch.randn(2, 2, h, a + c + 8, dh, generator=g, dtype=torch.float64) * 0.5
    Kd, Vd = cache[0].float().to(DEV), cache[1].float().to(DEV)
    before = (Kd.clone(), Vd.clone())
    xc = x[:, a:a + c]
    o, K_rows, V_rows = chunk_cell_forward(attn, xc.float().to(DEV), c32[a:a + c].to(DEV), s32[a:a + c].to(DEV),
                                           Kd[:, :, :a] if a else None, Vd[:, :, :a] if a else None, k)
    torch.cuda.synchronize()
    assert torch.equal(Kd, before[0]) and torch.equal(Vd, before[1])   # committed rows untouched
    ref = O.chunk_cell_forward(cfg, sd, xc, c64[a:a + c], s64[a:a + c], cache[0][:, :, :a], cache[1][:, :, :a], k)
    errs = {"o": relerr(o, ref[0]), "K": relerr(K_rows, ref[1]), "V": relerr(V_rows, ref[2])}
    record(f"chunk_cell_forward a={a} c={c} K={k}", errs, TOL)
    assert max(errs.values()) < TOL, errs


def test_scan_loop_of_attend_one_and_refine_kv():
    """models/dualmod/scan.py:19-57 written with the module's own attend_one / refine_kv on the
    GPU, position by position, equals the oracle's sequential scan."""
    say("scan loop of attend_one + refine_kv")
    cfg = cfg_of(T=24)
    B, T = 2, 24
    sd, x, (c64, s64), (c32, s32) = setup(cfg, B, T)
    attn = _module(cfg, sd)
    h, dh = 4, 64
    xd = x.float().to(DEV)
    cos, sin = c32.to(DEV), s32.to(DEV)
    split = lambda z: z.view(B, -1, h, dh).transpose(1, 2)   # noqa: E731

    def rope(z, j):
        z1, z2 = z[..., :dh // 2], z[..., dh // 2:]
        c, s = cos[j], sin[j]
        return torch.cat([z1 * c - z2 * s, z2 * c + z1 * s], -1)

    with torch.no_grad():
        q = split(xd @ attn.wq.weight.t())
        kr = xd @ attn.wk.weight.t()
        vr = xd @ attn.wv.weight.t()
        Ks, Vs, outs = [], [], []
        for j in range(T):
            Kp = torch.cat(Ks, 2) if Ks else None
            Vp = torch.cat(Vs, 2) if Vs else None
            o, _ = attn.attend_one(rope(q[:, :, j:j + 1], j), rope(split(kr[:, j:j + 1]), j), split(vr[:, j:j + 1]),
                                   Kp, Vp)
            o_cat = o.transpose(1, 2).reshape(B, 1, -1)
            kpp, vpp = attn.refine_kv(xd[:, j:j + 1], o_cat, kr[:, j:j + 1], vr[:, j:j + 1])
            Ks.append(rope(split(kpp), j).contiguous())
            Vs.append(split(vpp).contiguous())
            outs.append(o_cat)
    torch.cuda.synchronize()
    o_ref, K_ref, V_ref = O.sequential_scan(cfg, sd, x, c64, s64, return_cache=True)
    errs = {"o": relerr(torch.cat(outs, 1), o_ref), "K": relerr(torch.cat(Ks, 2), K_ref),
            "V": relerr(torch.cat(Vs, 2), V_ref)}
    record("scan loop attend_one + refine_kv", errs, TOL)
    assert max(errs.values()) < TOL, errs
