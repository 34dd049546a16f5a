"""GPU parity of the HIP reverse-scan backward (dm_layer_bwd) against autograd
through the CPU oracle.

The oracle's layer forward is written functionally (cat-grown caches), so torch
autograd through it is the reference's own gradient oracle for K < c
(engines/wavescan/tests/test_k1_k9.py:240-281) and, at K = c, autograd through the
sequential scan (the oracle's scan grads are pinned to the reference's golden
gradients in tests/test_oracle_golden.py). Tolerances: fp32 grads within 1e-5
relative (the reference's published exactness bar, README.md:203-204; measured
~1e-6), bf16 grads within 2e-2 relative of the fp64 oracle (measured <= 1.4e-2 at
the 340M shape, T=2048).
"""

import pytest
import torch

import oracle as O
from dual_mod_public_amd import _lib as L
from dual_mod_public_amd.autograd import dm_layer
from dual_mod_public_amd.engine import HipSweepCell, LayerGrads, uniform_chunks
from tests.hip_helpers import DEV, cfg_of, record, relerr, say, setup

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-5
BF16_TOL = 2e-2
BF16_FWD_TOL = 2e-2   # bf16 forward bar of BASELINE.json (2e-2 relative)


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    L.load()


def oracle_grads(cfg, sd, x, dy, cos, sin, sched, dtype=torch.float64, normalize=True, residual=True,
                 device="cpu", with_forward=False):
    """dx and parameter grads of y = [x +] W_O DM([attn_norm](x)) by autograd through the oracle
    (on the CPU, or with device="cuda" the same torch code on the GPU for the large shapes).
    with_forward also returns the forward's (o_cat, K, V)."""
    sdg = {k: v.to(device, dtype).clone().requires_grad_(True) for k, v in sd.items()}
    xg = x.to(device, dtype).clone().requires_grad_(True)
    with torch.enable_grad():
        if normalize:
            xh = O.rms_norm(xg, sdg["attn_norm.weight"], 1e-5)
        else:
            xh = xg
        o, K, V = O.layer_forward(cfg, sdg, xh, cos.to(device, dtype), sin.to(device, dtype), sched)
        y = O.dm_oracle._lin(o, sdg, "wo")
        if residual:
            y = y + xg
        (y * dy.to(device, dtype)).sum().backward()
    g = {k: v.grad for k, v in sdg.items() if v.grad is not None}
    if with_forward:
        return xg.grad, g, (o.detach(), K.detach(), V.detach())
    return xg.grad, g


def hip_grads(cfg, sd, x, dy, cos, sin, sched, dtype, normalize=True, residual=True, tape=False,
              full=False):
    B, T, d = x.shape
    cell = HipSweepCell(cfg, B, T, device=DEV, dtype=dtype)
    cell.pack({k: v.to(DEV, dtype) for k, v in sd.items()})
    bufs = cell.new_bufs(T)
    xd = x.to(DEV, dtype).contiguous()
    y = torch.empty_like(xd)
    K = torch.empty(B, cfg.n_heads, T, cfg.head_dim, device=DEV, dtype=dtype)
    V = torch.empty_like(K)
    ocat = torch.empty_like(xd)
    tp = cell.new_tape(sched) if tape else None
    cell.layer_forward(xd, y, cos, sin, sched, K, V, ocat, bufs, normalize=normalize, residual=residual,
                       tape=tp)
    grads = LayerGrads(cfg, DEV)
    dx = torch.empty_like(xd)
    cell.layer_backward(xd, dy.to(DEV, dtype).contiguous(), dx, cos, sin, sched, K, V, ocat, bufs, grads,
                        normalize=normalize, residual=residual, tape=tp)
    torch.cuda.synchronize()
    if full:
        return y, dx, grads, (K, V, ocat)
    return y, dx, grads


def compare(name, dx, g, dx_ref, g_ref, tol, skip=()):
    errs = {"x": relerr(dx, dx_ref)}
    for k, v in g_ref.items():
        if k in skip:
            continue
        errs[k] = relerr(g[k], v)
    worst = max(errs, key=errs.get)
    say(f"  {name}: worst {worst} {errs[worst]:.2e}; " +
        " ".join(f"{k.split('.')[0]}={v:.1e}" for k, v in errs.items()))
    record(name, errs, tol)
    for k, v in errs.items():
        assert v < tol, f"{k}: relerr {v:.3e} >= {tol} (all: {errs})"


@pytest.mark.parametrize("ctx_mod", ["mult_res", "linear", "mult", "fusion"])
@pytest.mark.parametrize("c,k", [(16, 16), (16, 4), (64, 4), (8, 3)])
def test_layer_grads_fp32(ctx_mod, c, k):
    """dm_layer_bwd vs autograd through the oracle (fp64), config-1 shape, fp32 storage."""
    say(f"bwd fp32 ctx_mod={ctx_mod} c={c} K={k}")
    cfg = cfg_of(ctx_mod=ctx_mod)
    B, T = 2, 64
    sd, x, (c64, s64), (c32, s32) = setup(cfg, B, T)
    dy = torch.randn(B, T, cfg.d_model, generator=torch.Generator().manual_seed(99), dtype=torch.float64)
    sched = uniform_chunks(T, c, k)
    _, dx, g = hip_grads(cfg, sd, x, dy, c32, s32, sched, torch.float32)
    dx_ref, g_ref = oracle_grads(cfg, sd, x, dy, c64, s64, sched)
    compare("fp32", dx, g, dx_ref, g_ref, FP32_TOL)


@pytest.mark.parametrize("taped", [False, True])
def test_layer_grads_fp32_batch3(taped):
    """B * h = 12 (attention-VJP blocks: one whole run of 16 role pairs plus a partial run)."""
    say(f"bwd fp32 B=3 taped={taped}")
    cfg = cfg_of()
    B, T = 3, 64
    sd, x, (c64, s64), (c32, s32) = setup(cfg, B, T)
    dy = torch.randn(B, T, cfg.d_model, generator=torch.Generator().manual_seed(97), dtype=torch.float64)
    sched = uniform_chunks(T, 16, 4)
    _, dx, g = hip_grads(cfg, sd, x, dy, c32, s32, sched, torch.float32, tape=taped)
    dx_ref, g_ref = oracle_grads(cfg, sd, x, dy, c64, s64, sched)
    compare("fp32 B=3", dx, g, dx_ref, g_ref, FP32_TOL)


@pytest.mark.parametrize("ctx_mod", ["mult_res", "linear", "fusion"])
def test_layer_grads_tape_fp32(ctx_mod):
    """Forward-saved tape instead of recompute: grads vs autograd through the oracle."""
    say(f"bwd fp32 tape ctx_mod={ctx_mod}")
    cfg = cfg_of(ctx_mod=ctx_mod)
    B, T = 2, 64
    sd, x, (c64, s64), (c32, s32) = setup(cfg, B, T)
    dy = torch.randn(B, T, cfg.d_model, generator=torch.Generator().manual_seed(98), dtype=torch.float64)
    sched = uniform_chunks(T, 16, 4)
    _, dx, g = hip_grads(cfg, sd, x, dy, c32, s32, sched, torch.float32, tape=True)
    dx_ref, g_ref = oracle_grads(cfg, sd, x, dy, c64, s64, sched)
    compare("fp32 tape", dx, g, dx_ref, g_ref, FP32_TOL)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("ctx_mod", ["mult_res", "linear", "mult", "fusion"])
@pytest.mark.parametrize("sched", [[(0, 16, 3), (16, 16, 1), (32, 7, 2), (39, 25, 4)], [(0, 64, 1)],
                                   [(0, 8, 8), (8, 56, 2)]])
def test_tape_equals_recompute(dtype, ctx_mod, sched):
    """Tape and exact recompute give bit-identical outputs, caches and gradients
    (deterministic kernels): the tape changes where the sweep states come from, not
    their values. Ragged, single-cell and K = c schedules."""
    say(f"tape == recompute {dtype} {ctx_mod} {sched}")
    cfg = cfg_of(ctx_mod=ctx_mod)
    B, T = 2, 64
    sd, x, _, (c32, s32) = setup(cfg, B, T)
    dy = torch.randn(B, T, cfg.d_model, generator=torch.Generator().manual_seed(5), dtype=torch.float64)
    y0, dx0, g0, st0 = hip_grads(cfg, sd, x, dy, c32, s32, sched, dtype, full=True)
    y1, dx1, g1, st1 = hip_grads(cfg, sd, x, dy, c32, s32, sched, dtype, tape=True, full=True)
    assert torch.equal(y0, y1)
    for a, b in zip(st0, st1):
        assert torch.equal(a, b)
    assert torch.equal(dx0, dx1)
    for name, t in g0.t.items():
        assert torch.equal(t, g1[name]), name


def test_tape_bytes_and_bounds():
    """dm_layer_tape_bytes grows with the schedule; an undersized tape is rejected."""
    cfg = cfg_of()
    B, T = 2, 64
    cell = HipSweepCell(cfg, B, T, device=DEV, dtype=torch.float32)
    a = cell.tape_bytes(uniform_chunks(T, 16, 2))
    b = cell.tape_bytes(uniform_chunks(T, 16, 4))
    assert 0 < a < b
    sd, x, _, (c32, s32) = setup(cfg, B, T)
    cell.pack({k: v.to(DEV, torch.float32) for k, v in sd.items()})
    bufs = cell.new_bufs(T)
    xd = x.float().to(DEV)
    y, ocat = torch.empty_like(xd), torch.empty_like(xd)
    K = torch.empty(B, cfg.n_heads, T, cfg.head_dim, device=DEV)
    V = torch.empty_like(K)
    small = torch.empty(a, device=DEV, dtype=torch.uint8)
    with pytest.raises(L.DMError, match="tape"):
        cell.layer_forward(xd, y, c32, s32, uniform_chunks(T, 16, 4), K, V, ocat, bufs, tape=small)


def test_layer_grads_no_norm_no_residual_fp32():
    """DualModAttention.forward's form: y = W_O DM(xhat)."""
    say("bwd fp32 no attn_norm, no residual")
    cfg = cfg_of()
    B, T = 2, 48
    sd, x, (c64, s64), (c32, s32) = setup(cfg, B, T)
    dy = torch.randn(B, T, cfg.d_model, generator=torch.Generator().manual_seed(7), dtype=torch.float64)
    sched = uniform_chunks(T, 16, 5)
    _, dx, g = hip_grads(cfg, sd, x, dy, c32, s32, sched, torch.float32, normalize=False, residual=False)
    dx_ref, g_ref = oracle_grads(cfg, sd, x, dy, c64, s64, sched, normalize=False, residual=False)
    compare("fp32 plain", dx, g, dx_ref, g_ref, FP32_TOL, skip=("attn_norm.weight",))


def test_grads_accumulate():
    """Two backward calls into the same LayerGrads add up (``.grad`` semantics)."""
    say("bwd accumulation")
    cfg = cfg_of()
    B, T = 2, 32
    sd, x, _, (c32, s32) = setup(cfg, B, T)
    dy = torch.randn(B, T, cfg.d_model, generator=torch.Generator().manual_seed(3), dtype=torch.float64)
    sched = uniform_chunks(T, 16, 4)
    cell = HipSweepCell(cfg, B, T, device=DEV, dtype=torch.float32)
    cell.pack({k: v.to(DEV, torch.float32) for k, v in sd.items()})
    bufs = cell.new_bufs(T)
    xd = x.float().to(DEV)
    y = torch.empty_like(xd)
    K = torch.empty(B, cfg.n_heads, T, cfg.head_dim, device=DEV)
    V = torch.empty_like(K)
    ocat = torch.empty_like(xd)
    cell.layer_forward(xd, y, c32, s32, sched, K, V, ocat, bufs)
    g1, g2 = LayerGrads(cfg, DEV), LayerGrads(cfg, DEV)
    dx = torch.empty_like(xd)
    dyd = dy.float().to(DEV)
    cell.layer_backward(xd, dyd, dx, c32, s32, sched, K, V, ocat, bufs, g1)
    cell.layer_backward(xd, dyd, dx, c32, s32, sched, K, V, ocat, bufs, g2)
    cell.layer_backward(xd, dyd, dx, c32, s32, sched, K, V, ocat, bufs, g2)
    torch.cuda.synchronize()
    for name, t in g1.t.items():
        assert relerr(g2[name], 2 * t) < 1e-6, name


@pytest.mark.parametrize("ctx_mod", ["mult_res", "linear", "fusion"])
def test_layer_grads_340m_shape_fp32(ctx_mod):
    """340M layer shape (d=1024, 16x64), c=64, K=4, T=256, fp32 storage (
    fp32 leg) vs autograd through the oracle in fp64."""
    say(f"bwd fp32 d=1024 T=256 c=64 K=4 ctx_mod={ctx_mod}")
    cfg = cfg_of(d=1024, h=16, T=256, ctx_mod=ctx_mod)
    B, T = 2, 256
    sd, x, (c64, s64), (c32, s32) = setup(cfg, B, T)
    dy = torch.randn(B, T, cfg.d_model, generator=torch.Generator().manual_seed(11), dtype=torch.float64)
    sched = uniform_chunks(T, 64, 4)
    _, dx, g = hip_grads(cfg, sd, x, dy, c32, s32, sched, torch.float32)
    dx_ref, g_ref = oracle_grads(cfg, sd, x, dy, c64, s64, sched)
    compare("fp32 340m", dx, g, dx_ref, g_ref, FP32_TOL)


def test_layer_grads_340m_shape_bf16():
    """bf16 storage / fp32 accumulate at the 340M layer shape, T=256, vs the fp32 oracle."""
    say("bwd bf16 d=1024 T=256 c=64 K=4")
    cfg = cfg_of(d=1024, h=16, T=256)
    B, T = 2, 256
    sd, x, _, (c32, s32) = setup(cfg, B, T)
    dy = torch.randn(B, T, cfg.d_model, generator=torch.Generator().manual_seed(11), dtype=torch.float64)
    sched = uniform_chunks(T, 64, 4)
    _, dx, g = hip_grads(cfg, sd, x, dy, c32, s32, sched, torch.bfloat16)
    dx_ref, g_ref = oracle_grads(cfg, {k: v.float() for k, v in sd.items()}, x.float(), dy.float(),
                                 c32, s32, sched, dtype=torch.float32)
    compare("bf16 340m", dx, g, dx_ref, g_ref, BF16_TOL)


def test_layer_grads_340m_shape_bf16_T2048():
    """BASELINE config 3's bf16 leg: the bench shape itself (B=8, T=2048, d=1024, 16x64,
    c=64, K=4), bf16 storage, forward tape, against autograd through the oracle's
    chunked-Jacobi layer at the same K, run in fp32 torch on the GPU (the CPU would
    take minutes at this size)."""
    say("bwd bf16 d=1024 B=8 T=2048 c=64 K=4 (tape) vs fp32 oracle on the GPU")
    torch.backends.cuda.matmul.allow_tf32 = False
    cfg = cfg_of(d=1024, h=16, T=2048)
    B, T = 8, 2048
    sd, x, _, (c32, s32) = setup(cfg, B, T)
    dy = torch.randn(B, T, cfg.d_model, generator=torch.Generator().manual_seed(13), dtype=torch.float32)
    sched = uniform_chunks(T, 64, 4)
    _, dx, g, (K, V, ocat) = hip_grads(cfg, sd, x, dy, c32, s32, sched, torch.bfloat16, tape=True, full=True)
    dx_ref, g_ref, (o_ref, K_ref, V_ref) = oracle_grads(
        cfg, {k: v.float() for k, v in sd.items()}, x.float(), dy, c32, s32, sched, dtype=torch.float32,
        device=DEV, with_forward=True)
    # the forward over the whole 32-chunk Gauss-Seidel chain (o_cat and the final K / V
    # rows of every chunk), against the 2e-2 bf16 bar
    fwd = {"o_cat": relerr(ocat, o_ref), "K": relerr(K, K_ref), "V": relerr(V, V_ref)}
    say(f"  bf16 T=2048 forward relerr " + " ".join(f"{k}={v:.2e}" for k, v in fwd.items()))
    record("bf16 340m T=2048 forward", fwd, BF16_FWD_TOL)
    for k, v in fwd.items():
        assert v < BF16_FWD_TOL, f"forward {k}: relerr {v:.3e} >= {BF16_FWD_TOL} (all: {fwd})"
    compare("bf16 340m T=2048", dx, g, dx_ref, g_ref, BF16_TOL)


@pytest.mark.parametrize("taped", [False, True])
def test_bf16_grads_odd_stacked_rows(taped):
    """Batch 1 with a schedule whose stacked weight-grad rows B * sum(K c) = 256 + 105 = 361
    are odd: the rows padding the stack to a whole k-tile must be zeroed also when their
    count is odd. The backward workspace and the tape are filled with 0xFF (bf16 NaN)
    beforehand, so a padding row left unzeroed turns the sweep weight grads into NaN."""
    say(f"bwd bf16 B=1 odd stacked rows taped={taped}")
    cfg = cfg_of(d=256, h=4, T=99)
    B, T = 1, 99
    sched = [(0, 64, 4), (64, 35, 3)]
    sd, x, (c64, s64), (c32, s32) = setup(cfg, B, T)
    dy = torch.randn(B, T, cfg.d_model, generator=torch.Generator().manual_seed(17), dtype=torch.float64)
    dt = torch.bfloat16
    cell = HipSweepCell(cfg, B, T, device=DEV, dtype=dt)
    cell.pack({k: v.to(DEV, dt) for k, v in sd.items()})
    bufs = cell.new_bufs(T)
    xd = x.to(DEV, dt).contiguous()
    y, ocat = torch.empty_like(xd), torch.empty_like(xd)
    K = torch.empty(B, cfg.n_heads, T, cfg.head_dim, device=DEV, dtype=dt)
    V = torch.empty_like(K)
    tp = cell.new_tape(sched).fill_(255) if taped else None
    cell.layer_forward(xd, y, c32, s32, sched, K, V, ocat, bufs, tape=tp)
    cell._bwd_workspace(T, T, max(k for _, _, k in sched)).fill_(255)
    grads = LayerGrads(cfg, DEV)
    dx = torch.empty_like(xd)
    cell.layer_backward(xd, dy.to(DEV, dt).contiguous(), dx, c32, s32, sched, K, V, ocat, bufs, grads, tape=tp)
    torch.cuda.synchronize()
    for name, t in grads.t.items():
        assert torch.isfinite(t).all(), name
    dx_ref, g_ref = oracle_grads(cfg, sd, x, dy, c64, s64, sched)
    compare("bf16 odd rows", dx, grads, dx_ref, g_ref, BF16_TOL)


def test_module_autograd_matches_oracle():
    """DualModAttention (reference signature) forward + loss.backward() through the HIP path."""
    from dual_mod_public_amd.attention import DualModAttention
    say("DualModAttention autograd fp32")
    cfg = cfg_of(T=64)
    B, T = 2, 64
    sd, x, (c64, s64), (c32, s32) = setup(cfg, B, T)
    attn = DualModAttention(cfg).to(DEV)
    attn.load_state_dict({k: v.float() for k, v in sd.items() if k != "attn_norm.weight"})
    xd = x.float().to(DEV).requires_grad_(True)
    dy = torch.randn(B, T, cfg.d_model, generator=torch.Generator().manual_seed(5), dtype=torch.float64)
    y = attn(xd, c32.to(DEV), s32.to(DEV), n_sweeps=4)
    (y * dy.float().to(DEV)).sum().backward()
    torch.cuda.synchronize()
    sched = uniform_chunks(T, attn.CHUNK, 4)
    dx_ref, g_ref = oracle_grads(cfg, sd, x, dy, c64, s64, sched, normalize=False, residual=False)
    got = {n: p.grad for n, p in attn.named_parameters()}
    compare("module", xd.grad, got, dx_ref, g_ref, FP32_TOL, skip=("attn_norm.weight",))
