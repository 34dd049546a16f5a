"""GPU parity of the HIP forward path against the CPU oracle.

Bars: fp32 within 1e-5 relative of the sequential
scan at K = c and of the chunked Jacobi result at K < c; bf16 within 2e-2.
All calls go through libdm_hip.so's C ABI.
"""

import pytest
import torch

import oracle as O
from dual_mod_public_amd import _lib as L
from dual_mod_public_amd.engine import HipSweepCell, uniform_chunks
from tests.hip_helpers import DEV, cfg_of, relerr, say, setup, to_dev

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-5
BF16_TOL = 2e-2


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    L.load()
    torch.backends.cuda.matmul.allow_tf32 = False


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("M,N,K", [(128, 128, 64), (256, 384, 320), (128, 256, 1024), (512, 256, 192)])
def test_gemm_matches_fp64(dtype, ta, tb, M, N, K):
    """dm_gemm: C = op(A) op(B)^T (+C) for the four operand layouts the backward uses."""
    say(f"gemm dtype={dtype} ta={ta} tb={tb} M={M} N={N} K={K}")
    g = torch.Generator().manual_seed(M + N + K + 7 * ta + 3 * tb)
    A = torch.randn(M, K, generator=g).to(dtype)
    B = torch.randn(N, K, generator=g).to(dtype)
    C0 = torch.randn(M, N, generator=g)
    Ad = (A.T if ta else A).contiguous().to(DEV)
    Bd = (B.T if tb else B).contiguous().to(DEV)
    C = C0.clone().to(DEV)
    L.check(L.lib().dm_gemm(L.dtype_code(dtype), ta, tb, Ad.data_ptr(), Bd.data_ptr(), C.data_ptr(),
                            M, N, K, 1, L.stream_ptr()))
    torch.cuda.synchronize()
    ref = A.double() @ B.double().T + C0.double()
    assert relerr(C, ref) < (1e-6 if dtype == torch.float32 else 1e-5)


def _cell(cfg, B, cache_T, sd, dtype):
    cell = HipSweepCell(cfg, B, cache_T, device=DEV, dtype=dtype)
    cell.pack(to_dev(sd, dtype))
    return cell


@pytest.mark.parametrize("ctx_mod", ["mult_res", "linear", "mult", "fusion"])
def test_layer_proj_matches_oracle(ctx_mod):
    say(f"layer_proj fp32 ctx_mod={ctx_mod}")
    cfg = cfg_of(ctx_mod=ctx_mod)
    B, T = 2, 64
    sd, x, (c64, s64), (c32, s32) = setup(cfg, B, T)
    cell = _cell(cfg, B, T, sd, torch.float32)
    bufs = cell.new_bufs(T)
    cell.layer_proj(x.float().to(DEV), bufs, c32, s32, normalize=True)
    torch.cuda.synchronize()
    xhat = O.rms_norm(x, sd["attn_norm.weight"])
    q_r, k, k_self_r, v = O.dm_oracle._projections(cfg, sd, xhat, c64, s64)
    assert relerr(bufs.xhat, xhat) < 1e-6
    assert relerr(bufs.qr, q_r) < 1e-6
    assert relerr(bufs.kraw, k) < 1e-6
    assert relerr(bufs.kself, k_self_r) < 1e-6
    assert relerr(bufs.vraw, v) < 1e-6
    gx = torch.cat([xhat @ sd["w_gk.weight"][:, :cfg.d_model].T + sd["w_gk.bias"],
                    xhat @ sd["w_gv.weight"][:, :cfg.d_model].T + sd["w_gv.bias"]], -1)
    assert relerr(bufs.glogx, gx) < 1e-6
    if ctx_mod == "fusion":   # the x-half pre-activation of v_pre (no bias, no activation)
        assert relerr(bufs.sig, xhat @ sd["v_pre.weight"][:, :cfg.d_model].T) < 1e-6
    elif ctx_mod != "linear":
        assert relerr(bufs.sig, torch.sigmoid(xhat @ sd["v_gate.weight"].T + sd["v_gate.bias"])) < 1e-6


def _hip_layer(cfg, sd, x, cos, sin, schedule, dtype, cache_T=None, fill=0.0):
    B, T, d = x.shape
    cache_T = cache_T or T
    cell = _cell(cfg, B, cache_T, sd, dtype)
    bufs = cell.new_bufs(T)
    xd = x.to(DEV, dtype).contiguous()
    cell.layer_proj(xd, bufs, cos, sin, normalize=False)
    K = torch.full((B, cfg.n_heads, cache_T, cfg.head_dim), fill, device=DEV, dtype=dtype)
    V = torch.full_like(K, fill)
    ocat = torch.empty(B, T, d, device=DEV, dtype=dtype)
    for pos0, c, k in schedule:
        cell.cell_forward(bufs, cos, sin, K, V, pos0, c, k, ocat=ocat)
    torch.cuda.synchronize()
    return ocat, K, V


@pytest.mark.parametrize("ctx_mod", ["mult_res", "linear", "mult", "fusion"])
@pytest.mark.parametrize("c", [16, 64])
def test_cell_exact_equals_scan_fp32(ctx_mod, c):
    """K = c Jacobi cells == the exact sequential scan (config 1 shape)."""
    say(f"cell K=c fp32 ctx_mod={ctx_mod} c={c}")
    cfg = cfg_of(ctx_mod=ctx_mod)
    B, T = 2, 64
    sd, x, (c64, s64), (c32, s32) = setup(cfg, B, T)
    ocat, K, V = _hip_layer(cfg, sd, x, c32, s32, uniform_chunks(T, c), torch.float32)
    o_ref, K_ref, V_ref = O.sequential_scan(cfg, sd, x, c64, s64, return_cache=True)
    assert relerr(ocat, o_ref) < FP32_TOL
    assert relerr(K, K_ref) < FP32_TOL
    assert relerr(V, V_ref) < FP32_TOL


@pytest.mark.parametrize("ctx_mod", ["mult_res", "linear", "fusion"])
@pytest.mark.parametrize("c,k", [(16, 4), (16, 1), (64, 4), (8, 3)])
def test_cell_jacobi_equals_oracle_fp32(ctx_mod, c, k):
    """K < c: the HIP cells reproduce the chunked Jacobi result at the same K."""
    say(f"cell Jacobi fp32 ctx_mod={ctx_mod} c={c} K={k}")
    cfg = cfg_of(ctx_mod=ctx_mod)
    B, T = 2, 64
    sd, x, (c64, s64), (c32, s32) = setup(cfg, B, T)
    sched = uniform_chunks(T, c, k)
    ocat, K, V = _hip_layer(cfg, sd, x, c32, s32, sched, torch.float32)
    o_ref, K_ref, V_ref = O.layer_forward(cfg, sd, x, c64, s64, sched)
    assert relerr(ocat, o_ref) < FP32_TOL
    assert relerr(K, K_ref) < FP32_TOL
    assert relerr(V, V_ref) < FP32_TOL


def test_cell_matches_golden_vectors(golden):
    """The HIP cells against the reference's own outputs (tests/golden)."""
    from tests.golden.make_golden import CASES
    for name in ("c1_mult_res", "c1_linear"):
        case = CASES[name]
        say(f"golden {name}")
        cc = dict(case["cfg"])
        cfg = cfg_of(d=cc.pop("d_model"), h=cc.pop("n_heads"), T=case["T"], **cc)
        sd, x, _, (c32, s32) = setup(cfg, case["B"], case["T"], wseed=case["wseed"],
                                     xseed=case["xseed"])
        ocat, K, V = _hip_layer(cfg, sd, x, c32, s32, uniform_chunks(case["T"], case["c"]),
                                torch.float32)
        assert relerr(ocat, torch.from_numpy(golden[f"{name}/scan_o"])) < FP32_TOL
        sched = uniform_chunks(case["T"], case["c"], case["K"])
        ocat, K, V = _hip_layer(cfg, sd, x, c32, s32, sched, torch.float32)
        assert relerr(ocat, torch.from_numpy(golden[f"{name}/jacobi_o"])) < FP32_TOL
        if f"{name}/jacobi_K" in golden:
            assert relerr(K, torch.from_numpy(golden[f"{name}/jacobi_K"])) < FP32_TOL
            assert relerr(V, torch.from_numpy(golden[f"{name}/jacobi_V"])) < FP32_TOL


def test_append_only_and_bounds():
    """T-K9 (test_k1_k9.py:155-181): earlier rows never change, rows >= T untouched."""
    say("append-only / bounds")
    cfg = cfg_of()
    B, T, cache_T = 2, 40, 64
    sd, x, _, (c32, s32) = setup(cfg, B, T)
    cell = _cell(cfg, B, cache_T, sd, torch.float32)
    bufs = cell.new_bufs(T)
    cell.layer_proj(x.float().to(DEV), bufs, c32, s32, normalize=False)
    K = torch.full((B, cfg.n_heads, cache_T, cfg.head_dim), 7.0, device=DEV)
    V = torch.full_like(K, 7.0)
    snaps = {}
    for pos0, c, k in uniform_chunks(T, 8):
        snaps[pos0] = (K[:, :, :pos0].clone(), V[:, :, :pos0].clone())
        cell.cell_forward(bufs, c32, s32, K, V, pos0, c, k)
    torch.cuda.synchronize()
    for pos0, (k0, v0) in snaps.items():
        assert torch.equal(K[:, :, :pos0], k0) and torch.equal(V[:, :, :pos0], v0)
    assert torch.all(K[:, :, T:] == 7.0) and torch.all(V[:, :, T:] == 7.0)


def test_layer_fwd_matches_oracle_fp32():
    """dm_layer_fwd: y = x + W_O DM(attn_norm(x)) through the schedule."""
    say("layer_fwd fp32")
    cfg = cfg_of()
    B, T = 2, 64
    sd, x, (c64, s64), (c32, s32) = setup(cfg, B, T)
    cell = _cell(cfg, B, T, sd, torch.float32)
    bufs = cell.new_bufs(T)
    xd = x.float().to(DEV)
    y = torch.empty_like(xd)
    K = torch.zeros(B, cfg.n_heads, T, cfg.head_dim, device=DEV)
    V = torch.zeros_like(K)
    ocat = torch.empty_like(xd)
    sched = uniform_chunks(T, 16, 4)
    cell.layer_forward(xd, y, c32, s32, sched, K, V, ocat, bufs)
    torch.cuda.synchronize()
    y_ref = O.dm_layer(cfg, sd, x, c64, s64, schedule=sched)
    assert relerr(y - xd, (y_ref - x)) < FP32_TOL


@pytest.mark.parametrize("ctx_mod", ["mult_res", "linear", "fusion"])
def test_bf16_340m_shape_within_tolerance(ctx_mod):
    """bf16 storage, fp32 accumulate, 340M layer shape (d=1024, 16x64), c=64, K=4,
    against the fp32/fp64 oracle's Jacobi result at the same K (T=256)."""
    say(f"bf16 d=1024 T=256 c=64 K=4 ctx_mod={ctx_mod}")
    cfg = cfg_of(d=1024, h=16, T=256, ctx_mod=ctx_mod)
    B, T = 2, 256
    sd, x, (c64, s64), (c32, s32) = setup(cfg, B, T)
    sched = uniform_chunks(T, 64, 4)
    ocat, K, V = _hip_layer(cfg, sd, x, c32, s32, sched, torch.bfloat16)
    o_ref, K_ref, V_ref = O.layer_forward(cfg, sd, x.float(), c32, s32, sched)
    e = (relerr(ocat, o_ref), relerr(K, K_ref), relerr(V, V_ref))
    say(f"  bf16 relerr o={e[0]:.2e} K={e[1]:.2e} V={e[2]:.2e}")
    assert max(e) < BF16_TOL


def test_attention_module_forward_matches_oracle():
    """DualModAttention.forward (reference signature) == W_O . sequential_scan."""
    from dual_mod_public_amd.attention import DualModAttention
    say("DualModAttention.forward fp32")
    cfg = cfg_of(T=96)
    B, T = 2, 96
    sd, x, (c64, s64), (c32, s32) = setup(cfg, B, T)
    attn = DualModAttention(cfg).to(DEV)
    attn.load_state_dict({k: v.float() for k, v in sd.items() if k != "attn_norm.weight"})
    y = attn(x.float().to(DEV), c32.to(DEV), s32.to(DEV))
    torch.cuda.synchronize()
    y_ref = O.dm_oracle._lin(O.sequential_scan(cfg, sd, x, c64, s64), sd, "wo")
    assert relerr(y, y_ref) < FP32_TOL
