"""GPU tests of the trunk training step (trunk.HipTrunk): the single-GPU WaveScanEngine.train_step
(engines/wavescan/engine/graphs.py:36-792) — embedding, per layer the HIP attention sublayer and the
SwiGLU MLP, norm_f, the tied head and the cross-entropy loss, and the whole backward into one flat
fp32 gradient buffer.

* fp32: the loss and every parameter gradient against autograd through the oracle's fp64 model
  (oracle.lm_forward, pinned to the reference's scan by the golden vectors; with a chunk schedule
  each layer is the oracle's chunked Jacobi layer) within 1e-5, at K = c (exact) and K < c;
* bf16: against the same fp64 oracle within the bf16 bar 2e-2;
* the captured step's replays equal eager steps bit for bit, with eager steps between the replays;
* T-K8 (engines/wavescan/tests/test_k1_k9.py:346-373): two runs of 8 SGD steps from the same
  weights give the same bits (every kernel of the step, the library GEMMs included, is
  deterministic);
* forward tapes and exact recompute give the same bits;
* the layer-batched trunk (dm_stack_fwd / dm_stack_bwd with the MLP as each block's tail,
  engines/wave3d/wave3d.py:26-28) equals the layer-by-layer trunk bit for bit;
* the MLP sublayer alone (dm_mlp_fwd / dm_mlp_bwd): output and every gradient against autograd
  through the oracle's fp64 SwiGLU and RMSNorm (models/dualmod/model.py:102-131).
"""

import pytest
import torch
import torch.nn.functional as F

import oracle as O
from dual_mod_public_amd import _lib as L
from dual_mod_public_amd.config import DualModConfig
from dual_mod_public_amd.engine import uniform_chunks
from dual_mod_public_amd.model import DualModLM
from dual_mod_public_amd.synthetic import make_lm_state_dict
from dual_mod_public_amd.trunk import HipTrunk
from tests.hip_helpers import DEV, record, relerr, say
from dual_mod_public_amd.trunk import MlpBufs, MlpWeights

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    L.load()
    torch.backends.cuda.matmul.allow_tf32 = False


def _cfg(**kw):
    base = dict(d_model=256, n_heads=4, n_layers=2, vocab_size=512, max_seq_len=64, mlp_hidden_override=512,
                checkpoint_chunk=0, dtype="fp32", ctx_mod="mult_res")
    base.update(kw)
    return DualModConfig(**base)


def _model(cfg, dtype, seed=7):
    sd = make_lm_state_dict(cfg, seed=seed, std=0.02)
    m = DualModLM(cfg, dtype=dtype).to(DEV)
    m.load_state_dict({k: v.to(DEV) for k, v in sd.items()})
    return m, sd


def _batch(cfg, B, T, seed=3):
    g = torch.Generator().manual_seed(seed)
    idx = torch.randint(0, cfg.vocab_size, (B, T), generator=g)
    tg = torch.randint(0, cfg.vocab_size, (B, T), generator=g)
    tg[0, :3] = -1   # ignored targets (ignore_index=-1, model.py:279-281)
    return idx, tg


def _oracle(cfg, sd, idx, tg, T, schedule):
    """Loss and gradients of every parameter by autograd through the oracle's fp64 LM."""
    leaves = {}
    for k, v in sd.items():
        if k == "lm_head.weight":
            continue
        leaves[k] = v.double().clone().requires_grad_(True)
    full = dict(leaves)
    full["lm_head.weight"] = leaves["tok_emb.weight"]   # tied
    c64, s64 = O.build_rope_cache(T, cfg.head_dim, cfg.rope_theta, dtype=torch.float64)
    logits = O.lm_forward(cfg, full, idx, c64, s64, schedule=schedule)
    loss = F.cross_entropy(logits.view(-1, cfg.vocab_size), tg.reshape(-1), ignore_index=-1)
    loss.backward()
    return loss.detach(), {k: v.grad for k, v in leaves.items()}


def _compare(name, tr, loss_ref, g_ref, tol):
    errs = {"loss": relerr(tr.loss, loss_ref)}
    for k, v in g_ref.items():
        errs[k] = relerr(tr.grad[k], v)
    worst = max(errs, key=errs.get)
    say(f"  {name}: worst {worst} {errs[worst]:.2e}; loss {float(tr.loss):.6f} vs {float(loss_ref):.6f}")
    record(name, errs, tol)
    for k, v in errs.items():
        assert v < tol, f"{k}: relerr {v:.3e} >= {tol}"


@pytest.mark.parametrize("c,k", [(16, 16), (16, 4)])
def test_trunk_step_matches_oracle_fp32(c, k):
    say(f"trunk step fp32 vs oracle autograd, c={c} K={k}")
    cfg = _cfg()
    B, T = 2, 64
    m, sd = _model(cfg, torch.float32)
    sched = uniform_chunks(T, c, k)
    tr = HipTrunk(m, B, T, schedule=sched, loss_chunk=48)   # head chunks that split a batch row
    idx, tg = _batch(cfg, B, T)
    tr.train_step(idx.to(DEV), tg.to(DEV))
    torch.cuda.synchronize()
    loss_ref, g_ref = _oracle(cfg, sd, idx, tg, T, sched)
    _compare(f"trunk fp32 c={c} K={k}", tr, loss_ref, g_ref, 1e-5)


def test_trunk_step_exact_equals_sequential_scan_oracle():
    """K = c cells against the oracle's sequential scan itself (the reference's scan.py)."""
    say("trunk step fp32 K = c vs the sequential-scan LM")
    cfg = _cfg()
    B, T = 2, 64
    m, sd = _model(cfg, torch.float32, seed=9)
    tr = HipTrunk(m, B, T, schedule=uniform_chunks(T, 16))
    idx, tg = _batch(cfg, B, T, seed=5)
    tr.train_step(idx.to(DEV), tg.to(DEV))
    torch.cuda.synchronize()
    loss_ref, g_ref = _oracle(cfg, sd, idx, tg, T, None)
    _compare("trunk fp32 vs sequential scan", tr, loss_ref, g_ref, 1e-5)


def test_trunk_step_bf16_within_tolerance():
    say("trunk step bf16 vs the fp64 oracle")
    cfg = _cfg(dtype="bf16")
    B, T = 2, 64
    m, sd = _model(cfg, torch.bfloat16)
    sched = uniform_chunks(T, 16, 4)
    tr = HipTrunk(m, B, T, schedule=sched)
    idx, tg = _batch(cfg, B, T)
    tr.train_step(idx.to(DEV), tg.to(DEV))
    torch.cuda.synchronize()
    loss_ref, g_ref = _oracle(cfg, sd, idx, tg, T, sched)
    _compare("trunk bf16 c=16 K=4", tr, loss_ref, g_ref, 2e-2)


def _snapshot(tr):
    return tr.loss.clone(), tr.flat.clone(), tr.xs[-1].clone(), tr.dxs[0].clone()


def _same(a, b):
    return all(torch.equal(x, y) for x, y in zip(a, b))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_trunk_graph_replays_equal_eager(dtype):
    """Every replay of the captured step equals an eager step on the same batch, bit for bit,
    with eager steps on other batches between the replays."""
    say(f"trunk graph replays vs eager, {dtype}")
    cfg = _cfg()
    B, T = 2, 64
    m, _ = _model(cfg, dtype)
    tr = HipTrunk(m, B, T, schedule=uniform_chunks(T, 16, 4))
    batches = [tuple(t.to(DEV) for t in _batch(cfg, B, T, seed=s)) for s in (11, 12, 13)]
    ref = []
    for idx, tg in batches:
        tr.train_step(idx, tg)
        torch.cuda.synchronize()
        ref.append(_snapshot(tr))
    tr.capture()
    for rep in range(2):
        for i, (idx, tg) in enumerate(batches):
            tr.train_step(idx, tg)          # replay
            torch.cuda.synchronize()
            assert _same(_snapshot(tr), ref[i]), (rep, i)
            g, tr.graph = tr.graph, None    # an eager step between the replays
            tr.train_step(*batches[(i + 1) % 3])
            torch.cuda.synchronize()
            assert _same(_snapshot(tr), ref[(i + 1) % 3]), (rep, i, "eager")
            tr.graph = g


def test_trunk_tape_equals_recompute():
    say("trunk step: forward tapes vs exact recompute, bf16")
    cfg = _cfg()
    B, T = 2, 64
    m, _ = _model(cfg, torch.bfloat16)
    sched = uniform_chunks(T, 16, 4)
    a = HipTrunk(m, B, T, schedule=sched)
    b = HipTrunk(m, B, T, schedule=sched, tape_budget=0)
    assert a.n_tape == cfg.n_layers and b.n_tape == 0
    idx, tg = (t.to(DEV) for t in _batch(cfg, B, T))
    a.train_step(idx, tg)
    b.train_step(idx, tg)
    torch.cuda.synchronize()
    assert _same(_snapshot(a), _snapshot(b))


def test_trunk_tk8_bitwise_determinism():
    """T-K8: 8 SGD steps (update the fp32 masters, refresh) twice from the same weights, through the
    captured step: identical losses and weights bit for bit."""
    say("trunk T-K8: two runs of 8 SGD steps, bf16, graph")
    cfg = _cfg()
    B, T = 2, 64
    sched = uniform_chunks(T, 16, 4)
    runs = []
    for _ in range(2):
        m, _ = _model(cfg, torch.bfloat16)
        tr = HipTrunk(m, B, T, schedule=sched).capture()
        losses = []
        idx, tg = (t.to(DEV) for t in _batch(cfg, B, T, seed=100))
        for s in range(8):
            losses.append(float(tr.train_step(idx, tg)))
            with torch.no_grad():
                for n, p in m.named_parameters():
                    p.add_(tr.grad[n], alpha=-0.05)
            tr.refresh()
        torch.cuda.synchronize()
        runs.append((losses, [p.detach().clone() for p in m.parameters()]))
        del tr
    assert runs[0][0] == runs[1][0]
    assert all(torch.equal(x, y) for x, y in zip(runs[0][1], runs[1][1]))
    say(f"  losses {['%.4f' % v for v in runs[0][0]]}")
    assert runs[0][0][-1] < runs[0][0][0]   # the steps descend on the repeated batch


@pytest.mark.parametrize("dtype,tape", [(torch.float32, True), (torch.bfloat16, True), (torch.bfloat16, False)])
def test_trunk_wavefront_equals_layer_by_layer(dtype, tape):
    """The blocks layer-batched, each block's MLP its tail, against the layer-by-layer step: loss,
    every gradient, the trunk's output and dx, bit for bit (3 layers, 4 cells)."""
    say(f"trunk wavefront vs layer by layer, {dtype}, tape={tape}")
    cfg = _cfg(n_layers=3)
    B, T = 2, 64
    m, _ = _model(cfg, dtype)
    sched = uniform_chunks(T, 16, 4)
    budget = None if tape else 0
    a = HipTrunk(m, B, T, schedule=sched, tape_budget=budget)
    b = HipTrunk(m, B, T, schedule=sched, tape_budget=budget, wavefront=True)
    assert b.n_tape == (cfg.n_layers if tape else 0)
    for seed in (21, 22):
        idx, tg = (t.to(DEV) for t in _batch(cfg, B, T, seed=seed))
        a.train_step(idx, tg)
        b.train_step(idx, tg)
        torch.cuda.synchronize()
        assert _same(_snapshot(a), _snapshot(b)), seed
    b.capture()   # the captured layer-batched step replays the same bits
    idx, tg = (t.to(DEV) for t in _batch(cfg, B, T, seed=23))
    a.train_step(idx, tg)
    b.train_step(idx, tg)
    torch.cuda.synchronize()
    assert _same(_snapshot(a), _snapshot(b))


@pytest.mark.parametrize("dtype,tol,M", [(torch.float32, 1e-5, 128), (torch.float32, 1e-5, 100),
                                         (torch.bfloat16, 2e-2, 300)])
def test_mlp_sublayer_matches_oracle(dtype, tol, M):
    """dm_mlp_fwd / dm_mlp_bwd on M rows (also a count that is no multiple of the tiles) against
    autograd through the oracle's fp64 z = y + swiglu(rms_norm(y))."""
    say(f"MLP sublayer {dtype} M={M}")
    d, H = 256, 384
    g = torch.Generator().manual_seed(31)
    y = torch.randn(M, d, generator=g, dtype=torch.float64)
    dz = torch.randn(M, d, generator=g, dtype=torch.float64)
    sd = {"mlp.w1.weight": 0.05 * torch.randn(H, d, generator=g, dtype=torch.float64),
          "mlp.w3.weight": 0.05 * torch.randn(H, d, generator=g, dtype=torch.float64),
          "mlp.w2.weight": 0.05 * torch.randn(d, H, generator=g, dtype=torch.float64),
          "mlp_norm.weight": 1.0 + 0.1 * torch.randn(d, generator=g, dtype=torch.float64)}

    class _Blk:   # the module attributes MlpWeights.pack reads
        pass
    blk = _Blk()
    blk.mlp = _Blk()
    for n in ("w1", "w3", "w2"):
        setattr(blk.mlp, n, _Blk())
        getattr(blk.mlp, n).weight = sd[f"mlp.{n}.weight"].to(DEV, dtype)
    blk.mlp_norm = _Blk()
    blk.mlp_norm.weight = sd["mlp_norm.weight"].to(DEV, dtype)
    mw = MlpWeights(d, H, DEV, dtype)
    mw.pack(blk)
    mb = MlpBufs(1, M, d, H, DEV, dtype)
    yd, dzd = y.to(DEV, dtype).contiguous(), dz.to(DEV, dtype).contiguous()
    z = torch.empty_like(yd)
    dy = torch.empty_like(yd)
    grads = {k: torch.zeros(v.shape, device=DEV, dtype=torch.float32) for k, v in sd.items()}
    gs = L.dm_mlp_grads()
    gs.w1, gs.w3, gs.w2 = (L.ptr(grads[f"mlp.{n}.weight"]) for n in ("w1", "w3", "w2"))
    gs.norm_w = L.ptr(grads["mlp_norm.weight"])
    code = L.dtype_code(dtype)
    import ctypes
    L.check(L.lib().dm_mlp_fwd(code, ctypes.byref(mw.s), L.ptr(yd), L.ptr(z), ctypes.byref(mb.s), M, d, H, 1e-5,
                               L.stream_ptr()))
    nb = L.lib().dm_mlp_workspace_bytes(code, M, d, H)
    ws = torch.empty(nb, device=DEV, dtype=torch.uint8)
    L.check(L.lib().dm_mlp_bwd(code, ctypes.byref(mw.s), L.ptr(yd), L.ptr(dzd), L.ptr(dy), ctypes.byref(mb.s),
                               ctypes.byref(gs), M, d, H, 1e-5, L.ptr(ws), nb, L.stream_ptr()))
    torch.cuda.synchronize()
    leaves = {k: v.clone().requires_grad_(True) for k, v in sd.items()}
    yl = y.clone().requires_grad_(True)
    z_ref = yl + O.swiglu(leaves, O.rms_norm(yl, leaves["mlp_norm.weight"], 1e-5))
    (z_ref * dz).sum().backward()
    errs = {"z": relerr(z, z_ref.detach()), "dy": relerr(dy, yl.grad)}
    for k, v in leaves.items():
        errs[k] = relerr(grads[k], v.grad)
    say("  " + " ".join(f"{k}={v:.1e}" for k, v in errs.items()))
    record(f"mlp sublayer {dtype} M={M}", errs, tol)
    for k, v in errs.items():
        assert v < tol, f"{k}: relerr {v:.3e}"


@pytest.mark.parametrize("W", [10, 24])
def test_windowed_trunk_step_matches_oracle_fp32(W):
    """local_window W (inside a 16-row cell, and across cells) on every layer of the trunk step:
    the loss and every gradient against autograd through the oracle's windowed fp64 LM, K = 4;
    the layer-batched step equals the layer-by-layer one bit for bit."""
    say(f"windowed trunk step fp32 vs oracle autograd, W={W}")
    cfg = _cfg(local_window=W)
    B, T = 2, 64
    m, sd = _model(cfg, torch.float32)
    sched = uniform_chunks(T, 16, 4)
    tr = HipTrunk(m, B, T, schedule=sched)
    idx, tg = _batch(cfg, B, T)
    tr.train_step(idx.to(DEV), tg.to(DEV))
    torch.cuda.synchronize()
    loss_ref, g_ref = _oracle(cfg, sd, idx, tg, T, sched)
    _compare(f"trunk fp32 W={W}", tr, loss_ref, g_ref, 1e-5)
    wf = HipTrunk(m, B, T, schedule=sched, wavefront=True)
    wf.train_step(idx.to(DEV), tg.to(DEV))
    torch.cuda.synchronize()
    assert _same(_snapshot(tr), _snapshot(wf))
