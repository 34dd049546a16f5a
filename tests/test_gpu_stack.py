"""GPU tests of the multi-layer step on one GPU (dual_mod_public_amd.stack.HipLayerStack,
the single-GPU part of engines/wavescan/engine/graphs.py:36-792): L attention sublayers
forward + backward with one flat fp32 gradient buffer; against autograd through the oracle's
chained layers; the captured HIP graph's replays equal the eager step bit for bit (replayed
several times with eager work in between); the layer-batched (wavefront) forward equals the
layer-by-layer forward bit for bit (outputs, caches, layer buffers, tapes, and the gradients
of the backward that follows); and the T-K8 determinism check
(engines/wavescan/tests/test_k1_k9.py:346-373): two reruns of a short training loop give
bit-identical losses and weights."""

import hashlib
import math

import pytest
import torch

import oracle as O
from dual_mod_public_amd import _lib as L
from dual_mod_public_amd.stack import HipLayerStack
from dual_mod_public_amd.synthetic import make_state_dict
from tests.hip_helpers import DEV, cfg_of, record, relerr, say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    L.load()


def _digest(t):
    return hashlib.sha1(t.detach().contiguous().view(torch.uint8).cpu().numpy().tobytes()).hexdigest()[:12]


def _stack(cfg, n, B, T, dtype, seeds, sched, graph=False, wavefront=False, tape=True):
    sds = [make_state_dict(cfg, seed=s, std=0.02) for s in seeds]
    cos, sin = O.build_rope_cache(T, cfg.head_dim, cfg.rope_theta)
    st = HipLayerStack(cfg, n, B, T, schedule=sched, device=DEV, dtype=dtype, wavefront=wavefront, tape=tape)
    st.load([{k: v.to(DEV) for k, v in sd.items()} for sd in sds], cos, sin)
    if graph:
        st.capture()
    return st, sds


def test_stack_matches_oracle_fp32():
    say("stack of 3 layers fp32 vs oracle autograd")
    cfg = cfg_of(T=64)
    B, T, n = 2, 64, 3
    sched = [(0, 16, 4), (16, 16, 4), (32, 32, 3)]
    st, sds = _stack(cfg, n, B, T, torch.float32, (41, 42, 43), sched)
    g = torch.Generator().manual_seed(4)
    x = torch.randn(B, T, cfg.d_model, generator=g, dtype=torch.float64)
    dy = torch.randn(B, T, cfg.d_model, generator=g, dtype=torch.float64)
    y, dx, grads = st.step(x.float().to(DEV), dy.float().to(DEV))
    torch.cuda.synchronize()
    c64, s64 = O.build_rope_cache(T, cfg.head_dim, cfg.rope_theta, dtype=torch.float64)
    sdg = [{k: v.double().clone().requires_grad_(True) for k, v in sd.items()} for sd in sds]
    xg = x.clone().requires_grad_(True)
    h = xg
    for sd in sdg:
        h = O.dm_layer(cfg, sd, h, c64, s64, schedule=sched)
    (h * dy).sum().backward()
    errs = {"y": relerr(y, h.detach()), "x": relerr(dx, xg.grad)}
    for l, sd in enumerate(sdg):
        for k, v in sd.items():
            errs[f"L{l}.{k}"] = relerr(grads[l][k], v.grad)
    record("stack 3 layers fp32", errs, 1e-5)
    assert max(errs.values()) < 1e-5, max(errs.items(), key=lambda kv: kv[1])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_graph_replays_equal_eager(dtype):
    """Every replay of the captured step equals an eager step on the same inputs bit for bit,
    with eager work and synchronisations between the replays."""
    say(f"stack graph replay == eager {dtype}")
    cfg = cfg_of(T=64)
    B, T, n = 2, 64, 2
    sched = [(0, 16, 4), (16, 48, 2)]
    st_g, _ = _stack(cfg, n, B, T, dtype, (51, 52), sched, graph=True)
    st_e, _ = _stack(cfg, n, B, T, dtype, (51, 52), sched)
    g = torch.Generator(device=DEV).manual_seed(6)
    for rep in range(4):
        x = torch.randn(B, T, cfg.d_model, generator=g, device=DEV).to(dtype)
        dy = torch.randn(B, T, cfg.d_model, generator=g, device=DEV).to(dtype)
        y1, dx1, _ = st_g.step(x, dy)
        torch.cuda.synchronize()
        y1, dx1, f1 = y1.clone(), dx1.clone(), st_g.flat.clone()
        y2, dx2, _ = st_e.step(x, dy)
        torch.cuda.synchronize()
        assert torch.equal(y1, y2) and torch.equal(dx1, dx2), rep
        assert torch.equal(f1, st_e.flat), rep
        _ = (x.float() @ x.float().transpose(1, 2)).sum().item()   # unrelated eager work between replays


def test_k8_determinism_training_loop():
    """T-K8 analogue: two reruns of 8 steps of SGD on fp32 master weights (bf16 packed copies
    repacked each step, the step replayed from its HIP graph) give identical losses and final
    weights, bit for bit."""
    say("T-K8 determinism, 2 reruns x 8 steps")
    cfg = cfg_of(d=256, h=4, T=128)
    B, T, n, steps, lr = 2, 128, 2, 8, 5.0
    sched = [(0, 64, 4), (64, 64, 4)]
    runs = []
    for rep in range(2):
        st, sds = _stack(cfg, n, B, T, torch.bfloat16, (61, 62), sched)
        masters = [{k: v.float().to(DEV).clone() for k, v in sd.items()} for sd in sds]
        cos, sin = O.build_rope_cache(T, cfg.head_dim, cfg.rope_theta)
        st.capture()
        g = torch.Generator(device=DEV).manual_seed(9)
        losses, hashes = [], []
        for _ in range(steps):
            x = torch.randn(B, T, cfg.d_model, generator=g, device=DEV).to(torch.bfloat16)
            tgt = torch.randn(B, T, cfg.d_model, generator=g, device=DEV)
            # loss = 0.5 mean |y - tgt|^2: dy = (y - tgt) / numel (y from this step's forward, the
            # step replayed twice: once to get y, once with the gradient)
            y, _, _ = st.step(x, torch.zeros_like(x))
            dy = ((y.float() - tgt) / y.numel()).to(torch.bfloat16)
            losses.append(0.5 * float(((y.float() - tgt) ** 2).mean()))
            _, dx, grads = st.step(x, dy)
            hashes.append((_digest(y), _digest(dx), _digest(st.flat)))
            for l in range(n):
                for k, w in masters[l].items():
                    w.sub_(lr * grads[l][k])
            st.load(masters, cos, sin)
        runs.append((losses, [{k: v.clone() for k, v in m.items()} for m in masters], hashes))
    assert all(math.isfinite(v) for v in runs[0][0]), runs[0][0]
    for i, (ha, hb) in enumerate(zip(runs[0][2], runs[1][2])):
        assert ha == hb, f"step {i}: (y, dx, grads) digests {ha} vs {hb}"
    assert runs[0][0] == runs[1][0], (runs[0][0], runs[1][0])
    for a, b in zip(runs[0][1], runs[1][1]):
        for k in a:
            assert torch.isfinite(a[k]).all(), k
            assert torch.equal(a[k], b[k]), (k, float((a[k] - b[k]).abs().max()))
    assert runs[0][0][-1] != runs[0][0][0]   # the weights did move


def _bufs_equal(a, b):
    for n in ("xhat", "qr", "kraw", "kself", "vraw", "glogx", "sig"):
        ta, tb = getattr(a, n), getattr(b, n)
        if ta is None and tb is None:
            continue
        if not torch.equal(ta, tb):
            return n
    return None


@pytest.mark.parametrize("dtype,ctx_mod,n,B,T,c,K,d,h,tape", [
    (torch.float32, "mult_res", 3, 2, 64, 16, 4, 256, 4, True),
    (torch.bfloat16, "mult_res", 4, 2, 128, 32, 3, 256, 4, True),
    (torch.bfloat16, "linear", 3, 2, 128, 64, 2, 256, 4, False),
    (torch.bfloat16, "fusion", 3, 1, 128, 64, 4, 256, 2, True),
    (torch.bfloat16, "mult_res", 5, 8, 512, 64, 4, 1024, 16, True),
    (torch.bfloat16, "mult_res", 3, 2, 256, 64, 4, 2048, 16, True),
    (torch.float32, "mult", 2, 2, 64, 64, 3, 256, 4, True),        # one cell
    (torch.float32, "linear", 2, 2, 64, 8, 2, 256, 4, False),      # 8-row cells
])
def test_wavefront_forward_equals_layer_by_layer(dtype, ctx_mod, n, B, T, c, K, d, h, tape):
    say(f"wavefront forward vs layer by layer: {dtype} {ctx_mod} L={n} B={B} T={T} c={c} K={K} d={d} h={h} "
        f"tape={tape}")
    cfg = cfg_of(d=d, h=h, T=T, ctx_mod=ctx_mod)
    sched = [(p, c, K) for p in range(0, T, c)]
    seeds = tuple(70 + i for i in range(n))
    st_w, _ = _stack(cfg, n, B, T, dtype, seeds, sched, wavefront=True, tape=tape)
    st_l, _ = _stack(cfg, n, B, T, dtype, seeds, sched, tape=tape)
    if tape:   # slots a cell shorter than 64 rows leaves unwritten compare equal too
        for t in st_w.tapes + st_l.tapes:
            t.zero_()
    g = torch.Generator(device=DEV).manual_seed(8)
    x = torch.randn(B, T, d, generator=g, device=DEV).to(dtype)
    dy = torch.randn(B, T, d, generator=g, device=DEV).to(dtype)
    for rep in range(2):   # the second step launches from the plan the first one wrote
        y1, dx1, _ = st_w.step(x, dy)
        torch.cuda.synchronize()
        y2, dx2, _ = st_l.step(x, dy)
        torch.cuda.synchronize()
        for l in range(n):
            assert torch.equal(st_w.xs[l + 1], st_l.xs[l + 1]), (rep, l, "y")
            assert torch.equal(st_w.K[l], st_l.K[l]) and torch.equal(st_w.V[l], st_l.V[l]), (rep, l, "K/V")
            assert torch.equal(st_w.ocat[l], st_l.ocat[l]), (rep, l, "ocat")
            assert _bufs_equal(st_w.bufs[l], st_l.bufs[l]) is None, (rep, l, _bufs_equal(st_w.bufs[l], st_l.bufs[l]))
            if tape:
                assert torch.equal(st_w.tapes[l], st_l.tapes[l]), (rep, l, "tape")
        assert torch.equal(dx1, dx2) and torch.equal(st_w.flat, st_l.flat), rep


def test_wavefront_graph_replays_equal_eager():
    """The wavefront step captured as a HIP graph: every replay equals the eager layer-by-layer
    step bit for bit, with eager work between the replays."""
    say("wavefront stack graph replay == eager layer-by-layer step")
    cfg = cfg_of(T=128)
    B, T, n = 2, 128, 3
    sched = [(p, 32, 3) for p in range(0, T, 32)]
    st_g, _ = _stack(cfg, n, B, T, torch.bfloat16, (81, 82, 83), sched, graph=True, wavefront=True)
    st_e, _ = _stack(cfg, n, B, T, torch.bfloat16, (81, 82, 83), sched)
    g = torch.Generator(device=DEV).manual_seed(3)
    for rep in range(3):
        x = torch.randn(B, T, cfg.d_model, generator=g, device=DEV).to(torch.bfloat16)
        dy = torch.randn(B, T, cfg.d_model, generator=g, device=DEV).to(torch.bfloat16)
        y1, dx1, _ = st_g.step(x, dy)
        torch.cuda.synchronize()
        y1, dx1, f1 = y1.clone(), dx1.clone(), st_g.flat.clone()
        y2, dx2, _ = st_e.step(x, dy)
        torch.cuda.synchronize()
        assert torch.equal(y1, y2) and torch.equal(dx1, dx2) and torch.equal(f1, st_e.flat), rep
        _ = (x.float() @ x.float().transpose(1, 2)).sum().item()


def test_wavefront_rejects_unequal_cells():
    cfg = cfg_of(T=64)
    st, _ = _stack(cfg, 2, 2, 64, torch.bfloat16, (1, 2), [(0, 16, 4), (16, 48, 2)], wavefront=True)
    with pytest.raises(L.DMError):
        st.forward_wavefront()


def test_wavefront_plan_refused_unless_built_for_the_arguments():
    """dm_stack_fwd / dm_stack_bwd with build == 0 launch from a plan written earlier: a plan
    never written, or written for other buffers, is refused (DM_ERR_INVALID, nothing launched);
    the same arguments go through and give the same results."""
    say("wavefront plans: build == 0 needs a plan written for the same arguments")
    cfg = cfg_of(T=64)
    B, T, n = 2, 64, 2
    st, _ = _stack(cfg, n, B, T, torch.bfloat16, (5, 6), [(p, 16, 2) for p in range(0, T, 16)], wavefront=True)
    g = torch.Generator(device=DEV).manual_seed(8)
    x = torch.randn(B, T, cfg.d_model, generator=g, device=DEV).to(torch.bfloat16)
    dy = torch.randn(B, T, cfg.d_model, generator=g, device=DEV).to(torch.bfloat16)
    y0, dx0, _ = st.step(x, dy)          # writes both plans
    torch.cuda.synchronize()
    y0, dx0 = y0.clone(), dx0.clone()
    plan, bplan = st._plan, st._bplan
    st._plan = torch.empty_like(plan)    # never written
    with pytest.raises(L.DMError):
        st.forward_wavefront()
    st._plan = plan
    x_saved = st.xs[0]
    st.xs[0] = x_saved.clone()            # another input buffer than the plan was written for
    with pytest.raises(L.DMError):
        st.forward_wavefront()
    st.xs[0] = x_saved
    st._bplan = torch.empty_like(bplan)
    with pytest.raises(L.DMError):
        st.backward_wavefront()
    st._bplan = bplan
    y1, dx1, _ = st.step(x, dy)          # the written plans, the same arguments
    torch.cuda.synchronize()
    assert torch.equal(y1, y0) and torch.equal(dx1, dx0)
