"""GPU tests of the multi-layer step on one GPU (dual_mod_public_amd.stack.HipLayerStack,
the single-GPU part of engines/wavescan/engine/graphs.py:36-792): L attention sublayers
forward + backward with one flat fp32 gradient buffer; against autograd through the oracle's
chained layers; the captured HIP graph's replays equal the eager step bit for bit (replayed
several times with eager work in between); and the T-K8 determinism check
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


def _stack(cfg, n, B, T, dtype, seeds, sched, graph=False):
    sds = [make_state_dict(cfg, seed=s, std=0.02) for s in seeds]
    cos, sin = O.build_rope_cache(T, cfg.head_dim, cfg.rope_theta)
    st = HipLayerStack(cfg, n, B, T, schedule=sched, device=DEV, dtype=dtype)
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
    record("stack 3 layers fp32", errs, 1e-4)
    assert max(errs.values()) < 1e-4, max(errs.items(), key=lambda kv: kv[1])


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
