"""Benchmark of the Dual-Mod attention hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload fwdbwd|fwd|c4]
                    [--no-cpu-baseline] [--no-decode] [--no-c1] [--no-c4] [--c4-stack-layers L] [--no-stack]
                    [--stack-layers L]
                    [--no-graph-decode]

One step = one DM attention layer of the 340M shape (B=8, T=2048, d=1024,
16 heads x 64, c=64, K=4 Jacobi sweeps chained over 32 chunks, bf16 storage /
fp32 accumulate) through libdm_hip.so: the forward (attn_norm + projections,
the 32 chunk cells = committed accumulator + 4 sweeps each, W_O with the
residual) and, for the default fwdbwd workload, the
reverse-scan backward producing dx and every parameter gradient for an upstream
dy ~ N(0,1). The forward keeps every cell's sweep states in an HBM tape (1.2 GB
for this layer) that the backward reads instead of recomputing them; the
reference's exact-recompute mode (same values bit for bit) is timed beside it in
the same run and reported with the same fields ("recompute"; --recompute makes it
the headline). Inputs (x, dy, weights, RoPE tables) are resident in HBM before
timing starts.

Prints ONE JSON line: the headline sweep throughput in tokens/s, the roofline of
the dominant kernel (sweep GEMM 1) timed with HIP events stamped by its own launches inside a
second pass of the timed steps, the path-level roofline, config 4 (one layer of the d=2048
trunk, fwd+bwd for K in {1, 2, 4, 8}; the whole 24-layer trunk training step with SwiGLU MLPs and
the tied 32000-token head, layer by layer and layer-batched, its per-layer cell timed inside it;
8 attention layers layer-batched), a stack of the 340M layer at the model's depth (24 layers,
--stack-layers) fwd+bwd layer by layer and layer-batched (wavefront), the 24-layer model's greedy
decode
through the one-graph-per-token decoder against the eager one, the decode sub-benchmark
(batch 64, bf16 tape of 32768 positions, HBM GB/s)
whole (B=2, T=64, d=256, fp32, c=16, K=16) and the CPU baselines (the oracle on this host's
cores, warm-up then the median of 3: C1 whole by the sequential scan, the C2 forward and the C3
forward + backward over the whole workload, C5 over 8 of the 64 batch rows).
"""

import argparse
import json
import os
import re
import statistics
import sys
import time

import torch

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

from dual_mod_public_amd import _lib as L  # noqa: E402
from dual_mod_public_amd.config import DualModConfig  # noqa: E402
from dual_mod_public_amd.decode import StaticTape  # noqa: E402
from dual_mod_public_amd.engine import HipSweepCell, LayerGrads, uniform_chunks  # noqa: E402
from dual_mod_public_amd.rope import build_rope_cache  # noqa: E402
from dual_mod_public_amd.synthetic import make_input, make_state_dict  # noqa: E402

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
COPY_CAL_BYTES = 256 << 20  # --copy-calibration: bytes read (and written) per copy dispatch
# HBM bytes per launch of the roofline kernels are read from the committed counter summary
# (rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE passes over this script, each scaled by what the
# counter reads for the 256 MiB --copy-calibration copy; the file has the commands).
TRAFFIC_PROFILE = os.path.join(REPO, "profiles", "traffic_sweep1_decode.md")
TIMING_NOTE = ("avg_launch_ms: a HIP event pair stamped by each launch of the kernel itself "
               "(hipExtLaunchKernel start/stop events on its own stream: the dispatch's begin and end, "
               "the interval rocprofv3's kernel trace reports), over a second pass of the timed steps "
               "(instrumented_ms_per_step); avg_launch_ms_device: first block start to last block end "
               "on the device clock (s_memrealtime), the kernel's execution without dispatch and drain")

# BASELINE config 2 (forward) — the 340M-shape DM layer
C2 = dict(B=8, T=2048, d=1024, h=16, c=64, K=4, wseed=1, xseed=2)
# BASELINE config 4 — one layer of the 24-layer d=2048 trunk (16 heads x 128), K ladder
C4 = dict(B=4, T=4096, d=2048, h=16, c=64, K=4, wseed=1, xseed=2, ladder=(1, 2, 4, 8))
# BASELINE config 5 — incremental decode
C5 = dict(B=64, d=1024, h=16, P0=32768, steps=256, wseed=3, xseed=4, tseed=5)


def traffic_from_profile(kernel):
    """HBM bytes per launch of a kernel row ("| sweep1 | ... | <MB/launch> |") of the committed
    counter summary, or None when the file or the row is missing."""
    try:
        text = open(TRAFFIC_PROFILE).read()
    except OSError:
        return None
    m = re.search(r"^\|\s*" + re.escape(kernel) + r"\s*\|.*\|\s*([0-9.]+)\s*\|\s*$", text, re.M)
    return float(m.group(1)) * 1e6 if m else None


def host_info():
    model = None
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                model = ln.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"host_cpus": os.cpu_count(), "cpu_model": model}


def fwd_flops_per_token(d, T, c, K, ctx_mod="mult_res"):
    """Algorithmic forward FLOPs per token of one DM layer (recompute excluded):
    projections q,k,v,W_O + gate x-halves + v_gate (14 d^2), per sweep the packed
    ctx/gate GEMM (8 d^2) and w_vctx (2 d^2), committed attention averaged over
    chunks 2d(T-c), causal intra pairs 2d(c-1) and the raw-self column 4d per sweep."""
    proj = 14 if ctx_mod != "linear" else 12
    per_sweep = 10 if ctx_mod != "linear" else 8
    return (proj + per_sweep * K) * d * d + 2 * d * (T - c) + 2 * K * d * (c - 1) + 4 * K * d


def fwdbwd_flops_per_token(d, T, c, K, ctx_mod="mult_res"):
    """Algorithmic forward + backward FLOPs per token: the backward of every product
    is two products of the same size, so 3x the forward; the backward's exact
    recompute of the forward is not useful work and is not counted."""
    return 3 * fwd_flops_per_token(d, T, c, K, ctx_mod)


def sweep1_flops(N, d):
    """Useful FLOPs of one sweep GEMM 1 launch: N rows x (w_kctx, g_k u-half, v_map,
    g_v u-half) = 4 d x d products."""
    return 2.0 * N * d * 4 * d


def build_layer(cfg, B, T, dev, seeds=C2):
    sd = make_state_dict(cfg, seed=seeds["wseed"])
    cell = HipSweepCell(cfg, B, T, device=dev, dtype=torch.bfloat16)
    cell.pack({k: v.to(dev) for k, v in sd.items()})
    x = make_input((B, T, cfg.d_model), seed=seeds["xseed"]).to(dev, torch.bfloat16)
    cos, sin = build_rope_cache(T, cfg.head_dim, cfg.rope_theta, device=dev)
    bufs = cell.new_bufs(T)
    K = torch.zeros(B, cfg.n_heads, T, cfg.head_dim, device=dev, dtype=torch.bfloat16)
    V = torch.zeros_like(K)
    ocat = torch.empty_like(x)
    y = torch.empty_like(x)
    return sd, cell, x, cos.contiguous(), sin.contiguous(), bufs, K, V, ocat, y


def timed(fn, steps):
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps


def median_wall(fn, reps=3, warmup=1):
    """One untimed warm-up call, then the median wall time of `reps` calls (and all of them)."""
    for _ in range(warmup):
        fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts), ts


def cpu_threads():
    """Threads of the CPU baselines: every host core, capped at the 16 a one-GPU share of the box has."""
    return min(os.cpu_count() or 1, 16)


def cpu_baseline(cfg, sd, T, B, fwdbwd, cpu_T):
    """The oracle's chunked-Jacobi layer (same schedule, fp32 torch) on this host's cores over a
    T-prefix of the workload (the same per-token GEMM work, a shorter committed prefix), forward
    or forward + autograd backward: one warm-up, then the median of 3."""
    import oracle as O
    nthr = cpu_threads()
    torch.set_num_threads(nthr)
    Ts = min(T, cpu_T) if cpu_T else T
    x = make_input((B, Ts, cfg.d_model), seed=C2["xseed"])
    cos, sin = O.build_rope_cache(Ts, cfg.head_dim, cfg.rope_theta)
    sched = O.uniform_chunks(Ts, C2["c"], C2["K"])
    dy = make_input((B, Ts, cfg.d_model), seed=C2["xseed"] + 100)

    def run():
        if fwdbwd:
            sdf = {k: v.float().clone().requires_grad_(True) for k, v in sd.items()}
            xg = x.clone().requires_grad_(True)
            y = O.dm_layer(cfg, sdf, xg, cos, sin, schedule=sched)
            (y * dy).sum().backward()
        else:
            with torch.no_grad():
                O.dm_layer(cfg, {k: v.float() for k, v in sd.items()}, x, cos, sin, schedule=sched)

    med, ts = median_wall(run)
    span = "the whole workload" if Ts == T else f"a T-prefix of the T={T} workload"
    what = ("layer forward + autograd backward" if fwdbwd else "layer forward") + \
        f" at B={B}, T={Ts} ({span}; c=64, K=4)"
    return dict(value=B * Ts / med, unit="tokens/s", cores=nthr, kind="port",
                sample=f"{what}, fp32 torch CPU oracle, median of 3 after a warm-up: "
                       + ", ".join(f"{t:.2f}" for t in ts) + " s", **host_info())


def cpu_decode_baseline(cfg, sd, rows=8, steps=3):
    """The oracle's static-tape decode step (lm/eval/graph_decode.py:33-51 restated, fp32 torch)
    on this host's cores for `rows` of the 64 batch rows of BASELINE config 5 (tape of 32768
    positions): one warm-up step, then the median of `steps`; GB/s of the same algorithmic bytes
    as the GPU figure (the bf16 tape rows read, the weights, the row writes)."""
    import oracle as O
    nthr = cpu_threads()
    torch.set_num_threads(nthr)
    P0, h, d = C5["P0"], C5["h"], C5["d"]
    dh = d // h
    P = P0 + steps + 1
    g = torch.Generator().manual_seed(C5["tseed"])
    Kb = torch.randn(rows, h, P, dh, generator=g).bfloat16().float()
    Vb = torch.randn(rows, h, P, dh, generator=g).bfloat16().float()
    x = torch.randn(steps + 1, rows, 1, d, generator=g).bfloat16().float()
    cos, sin = O.build_rope_cache(P, dh, cfg.rope_theta)
    sdf = {k: v.float() for k, v in sd.items()}
    pos = [P0]

    def run():
        with torch.no_grad():
            O.static_decode_step(cfg, sdf, x[pos[0] - P0], pos[0], Kb, Vb, cos, sin)
        pos[0] += 1

    med, ts = median_wall(run, reps=steps)
    step_bytes = 2.0 * rows * h * (P0 + 2) * dh * 2 + 12.0 * d * d * 2 + 2.0 * rows * d * 2
    return dict(value=step_bytes / med / 1e9, unit="GB/s", tokens_per_s=rows / med, cores=nthr, kind="port",
                sample=f"static-tape decode steps of {rows} of the 64 batch rows at P = {P0}.., fp32 torch "
                       "CPU oracle, median of 3 after a warm-up: " + ", ".join(f"{t * 1e3:.0f}" for t in ts) + " ms",
                **host_info())


def bench_c1(dev, steps=50, warmup=5, with_cpu=True):
    """BASELINE config 1, whole: one DM layer at B=2, T=64, d=256, 4 x 64, fp32, c=16, K=16 (exact).
    The HIP layer forward (dm_layer_fwd, one call) timed over `steps` calls, and beside it the
    reference's CPU path for the same case, the oracle's sequential scan (scan.py:19-95 restated,
    fp32 torch) on this host's cores over the whole workload: one warm-up, then the median of 3."""
    B, T, d, h, c, K = 2, 64, 256, 4, 16, 16
    cfg = DualModConfig(d_model=d, n_heads=h, ctx_mod="mult_res", max_seq_len=T, dtype="fp32")
    sd = make_state_dict(cfg, seed=C2["wseed"])
    cell = HipSweepCell(cfg, B, T, device=dev, dtype=torch.float32)
    cell.pack({k: v.to(dev) for k, v in sd.items()})
    x = make_input((B, T, d), seed=C2["xseed"]).to(dev, torch.float32)
    cos, sin = build_rope_cache(T, cfg.head_dim, cfg.rope_theta, device=dev)
    cos, sin = cos.contiguous(), sin.contiguous()
    bufs = cell.new_bufs(T)
    Kc = torch.zeros(B, h, T, cfg.head_dim, device=dev, dtype=torch.float32)
    Vc, ocat, y = torch.zeros_like(Kc), torch.empty_like(x), torch.empty_like(x)
    sched = uniform_chunks(T, c, K)

    def step():
        cell.layer_forward(x, y, cos, sin, sched, Kc, Vc, ocat, bufs)
    for _ in range(warmup):
        step()
    dt = timed(step, steps)
    out = {"workload": f"C1: one DM layer forward, B={B} T={T} d={d} {h}x{d // h}, fp32, c={c} K={K} (exact)",
           "ms_per_step": dt * 1e3, "tokens_per_s": B * T / dt, "steps": steps}
    if with_cpu:
        import oracle as O
        nthr = cpu_threads()
        torch.set_num_threads(nthr)
        xc = make_input((B, T, d), seed=C2["xseed"])
        c32, s32 = O.build_rope_cache(T, cfg.head_dim, cfg.rope_theta)
        sdf = {k: v.float() for k, v in sd.items()}

        def run():
            with torch.no_grad():
                O.dm_layer(cfg, sdf, xc, c32, s32, schedule=None)
        med, ts = median_wall(run)
        out["cpu_baseline"] = dict(
            value=B * T / med, unit="tokens/s", cores=nthr, kind="port",
            sample=f"the whole C1 workload (B={B}, T={T}): the sequential scan (scan.py), fp32 torch CPU oracle, "
                   "median of 3 after a warm-up: " + ", ".join(f"{t * 1e3:.1f}" for t in ts) + " ms",
            **host_info())
    del cell, bufs, Kc, Vc, ocat, y, x
    return out


def bench_decode(dev, steps_override=None, with_cpu=True):
    cfg = DualModConfig(d_model=C5["d"], n_heads=C5["h"], ctx_mod="mult_res", max_seq_len=8,
                        dtype="bf16")
    B, P0 = C5["B"], C5["P0"]
    steps = steps_override or C5["steps"]
    P = P0 + steps
    sd = make_state_dict(cfg, seed=C5["wseed"], with_attn_norm=False)
    tape = StaticTape(cfg, B, P, dev, torch.bfloat16,
                      sd={k: v.to(dev) for k, v in sd.items()})
    g = torch.Generator(device=dev).manual_seed(C5["tseed"])
    tape.K.normal_(generator=g)
    tape.V.normal_(generator=g)
    x = torch.randn(steps, B, cfg.d_model, generator=g, device=dev).to(torch.bfloat16)
    cos, sin = build_rope_cache(P, cfg.head_dim, cfg.rope_theta, device=dev)
    cos, sin = cos.contiguous(), sin.contiguous()
    dh, h, d = cfg.head_dim, cfg.n_heads, cfg.d_model

    def run_all():
        for t in range(steps):
            tape.step(x[t], P0 + t, cos, sin, with_wo=True)

    # warm-up pass over the first few slots (the slots are rewritten by the timed pass)
    for t in range(4):
        tape.step(x[t], P0 + t, cos, sin, with_wo=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    run_all()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    # the same steps again (rewriting the same tape slots) with the tape read's timing armed
    with L.KernelTimer("dec_read", max_launches=steps + 8) as kt:
        run_all()
        torch.cuda.synchronize()
    tape_bytes = sum(2.0 * B * h * (P0 + t) * dh * 2 for t in range(steps))
    weight_bytes = steps * 12.0 * d * d * 2
    write_bytes = steps * 2.0 * B * d * 2
    total = tape_bytes + weight_bytes + write_bytes
    read_bytes_per_launch = tape_bytes / steps
    ev_s = kt.avg_ms / 1e3
    out = {
        "metric": "decode HBM GB/s (attend_one+refine_kv over the tape, append)",
        "value": total / wall / 1e9, "unit": "GB/s", "steps": steps, "ms_per_step": wall / steps * 1e3,
        "tokens_per_s": B * steps / wall,
        "config": {"workload": "C5 decode: B=64, bf16 tape 32768..33023 positions, d=1024, 16x64",
                   "algorithmic_bytes": total},
        "roofline": {"bound": "hbm", "achieved": read_bytes_per_launch / ev_s / 1e9,
                     "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": read_bytes_per_launch / ev_s / 1e9 / PEAK_HBM_GBS,
                     "traffic": traffic_from_profile("dec_read"), "kernel": "k_decode_partial",
                     "bytes_per_launch": read_bytes_per_launch,
                     "avg_launch_ms": kt.avg_ms, "avg_launch_ms_device": kt.device_avg_ms,
                     "timing": TIMING_NOTE, "launches": kt.n},
        "path_frac_of_hbm_peak": total / wall / 1e9 / PEAK_HBM_GBS,
    }
    del tape
    torch.cuda.empty_cache()
    if with_cpu:
        out["cpu_baseline"] = cpu_decode_baseline(cfg, sd)
    return out


def bench_c4_ladder(dev, steps=3, warmup=1):
    """BASELINE config 4's workload: one layer of the d=2048, 16 x 128 trunk at B=4, T=4096, c=64,
    forward (tape) + reverse-scan backward per K in the ladder (1, 2, 4, 8). The cell's algorithmic
    FLOPs (fwd_flops_per_token; the trunk's SwiGLU MLP and tied head are outside the layer)."""
    B, T, d, h, c = C4["B"], C4["T"], C4["d"], C4["h"], C4["c"]
    cfg = DualModConfig(d_model=d, n_heads=h, ctx_mod="mult_res", max_seq_len=T, dtype="bf16")
    sd, cell, x, cos, sin, bufs, Kc, Vc, ocat, y = build_layer(cfg, B, T, dev, seeds=C4)
    grads = LayerGrads(cfg, dev)
    dy = make_input((B, T, d), seed=C4["xseed"] + 100).to(dev, torch.bfloat16)
    dx = torch.empty_like(x)
    ladder = []
    for K in C4["ladder"]:
        sched = uniform_chunks(T, c, K)
        tape = cell.new_tape(sched)

        def step():
            cell.layer_forward(x, y, cos, sin, sched, Kc, Vc, ocat, bufs, tape=tape)
            cell.layer_backward(x, dy, dx, cos, sin, sched, Kc, Vc, ocat, bufs, grads, tape=tape)

        def fwd():
            cell.layer_forward(x, y, cos, sin, sched, Kc, Vc, ocat, bufs, tape=tape)

        for _ in range(warmup):
            step()
        dt = timed(step, steps)
        dtf = timed(fwd, steps)
        fpt = fwd_flops_per_token(d, T, c, K)
        ladder.append({"K": K, "ms_per_layer_fwdbwd": dt * 1e3, "tokens_per_s": B * T / dt,
                       "fwd_mflop_per_token": fpt / 1e6,
                       "frac_fwdbwd": 3 * fpt * B * T / dt / 1e12 / PEAK_BF16_TFLOPS,
                       "ms_per_layer_fwd": dtf * 1e3, "frac_fwd": fpt * B * T / dtf / 1e12 / PEAK_BF16_TFLOPS,
                       "tape_bytes": tape.numel()})
        del tape
        torch.cuda.empty_cache()
    del cell, bufs, Kc, Vc, ocat, y, x, dx, dy, grads
    torch.cuda.empty_cache()
    return {"workload": f"C4: one layer of the d=2048 trunk (16x128), B={B} T={T} c={c}, forward (tape) + "
                        "reverse-scan backward per K; the per-layer cell of the 24-layer trunk",
            "steps": steps, "warmup": warmup, "ladder": ladder}


def bench_c4_trunk(dev, n_layers=24, steps=2, warmup=1):
    """BASELINE config 4 as written: the 24-layer d=2048 trunk (16 x 128 heads, SwiGLU ffn 5632, tied
    embeddings, vocab 32000) at B=4, T=4096, token ids uniform random, bf16, one training step (forward
    + backward, trunk.HipTrunk captured as one HIP graph) per K in the ladder; the per-layer DM cell
    timed inside the step (HIP events around each layer's attention forward and backward in an eager
    step). Forward tapes for as many layers as fit in the memory left (HipTrunk's tape_budget "auto");
    the others recompute their cells (same results)."""
    from dual_mod_public_amd.model import DualModLM
    from dual_mod_public_amd.trunk import CellTimer, HipTrunk
    B, T, d, h, c = C4["B"], C4["T"], C4["d"], C4["h"], C4["c"]
    cfg = DualModConfig(d_model=d, n_heads=h, n_layers=n_layers, vocab_size=32000, max_seq_len=T, ctx_mod="mult_res",
                        mlp_hidden_override=5632, dtype="bf16")
    torch.manual_seed(C4["wseed"])
    with torch.device(dev):
        m = DualModLM(cfg, dtype=torch.bfloat16)
    with torch.no_grad():
        m.tok_emb.weight.normal_(0.0, 0.02)   # model.py:187-195 init scale (nn.Embedding's default is N(0, 1))
    n_params = sum(p.numel() for p in m.parameters())
    g = torch.Generator(device=dev).manual_seed(C4["xseed"])
    idx = torch.randint(0, cfg.vocab_size, (B, T), generator=g, device=dev)
    tg = torch.randint(0, cfg.vocab_size, (B, T), generator=g, device=dev)
    Fh = cfg.mlp_hidden
    ladder = []
    for K in C4["ladder"]:
        sched = uniform_chunks(T, c, K)
        torch.cuda.empty_cache()
        tr = HipTrunk(m, B, T, schedule=sched, tape_budget="auto")
        for _ in range(warmup):
            tr.train_step(idx, tg)
        tr.timer = CellTimer(n_layers)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        tr.train_step(idx, tg)                 # eager, the cells timed in place
        torch.cuda.synchronize()
        eager = time.perf_counter() - t0
        cells = tr.timer.ms()
        tr.timer = None
        tr.capture()
        dt = timed(lambda: tr.train_step(idx, tg), steps)
        loss = float(tr.loss)
        fpt = fwd_flops_per_token(d, T, c, K)
        cell_ms = [f + b for f, b in cells]
        mean_cell = sum(cell_ms) / n_layers
        mlp_f, head_f = 2 * 3 * d * Fh, 2 * d * cfg.vocab_size
        trunk_f = 3 * (n_layers * (fpt + mlp_f) + head_f)
        ladder.append({"K": K, "step_ms": dt * 1e3, "tokens_per_s": B * T / dt, "loss": loss,
                       "cell_ms_per_layer_fwdbwd": mean_cell,
                       "cell_fwd_ms_per_layer": sum(f for f, _ in cells) / n_layers,
                       "cell_bwd_ms_per_layer": sum(b for _, b in cells) / n_layers,
                       "cell_frac": 3 * fpt * B * T / (mean_cell / 1e3) / 1e12 / PEAK_BF16_TFLOPS,
                       "cells_share_of_eager_step": sum(cell_ms) / (eager * 1e3), "eager_step_ms": eager * 1e3,
                       "trunk_frac": trunk_f * B * T / dt / 1e12 / PEAK_BF16_TFLOPS,
                       "tape_layers": tr.n_tape})
        del tr
        torch.cuda.empty_cache()
    # the same step layer-batched: every block (attention + its MLP tail) in the wavefront, the
    # forward tapes kept when every layer's fits (else every cell recomputed in the backward)
    wf = []
    for K in C4["ladder"]:
        sched = uniform_chunks(T, c, K)
        torch.cuda.empty_cache()
        tr = HipTrunk(m, B, T, schedule=sched, tape_budget="auto", wavefront=True)
        for _ in range(warmup):
            tr.train_step(idx, tg)
        tr.capture()
        dt = timed(lambda: tr.train_step(idx, tg), steps)
        fpt = fwd_flops_per_token(d, T, c, K)
        mlp_f, head_f = 2 * 3 * d * Fh, 2 * d * cfg.vocab_size
        trunk_f = 3 * (n_layers * (fpt + mlp_f) + head_f)
        wf.append({"K": K, "step_ms": dt * 1e3, "tokens_per_s": B * T / dt, "loss": float(tr.loss),
                   "trunk_frac": trunk_f * B * T / dt / 1e12 / PEAK_BF16_TFLOPS, "tape_layers": tr.n_tape,
                   "speedup_vs_layer_by_layer": next(e["step_ms"] for e in ladder if e["K"] == K) / (dt * 1e3)})
        del tr
        torch.cuda.empty_cache()
    del m
    torch.cuda.empty_cache()
    return {"workload": f"C4: {n_layers}-layer d={d} trunk ({h}x{d // h}, SwiGLU {Fh}, tied vocab 32000, "
                        f"{n_params / 1e9:.2f}B params), B={B} T={T} c={c}, one training step (embedding, attention + "
                        "MLP per layer, head + CE loss, full backward into a flat fp32 gradient buffer) per K, "
                        "captured as one HIP graph; the DM cell timed per layer inside an eager step",
            "flops": "cell: 3 x fwd_flops_per_token per layer; trunk_frac adds the MLP (3 x 6 d ffn) and head "
                     "(3 x 2 d V) per token",
            "steps": steps, "warmup": warmup, "ladder": ladder,
            "wavefront": {"what": "the same step with the blocks layer-batched (dm_stack_fwd / dm_stack_bwd, "
                                  "each block's MLP its tail; the same results bit for bit)", "ladder": wf}}


def bench_c4_wavefront(dev, n_layers=8, steps=2, warmup=1):
    """Config 4's trunk attention sublayers as a layer-batched stack: n_layers d=2048, 16 x 128
    sublayers (one weight set) at B=4, T=4096, c=64, forward (tape) + reverse-scan backward per
    step, HipLayerStack(wavefront=True), per K in the ladder; ms per layer and the cell's MFMA
    fraction. 8 layers by default: at K = 8 a layer holds ~12 GB (tape and backward workspace)."""
    from dual_mod_public_amd.stack import HipLayerStack
    B, T, d, h, c = C4["B"], C4["T"], C4["d"], C4["h"], C4["c"]
    cfg = DualModConfig(d_model=d, n_heads=h, ctx_mod="mult_res", max_seq_len=T, dtype="bf16")
    sd = {k: v.to(dev) for k, v in make_state_dict(cfg, seed=C4["wseed"]).items()}
    cos, sin = build_rope_cache(T, d // h, cfg.rope_theta)
    x = make_input((B, T, d), seed=C4["xseed"]).to(dev, torch.bfloat16)
    dy = make_input((B, T, d), seed=C4["xseed"] + 100).to(dev, torch.bfloat16)
    ladder = []
    for K in C4["ladder"]:
        st = HipLayerStack(cfg, n_layers, B, T, schedule=uniform_chunks(T, c, K), device=dev, tape=True,
                           wavefront=True)
        st.load([sd] * n_layers, cos, sin)
        for _ in range(warmup):
            st.step(x, dy)
        dt = timed(lambda: st.step(x, dy), steps)
        fpt = fwd_flops_per_token(d, T, c, K)
        ladder.append({"K": K, "ms_per_layer_fwdbwd": dt * 1e3 / n_layers,
                       "layer_tokens_per_s": B * T * n_layers / dt,
                       "frac_fwdbwd": 3 * fpt * B * T * n_layers / dt / 1e12 / PEAK_BF16_TFLOPS})
        del st
        torch.cuda.empty_cache()
    return {"workload": f"C4: {n_layers} attention sublayers of the d=2048 trunk (16x128), B={B} T={T} c={c}, "
                        "layer-batched (wavefront) forward (tape) + reverse-scan backward per K",
            "n_layers": n_layers, "steps": steps, "warmup": warmup, "ladder": ladder}


def bench_stack(dev, n_layers=8, steps=3, warmup=1):
    """A stack of n_layers 340M-shape attention sublayers (BASELINE config 3's layer, one seed per
    layer), forward (tape) + reverse-scan backward per step, layer by layer and layer-batched
    (HipLayerStack(wavefront=True): each kernel of a wavefront step one launch over every active
    layer; bit-identical results). Throughput in layer-tokens/s (B*T tokens through one layer)."""
    from dual_mod_public_amd.stack import HipLayerStack
    B, T, d, h, c, K = C2["B"], C2["T"], C2["d"], C2["h"], C2["c"], C2["K"]
    cfg = DualModConfig(d_model=d, n_heads=h, ctx_mod="mult_res", max_seq_len=T, dtype="bf16")
    sds = [{k: v.to(dev) for k, v in make_state_dict(cfg, seed=C2["wseed"] + l).items()} for l in range(n_layers)]
    cos, sin = build_rope_cache(T, d // h, cfg.rope_theta)
    st = HipLayerStack(cfg, n_layers, B, T, schedule=uniform_chunks(T, c, K), device=dev, tape=True)
    st.load(sds, cos, sin)
    x = make_input((B, T, d), seed=C2["xseed"]).to(dev, torch.bfloat16)
    dy = make_input((B, T, d), seed=C2["xseed"] + 100).to(dev, torch.bfloat16)
    out = {"workload": f"{n_layers} attention sublayers of the 340M shape (B={B} T={T} d={d} {h}x{d // h} c={c} "
                       f"K={K}), forward (tape) + reverse-scan backward per step",
           "n_layers": n_layers, "steps": steps, "warmup": warmup}
    fpt = fwd_flops_per_token(d, T, c, K)
    for mode in (False, True):
        st.wavefront = mode
        for _ in range(warmup):
            st.step(x, dy)
        dt = timed(lambda: st.step(x, dy), steps)
        key = "wavefront" if mode else "layer_by_layer"
        out[key] = {"ms_per_step": dt * 1e3, "ms_per_layer": dt * 1e3 / n_layers,
                    "layer_tokens_per_s": B * T * n_layers / dt,
                    "path_frac": 3 * fpt * B * T * n_layers / dt / 1e12 / PEAK_BF16_TFLOPS}
    out["speedup"] = out["layer_by_layer"]["ms_per_step"] / out["wavefront"]["ms_per_step"]
    del st
    torch.cuda.empty_cache()
    return out


def bench_graph_decode(dev, B=8, n_layers=24, P_max=2048, steps=100, warmup=5):
    """Greedy decode of a 24-layer 340M-shape DualModLM (vocab 32000, random weights) through the
    one-graph-per-token GraphDecoder against the eager decode_step, ms per token at B rows."""
    from dual_mod_public_amd.graph_decode import GraphDecoder
    from dual_mod_public_amd.model import DualModLM
    from dual_mod_public_amd.synthetic import make_lm_state_dict
    cfg = DualModConfig(d_model=C2["d"], n_heads=C2["h"], n_layers=n_layers, vocab_size=32000, max_seq_len=P_max,
                        ctx_mod="mult_res")
    m = DualModLM(cfg).to(dev).eval()
    m.load_state_dict({k: v.to(dev) for k, v in make_lm_state_dict(cfg, seed=C2["wseed"]).items()})
    dec = GraphDecoder(m, B, P_max).capture()
    tok = torch.randint(0, cfg.vocab_size, (B, 1), generator=torch.Generator().manual_seed(3)).to(dev)
    dec.reset()
    dec.tok.copy_(tok)
    for _ in range(warmup):
        dec.step()
    dt_g = timed(dec.step, steps)
    caches = m.decode_init()
    with torch.no_grad():
        for p in range(warmup):
            m.decode_step(tok, p, caches)
        pos = [warmup]

        def eager():
            m.decode_step(tok, pos[0], caches)
            pos[0] += 1
        dt_e = timed(eager, max(10, steps // 5))
    del dec, caches, m
    torch.cuda.empty_cache()
    return {"workload": f"greedy decode, {n_layers}-layer 340M-shape DualModLM (vocab 32000), B={B}, "
                        f"tape {P_max} rows, positions {warmup}..{warmup + steps}",
            "graph_ms_per_token": dt_g * 1e3, "graph_tokens_per_s": B / dt_g,
            "eager_ms_per_token": dt_e * 1e3, "speedup": dt_e / dt_g}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-T", type=int, default=0,
                    help="T-prefix of the CPU baseline sample (0: the whole T)")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-c1", action="store_true", help="skip BASELINE config 1 (the CPU-runnable layer)")
    ap.add_argument("--no-c4", action="store_true", help="skip the config-4 K ladder")
    ap.add_argument("--no-stack", action="store_true", help="skip the layer-stack (layer-batched) sub-benchmark")
    ap.add_argument("--c4-trunk-layers", type=int, default=24,
                    help="layers of the config-4 trunk training step (0: skip)")
    ap.add_argument("--c4-stack-layers", type=int, default=8,
                    help="layers of the config-4 layer-batched K ladder (0: skip)")
    ap.add_argument("--stack-layers", type=int, default=24,
                    help="layers of the stack sub-benchmark (24: the 340M model's depth)")
    ap.add_argument("--no-graph-decode", action="store_true", help="skip the model-level graph decode")
    ap.add_argument("--decode-steps", type=int, default=0)
    ap.add_argument("--kernel", default="sweep1", help="kernel class timed for the roofline")
    ap.add_argument("--workload", default="fwdbwd", choices=["fwdbwd", "fwd", "c4"],
                    help="fwdbwd: C3 (340M-shape layer fwd+bwd, the headline); fwd: C2 forward; "
                         "c4: one layer of the config-4 trunk (d=2048, 16x128, B=4, T=4096) fwd+bwd")
    ap.add_argument("--sweeps", type=int, default=0, help="Jacobi sweeps K per chunk (default 4)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first run a plain 256 MiB device copy 3x (the known-size kernel that "
                         "scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings to bytes)")
    ap.add_argument("--headline-only", action="store_true",
                    help="time only the headline mode (no forward-only / other-backward-mode lines)")
    ap.add_argument("--recompute", action="store_true",
                    help="headline without the forward tape (backward recomputes every cell)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build runs on one GPU only: the DM hot path is measured "
                                   "on one MI355X (see the sharding notes); --gpus must be 1"}))
        sys.exit(2)
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        sys.exit(1)
    dev = torch.device("cuda:0")
    L.load()
    t_start = time.time()

    def note(what):   # progress on stderr (stdout carries the one JSON line)
        print(f"[bench] {what} done at {time.time() - t_start:.0f} s", file=sys.stderr, flush=True)

    if args.copy_calibration:
        src = torch.ones(COPY_CAL_BYTES // 2, device=dev, dtype=torch.bfloat16)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    shape = C4 if args.workload == "c4" else C2
    B, T, d, h, c, K = shape["B"], shape["T"], shape["d"], shape["h"], shape["c"], shape["K"]
    K = args.sweeps or K
    cfg = DualModConfig(d_model=d, n_heads=h, ctx_mod="mult_res", max_seq_len=T, dtype="bf16")
    sd, cell, x, cos, sin, bufs, Kc, Vc, ocat, y = build_layer(cfg, B, T, dev, seeds=shape)
    sched = uniform_chunks(T, c, K)

    grads = LayerGrads(cfg, dev)
    dy = make_input((B, T, d), seed=shape["xseed"] + 100).to(dev, torch.bfloat16)
    dx = torch.empty_like(x)
    fwdbwd = args.workload in ("fwdbwd", "c4")

    use_tape = fwdbwd and not args.recompute
    tape = cell.new_tape(sched) if fwdbwd else None

    def step_fwd():
        cell.layer_forward(x, y, cos, sin, sched, Kc, Vc, ocat, bufs)

    def make_step(taped):
        tp = tape if taped else None

        def step():
            cell.layer_forward(x, y, cos, sin, sched, Kc, Vc, ocat, bufs, tape=tp)
            if fwdbwd:
                cell.layer_backward(x, dy, dx, cos, sin, sched, Kc, Vc, ocat, bufs, grads, tape=tp)
        return step

    step = make_step(use_tape)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    sweeps = sum(k for _, _, k in sched)
    per_step_launches = sweeps * (2 if fwdbwd else 1)
    # the headline: the timed steps with nothing armed; then the same steps again with the
    # roofline kernel's launches stamping their event pairs (the kernels unmodified), and once
    # more with the kernels' own device-clock stamps (these cost ~0.5 us per launch, so they
    # get a pass of their own)
    dt = timed(step, args.steps)
    cap = args.steps * per_step_launches * 2 + 64
    with L.KernelTimer(args.kernel, max_launches=cap, device_clock=False) as kt:
        dt_instr = timed(step, args.steps)
    with L.KernelTimer(args.kernel, max_launches=cap) as kt_dev:
        timed(step, args.steps)
    # forward alone, and the other backward mode (reported beside the headline)
    dt_fwd = dt_other = None
    if not args.headline_only:
        dt_fwd = timed(step_fwd, args.steps)
    if fwdbwd and not args.headline_only:
        other = make_step(not use_tape)
        other()
        dt_other = timed(other, args.steps)
    tokens = B * T
    fpt = fwdbwd_flops_per_token(d, T, c, K) if fwdbwd else fwd_flops_per_token(d, T, c, K)
    if args.kernel == "sweep1":
        per_launch = sweep1_flops(B * c, d)
        kname = ("k_gemm<SrcRowsRs, EpiSweep1> (sweep GEMM 1: RMSNorm(o) . [w_kctx|g_k|v_map|g_v]^T, "
                 "norm weight folded into W, row scale in the epilogue)")
    elif args.kernel == "layer":
        per_launch = fwd_flops_per_token(d, T, c, K) * tokens
        kname = "whole dm_layer_fwd call"
    else:
        per_launch = float("nan")
        kname = args.kernel
    avg_ms = kt.avg_ms
    achieved = per_launch / (avg_ms / 1e3) / 1e12 if kt.n else None
    mode = "exact recompute" if not use_tape else "sweep states from the forward's HBM tape"
    if args.workload == "c4":
        wl = f"C4: one layer of the d=2048 trunk, forward + reverse-scan backward ({mode})"
    elif fwdbwd:
        wl = f"C3: 340M-shape DM layer forward + reverse-scan backward ({mode})"
    else:
        wl = "C2: 340M-shape DM layer forward"
    out = {
        "metric": f"DM sweep tokens/s/GPU ({'fwd+bwd' if fwdbwd else 'forward'}, c={c}, K={K})" +
                  (" per layer, C4" if args.workload == "c4" else ""),
        "value": tokens / dt, "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": dt * 1e3, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic (seeded N(0,1) x and dy, N(0,0.02) weights)",
        "config": {"workload": wl + f", B={B} T={T} d={d} {h}x{d // h} c={c} K={K}, {T // c} chunks "
                               "Gauss-Seidel",
                   "global_batch": B, "seq_len": T, "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": achieved, "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": (achieved / PEAK_BF16_TFLOPS) if achieved else None,
                     "traffic": traffic_from_profile(args.kernel), "kernel": kname,
                     "flops_per_launch": per_launch, "avg_launch_ms": avg_ms,
                     "avg_launch_ms_device": kt_dev.device_avg_ms,
                     "frac_device_span": (per_launch / (kt_dev.device_avg_ms / 1e3) / 1e12 / PEAK_BF16_TFLOPS
                                          if kt_dev.device_avg_ms else None),
                     "timing": TIMING_NOTE, "launches": kt.n, "instrumented_ms_per_step": dt_instr * 1e3},
        "path_roofline": {"flops_per_token": fpt, "achieved_tflops": fpt * tokens / dt / 1e12,
                          "frac": fpt * tokens / dt / 1e12 / PEAK_BF16_TFLOPS},
    }
    if dt_fwd is not None:
        out["forward_only"] = {"ms_per_step": dt_fwd * 1e3, "tokens_per_s": tokens / dt_fwd,
                               "frac": fwd_flops_per_token(d, T, c, K) * tokens / dt_fwd / 1e12 / PEAK_BF16_TFLOPS}
    if fwdbwd:
        out["tape_bytes"] = tape.numel()
    if dt_other is not None:
        # the other backward mode, with the headline's fields (C3 as BASELINE words it is the
        # exact-recompute mode; the tape holds the same sweep states bit for bit)
        out["recompute" if use_tape else "tape"] = {
            "value": tokens / dt_other, "unit": "tokens/s", "ms_per_step": dt_other * 1e3,
            "tokens_per_s": tokens / dt_other,
            "path_frac": fpt * tokens / dt_other / 1e12 / PEAK_BF16_TFLOPS,
            "workload": wl.replace(mode, "exact recompute" if use_tape else "sweep states from the forward's HBM tape")}
    del cell, bufs, Kc, Vc, ocat, y, x, dx, dy, grads, tape
    torch.cuda.empty_cache()
    note("headline")
    if not args.no_c4 and args.workload != "c4":
        out["c4"] = bench_c4_ladder(dev)
        note("c4 ladder")
        if args.c4_trunk_layers > 0:
            out["c4"]["trunk"] = bench_c4_trunk(dev, n_layers=args.c4_trunk_layers)
            note("c4 trunk")
        if args.c4_stack_layers > 0:
            out["c4"]["wavefront"] = bench_c4_wavefront(dev, n_layers=args.c4_stack_layers)
            note("c4 wavefront")
    if not args.no_stack and args.workload != "c4":
        out["stack"] = bench_stack(dev, n_layers=args.stack_layers)
        note("stack")
    if not args.no_graph_decode and args.workload != "c4":
        out["graph_decode"] = bench_graph_decode(dev)
        note("graph decode")
    if not args.no_decode:
        out["decode"] = bench_decode(dev, args.decode_steps or None, with_cpu=not args.no_cpu_baseline)
        note("decode")
    if not args.no_c1 and args.workload != "c4":
        out["c1"] = bench_c1(dev, with_cpu=not args.no_cpu_baseline)
        note("c1")
    if not args.no_cpu_baseline and args.workload != "c4":
        out["cpu_baseline"] = cpu_baseline(cfg, sd, T, B, fwdbwd, args.cpu_T)
        if fwdbwd and "forward_only" in out:
            # BASELINE config 2 (the forward of the same layer) on the same cores
            out["forward_only"]["cpu_baseline"] = cpu_baseline(cfg, sd, T, B, False, args.cpu_T)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
