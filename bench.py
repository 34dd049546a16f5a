"""Benchmark of the Dual-Mod attention hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload fwdbwd|fwd]
                    [--no-cpu-baseline] [--no-decode]

One step = one DM attention layer of the 340M shape (B=8, T=2048, d=1024,
16 heads x 64, c=64, K=4 Jacobi sweeps chained over 32 chunks, bf16 storage /
fp32 accumulate) through libdm_hip.so: the forward (attn_norm + projections,
the 32 chunk cells = committed accumulator + 4 sweeps each, W_O with the
residual) and, for the default fwdbwd workload, the
reverse-scan backward producing dx and every parameter gradient for an upstream
dy ~ N(0,1). The forward keeps every cell's sweep states in an HBM tape (1.9 GB
for this layer) that the backward reads instead of recomputing them; the
reference's exact-recompute mode (same values bit for bit) is timed beside it
(--recompute makes it the headline). Inputs (x, dy, weights, RoPE tables) are
resident in HBM before timing starts.

Prints ONE JSON line (rank 0): the headline sweep throughput in tokens/s, the
roofline of the dominant kernel timed with HIP events inside the timed region,
the path-level roofline, the CPU baseline (the oracle's chunked-Jacobi layer
forward timed on this host's cores on a bounded sample) and the decode
sub-benchmark (batch 64, bf16 tape of 32768 positions, HBM GB/s).
"""

import argparse
import json
import os
import sys
import time

import torch

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

from dual_mod_public_amd import _lib as L  # noqa: E402
from dual_mod_public_amd.config import DualModConfig  # noqa: E402
from dual_mod_public_amd.decode import StaticTape  # noqa: E402
from dual_mod_public_amd.engine import HipSweepCell, uniform_chunks  # noqa: E402
from dual_mod_public_amd.rope import build_rope_cache  # noqa: E402
from dual_mod_public_amd.synthetic import make_input, make_state_dict  # noqa: E402

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
COPY_CAL_BYTES = 256 << 20  # --copy-calibration: bytes read (and written) per copy dispatch
# HBM bytes per launch of the roofline kernels (read + written), from rocprofv3 --pmc FETCH_SIZE and
# WRITE_SIZE passes over this script (profiles/traffic_sweep1_decode.md has the commands and raw
# readings), each scaled by what the counter reads for the 256 MiB --copy-calibration copy.
# sweep1: the N = B*c = 512-row launches at C3 (tape mode); dec_read: launches at P = 32768..32783.
TRAFFIC_BYTES = {"sweep1": 34.96e6, "dec_read": 8613.0e6}
TIMING_NOTE = ("avg_launch_ms: per-dispatch span from the device clock (s_memrealtime, first block "
               "start to last block end), recorded by the kernel itself over a second pass of the timed "
               "steps (instrumented_ms_per_step); avg_launch_ms_events: HIP event pair around each launch "
               "on its stream (adds queue time)")

# BASELINE config 2 (forward) — the 340M-shape DM layer
C2 = dict(B=8, T=2048, d=1024, h=16, c=64, K=4, wseed=1, xseed=2)
# BASELINE config 4 — one layer of the 24-layer d=2048 trunk (16 heads x 128), K from --sweeps
C4 = dict(B=4, T=4096, d=2048, h=16, c=64, K=4, wseed=1, xseed=2)
# BASELINE config 5 — incremental decode
C5 = dict(B=64, d=1024, h=16, P0=32768, steps=256, wseed=3, xseed=4, tseed=5)


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


def build_layer(cfg, B, T, dev):
    sd = make_state_dict(cfg, seed=C2["wseed"])
    cell = HipSweepCell(cfg, B, T, device=dev, dtype=torch.bfloat16)
    cell.pack({k: v.to(dev) for k, v in sd.items()})
    x = make_input((B, T, cfg.d_model), seed=C2["xseed"]).to(dev, torch.bfloat16)
    cos, sin = build_rope_cache(T, cfg.head_dim, cfg.rope_theta, device=dev)
    bufs = cell.new_bufs(T)
    K = torch.zeros(B, cfg.n_heads, T, cfg.head_dim, device=dev, dtype=torch.bfloat16)
    V = torch.zeros_like(K)
    ocat = torch.empty_like(x)
    y = torch.empty_like(x)
    return sd, cell, x, cos.contiguous(), sin.contiguous(), bufs, K, V, ocat, y


def cpu_baseline(cfg, sd, T, B, fwdbwd, cpu_T=0):
    """The oracle's chunked-Jacobi layer (same schedule, fp32 torch) on this host's cores:
    forward only, or forward + autograd backward, over the whole workload or, with
    cpu_T < T, a T-prefix sample (the same per-token work at a shorter committed prefix)."""
    import oracle as O
    nthr = min(os.cpu_count() or 1, 16)
    torch.set_num_threads(nthr)
    Ts = min(T, cpu_T) if cpu_T else T
    x = make_input((B, Ts, cfg.d_model), seed=C2["xseed"])
    cos, sin = O.build_rope_cache(Ts, cfg.head_dim, cfg.rope_theta)
    sched = O.uniform_chunks(Ts, C2["c"], C2["K"])
    if fwdbwd:
        sdf = {k: v.float().clone().requires_grad_(True) for k, v in sd.items()}
        x.requires_grad_(True)
        dy = make_input((B, Ts, cfg.d_model), seed=C2["xseed"] + 100)
        t0 = time.perf_counter()
        y = O.dm_layer(cfg, sdf, x, cos, sin, schedule=sched)
        (y * dy).sum().backward()
        dt = time.perf_counter() - t0
        span = "the whole workload" if Ts == T else f"T-prefix of {T}"
        what = f"layer forward + autograd backward at B={B}, T={Ts} ({span}; c=64, K=4)"
    else:
        sdf = {k: v.float() for k, v in sd.items()}
        with torch.no_grad():
            t0 = time.perf_counter()
            O.dm_layer(cfg, sdf, x, cos, sin, schedule=sched)
            dt = time.perf_counter() - t0
        what = f"layer forward at B={B}, T={Ts} (c=64, K=4)"
    return dict(value=B * Ts / dt, unit="tokens/s", cores=nthr, kind="port",
                sample=f"{what}, fp32 torch CPU oracle, {dt:.2f} s wall")


def bench_decode(dev, steps_override=None):
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

    # warm-up pass over the first few slots, then restore nothing (slots are rewritten)
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
    read_avg_ms = kt.device_avg_ms if kt.device_avg_ms is not None else kt.avg_ms
    read_avg_s = read_avg_ms / 1e3
    read_bytes_per_launch = tape_bytes / steps
    return {
        "metric": "decode HBM GB/s (attend_one+refine_kv over the tape, append)",
        "value": total / wall / 1e9, "unit": "GB/s", "steps": steps, "ms_per_step": wall / steps * 1e3,
        "tokens_per_s": B * steps / wall,
        "config": {"workload": "C5 decode: B=64, bf16 tape 32768..33023 positions, d=1024, 16x64",
                   "algorithmic_bytes": total},
        "roofline": {"bound": "hbm", "achieved": read_bytes_per_launch / read_avg_s / 1e9,
                     "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": read_bytes_per_launch / read_avg_s / 1e9 / PEAK_HBM_GBS,
                     "traffic": TRAFFIC_BYTES["dec_read"], "kernel": "k_decode_partial",
                     "avg_launch_ms": read_avg_ms, "avg_launch_ms_events": kt.avg_ms,
                     "timing": TIMING_NOTE, "launches": kt.n},
        "path_frac_of_hbm_peak": total / wall / 1e9 / PEAK_HBM_GBS,
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-T", type=int, default=0,
                    help="CPU baseline over a T-prefix of the workload (default: the whole T)")
    ap.add_argument("--no-decode", action="store_true")
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
    sd, cell, x, cos, sin, bufs, Kc, Vc, ocat, y = build_layer(cfg, B, T, dev)
    sched = uniform_chunks(T, c, K)

    from dual_mod_public_amd.engine import LayerGrads
    grads = LayerGrads(cfg, dev)
    dy = make_input((B, T, d), seed=C2["xseed"] + 100).to(dev, torch.bfloat16)
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

    def timed(fn, steps):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / steps

    step = make_step(use_tape)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    sweeps = sum(k for _, _, k in sched)
    per_step_launches = sweeps * (2 if fwdbwd else 1)
    # the headline: the timed steps with nothing armed; then the same steps again with
    # the roofline kernel's per-dispatch timing armed (its device-clock stamps and event
    # pairs cost ~5% of the step, so they stay out of the headline's clock)
    dt = timed(step, args.steps)
    with L.KernelTimer(args.kernel, max_launches=args.steps * per_step_launches * 2 + 64) as kt:
        dt_instr = timed(step, args.steps)
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
    avg_ms = kt.device_avg_ms if kt.device_avg_ms is not None else kt.avg_ms
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
                     "traffic": TRAFFIC_BYTES.get(args.kernel), "kernel": kname, "flops_per_launch": per_launch,
                     "avg_launch_ms": avg_ms, "avg_launch_ms_events": kt.avg_ms,
                     "timing": TIMING_NOTE if kt.device_avg_ms is not None else "HIP event pairs",
                     "launches": kt.n, "instrumented_ms_per_step": dt_instr * 1e3},
        "path_roofline": {"flops_per_token": fpt, "achieved_tflops": fpt * tokens / dt / 1e12,
                          "frac": fpt * tokens / dt / 1e12 / PEAK_BF16_TFLOPS},
    }
    if dt_fwd is not None:
        out["forward_only"] = {"ms_per_step": dt_fwd * 1e3, "tokens_per_s": tokens / dt_fwd,
                               "frac": fwd_flops_per_token(d, T, c, K) * tokens / dt_fwd / 1e12 / PEAK_BF16_TFLOPS}
    if fwdbwd:
        out["tape_bytes"] = tape.numel()
    if dt_other is not None:
        out["recompute" if use_tape else "tape"] = {"ms_per_step": dt_other * 1e3,
                                                    "tokens_per_s": tokens / dt_other}
    if not args.no_decode:
        del cell, bufs, Kc, Vc, ocat, y, x, dx, dy, grads, tape
        torch.cuda.empty_cache()
        out["decode"] = bench_decode(dev, args.decode_steps or None)
    if not args.no_cpu_baseline and args.workload != "c4":
        out["cpu_baseline"] = cpu_baseline(cfg, sd, T, B, fwdbwd, args.cpu_T)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
