"""Shared helpers for the GPU parity tests (HIP path vs the CPU oracle)."""

import json
import os
import sys

import torch

import oracle as O
from dual_mod_public_amd.config import DualModConfig
from dual_mod_public_amd.synthetic import make_input, make_state_dict

DEV = "cuda"


# measured parity errors of this session: (test, {quantity: relerr}, tolerance)
MARGINS = []


def say(msg):
    print(f"[gpu-test] {msg}", flush=True)
    sys.stdout.flush()


def record(test, errs, tol):
    """Keep a test's measured relative errors (written to parity_margins.json in the run's
    output folder at the end of the session)."""
    node = os.environ.get("PYTEST_CURRENT_TEST", "").split(" ")[0].split("::")[-1]
    MARGINS.append({"test": test, "node": node, "tol": tol, "relerr": {k: float(v) for k, v in errs.items()}})


def write_margins(repo):
    """parity_margins.json (every recorded error) and parity_margins.md (one row per recorded
    check: tolerance, worst relative error, the quantity it was measured on, worst / tolerance)."""
    if not MARGINS:
        return
    out = os.path.join(repo, os.environ.get("DM_RESULTS_DIR", "gpurun_out"))
    os.makedirs(out, exist_ok=True)
    with open(os.path.join(out, "parity_margins.json"), "w") as f:
        json.dump(MARGINS, f, indent=1)
    rows = ["| test | check | tolerance | worst relerr | on | worst / tol |", "|---|---|---|---|---|---|"]
    for m in MARGINS:
        if not m["relerr"]:
            continue
        k = max(m["relerr"], key=m["relerr"].get)
        v = m["relerr"][k]
        rows.append(f"| {m.get('node', '')} | {m['test']} | {m['tol']:.0e} | {v:.2e} | {k} | {v / m['tol']:.2f} |")
    with open(os.path.join(out, "parity_margins.md"), "w") as f:
        f.write("\n".join(rows) + "\n")


def cfg_of(d=256, h=4, ctx_mod="mult_res", T=64, **kw):
    return DualModConfig(d_model=d, n_heads=h, n_layers=1, max_seq_len=T, checkpoint_chunk=0,
                         ctx_mod=ctx_mod, dtype="fp32", **kw)


def setup(cfg, B, T, wseed=11, xseed=12, std=0.02):
    """(sd fp64 CPU, x fp64 CPU, cos/sin fp64 CPU, cos/sin fp32 CPU)."""
    sd = {k: v.double() for k, v in make_state_dict(cfg, seed=wseed, std=std).items()}
    x = make_input((B, T, cfg.d_model), seed=xseed, dtype=torch.float64)
    cos64, sin64 = O.build_rope_cache(T, cfg.head_dim, cfg.rope_theta, dtype=torch.float64)
    cos32, sin32 = O.build_rope_cache(T, cfg.head_dim, cfg.rope_theta, dtype=torch.float32)
    return sd, x, (cos64, sin64), (cos32, sin32)


def to_dev(sd, dtype):
    return {k: v.to(device=DEV, dtype=dtype) for k, v in sd.items()}


def relerr(a, b):
    a = a.double().cpu()
    b = b.double().cpu()
    return ((a - b).norm() / (b.norm() + 1e-30)).item()
