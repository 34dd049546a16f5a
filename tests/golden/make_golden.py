"""Write golden vectors for the DM attention path from the reference itself.

Run in the build container only (the reference is not on the GPU box):

    python tests/golden/make_golden.py /path/to/reference [--only case ...]

The reference's own tests never exercise ctx_mod="mult_res" and hold no stored
vectors, so the absolute numerics of refine_kv / sequential_scan / the Jacobi
cell / decode_step are pinned here by running the reference's own functions
on seeded inputs and storing inputs-by-seed + outputs as fixtures:

  * models/dualmod/scan.py:60 ``sequential_scan`` and the eager per-position
    oracle ``engines/wavescan/cells/reference.py:15 eager_layer`` (o, K, V rows)
  * engines/wavescan/engine/forward.py:95 ``layer_forward`` with
    ``uniform_chunks(T, c, K<c)`` (chunked Jacobi, the K<c oracle)
  * models/dualmod/attention.py:564 ``decode_step`` over T steps
  * autograd through ``sequential_scan`` at a tiny config (all param grads)

Weights/inputs come from dual_mod_public_amd.synthetic (numpy seeds), so the
fixture stores only seeds, config and outputs. Outputs are float32.
"""

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)

from dual_mod_public_amd.config import DualModConfig  # noqa: E402
from dual_mod_public_amd.synthetic import make_input, make_state_dict  # noqa: E402

# the configurations the fixtures cover (also read back by the tests)
CASES = {
    # B=2, T=64, d=256, 4 heads x 64, mult_res, c=16
    "c1_mult_res": dict(cfg=dict(d_model=256, n_heads=4, ctx_mod="mult_res"),
                        B=2, T=64, c=16, K=4, wseed=11, xseed=12, dtype="float32"),
    # linear ctx_mod (the reference tests' arm), same shape
    "c1_linear": dict(cfg=dict(d_model=256, n_heads=4, ctx_mod="linear"),
                      B=2, T=64, c=16, K=4, wseed=21, xseed=22, dtype="float32",
                      full=False),
    # ctx_mod fusion (attention.py:341-342), v_pre live (random, not the reference's zero init)
    "c1_fusion": dict(cfg=dict(d_model=256, n_heads=4, ctx_mod="fusion"),
                      B=2, T=64, c=16, K=4, wseed=51, xseed=52, dtype="float32"),
    # knob combo: lambda leak, K-norm, V-ctx-norm, kmod raw heads, clamp
    "knobs_mult_res": dict(cfg=dict(d_model=128, n_heads=4, ctx_mod="mult_res",
                                    mult_res_lambda=0.97, k_ctx_norm="rms",
                                    v_ctx_norm="rms", kmod_vraw_heads=1,
                                    v_clamp_tau=1.0),
                           B=2, T=32, c=8, K=3, wseed=31, xseed=32, dtype="float32"),
}
# autograd through the scan (tiny, all grads stored)
GRAD_CASE = dict(cfg=dict(d_model=64, n_heads=2, ctx_mod="mult_res"),
                 B=2, T=24, wseed=41, xseed=42, gseed=43)


def _ref_modules(ref_root):
    sys.path.insert(0, ref_root)
    from models.dualmod.config import DualModConfig as RefCfg
    from models.dualmod.attention import DualModAttention, RMSNorm
    from models.dualmod.rope import build_rope_cache
    from models.dualmod.scan import sequential_scan
    from engines.wavescan.cells.reference import eager_layer
    from engines.wavescan.engine.forward import MaskCache, layer_forward
    from engines.wavescan.engine.schedule import uniform_chunks
    return dict(RefCfg=RefCfg, DualModAttention=DualModAttention, RMSNorm=RMSNorm,
                build_rope_cache=build_rope_cache, sequential_scan=sequential_scan,
                eager_layer=eager_layer, MaskCache=MaskCache,
                layer_forward=layer_forward, uniform_chunks=uniform_chunks)


def _build_attn(R, kw, wseed, T):
    cfg_kw = dict(n_layers=1, max_seq_len=max(T, 8), checkpoint_chunk=0, dtype="fp32")
    cfg_kw.update(kw)
    ref_cfg = R["RefCfg"](**cfg_kw)
    my_cfg = DualModConfig(**cfg_kw)
    sd = make_state_dict(my_cfg, seed=wseed)
    attn = R["DualModAttention"](ref_cfg).eval()
    attn_sd = {k: v for k, v in sd.items() if not k.startswith("attn_norm")}
    missing, unexpected = attn.load_state_dict(attn_sd, strict=True), None
    del missing, unexpected
    return ref_cfg, attn, sd


def main(ref_root, only=None):
    """Write every case, or with ``only`` just those cases, merged into the existing
    fixture (its other arrays are kept as they are)."""
    torch.set_grad_enabled(False)
    R = _ref_modules(ref_root)
    out = {}
    path = os.path.join(HERE, "dm_golden.npz")
    if only:
        with np.load(path) as old:
            out = {k: old[k] for k in old.files}
    for name, case in CASES.items():
        if only and name not in only:
            continue
        B, T, c, K = case["B"], case["T"], case["c"], case["K"]
        ref_cfg, attn, sd = _build_attn(R, case["cfg"], case["wseed"], T)
        d = ref_cfg.d_model
        cos, sin = R["build_rope_cache"](T, ref_cfg.head_dim, ref_cfg.rope_theta)
        xhat = make_input((B, T, d), seed=case["xseed"])
        # exact scan: o_cat from sequential_scan, cache rows from eager_layer
        o_cat = R["sequential_scan"](attn, xhat, cos, sin)
        o_h, K_rows, V_rows = R["eager_layer"](attn, xhat, cos, sin)
        assert torch.equal(attn._merge(o_h), o_cat)
        out[f"{name}/scan_o"] = o_cat.numpy().astype(np.float32)
        if case.get("full", True):
            out[f"{name}/scan_K"] = K_rows.numpy().astype(np.float32)
            out[f"{name}/scan_V"] = V_rows.numpy().astype(np.float32)
        # chunked Jacobi at K < c
        masks = R["MaskCache"]("cpu")
        Kc = torch.zeros(B, ref_cfg.n_heads, T, ref_cfg.head_dim)
        Vc = torch.zeros_like(Kc)
        o_j = R["layer_forward"](attn, xhat, cos, sin, R["uniform_chunks"](T, c, K),
                                 Kc, Vc, masks)
        out[f"{name}/jacobi_o"] = o_j.numpy().astype(np.float32)
        if not case.get("full", True):
            continue
        out[f"{name}/jacobi_K"] = Kc.numpy().astype(np.float32)
        out[f"{name}/jacobi_V"] = Vc.numpy().astype(np.float32)
        # decode: T steps from an empty cache
        cache = {"K": None, "V": None}
        ys = [attn.decode_step(xhat[:, t:t + 1], t, cache, cos, sin) for t in range(T)]
        out[f"{name}/decode_y"] = torch.cat(ys, dim=1).numpy().astype(np.float32)
        assert torch.allclose(cache["K"], K_rows, rtol=1e-4, atol=1e-5)

    if only:
        np.savez_compressed(path, **out)
        print(f"wrote {path}: {len(out)} arrays ({', '.join(only)} rewritten)")
        return
    # gradients through the exact scan: y = x + wo(scan(attn_norm(x)))
    g = GRAD_CASE
    B, T = g["B"], g["T"]
    ref_cfg, attn, sd = _build_attn(R, g["cfg"], g["wseed"], T)
    d = ref_cfg.d_model
    norm = R["RMSNorm"](d)
    norm.weight.data.copy_(sd["attn_norm.weight"])
    cos, sin = R["build_rope_cache"](T, ref_cfg.head_dim, ref_cfg.rope_theta)
    x = make_input((B, T, d), seed=g["xseed"]).requires_grad_(True)
    dy = make_input((B, T, d), seed=g["gseed"])
    with torch.enable_grad():
        attn.train()
        y = x + attn.wo(R["sequential_scan"](attn, norm(x), cos, sin))
        (y * dy).sum().backward()
    out["grad/y"] = y.detach().numpy().astype(np.float32)
    out["grad/x"] = x.grad.numpy().astype(np.float32)
    for pname, p in attn.named_parameters():
        out[f"grad/{pname}"] = p.grad.numpy().astype(np.float32)
    out["grad/attn_norm.weight"] = norm.weight.grad.numpy().astype(np.float32)

    np.savez_compressed(path, **out)
    print(f"wrote {path}: {len(out)} arrays, {os.path.getsize(path) / 1024:.0f} KiB")


if __name__ == "__main__":
    # python tests/golden/make_golden.py [/path/to/reference] [--only case ...]
    args = sys.argv[1:]
    only = args[args.index("--only") + 1:] if "--only" in args else None
    pos = [a for a in (args[:args.index("--only")] if "--only" in args else args)]
    main(pos[0] if pos else "/root/reference", only)
