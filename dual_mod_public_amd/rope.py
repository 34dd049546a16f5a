"""RoPE tables (models/dualmod/rope.py:13-19): cos/sin [T, dh/2] fp32,
inv_freq = theta^(-2i/dh), half-split pairs (i, i + dh/2). The rotation itself
is applied inside the HIP kernels (projection epilogue for q / raw k, sweep
epilogue for the blended key)."""

import torch


def build_rope_cache(max_seq_len, head_dim, theta, device=None, use_rope=True):
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, device=device, dtype=torch.float32)
                                / head_dim))
    t = torch.arange(max_seq_len, device=device, dtype=torch.float32)
    freqs = torch.outer(t, inv_freq)
    cos, sin = freqs.cos(), freqs.sin()
    if not use_rope:                      # NoPE (model.py:146-147): identity rotation
        cos, sin = torch.ones_like(cos), torch.zeros_like(sin)
    return cos, sin
