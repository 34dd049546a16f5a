"""Low-rank (factored) gates and context operators: the ``gate_rank`` / ``ctx_rank`` knobs.

The reference factors the two gate projections and the four context operators:

* LoRAGate (models/dualmod/attention.py:24-42), ``w_gk`` / ``w_gv`` when gate_rank > 0:
  in -> r -> out with ``a.weight`` [r, 2d], ``b.weight`` [d, r], ``b.bias`` [d];
  effective weight ``b.weight @ a.weight``.
* LoRALinear (attention.py:45-75), ``w_kctx``, ``w_vctx``, ``v_gate``, ``v_map`` when
  ctx_rank > 0 (attention.py:125-132, 182-183): ``down.weight`` [r, d],
  ``up.weight`` [d, r] (+ ``up.bias`` for v_gate); effective weight
  ``up.weight @ down.weight``.

Its fused engine hands its kernels the dense products (fused_sweep.py:1266-1275) and
chains the dense weight gradients back onto the factors: dA = B^T dW, dB = dW A^T for
W = B A (``_accum_ctx_dW``, fused_sweep.py:43-56; the gate chain, fused_sweep.py:1882-1936).
The HIP path does the same, here on the host side of the boundary: the C ABI only ever
sees dense weights (``dense_params`` before packing) and returns dense gradients
(``factor_grads`` after the backward). The products are r-rank glue outside the sweep
loop, computed once per pack / per backward in fp32 (fp64 for fp64 operands).
"""

import torch

CTX_MATS = ("w_kctx", "w_vctx", "v_gate", "v_map")
GATES = ("w_gk", "w_gv")


def is_factored(sd):
    return any(f"{n}.down.weight" in sd for n in CTX_MATS) or any(f"{n}.a.weight" in sd for n in GATES)


def _mm(a, b):
    """a @ b in fp32, or fp64 when an operand is fp64."""
    t = torch.promote_types(torch.promote_types(a.dtype, b.dtype), torch.float32)
    return a.detach().to(t) @ b.detach().to(t)


def dense_params(sd):
    """A copy of ``sd`` (reference parameter names) in which every factored gate or context
    operator also appears as its dense ``<name>.weight`` (and ``<name>.bias``)."""
    if not is_factored(sd):
        return sd
    out = dict(sd)
    for n in CTX_MATS:
        if f"{n}.down.weight" in sd:
            up = sd[f"{n}.up.weight"]
            out[f"{n}.weight"] = _mm(up, sd[f"{n}.down.weight"]).to(up.dtype)
            if f"{n}.up.bias" in sd:
                out[f"{n}.bias"] = sd[f"{n}.up.bias"]
    for n in GATES:
        if f"{n}.a.weight" in sd:
            b = sd[f"{n}.b.weight"]
            out[f"{n}.weight"] = _mm(b, sd[f"{n}.a.weight"]).to(b.dtype)
            out[f"{n}.bias"] = sd[f"{n}.b.bias"]
    return out


def factor_grads(sd, dense, names):
    """Gradients of the parameters ``names`` of ``sd`` from the dense-layout gradients
    ``dense`` (name -> fp32 tensor, as LayerGrads holds them). Factored names get the
    chain rule through W = up @ down (or b @ a); every other name is looked up as is."""
    g = {}
    for n in names:
        if n in dense:
            g[n] = dense[n]
            continue
        base, _, leaf = n.partition(".")
        if leaf in ("down.weight", "up.weight", "up.bias"):
            if leaf == "up.bias":
                g[n] = dense[f"{base}.bias"]
                continue
            dW = dense[f"{base}.weight"]
            up, down = sd[f"{base}.up.weight"], sd[f"{base}.down.weight"]
            g[n] = _mm(up.t(), dW) if leaf == "down.weight" else _mm(dW, down.t())
        elif leaf in ("a.weight", "b.weight", "b.bias"):
            if leaf == "b.bias":
                g[n] = dense[f"{base}.bias"]
                continue
            dW = dense[f"{base}.weight"]
            a, b = sd[f"{base}.a.weight"], sd[f"{base}.b.weight"]
            g[n] = _mm(b.t(), dW) if leaf == "a.weight" else _mm(dW, a.t())
        else:
            raise KeyError(f"no gradient for parameter {n}")
    return g


class LoRAGate(torch.nn.Module):
    """attention.py:24-42: in -> r -> out, parameters a.weight, b.weight, b.bias."""

    def __init__(self, din, r, dout):
        super().__init__()
        self.a = torch.nn.Linear(din, r, bias=False)
        self.b = torch.nn.Linear(r, dout, bias=True)

    def forward(self, x):
        return self.b(self.a(x))


class LoRALinear(torch.nn.Module):
    """attention.py:45-75: down (din -> r) then up (r -> dout, optional bias)."""

    def __init__(self, din, r, dout, bias=False):
        super().__init__()
        self.down = torch.nn.Linear(din, r, bias=False)
        self.up = torch.nn.Linear(r, dout, bias=bias)

    def forward(self, x):
        return self.up(self.down(x))

    @property
    def weight(self):
        return self.up.weight @ self.down.weight
