"""ctypes binding of libdm_hip.so (the C ABI in include/dm_abi.h).

The library is loaded from the package directory. There is no fallback:
if it is missing or fails to load, every compute entry point raises.
Tensors cross the boundary as raw device pointers; the stream is torch's
current HIP stream.
"""

import ctypes
import os

import torch

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libdm_hip.so")

DM_F32, DM_BF16 = 0, 1
CTX_MOD = {"linear": 0, "mult_res": 1, "mult": 2, "fusion": 3}

c_i32 = ctypes.c_int32
c_vp = ctypes.c_void_p
c_fp = ctypes.c_void_p


class dm_config(ctypes.Structure):
    _fields_ = [("dtype", c_i32), ("B", c_i32), ("d", c_i32), ("h", c_i32), ("dh", c_i32),
                ("ctx_mod", c_i32), ("mult_res_lambda", ctypes.c_float), ("rms_eps", ctypes.c_float),
                ("local_window", c_i32), ("flags", c_i32), ("kmod_vraw_heads", c_i32),
                ("kmod_mode", c_i32), ("v_clamp_tau", ctypes.c_float), ("norms", c_i32),
                ("reserved", c_i32 * 2)]


DM_DECODE_SCRATCH_MAX = 32 << 20   # include/dm_abi.h: static scratch of dm_decode_step_noalloc
DM_FLAG_NO_RESIDUAL = 1
DM_FLAG_FUSED_ATTEND = 2
DM_FLAG_UNFUSED_ATTEND = 4
# per-head RMS norms (dm_config.norms bits) and the gain parameter of each (attention.py:113-166)
DM_NORM_K_CTX, DM_NORM_V_CTX, DM_NORM_V = 1, 2, 4
NORM_KNOBS = (("k_ctx_norm", DM_NORM_K_CTX, "k_gain"), ("v_ctx_norm", DM_NORM_V_CTX, "ctx_gain"),
              ("v_norm", DM_NORM_V, "v_gain"))

# dm_grads fields and the reference parameter each one accumulates
GRAD_FIELDS = (("wq", "wq.weight"), ("wk", "wk.weight"), ("wv", "wv.weight"), ("wo", "wo.weight"),
               ("w_kctx", "w_kctx.weight"), ("w_vctx", "w_vctx.weight"), ("w_gk", "w_gk.weight"),
               ("w_gv", "w_gv.weight"), ("b_gk", "w_gk.bias"), ("b_gv", "w_gv.bias"),
               ("v_gate", "v_gate.weight"), ("b_vgate", "v_gate.bias"), ("v_map", "v_map.weight"),
               ("norm_ctx_w", "norm_ctx.weight"), ("attn_norm_w", "attn_norm.weight"),
               ("v_pre", "v_pre.weight"), ("k_gain", "k_gain"), ("ctx_gain", "ctx_gain"),
               ("v_gain", "v_gain"))


class dm_grads(ctypes.Structure):
    _fields_ = [(f, c_vp) for f, _ in GRAD_FIELDS]


class dm_params(ctypes.Structure):
    _fields_ = [(n, c_vp) for n in ("wq", "wk", "wv", "wo", "w_kctx", "w_vctx", "w_gk", "w_gv",
                                    "b_gk", "b_gv", "v_gate", "b_vgate", "v_map", "norm_ctx_w",
                                    "attn_norm_w", "v_pre", "k_gain", "ctx_gain", "v_gain")]


class dm_packed(ctypes.Structure):
    _fields_ = [(n, c_vp) for n in ("w_proj", "b_proj", "w_sweep", "w_vctx", "norm_ctx_w",
                                    "attn_norm_w", "wo", "w_proj_t", "w_sweep_t", "w_vctx_t",
                                    "wo_t", "gains")]


class dm_layer_bufs(ctypes.Structure):
    _fields_ = [("T", c_i32), ("xhat", c_vp), ("qr", c_vp), ("kraw", c_vp), ("kself", c_vp),
                ("vraw", c_vp), ("glogx", c_vp), ("sig", c_vp), ("vpre", c_vp)]


class dm_cell_args(ctypes.Structure):
    _fields_ = [("pos0", c_i32), ("c", c_i32), ("n_sweeps", c_i32), ("cache_T", c_i32),
                ("K_cache", c_vp), ("V_cache", c_vp), ("ocat", c_vp), ("o_last", c_vp),
                ("workspace", c_vp), ("workspace_bytes", ctypes.c_size_t), ("K_rows", c_vp),
                ("V_rows", c_vp), ("rows_T", c_i32), ("reserved_", c_i32)]


class dm_cell_bwd_args(ctypes.Structure):
    _fields_ = [("sched", ctypes.POINTER(c_i32)), ("n_cells", c_i32), ("cell", c_i32), ("cache_T", c_i32),
                ("K_cache", c_vp), ("V_cache", c_vp), ("dK_gc", c_vp), ("dV_gc", c_vp), ("tape", c_vp),
                ("tape_bytes", ctypes.c_size_t), ("workspace", c_vp), ("workspace_bytes", ctypes.c_size_t)]


class dm_decode_args(ctypes.Structure):
    _fields_ = [("pos", c_i32), ("tape_T", c_i32), ("xhat", c_vp), ("K_tape", c_vp),
                ("V_tape", c_vp), ("o_cat", c_vp), ("y", c_vp), ("workspace", c_vp),
                ("workspace_bytes", ctypes.c_size_t), ("pos_dev", c_vp)]


class dm_mlp_packed(ctypes.Structure):
    _fields_ = [(n, c_vp) for n in ("w13", "w2", "w13_t", "w2_t", "norm_w")]


class dm_mlp_bufs(ctypes.Structure):
    _fields_ = [(n, c_vp) for n in ("h", "ab", "mid", "dab", "dh")]


class dm_mlp_grads(ctypes.Structure):
    _fields_ = [(n, c_vp) for n in ("w1", "w3", "w2", "norm_w")]


class dm_stack_layer(ctypes.Structure):
    _fields_ = [("w", c_vp), ("bufs", c_vp), ("x", c_vp), ("y", c_vp), ("K_cache", c_vp), ("V_cache", c_vp),
                ("ocat", c_vp), ("tape", c_vp), ("tape_bytes", ctypes.c_size_t), ("workspace", c_vp),
                ("workspace_bytes", ctypes.c_size_t), ("mlp_w", c_vp), ("mlp_bufs", c_vp), ("z", c_vp),
                ("mlp_H", c_i32)]


class dm_stack_bwd_layer(ctypes.Structure):
    _fields_ = [("w", c_vp), ("bufs", c_vp), ("x", c_vp), ("dy", c_vp), ("dx", c_vp), ("K_cache", c_vp),
                ("V_cache", c_vp), ("ocat", c_vp), ("tape", c_vp), ("tape_bytes", ctypes.c_size_t), ("grads", c_vp),
                ("workspace", c_vp), ("workspace_bytes", ctypes.c_size_t), ("mlp_w", c_vp), ("mlp_bufs", c_vp),
                ("mlp_grads", c_vp), ("dz", c_vp), ("mlp_y", c_vp), ("mlp_H", c_i32), ("mlp_workspace", c_vp),
                ("mlp_workspace_bytes", ctypes.c_size_t)]


P = ctypes.POINTER

# name -> (restype, argtypes); every symbol include/dm_abi.h declares
SIGNATURES = {
    "dm_abi_version": (ctypes.c_int, []),
    "dm_last_error": (ctypes.c_char_p, []),
    "dm_pack_weights": (ctypes.c_int, [P(dm_config), P(dm_params), P(dm_packed), c_vp]),
    "dm_layer_proj": (ctypes.c_int, [P(dm_config), P(dm_packed), c_vp, c_fp, c_fp,
                                     P(dm_layer_bufs), c_vp]),
    "dm_cell_workspace_bytes": (ctypes.c_size_t, [P(dm_config), c_i32]),
    "dm_cell_fwd": (ctypes.c_int, [P(dm_config), P(dm_packed), P(dm_layer_bufs), c_fp, c_fp,
                                   P(dm_cell_args), c_vp]),
    "dm_layer_tape_bytes": (ctypes.c_size_t, [P(dm_config), P(c_i32), c_i32]),
    "dm_layer_fwd": (ctypes.c_int, [P(dm_config), P(dm_packed), c_vp, c_vp, c_fp, c_fp,
                                    P(dm_layer_bufs), P(c_i32), c_i32, c_vp, c_vp, c_i32, c_vp,
                                    c_vp, ctypes.c_size_t, c_vp, ctypes.c_size_t, c_vp]),
    "dm_layer_bwd_workspace_bytes": (ctypes.c_size_t, [P(dm_config), c_i32, c_i32, c_i32]),
    "dm_layer_bwd": (ctypes.c_int, [P(dm_config), P(dm_packed), c_vp, c_vp, c_vp, c_fp, c_fp,
                                    P(dm_layer_bufs), P(c_i32), c_i32, c_vp, c_vp, c_i32, c_vp,
                                    c_vp, ctypes.c_size_t, P(dm_grads), c_vp, ctypes.c_size_t,
                                    c_vp]),
    "dm_layer_bwd_begin": (ctypes.c_int, [P(dm_config), P(dm_packed), c_vp, c_vp, P(dm_layer_bufs), P(c_i32),
                                          c_i32, c_i32, P(dm_grads), c_vp, ctypes.c_size_t, c_vp]),
    "dm_cell_bwd": (ctypes.c_int, [P(dm_config), P(dm_packed), P(dm_layer_bufs), c_fp, c_fp,
                                   P(dm_cell_bwd_args), c_vp]),
    "dm_layer_bwd_end": (ctypes.c_int, [P(dm_config), P(dm_packed), c_vp, c_vp, c_vp, c_fp, c_fp,
                                        P(dm_layer_bufs), P(c_i32), c_i32, c_vp, c_vp, c_i32, c_vp,
                                        ctypes.c_size_t, P(dm_grads), c_vp, ctypes.c_size_t, c_vp]),
    "dm_decode_workspace_bytes": (ctypes.c_size_t, [P(dm_config), c_i32]),
    "dm_decode_step": (ctypes.c_int, [P(dm_config), P(dm_packed), c_fp, c_fp,
                                      P(dm_decode_args), c_vp]),
    "dm_decode_step_noalloc": (ctypes.c_int, [P(dm_config), P(dm_packed), c_fp, c_fp,
                                              P(dm_decode_args), c_vp]),
    "dm_attend_one": (ctypes.c_int, [P(dm_config), c_vp, c_vp, c_vp, c_vp, c_vp, c_i32, c_i32, c_vp, c_vp,
                                     ctypes.c_size_t, c_vp]),
    "dm_refine_kv_workspace_bytes": (ctypes.c_size_t, [P(dm_config), c_i32]),
    "dm_refine_kv": (ctypes.c_int, [P(dm_config), P(dm_packed), P(dm_layer_bufs), c_vp, c_fp, c_fp, c_vp, c_vp,
                                    c_vp, ctypes.c_size_t, c_vp]),
    "dm_linear": (ctypes.c_int, [c_i32, c_vp, c_vp, c_vp, c_vp, c_i32, c_i32, c_i32, c_vp]),
    "dm_argmax_rows": (ctypes.c_int, [c_i32, c_vp, c_i32, c_i32, ctypes.c_int64, c_vp, c_vp]),
    "dm_stack_fwd_plan_bytes": (ctypes.c_size_t, [P(dm_config), c_i32, P(dm_stack_layer), P(c_i32), c_i32, c_i32]),
    "dm_stack_fwd": (ctypes.c_int, [P(dm_config), c_i32, P(dm_stack_layer), c_fp, c_fp, P(c_i32), c_i32, c_i32,
                                    c_vp, ctypes.c_size_t, c_i32, c_vp]),
    "dm_stack_bwd_plan_bytes": (ctypes.c_size_t, [P(dm_config), c_i32, P(dm_stack_bwd_layer), P(c_i32), c_i32,
                                                  c_i32]),
    "dm_stack_bwd": (ctypes.c_int, [P(dm_config), c_i32, P(dm_stack_bwd_layer), c_fp, c_fp, P(c_i32), c_i32, c_i32,
                                    c_vp, ctypes.c_size_t, c_i32, c_vp]),
    "dm_residual_rmsnorm": (ctypes.c_int, [c_i32, c_vp, c_vp, c_vp, c_vp, c_i32, c_i32, ctypes.c_float, c_vp]),
    "dm_pack_mlp": (ctypes.c_int, [c_i32, c_vp, c_vp, c_vp, c_vp, c_i32, c_i32, P(dm_mlp_packed), c_vp]),
    "dm_mlp_fwd": (ctypes.c_int, [c_i32, P(dm_mlp_packed), c_vp, c_vp, P(dm_mlp_bufs), c_i32, c_i32, c_i32,
                                  ctypes.c_float, c_vp]),
    "dm_mlp_workspace_bytes": (ctypes.c_size_t, [c_i32, c_i32, c_i32, c_i32]),
    "dm_mlp_bwd": (ctypes.c_int, [c_i32, P(dm_mlp_packed), c_vp, c_vp, c_vp, P(dm_mlp_bufs), P(dm_mlp_grads), c_i32,
                                  c_i32, c_i32, ctypes.c_float, c_vp, ctypes.c_size_t, c_vp]),
    "dm_swiglu_rows": (ctypes.c_int, [c_i32, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_i32, c_i32, c_i32, c_vp]),
    "dm_gemm": (ctypes.c_int, [c_i32, c_i32, c_i32, c_vp, c_vp, c_fp, c_i32, c_i32, c_i32, c_i32,
                               c_vp]),
    "dm_check_schedule": (ctypes.c_int, [P(c_i32), c_i32, c_i32]),
    "dm_prof_start": (ctypes.c_int, [c_i32, c_i32]),
    "dm_prof_stop2": (ctypes.c_int, [P(ctypes.c_float), P(ctypes.c_float), P(c_i32)]),
    "dm_prof_stop": (ctypes.c_int, [P(ctypes.c_float), P(c_i32)]),
}

# kernel classes of dm_prof_start (include/dm_abi.h)
PROF = {"proj": 1, "comm": 2, "attend": 3, "sweep1": 4, "sweep2": 5, "wo": 6, "dec_read": 7,
        "dec_merge": 8, "dec_refine": 9, "bwd": 10, "layer": 11}


DM_PROF_EVENTS_ONLY = 0x100


class KernelTimer:
    """Times every launch of one kernel class with HIP events stamped by the launches
    (dm_prof_*); device_clock=False leaves the kernels' own device-clock stamps out."""

    def __init__(self, kernel_class, max_launches=8192, device_clock=True):
        self.cls = PROF[kernel_class] if isinstance(kernel_class, str) else int(kernel_class)
        if not device_clock:
            self.cls |= DM_PROF_EVENTS_ONLY
        self.cap = max_launches
        self.total_ms, self.n, self.device_total_ms = 0.0, 0, None

    def __enter__(self):
        check(lib().dm_prof_start(self.cls, self.cap))
        return self

    def __exit__(self, *exc):
        ms, dms, n = ctypes.c_float(), ctypes.c_float(), c_i32()
        check(lib().dm_prof_stop2(ctypes.byref(ms), ctypes.byref(dms), ctypes.byref(n)))
        self.total_ms, self.n = float(ms.value), int(n.value)
        self.device_total_ms = float(dms.value) if dms.value >= 0 else None
        return False

    @property
    def avg_ms(self):
        """Mean per-launch time from the HIP event pairs (each dispatch's begin to end)."""
        return self.total_ms / max(self.n, 1)

    @property
    def device_avg_ms(self):
        """Mean per-dispatch span from the device clock (None for classes without it)."""
        if self.device_total_ms is None:
            return None
        return self.device_total_ms / max(self.n, 1)

_lib = None
_lib_err = None


def load(path=LIB_PATH):
    """Load libdm_hip.so and bind every declared symbol (no GPU needed)."""
    global _lib, _lib_err
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        _lib_err = f"{path} not built (run dual_mod_public_amd._build.build())"
        raise RuntimeError(_lib_err)
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def lib():
    return _lib if _lib is not None else load()


class DMError(RuntimeError):
    pass


def check(rc):
    if rc != 0:
        msg = lib().dm_last_error().decode(errors="replace")
        raise DMError(f"libdm_hip error {rc}: {msg}")


def ptr(t):
    """Device pointer of a tensor (None -> NULL)."""
    if t is None:
        return None
    return t.data_ptr()


def stream_ptr():
    return torch.cuda.current_stream().cuda_stream


def dtype_code(dt):
    if dt == torch.float32:
        return DM_F32
    if dt == torch.bfloat16:
        return DM_BF16
    raise NotImplementedError(f"storage dtype {dt} (fp32 or bf16)")


def linear(x, W, residual=None, out=None):
    """y = x W^T (+ residual) through dm_linear; x [..., K], W [N, K]."""
    K = x.shape[-1]
    N = W.shape[0]
    x2 = x.reshape(-1, K).contiguous()
    W = W.to(dtype=x.dtype).contiguous()
    y = out if out is not None else torch.empty(*x.shape[:-1], N, device=x.device, dtype=x.dtype)
    r = residual.reshape(-1, N).contiguous() if residual is not None else None
    check(lib().dm_linear(dtype_code(x.dtype), ptr(x2), ptr(W), ptr(r), ptr(y), x2.shape[0], N, K,
                          stream_ptr()))
    return y


def residual_rmsnorm(x, delta=None, w=None, dtype=torch.bfloat16, y=None, eps=1e-5):
    """dm_residual_rmsnorm on contiguous device tensors: x (fp32 [.., d], updated in place)
    += delta (``dtype``); returns y = rmsnorm(x) * w in ``dtype`` (a new tensor unless y is
    given), or None when w is None."""
    d = x.shape[-1]
    M = x.numel() // d
    assert x.dtype == torch.float32 and x.is_contiguous()
    if delta is not None:
        assert delta.dtype == dtype and delta.is_contiguous() and delta.numel() == x.numel()
    if w is not None:
        assert w.dtype == torch.float32 and w.is_contiguous() and w.numel() == d
        if y is None:
            y = torch.empty(x.shape, device=x.device, dtype=dtype)
        assert y.dtype == dtype and y.is_contiguous() and y.numel() == x.numel()
    check(lib().dm_residual_rmsnorm(dtype_code(dtype), ptr(x), ptr(delta) if delta is not None else None,
                                    ptr(w) if w is not None else None, ptr(y) if w is not None else None, M, d,
                                    float(eps), stream_ptr()))
    return y if w is not None else None


MLP_ROWS = 64   # rows dm_swiglu_rows takes per call


def swiglu_rows_ok(x, w1, w2):
    """Whether dm_swiglu_rows takes this product: bf16, at most MLP_ROWS rows, d a multiple of
    128 and H of 32."""
    d = x.shape[-1]
    M = x.numel() // d
    H = w1.shape[0]
    return x.dtype == torch.bfloat16 and 1 <= M <= MLP_ROWS and d % 128 == 0 and H % 32 == 0


def swiglu_rows(x, w1, w3, w2, act=None, out=None):
    """(silu(x w1^T) * (x w3^T)) w2^T through dm_swiglu_rows (models/dualmod/model.py:102-112 on
    a decode step's rows): x [.., d] bf16 with at most MLP_ROWS rows, w1 / w3 [H, d], w2 [d, H]
    bf16 contiguous; act [M, H] / out (shape of x) optional preallocated buffers."""
    d = x.shape[-1]
    M = x.numel() // d
    H = w1.shape[0]
    assert x.is_contiguous() and w1.is_contiguous() and w3.is_contiguous() and w2.is_contiguous()
    assert w1.shape == (H, d) and w3.shape == (H, d) and w2.shape == (d, H)
    assert x.dtype == w1.dtype == w3.dtype == w2.dtype
    if act is None:
        act = torch.empty(M, H, device=x.device, dtype=x.dtype)
    if out is None:
        out = torch.empty(x.shape, device=x.device, dtype=x.dtype)
    assert act.is_contiguous() and act.numel() >= M * H and out.is_contiguous() and out.numel() == x.numel()
    check(lib().dm_swiglu_rows(dtype_code(x.dtype), ptr(x), ptr(w1), ptr(w3), ptr(w2), ptr(act), ptr(out), M, d, H,
                               stream_ptr()))
    return out


def make_config(cfg, B, dtype):
    """dm_config from a DualModConfig (the knob subset the ABI carries)."""
    c = dm_config()
    c.dtype = dtype_code(dtype)
    c.B = B
    c.d = cfg.d_model
    c.h = cfg.n_heads
    c.dh = cfg.head_dim
    c.ctx_mod = CTX_MOD[cfg.ctx_mod]
    c.mult_res_lambda = float(getattr(cfg, "mult_res_lambda", 1.0))
    c.rms_eps = 1e-5
    c.local_window = int(getattr(cfg, "local_window", 0) or 0)
    # kmod heads (attention.py:362-384): 0 raw, 1 raw with the tanh bound, 2 gated_norm
    c.kmod_vraw_heads = int(getattr(cfg, "kmod_vraw_heads", 0) or 0)
    if getattr(cfg, "kmod_mode", "raw") == "gated_norm":
        c.kmod_mode = 2
    else:
        c.kmod_mode = 1 if getattr(cfg, "kmod_vraw_bound", "none") == "tanh" else 0
    c.v_clamp_tau = float(getattr(cfg, "v_clamp_tau", 0.0) or 0.0)
    c.norms = norm_bits(cfg)
    return c


def norm_bits(cfg):
    """dm_config.norms of a config: the per-head RMS norms set to "rms"."""
    bits = 0
    for knob, bit, _ in NORM_KNOBS:
        if getattr(cfg, knob, "none") == "rms":
            bits |= bit
    return bits
