"""DualModConfig — the knob surface of the reference, same names and defaults.

Mirrors models/dualmod/config.py:7-226 field for field so a reference config
(or its ``to_dict()``) constructs one of these unchanged. Validation follows
config.py:164-199. Which knobs the HIP path honours is decided in
``dual_mod_public_amd.engine.check_supported`` (NotImplementedError for the
rest — there is no fallback backend).
"""

from dataclasses import asdict, dataclass


@dataclass
class DualModConfig:
    # architecture (config.py:10-24)
    d_model: int = 512
    n_layers: int = 8
    n_heads: int = 8
    n_kv_heads: int = 0
    head_dim_override: int = 0
    vocab_size: int = 50257
    max_seq_len: int = 512
    local_window: int = 0
    rope_theta: float = 10000.0
    use_rope: bool = True
    mlp_ratio: str = "swiglu_8_3"
    mlp_hidden_override: int = 0
    tie_embeddings: bool = True

    # dual-mod (config.py:27-159)
    attn_mode: str = "sequential"
    enable_key_mod: bool = True
    enable_value_mod: bool = True
    gate_type: str = "convex_sigmoid"
    gate_type_v: str = "convex"
    gate_input: str = "xu"
    gate_bias_init: float = 4.0
    gate_bias_init_k: str = "scalar"
    gate_bias_init_v: str = "scalar"
    ugi_eps: float = 0.04
    key_commit_bias: float = 3.0
    key_frontier_pairs: int = 6
    key_frontier_hi: float = 1.5
    value_band_lo: float = 0.2
    value_band_hi: float = 0.8
    ctx_reserved_init_std: float = 0.02
    gate_init_seed: int = 1337
    ctx_proj_init_std: float = 0.006
    rmsnorm_on_o: bool = True
    deq_sweeps: int = 4
    kmod_vraw_heads: int = 0
    ctx_mod: str = "linear"
    kmod_vraw_bound: str = "none"
    kmod_mode: str = "raw"
    gate_rank: int = 0
    ctx_rank: int = 0
    v_norm: str = "none"
    v_ctx_norm: str = "none"
    mult_res_lambda: float = 1.0
    k_ctx_norm: str = "none"
    attn_logn_ref: int = 0
    k_gain_init: float = 1.75
    v_clamp_tau: float = 0.0
    deterministic_bwd: bool = False
    # training (config.py:160-162)
    checkpoint_chunk: int = 64
    dtype: str = "bf16"

    def __post_init__(self):
        # config.py:164-199
        if self.head_dim_override == 0:
            assert self.d_model % self.n_heads == 0
        assert self.n_kv_heads_eff <= self.n_heads and self.n_heads % self.n_kv_heads_eff == 0
        if self.attn_mode != "vanilla":
            assert self.head_dim_override == 0 and self.n_kv_heads == 0, \
                "n_kv_heads / head_dim_override are vanilla-path only"
        assert self.attn_mode in ("vanilla", "sequential", "deq", "static")
        assert self.gate_type in ("convex_sigmoid", "independent", "unbounded")
        assert self.gate_type_v in ("convex", "independent")
        assert self.gate_bias_init_k in ("scalar", "ugi", "committed")
        assert self.gate_bias_init_v in ("scalar", "ugi", "band")
        assert self.gate_input in ("xu", "u", "x")
        assert self.kmod_vraw_bound in ("none", "tanh")
        assert self.v_norm in ("none", "rms")
        assert self.v_ctx_norm in ("none", "rms")
        assert self.k_ctx_norm in ("none", "rms")
        assert self.kmod_mode in ("raw", "gated_norm")
        assert not (self.kmod_mode == "gated_norm" and self.kmod_vraw_bound != "none"), \
            "kmod_vraw_bound applies to kmod_mode='raw' only"
        assert self.mlp_ratio == "swiglu_8_3", "only swiglu_8_3 is implemented"

    @property
    def head_dim(self) -> int:
        return self.head_dim_override or (self.d_model // self.n_heads)

    @property
    def n_kv_heads_eff(self) -> int:
        return self.n_kv_heads or self.n_heads

    @property
    def d_attn(self) -> int:
        return self.n_heads * self.head_dim

    @property
    def mlp_hidden(self) -> int:
        if self.mlp_hidden_override:
            return self.mlp_hidden_override
        return int(round(self.d_model * 8 / 3 / 64) * 64)

    @property
    def gate_in_dim(self) -> int:
        return 2 * self.d_model if self.gate_input == "xu" else self.d_model

    def to_dict(self) -> dict:
        return asdict(self)
