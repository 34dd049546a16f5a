"""CPU restatement of the Dual-Mod attention hot path — TEST INFRASTRUCTURE ONLY.

This package is the checker, never the product. Only `tests/`,
`__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may import
it. The product path (`dual_mod_public_amd`) never imports, links or calls
anything in here, and raises if its HIP library is missing.

Pinning status of each function (what independent check fixes it):
  * build_rope_cache / apply_rope  — closed form + pairing test + golden vectors
  * rms_norm                        — closed form (mean of squares) + golden vectors
  * attend_one                      — T1/T2 (reduces to SDPA) + golden vectors
  * refine_kv (linear, mult_res)    — golden vectors written by the reference
                                      itself (tests/golden/make_golden.py);
                                      special case v_map=0, lam=1 == linear
  * refine_kv knob branches         — closed forms in tests/test_oracle_invariants.py:
      mult                              mult == mult_res at lambda = 0 (and the
                                        lambda term == (1 - g_v) w_vctx(u))
      kmod gated_norm                   kmod heads' v'' == sigmoid(gate) * v_raw
      kmod raw / tanh bound             kmod heads' v'' == v_raw / tanh(v_raw)
      k_ctx_norm, v_ctx_norm, v_norm    per-head RMS written element by element
  * attend_one local_window         — scalar softmax over the last W-1 rows + self
  * sequential_scan                 — golden vectors + T1/T2/T5 invariants
  * chunk_cell_forward (Jacobi)     — golden vectors at K<c + nilpotency K=c
                                      == scan + frontier property
  * decode_step                     — golden vectors + T3 (decode == teacher forcing)
  * layer grads                     — golden vectors (autograd through the
                                      reference scan) at a tiny config
"""

from .dm_oracle import *  # noqa: F401,F403
