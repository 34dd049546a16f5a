/* dm_abi.h — C ABI of libdm_hip.so, the MI355X (gfx950) Dual-Mod attention hot path.
 *
 * Plain C: device pointers, sizes, enums. No torch, no HIP types in the
 * signatures (streams are passed as `void*` holding a hipStream_t; NULL =
 * the null stream). Every call validates its arguments, launches asynchronously
 * on the given stream, never allocates device memory, never synchronizes,
 * and returns 0 (DM_OK) or a negative dm_status; dm_last_error() then holds a
 * message (thread-local).
 *
 * Layouts (all contiguous, row-major):
 *   x, y        [B, T, d]        storage dtype
 *   head bufs   [B, h, T, dh]    storage dtype (qr, kraw, kself, vraw)
 *   K/V cache   [B, h, Tc, dh]   storage dtype, rows [0, pos0) committed
 *   glogx       [B, T, 2d] storage dtype  x-half of the key|value gate logits + bias
 *   sig         [B, T, d]  storage dtype  sigmoid(v_gate(xhat)) (ctx_mod mult/mult_res)
 *   cos, sin    [Tc, dh/2] fp32  RoPE tables (models/dualmod/rope.py:13-19)
 *
 * Reference interface each entry point replaces (paths in Atom-101/dual_mod_public):
 *   dm_pack_weights  engines/wavescan/cells/fused_sweep.py:1266-1291 (FusedSweepCell.pack)
 *   dm_layer_proj    engines/wavescan/cells/fused_sweep.py:1403-1436 (FusedSweepCell.layer_proj)
 *   dm_cell_fwd      engines/wavescan/cells/fused_sweep.py:1455-1553 (FusedSweepCell.cell_forward)
 *                    == engines/wavescan/cells/scan_cell_fwd.py:88-116 (chunk_cell_forward)
 *   dm_layer_fwd     engines/wavescan/engine/forward.py:95-113 (layer_forward) + W_O,
 *                    models/dualmod/model.py:123-124 (Block attention sublayer)
 *   dm_decode_step   models/dualmod/attention.py:564-588 (DualModAttention.decode_step),
 *                    lm/eval/graph_decode.py:33-51 (GraphDecoder._attn)
 */
#ifndef DM_ABI_H
#define DM_ABI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DM_ABI_VERSION 7

typedef enum dm_status {
  DM_OK = 0,
  DM_ERR_INVALID = -1,      /* bad shape / pointer / alignment */
  DM_ERR_UNSUPPORTED = -2,  /* knob or shape the HIP path does not implement */
  DM_ERR_WORKSPACE = -3,    /* workspace too small */
  DM_ERR_HIP = -4           /* a HIP runtime call failed */
} dm_status;

typedef enum dm_dtype { DM_F32 = 0, DM_BF16 = 1 } dm_dtype;

/* ctx_mod values (models/dualmod/config.py:61, attention.py:338-360) */
typedef enum dm_ctx_mod { DM_CTX_LINEAR = 0, DM_CTX_MULT_RES = 1, DM_CTX_MULT = 2, DM_CTX_FUSION = 3 } dm_ctx_mod;

/* Shape + knob set shared by every call (DualModConfig subset). */
typedef struct dm_config {
  int32_t dtype;            /* dm_dtype of activations, weights and caches */
  int32_t B, d, h, dh;      /* batch, d_model, heads, head_dim (d == h*dh) */
  int32_t ctx_mod;          /* dm_ctx_mod */
  float mult_res_lambda;    /* config.py:126 */
  float rms_eps;            /* RMSNorm eps of attn_norm / norm_ctx: 1e-5 */
  int32_t local_window;     /* W tokens incl. self (attention.py:291-293), 0 = full: a row at
                               position i reads keys >= i - W + 1 of the committed prefix and of
                               its own cell; W = 1 reads like 0, as attend_one's K_past[-(W-1):]
                               does; < 0 is rejected (DM_ERR_INVALID) */
  int32_t flags;            /* DM_FLAG_* */
  int32_t kmod_vraw_heads;  /* config.py kmod_vraw_heads: the first n heads keep raw values */
  int32_t kmod_mode;        /* dm_kmod_mode (kmod_mode + kmod_vraw_bound), attention.py:362-384 */
  float v_clamp_tau;        /* config.py v_clamp_tau: v'' <- v'' min(1, tau / ||v''||) per (position,
                               head), attention.py:389-402; 0 = off */
  int32_t norms;            /* DM_NORM_* bits: the per-head RMS norms that are on */
  int32_t reserved[2];
} dm_config;

/* Per-head RMS norms with a learned per-head gain, fp32, eps 1e-6 (attention.py:218-269):
 *   K_CTX  k_ctx_norm="rms": k_ctx = w_kctx(u) -> norm_kctx (gain k_gain), before the key blend
 *   V_CTX  v_ctx_norm="rms": v_ctx = w_vctx(v_in) -> norm_vctx (gain ctx_gain), before the value blend
 *   V      v_norm="rms": v_raw = wv(xhat) -> project_v's norm (gain v_gain)
 * y = gain * x * rsqrt(mean over the head's dh columns of x^2 + 1e-6); x is the projection's output
 * rounded to the storage dtype and y is rounded to it again, as the reference's eager path does. */
#define DM_NORM_K_CTX 1
#define DM_NORM_V_CTX 2
#define DM_NORM_V 4

/* kmod heads (value columns of heads < kmod_vraw_heads), attention.py:362-384:
 * RAW v'' = v_raw; RAW_TANH v'' = tanh(v_raw) (kmod_vraw_bound="tanh");
 * GATED_NORM v_ctx = 0 in the blend, v'' = g v_raw (kmod_mode="gated_norm"). */
typedef enum dm_kmod_mode { DM_KMOD_RAW = 0, DM_KMOD_RAW_TANH = 1, DM_KMOD_GATED_NORM = 2 } dm_kmod_mode;

/* dm_layer_fwd / dm_layer_bwd: without this flag y = x + W_O . DM(norm(x)) (the Block
 * attention sublayer, models/dualmod/model.py:123-124); with it y = W_O . DM(norm(x))
 * (DualModAttention.forward, attention.py:438-447). */
#define DM_FLAG_NO_RESIDUAL 1
/* Forward sweeps of 64-row cells run sweep s + 1's attention inside sweep s's GEMM 2 launch (one
 * launch per sweep less) when B*h >= 128 (enough blocks); these force it on / off (results agree
 * to rounding). */
#define DM_FLAG_FUSED_ATTEND 2
#define DM_FLAG_UNFUSED_ATTEND 4

/* The reference parameters of one DualModAttention layer (attention.py:100-202),
 * each as stored by torch (nn.Linear weight = [out, in]). Storage dtype unless noted. */
typedef struct dm_params {
  const void* wq; const void* wk; const void* wv; const void* wo;   /* [d, d] */
  const void* w_kctx; const void* w_vctx;                            /* [d, d] */
  const void* w_gk; const void* w_gv;                                /* [d, 2d] */
  const void* b_gk; const void* b_gv;                                /* [d] */
  const void* v_gate; const void* b_vgate; const void* v_map;        /* [d,d],[d],[d,d]; mult family */
  const void* norm_ctx_w;                                            /* [d] */
  const void* attn_norm_w;                                           /* [d] (layer entry points) */
  const void* v_pre;                                                 /* [d, 2d]; ctx_mod fusion (attention.py:341-342) */
  const void* k_gain; const void* ctx_gain; const void* v_gain;      /* [h] norm gains (attention.py:113-166),
                                                                        read when the DM_NORM_* bit is set */
} dm_params;

/* Packed weights (written by dm_pack_weights, read by every compute call).
 * The *_t fields are transposed copies used by the backward (may be NULL for
 * forward-only use; dm_layer_bwd requires them).
 *   w_proj  [6d, d]  rows: wq | wk | wv | w_gk[:, :d] | w_gv[:, :d] | v_gate (fusion: v_pre[:, :d])
 *                    (linear: 5d rows)
 *   b_proj  [3d] fp32: b_gk | b_gv | b_vgate
 *   w_sweep [4d, d]  per head g: [w_kctx rows of g ; w_gk[:, d:] rows of g] (2*dh rows each),
 *                    then mult family: v_map (fusion: v_pre[:, d:]) (d rows), w_gv[:, d:] (d rows);
 *                    linear: per head g: [w_vctx rows of g ; w_gv[:, d:] rows of g]
 *   w_vctx  [d, d]   (mult family), norm_ctx_w [d], attn_norm_w [d], wo [d, d]: copies */
typedef struct dm_packed {
  void* w_proj; float* b_proj; void* w_sweep; void* w_vctx;
  void* norm_ctx_w; void* attn_norm_w; void* wo;
  void* w_proj_t;   /* [d, 6d] (linear: [d, 5d]) */
  void* w_sweep_t;  /* [d, 4d] */
  void* w_vctx_t;   /* [d, d]  (mult family) */
  void* wo_t;       /* [d, d]  */
  float* gains;     /* [3h] fp32: k_gain | ctx_gain | v_gain (required when cfg->norms != 0) */
} dm_packed;

/* Per-layer projection buffers (fused_sweep.py:1179-1215 LayerBufs, own layout). */
typedef struct dm_layer_bufs {
  int32_t T;                /* sequence length of these buffers */
  void* xhat;               /* [B, T, d] attn_norm(x) (kept for the backward) */
  void* qr;                 /* [B, h, T, dh] rotated query */
  void* kraw;               /* [B, h, T, dh] unrotated raw key (blend space) */
  void* kself;              /* [B, h, T, dh] rotated raw key (self column) */
  void* vraw;               /* [B, h, T, dh] raw value */
  void* glogx;              /* [B, T, 2d] storage dtype (LayerBufs.glog_x, fused_sweep.py:1189) */
  void* sig;                /* [B, T, d] storage dtype, or NULL (linear) (fused_sweep.py:1207) */
  void* vpre;               /* [B, h, T, dh] v_raw before the v_norm (DM_NORM_V only, kept for the
                               backward; may be NULL for forward-only use) */
} dm_layer_bufs;

/* ---- version / errors ------------------------------------------------------ */
int dm_abi_version(void);
const char* dm_last_error(void);

/* ---- weights ----------------------------------------------------------------
 * Replaces FusedSweepCell.pack (engines/wavescan/cells/fused_sweep.py:1266-1291). */
int dm_pack_weights(const dm_config* cfg, const dm_params* p, const dm_packed* out, void* stream);

/* ---- layer projection pass --------------------------------------------------
 * Replaces FusedSweepCell.layer_proj (fused_sweep.py:1403-1436): xhat = RMSNorm(x),
 * q/k/v projections + RoPE, x-half gate logits (+bias), sigmoid(v_gate(xhat)).
 * x: [B, T, d]; cos/sin: [>=T, dh/2] fp32 tables, row t = position t.
 * With w->attn_norm_w == NULL, x is taken as already normalised (xhat) and
 * bufs->xhat is not written (DualModAttention.forward takes xhat, attention.py:438). */
int dm_layer_proj(const dm_config* cfg, const dm_packed* w, const void* x, const float* cos,
                  const float* sin, const dm_layer_bufs* bufs, void* stream);

/* ---- one forward cell ---------------------------------------------------------
 * Replaces FusedSweepCell.cell_forward (fused_sweep.py:1455-1553) and
 * chunk_cell_forward (scan_cell_fwd.py:88-116): chunk [pos0, pos0+c) of the
 * layer, n_sweeps Jacobi sweeps against the committed rows [0, pos0) of K/V
 * cache, writing the chunk's final refined rows into the cache (append-only)
 * and the last sweep's o_cat into ocat[:, pos0:pos0+c] (storage dtype, [B,T,d]).
 * Requires 1 <= c <= 64, pos0 + c <= bufs->T <= cache_T.
 * Chunk-local form (K_rows != NULL, chunk_cell_forward's K_comm / V_comm arguments): bufs,
 * the cos / sin rows and ocat hold only the chunk (row p = chunk row p, c <= bufs->T),
 * K_cache / V_cache are the committed rows [0, pos0) alone ([B, h, cache_T, dh], pos0 <=
 * cache_T; NULL when pos0 == 0), and the chunk's rows (rotated K, V) go to K_rows / V_rows
 * [B, h, rows_T, dh] rows [0, c) instead of the cache. */
typedef struct dm_cell_args {
  int32_t pos0, c, n_sweeps, cache_T;
  void* K_cache; void* V_cache;        /* [B, h, cache_T, dh] */
  void* ocat;                          /* [B, bufs->T, d] or NULL */
  float* o_last;                       /* [B*c, d] fp32 copy of the last sweep's o, or NULL */
  void* workspace; size_t workspace_bytes;
  void* K_rows; void* V_rows;          /* chunk-local form: [B, h, rows_T, dh], else NULL */
  int32_t rows_T;
  int32_t reserved_;
} dm_cell_args;
size_t dm_cell_workspace_bytes(const dm_config* cfg, int32_t cache_T);
int dm_cell_fwd(const dm_config* cfg, const dm_packed* w, const dm_layer_bufs* bufs,
                const float* cos, const float* sin, const dm_cell_args* a, void* stream);

/* ---- whole layer forward ------------------------------------------------------
 * Block attention sublayer (models/dualmod/model.py:123-124) run through the
 * chunk schedule (engines/wavescan/engine/forward.py:95-113, schedule.py:63-69):
 *   y = x + W_O . DM(RMSNorm(x)).  sched = n_cells triples (pos0, c, n_sweeps)
 * that tile [0, T) in order. Fills bufs, the caches and ocat [B, T, d].
 *
 * tape (may be NULL): device buffer of dm_layer_tape_bytes() bytes that receives
 * every sweep state of every cell (o, RMS sums, softmax row stats, raw sweep GEMM
 * outputs, v_in, the refined intra rows of sweeps 1..K-1, the committed row max).
 * The reference rebuilds these in the backward by exact recompute
 * (fused_sweep.py:1580-1659); with 288 GB of HBM per GPU this build can keep them
 * instead (about 58 MB per 64-token cell at d=1024, B=8, K=4). Every kernel is
 * deterministic, so the saved states equal the recomputed ones bit for bit. */
size_t dm_layer_tape_bytes(const dm_config* cfg, const int32_t* sched, int32_t n_cells);
int dm_layer_fwd(const dm_config* cfg, const dm_packed* w, const void* x, void* y,
                 const float* cos, const float* sin, const dm_layer_bufs* bufs,
                 const int32_t* sched, int32_t n_cells, void* K_cache, void* V_cache,
                 int32_t cache_T, void* ocat, void* tape, size_t tape_bytes, void* workspace,
                 size_t workspace_bytes, void* stream);

/* ---- SwiGLU MLP sublayer of a Block ---------------------------------------------------
 * z = y + W2 (silu(W1 h) * W3 h), h = mlp_norm(y) (models/dualmod/model.py:102-112, 127-128;
 * RMSNorm attention.py:74-83), over M rows [M, d] of the storage dtype, and its VJP. The
 * trunk's MLP in the reference engine's chunk body (engines/wavescan/engine/graphs.py:254-256,
 * the layer_blockmlp_bwd VJP fused_sweep.py:1854-1869); here on the library's own GEMM tiles,
 * so that the layer-by-layer trunk and the layer-batched stack (dm_stack_fwd / dm_stack_bwd
 * with a block tail) compute the same bits. Numerics as the reference's bf16 autocast: every
 * product with fp32 accumulation rounded to the storage dtype, silu(a) * b from the rounded
 * products, RMS statistics in fp32. H (the hidden width) a multiple of 32, d of 64.
 * dm_pack_mlp writes the packed weights from the reference's w1 / w3 [H, d], w2 [d, H] and
 * mlp_norm.weight [d] (storage dtype). */
typedef struct dm_mlp_packed {
  void* w13;      /* [2H, d] W1 / W3 rows interleaved in groups of 32 (W1 rows 32g.., then W3 rows 32g..) */
  void* w2;       /* [d, H] */
  void* w13_t;    /* [d, 2H] w13 transposed */
  void* w2_t;     /* [H, d] W2 transposed */
  void* norm_w;   /* [d] mlp_norm.weight */
} dm_mlp_packed;
/* The forward's saved state and the backward's intermediates, rows laid out as y's. */
typedef struct dm_mlp_bufs {
  void* h;        /* [rows, d]  mlp_norm(y) */
  void* ab;       /* [rows, 2H] W1 h | W3 h in w13's row order */
  void* mid;      /* [rows, H]  silu(W1 h) * W3 h */
  void* dab;      /* [rows, 2H] backward: the grads of ab */
  float* dh;      /* [rows, d]  backward: the grad of h */
} dm_mlp_bufs;
typedef struct dm_mlp_grads {
  float* w1; float* w3;   /* [H, d] */
  float* w2;              /* [d, H] */
  float* norm_w;          /* [d] */
} dm_mlp_grads;
int dm_pack_mlp(int32_t dtype, const void* w1, const void* w3, const void* w2, const void* norm_w, int32_t d,
                int32_t H, const dm_mlp_packed* out, void* stream);
int dm_mlp_fwd(int32_t dtype, const dm_mlp_packed* w, const void* y, void* z, const dm_mlp_bufs* bufs, int32_t M,
               int32_t d, int32_t H, float eps, void* stream);
/* dy = dz + the MLP branch's VJP (dy may not alias dz); the weight gradients are ADDED into g.
 * workspace: dm_mlp_workspace_bytes(dtype, M, d, H). */
size_t dm_mlp_workspace_bytes(int32_t dtype, int32_t M, int32_t d, int32_t H);
int dm_mlp_bwd(int32_t dtype, const dm_mlp_packed* w, const void* y, const void* dz, void* dy,
               const dm_mlp_bufs* bufs, const dm_mlp_grads* g, int32_t M, int32_t d, int32_t H, float eps,
               void* workspace, size_t workspace_bytes, void* stream);

/* ---- layer-batched (wavefront) forward of a stack of layers --------------------------
 * engines/wave3d/wave3d.py:1-47 (layer l at global step t works on step t - l, every active
 * layer's work batched into the same launches), applied to the chunk schedule above: layer l
 * runs cell t - l at global step t (its chunk's rows are final once that cell's K sweeps
 * are done, so layer l + 1 takes them one step later), and each kernel of a step is ONE launch
 * over all active layers (grid z = layer), its arguments read from `plan`. Per layer the
 * result is dm_layer_fwd's, bit for bit: the same bufs, caches, ocat, tape and output y (the
 * chunk's RMSNorm + projection, its cell, W_O + residual per chunk instead of per layer).
 * Layer l reads layers[l].x and writes layers[l].y (layers[l + 1].x is normally
 * layers[l].y). Every cell of the schedule has the same length c (a power of two <= 64) and
 * the same n_sweeps. Each layer has its own workspace (dm_cell_workspace_bytes(cfg,
 * cache_T)) and tape (optional, as dm_layer_fwd; all layers with or all without).
 * plan: device memory of dm_stack_fwd_plan_bytes() bytes holding every launch's argument
 * table. build != 0 writes it (a blocking host-to-device copy) before launching; build == 0
 * launches from a plan written by an earlier call with the same arguments (e.g. under graph
 * capture): the library keeps each written plan's launch list and a signature of its arguments,
 * keyed by the plan's address, so such a call only issues the launches; a build == 0 call whose
 * arguments differ from the plan's last build (or on a plan never built) returns
 * DM_ERR_INVALID and launches nothing. Kernel timing (dm_prof_start) does not cover this
 * entry point. */
typedef struct dm_stack_layer {
  const dm_packed* w;
  const dm_layer_bufs* bufs;
  const void* x; void* y;              /* [B, T, d] layer input / attention sublayer output */
  void* K_cache; void* V_cache;        /* [B, h, cache_T, dh] */
  void* ocat;                          /* [B, T, d] */
  void* tape; size_t tape_bytes;       /* NULL: no tape */
  void* workspace; size_t workspace_bytes;
  /* the block tail (engines/wave3d/wave3d.py:26-28: x + wo(o) + mlp(mlp_norm(.)) per step):
   * NULL mlp_w: the layer is the attention sublayer alone, its output y; else each cell's rows
   * also run the MLP sublayer (as dm_mlp_fwd) from y into z, the block output [B, T, d] (then
   * layers[l + 1].x is normally layers[l].z), with the state the backward reads in mlp_bufs */
  const dm_mlp_packed* mlp_w;
  const dm_mlp_bufs* mlp_bufs;
  void* z;
  int32_t mlp_H;
} dm_stack_layer;
size_t dm_stack_fwd_plan_bytes(const dm_config* cfg, int32_t n_layers, const dm_stack_layer* layers,
                               const int32_t* sched, int32_t n_cells, int32_t cache_T);
int dm_stack_fwd(const dm_config* cfg, int32_t n_layers, const dm_stack_layer* layers, const float* cos,
                 const float* sin, const int32_t* sched, int32_t n_cells, int32_t cache_T, void* plan,
                 size_t plan_bytes, int32_t build, void* stream);

/* ---- whole layer backward ---------------------------------------------------------
 * Reverse-scan backward of the layer forward above (engines/wavescan/engine/backward.py:92-123,
 * FusedSweepCell.cell_backward fused_sweep.py:1557-1850, layer_close :1873-1959):
 * cells in reverse order; each cell takes its n_sweeps sweep states from the
 * forward's tape (non-NULL, same schedule) or recomputes them exactly from the
 * forward's projections (bufs) and final cache rows (tape NULL, as the reference),
 * then runs the sweeps backward. Before a cell's sweeps, the grads its final rows
 * receive from the committed-prefix attention of every later row are summed (the
 * reference's grad cache, backward.py:27-123, without a running fp32 buffer); the
 * query side of that attention is computed for every row once, at the end.
 * Inputs are exactly what dm_layer_fwd produced / consumed (x, bufs, caches, ocat)
 * plus dy [B, T, d]. Writes dx [B, T, d] (storage dtype) and ADDS the parameter
 * gradients into g (fp32, reference layout). Needs the *_t fields of w. */
typedef struct dm_grads {
  float* wq; float* wk; float* wv; float* wo;        /* [d, d] */
  float* w_kctx; float* w_vctx;                      /* [d, d] */
  float* w_gk; float* w_gv;                          /* [d, 2d] */
  float* b_gk; float* b_gv;                          /* [d] */
  float* v_gate; float* b_vgate; float* v_map;       /* [d, d], [d], [d, d] (mult family) */
  float* norm_ctx_w;                                 /* [d] */
  float* attn_norm_w;                                /* [d] (when w->attn_norm_w != NULL) */
  float* v_pre;                                      /* [d, 2d] (fusion) */
  float* k_gain; float* ctx_gain; float* v_gain;     /* [h] (with the matching DM_NORM_* bit) */
} dm_grads;
size_t dm_layer_bwd_workspace_bytes(const dm_config* cfg, int32_t T, int32_t cache_T, int32_t max_sweeps);
int dm_layer_bwd(const dm_config* cfg, const dm_packed* w, const void* x, const void* dy, void* dx,
                 const float* cos, const float* sin, const dm_layer_bufs* bufs, const int32_t* sched,
                 int32_t n_cells, const void* K_cache, const void* V_cache, int32_t cache_T,
                 const void* ocat, const void* tape, size_t tape_bytes, const dm_grads* g,
                 void* workspace, size_t workspace_bytes, void* stream);

/* ---- layer-batched (wavefront) backward of a stack ---------------------------------------
 * The reverse of dm_stack_fwd: layer l takes its cells last first, the top layer leading, one
 * cell per step (layer l's cell i needs dy rows of that cell, written by layer l + 1's cell i
 * the step before); each kernel of a step is one launch over every active layer. Per layer the
 * result is dm_layer_bwd's (tape or recompute as given), bit for bit: dx, and the gradients
 * ADDED into grads. A cell's dx rows are made final right after its sweeps (its committed-prefix
 * query VJP, projection VJP rows, dxhat rows, attn_norm VJP + residual); the sums over a layer's
 * rows (weight grads, the bias / gain / norm-weight partials) run once its cell 0 is done.
 * Layer l reads layers[l].dy (normally layers[l + 1].dx). Equal cells of a power-of-two length,
 * attn_norm present. workspace: dm_layer_bwd_workspace_bytes(cfg, T, cache_T, n_sweeps) per
 * layer. plan / build as dm_stack_fwd (the argument tables of the grouped launches). */
typedef struct dm_stack_bwd_layer {
  const dm_packed* w;
  const dm_layer_bufs* bufs;
  const void* x; const void* dy; void* dx;   /* [B, T, d] */
  const void* K_cache; const void* V_cache;
  const void* ocat;
  const void* tape; size_t tape_bytes;
  const dm_grads* grads;
  void* workspace; size_t workspace_bytes;
  /* the block tail (as dm_stack_layer): with mlp_w, dz [B, T, d] is the grad of the block output
   * z, each cell's rows first run the MLP VJP (as dm_mlp_bwd) from dz into dy (then written, the
   * grad of the attention sublayer's output y = mlp_y), and the layer's close adds the MLP
   * weight grads into mlp_grads; mlp_workspace: dm_mlp_workspace_bytes(dtype, B T, d, mlp_H) */
  const dm_mlp_packed* mlp_w;
  const dm_mlp_bufs* mlp_bufs;
  const dm_mlp_grads* mlp_grads;
  const void* dz; const void* mlp_y;
  int32_t mlp_H;
  void* mlp_workspace; size_t mlp_workspace_bytes;
} dm_stack_bwd_layer;
size_t dm_stack_bwd_plan_bytes(const dm_config* cfg, int32_t n_layers, const dm_stack_bwd_layer* layers,
                               const int32_t* sched, int32_t n_cells, int32_t cache_T);
int dm_stack_bwd(const dm_config* cfg, int32_t n_layers, const dm_stack_bwd_layer* layers, const float* cos,
                 const float* sin, const int32_t* sched, int32_t n_cells, int32_t cache_T, void* plan,
                 size_t plan_bytes, int32_t build, void* stream);

/* ---- the same backward one cell at a time --------------------------------------------
 * The reference's engine drives the backward per cell (FusedSweepCell.layer_blockmlp_bwd,
 * cell_backward, layer_close: engines/wavescan/cells/fused_sweep.py:1557-1959, called from
 * engines/wavescan/engine/graphs.py:373-389) with an fp32 grad cache over the K/V rows
 * (engines/wavescan/engine/backward.py:92-123). These three calls do that:
 *   dm_layer_bwd_begin  zero the layer accumulators in `workspace`; W_O VJP (do_cat, dW_O += into g)
 *   dm_cell_bwd         one cell, called for cell = n_cells-1 .. 0 in that order: reads the grads of
 *                       its final rows from dK_gc / dV_gc rows [pos0, pos0+c) (complete once every
 *                       later cell ran), runs its sweeps backward (states from `tape`, or an exact
 *                       recompute when tape == NULL), and ADDS the grads of the committed rows
 *                       [0, pos0) it read into dK_gc / dV_gc; its rows' weight-grad operands and
 *                       projection grads stay in `workspace`
 *   dm_layer_bwd_end    sweep weight grads, projection VJP, attn_norm VJP: dx and the rest of g
 * Same arguments and results as dm_layer_bwd (dx, the ADDED grads), with one workspace
 * (dm_layer_bwd_workspace_bytes) and the same schedule / tape passed to all three. The caller
 * zeroes dK_gc / dV_gc (fp32 [B, h, cache_T, dh]) before the first cell. dm_layer_bwd computes
 * the committed-prefix grads without the running cache (per key cell, from every later row):
 * the results agree to fp32 rounding; the per-cell form reads and writes the cache once per
 * cell, O(T^2) bytes per layer. */
typedef struct dm_cell_bwd_args {
  const int32_t* sched; int32_t n_cells;  /* the layer's schedule (as given to dm_layer_fwd) */
  int32_t cell;                           /* index of this cell in sched */
  int32_t cache_T;
  const void* K_cache; const void* V_cache;   /* the forward's final rows [B, h, cache_T, dh] */
  float* dK_gc; float* dV_gc;             /* fp32 grad cache [B, h, cache_T, dh] */
  const void* tape; size_t tape_bytes;    /* the layer forward's tape, or NULL (recompute) */
  void* workspace; size_t workspace_bytes;
} dm_cell_bwd_args;
int dm_layer_bwd_begin(const dm_config* cfg, const dm_packed* w, const void* dy, const void* ocat,
                       const dm_layer_bufs* bufs, const int32_t* sched, int32_t n_cells, int32_t cache_T,
                       const dm_grads* g, void* workspace, size_t workspace_bytes, void* stream);
int dm_cell_bwd(const dm_config* cfg, const dm_packed* w, const dm_layer_bufs* bufs, const float* cos,
                const float* sin, const dm_cell_bwd_args* a, void* stream);
int dm_layer_bwd_end(const dm_config* cfg, const dm_packed* w, const void* x, const void* dy, void* dx,
                     const float* cos, const float* sin, const dm_layer_bufs* bufs, const int32_t* sched,
                     int32_t n_cells, const void* K_cache, const void* V_cache, int32_t cache_T,
                     const void* tape, size_t tape_bytes, const dm_grads* g, void* workspace,
                     size_t workspace_bytes, void* stream);

/* ---- decode ------------------------------------------------------------------
 * Replaces DualModAttention.decode_step (attention.py:564-588) on a static tape
 * (lm/eval/graph_decode.py:33-51): one token per batch row at position pos.
 * Reads tape rows [max(0, pos-W+1), pos) + the raw self pair, refines, and
 * writes the refined rotated key / refined value into tape slot pos.
 * xhat: [B, d] pre-normed input. o_cat: [B, d] storage dtype output (pre-W_O).
 * y: [B, d] = W_O o_cat, or NULL to skip. */
typedef struct dm_decode_args {
  int32_t pos, tape_T;
  const void* xhat;
  void* K_tape; void* V_tape;          /* [B, h, tape_T, dh] */
  void* o_cat; void* y;
  void* workspace; size_t workspace_bytes;
  /* Device position (lm/eval/graph_decode.py:24,44: GraphDecoder's device-side counter):
   * when non-NULL, pos is ignored and every kernel reads the position from this int32 in
   * device memory at run time, so one captured graph of the step serves every position.
   * The launch shapes then cover the whole tape (split blocks past the position return).
   * The RoPE tables must hold tape_T rows; a device position outside [0, tape_T) is
   * clamped into the tape (keeping it inside is the caller's job). */
  const int32_t* pos_dev;
} dm_decode_args;
size_t dm_decode_workspace_bytes(const dm_config* cfg, int32_t tape_T);
int dm_decode_step(const dm_config* cfg, const dm_packed* w, const float* cos, const float* sin,
                   const dm_decode_args* a, void* stream);

/* ---- decode step that allocates nothing ------------------------------------------
 * No counterpart in the reference. For callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid it):
 * dm_decode_step with its workspace taken from a static device array of
 * DM_DECODE_SCRATCH_MAX bytes inside the library (one per GPU, held until the process
 * ends) instead of a->workspace (ignored). Steps that need more scratch than that
 * (dm_decode_workspace_bytes > DM_DECODE_SCRATCH_MAX, e.g. B = 64, d = 1024 with
 * tape_T above ~56k) return DM_ERR_WORKSPACE. Calls no hipMalloc / hipFree; the
 * first call on a device looks up that device's address of the array
 * (hipGetSymbolAddress), so a caller that captures should make one call before
 * capturing. Every call on one GPU shares that GPU's array: calls that overlap on one
 * GPU (concurrent streams, threads) race. Nothing in it needs clearing between calls
 * (every scratch value a step reads is written earlier in the same step). */
#define DM_DECODE_SCRATCH_MAX ((size_t)32 << 20)
int dm_decode_step_noalloc(const dm_config* cfg, const dm_packed* w, const float* cos, const float* sin,
                           const dm_decode_args* a, void* stream);

/* ---- the per-position step as two calls ------------------------------------------
 * dm_attend_one replaces DualModAttention.attend_one (models/dualmod/attention.py:283-312):
 * each batch row's rotated query q_r against its refined tape rows K_past / V_past
 * [B, h, past_T, dh] (rows [max(0, P-W+1), P) with the config's local_window W, all P rows
 * when W == 0) plus its own raw self column (k_self_r, v_self), fp32 softmax; q_r, k_self_r,
 * v_self and the output o are [B, h, dh] (storage dtype). Workspace:
 * dm_decode_workspace_bytes(cfg, P) bytes. */
int dm_attend_one(const dm_config* cfg, const void* q_r, const void* k_self_r, const void* v_self,
                  const void* K_past, const void* V_past, int32_t P, int32_t past_T, void* o,
                  void* workspace, size_t workspace_bytes, void* stream);
/* dm_refine_kv replaces DualModAttention.refine_kv (attention.py:314-434) for t rows of every
 * batch row: u = RMSNorm_ctx(o_cat), the ctx projections, gates, value candidate, convex blends
 * (+ kmod heads, v'' clamp). bufs (T = t rows) hold the rows' gate x-halves and v_gate term
 * (glogx, sig: dm_layer_proj of xhat) and their raw key / value (kraw, vraw, [B, h, t, dh]);
 * o_cat [B, t, d]. Writes k'' and v'' to K_out / V_out [B, h, t, dh], the key rotated with the
 * cos / sin rows [t, dh/2] (identity tables give the reference's unrotated k''). Workspace:
 * dm_refine_kv_workspace_bytes(cfg, t). */
size_t dm_refine_kv_workspace_bytes(const dm_config* cfg, int32_t t);
int dm_refine_kv(const dm_config* cfg, const dm_packed* w, const dm_layer_bufs* bufs, const void* o_cat,
                 const float* cos, const float* sin, void* K_out, void* V_out, void* workspace,
                 size_t workspace_bytes, void* stream);

/* ---- linear layer -------------------------------------------------------------
 * y[M, N] = x[M, K] . W[N, K]^T (+ r[M, N] when r != NULL): nn.Linear without
 * bias (the W_O projection, attention.py:103), storage dtype, fp32 accumulate.
 * N multiple of 128, K multiple of 64, any M. */
int dm_linear(int32_t dtype, const void* x, const void* W, const void* r, void* y, int32_t M,
              int32_t N, int32_t K, void* stream);

/* ---- residual stream of the trunk's decode step -------------------------------------
 * The fp32 residual stream around one decode step of a Block (models/dualmod/model.py:
 * 127-130) with its RMSNorm (attention.py:74-83) in one pass per row: x[M, d] (fp32, in
 * place) += delta[M, d] (storage dtype; skipped when NULL), then, when w != NULL,
 * y[M, d] (storage dtype) = x * rsqrt(mean(x^2) + eps) * w (w fp32 [d]). */
int dm_residual_rmsnorm(int32_t dtype, float* x, const void* delta, const float* w, void* y, int32_t M,
                        int32_t d, float eps, void* stream);

/* ---- SwiGLU MLP of a decode step ---------------------------------------------------
 * out[M, d] = (silu(x W1^T) * (x W3^T)) W2^T, the Block's MLP (models/dualmod/model.py:
 * 102-112) on a decode step's rows (one token per sequence, M <= 64): bf16 x [M, d],
 * w1 / w3 [H, d], w2 [d, H], act [M, H] the caller's intermediate buffer, out [M, d]. The
 * products accumulate in fp32; act holds silu(g) * u rounded once to bf16. Deterministic
 * (fixed-order in-block sums). d must be a multiple of 128, H of 32, the operands 16-byte
 * aligned; DM_ERR_UNSUPPORTED for a dtype other than bf16. */
int dm_swiglu_rows(int32_t dtype, const void* x, const void* w1, const void* w3, const void* w2, void* act,
                   void* out, int32_t M, int32_t d, int32_t H, void* stream);

/* ---- row argmax ------------------------------------------------------------------
 * out[r] = the first index of the maximum of x[r, 0:cols) (row stride ld elements),
 * storage dtype bf16 or fp32: the greedy pick of lm/eval/graph_decode.py:62
 * (lg.argmax(-1)) as one block per row, with no multi-block reduction (nothing to
 * clear between graph replays). A NaN counts as the maximum (the first NaN's index), as
 * torch.argmax; a row of -inf gives 0. */
int dm_argmax_rows(int32_t dtype, const void* x, int32_t rows, int32_t cols, int64_t ld, int64_t* out,
                   void* stream);

/* ---- plain GEMM (test / utility) --------------------------------------------
 * C[M, N] (fp32) = op(A) . op(B)^T (+ C when accumulate != 0), storage dtype inputs,
 * fp32 accumulate. op(A) = A [M, K] (trans_a = 0) or A^T with A stored [K, M];
 * op(B) = B [N, K] (trans_b = 0) or B^T with B stored [K, N].
 * M, N multiples of 128, K multiple of 64. */
int dm_gemm(int32_t dtype, int32_t trans_a, int32_t trans_b, const void* A, const void* Bm, float* C,
            int32_t M, int32_t N, int32_t K, int32_t accumulate, void* stream);

/* ---- schedule check ------------------------------------------------------------
 * Validates a chunk schedule (engines/wavescan/engine/schedule.py:63-69 format):
 * n_cells triples (pos0, c, n_sweeps) tiling [0, T) in order, 1 <= c <= 64. */
int dm_check_schedule(const int32_t* sched, int32_t n_cells, int32_t T);

/* ---- optional kernel timing (benchmarks) -------------------------------------
 * No reference counterpart (the reference times with ad-hoc torch events,
 * engines/wave3d/wave3d_x.py:28-33). Arms one kernel class; every later launch of
 * that class (up to max_launches) stamps a HIP start/stop event pair from its own
 * dispatch (hipExtLaunchKernel: the interval a kernel-trace profiler reports), and
 * the GEMM classes (1, 4, 5, 6) and the decode tape read (7) also time themselves
 * from the device clock (first block start to last block end of each dispatch: the
 * execution without dispatch and drain) unless kernel_class carries
 * DM_PROF_EVENTS_ONLY (then the kernels write no timestamps and run unmodified).
 * dm_prof_stop2 waits, then returns the summed event time, the summed device-clock
 * time (-1 when some launch of the class has no device timing) and the launch
 * count; dm_prof_stop returns the event time only. dm_prof_start allocates its
 * timestamp buffer (2 * 1024 * 8 bytes per launch) and synchronizes the device.
 * Classes: 1 projection, 2 committed accumulator, 3 sweep attention, 4 sweep GEMM 1,
 * 5 sweep GEMM 2, 6 W_O, 7 decode tape read, 8 decode merge, 9 decode refine,
 * 10 backward, 11 whole entry-point call. */
#define DM_PROF_EVENTS_ONLY 0x100
int dm_prof_start(int32_t kernel_class, int32_t max_launches);
int dm_prof_stop(float* total_ms, int32_t* n_launches);
int dm_prof_stop2(float* event_ms, float* device_ms, int32_t* n_launches);

#ifdef __cplusplus
}
#endif
#endif /* DM_ABI_H */
