// Host-side launch sequences of the forward: layer projections and one chunk
// cell (committed accumulator + n_sweeps Jacobi sweeps). Shared by the forward
// entry points and by the backward's exact recompute (which keeps every sweep's
// state in a CellSave instead of overwriting it in place).
#pragma once

#include <vector>

#include "dm_host.h"

namespace dm {

// cell workspace (forward): per-sweep scratch reused across sweeps
struct CellWs {
  void* o; float* ssq;
  float* Ap; float* Zp; float* Mp;   // committed split partials
  float* A; float* Z; float* M;      // merged committed accumulator
  void* vin; void* gvu;              // v_in, g_v(u) [N, d] (storage dtype)
  size_t bytes;
};

inline CellWs carve_cell(const dm_config* c, int cache_T, void* base) {
  CellWs w{};
  const size_t N = (size_t)c->B * CMAX, BH = (size_t)c->B * c->h;
  const size_t ns = comm_splits_max(cache_T);
  Carver cv(base);
  w.o = cv.take<void>(N * c->d * esz(c->dtype));
  w.ssq = cv.take<float>(N * c->h * 4);
  w.Ap = cv.take<float>(ns * BH * CMAX * c->dh * 4);
  w.Zp = cv.take<float>(ns * BH * CMAX * 4);
  w.Mp = cv.take<float>(ns * BH * CMAX * 4);
  w.A = cv.take<float>(BH * CMAX * c->dh * 4);
  w.Z = cv.take<float>(BH * CMAX * 4);
  w.M = cv.take<float>(BH * CMAX * 4);
  w.vin = cv.take<void>(N * c->d * esz(c->dtype));
  w.gvu = cv.take<void>(N * c->d * esz(c->dtype));
  w.bytes = cv.off;
  return w;
}

// Every sweep's state of one cell, kept for the backward. Per-sweep arrays are
// stacked with the cell's own row count N = B*c (so the K sweeps of a [N, x]
// array form one [K*N, x] matrix); attention rows use B*h*CMAX slots.
template <typename T> struct CellSave {
  T* o;              // [K][N, d]      o of sweep s (storage dtype, as stored by the attention)
  float* ssq;        // [K][N, h]      per-head sums of squares of o
  float* stat_m;     // [K][BH, CMAX]  final row max of sweep s
  float* stat_z;     // [K][BH, CMAX]  final row sum of sweep s
  T* save1;          // [K][N, 4d]     raw sweep GEMM 1 outputs (rounded to the storage dtype,
  T* save2;          // [K][N, d]      raw v_ctx (mult family)    as the reference's GEMM outputs)
  T* vin;            // [K][N, d]      v_in (mult family): rows of the layer's stacked v_in
                     //   (the backward's cell order), assigned by the caller
  T* Kin; T* Vin;    // [K+1][BH, CMAX, DH]  intra rows read by sweep s (slot 0 unused: raw rows);
                     //   with last_to_cache only [K] slots: the last sweep writes the cache rows
  float* Mx;         // [BH, CMAX] committed row max (tape cells with pos0 > 0), else nullptr
  bool last_to_cache;
};

// Layout of one cell's saved state for N = B*cc rows and K sweeps. `tape` cells
// (forward-saved) drop the last K/V slot and add the committed row max.
template <typename T>
CellSave<T> carve_save(const dm_config* c, size_t N, int K, bool tape, bool has_comm, Carver& cv) {
  CellSave<T> w{};
  const size_t d = c->d, h = c->h, dh = c->dh, e = sizeof(T), BH = (size_t)c->B * c->h, k = K;
  const bool mult = c->ctx_mod != DM_CTX_LINEAR;
  w.o = cv.take<T>(k * N * d * e);
  w.ssq = cv.take<float>(k * N * h * 4);
  w.stat_m = cv.take<float>(k * BH * CMAX * 4);
  w.stat_z = cv.take<float>(k * BH * CMAX * 4);
  w.save1 = cv.take<T>(k * N * 4 * d * e);
  w.save2 = mult ? cv.take<T>(k * N * d * e) : nullptr;
  w.vin = nullptr;
  const size_t slots = tape ? k : k + 1;
  w.Kin = cv.take<T>(slots * BH * CMAX * dh * e);
  w.Vin = cv.take<T>(slots * BH * CMAX * dh * e);
  w.Mx = (tape && has_comm) ? cv.take<float>(BH * CMAX * 4) : nullptr;
  w.last_to_cache = tape;
  return w;
}

// Row of cell i's first v_in row in the layer's stacked v_in: the backward takes the
// cells last first, so the rows of cells i+1.. precede cell i's.
inline long vin_row(const dm_config* c, const int32_t* sched, int n_cells, int i) {
  long r = 0;
  for (int j = i + 1; j < n_cells; ++j) r += (long)sched[3 * j + 2] * c->B * sched[3 * j + 1];
  return r;
}

// Layout of a layer tape (n_cells + 2 entries): off[i] = cell i's saved state,
// off[n_cells] = the stacked v_in of every cell (mult family; rows in the backward's
// cell order, rounded up to a whole 64-row k-tile), off[n_cells + 1] = total bytes.
template <typename T>
std::vector<size_t> tape_offsets(const dm_config* c, const int32_t* sched, int n_cells) {
  std::vector<size_t> off(n_cells + 2, 0);
  for (int i = 0; i < n_cells; ++i) {
    Carver cv(nullptr);
    carve_save<T>(c, (size_t)c->B * sched[3 * i + 1], sched[3 * i + 2], true, sched[3 * i] > 0, cv);
    off[i + 1] = off[i] + cv.off;
  }
  const long rows = vin_row(c, sched, n_cells, -1);
  const size_t vin_bytes = c->ctx_mod != DM_CTX_LINEAR ? (size_t)((rows + 63) / 64 * 64) * c->d * sizeof(T) : 0;
  off[n_cells + 1] = off[n_cells] + align256(vin_bytes);
  return off;
}

// per-head norm gains of the packed weights (nullptr: that norm is off)
inline const float* kctx_gain(const dm_config* c, const dm_packed* w) {
  return (c->norms & DM_NORM_K_CTX) ? w->gains : nullptr;
}
inline const float* vctx_gain(const dm_config* c, const dm_packed* w) {
  return (c->norms & DM_NORM_V_CTX) ? w->gains + c->h : nullptr;
}
inline const float* v_gain(const dm_config* c, const dm_packed* w) {
  return (c->norms & DM_NORM_V) ? w->gains + 2 * c->h : nullptr;
}

// vpre: v_raw before the v_norm (nullptr: not kept); sa: the M input rows (x-hat);
// small_tiles: 128 x 128 blocks even where 256 x 256 ones fit (more blocks for a short M; the
// k-order of every output element, and so the result, is the same)
template <typename T, int DH, class SA>
void run_proj_src(const dm_config* c, const dm_packed* w, const SA& sa, int M, int Tl, int Tbuf, int buf_t0,
                  int rope_t0, const float* cos, const float* sin, T* qr, T* kraw, T* kself, T* vraw, T* vpre,
                  T* glogx, T* sig, hipStream_t s, bool small_tiles = false, const int* pos_dev = nullptr,
                  int pos_cap = 0) {
  const int nseg = (c->ctx_mod == DM_CTX_LINEAR) ? 5 : 6;
  SrcRows<T> sb{(const T*)w->w_proj, c->d, nseg * c->d};
  if (pos_dev != nullptr) {
    // a decode step at a device position (M <= 64 rows): the RoPE row read from device memory
    EpiProj<T, DH, true> epi{M, c->d, c->h, Tl, Tbuf, buf_t0, 0, cos, sin, w->b_proj, qr, kraw, kself, vraw,
                             glogx, sig, c->ctx_mod == DM_CTX_FUSION, v_gain(c, w), vpre, pos_dev, pos_cap};
    if constexpr (DH == 64)
      launch_gemm_auto<T, 64, 64, 2, 2, 3, 4>(sa, sb, M, nseg * c->d, c->d, epi, s, PROF_PROJ);
    else
      launch_gemm_auto<T, 64, 128, 2, 2, 3, 4>(sa, sb, M, nseg * c->d, c->d, epi, s, PROF_PROJ);
    return;
  }
  EpiProj<T, DH> epi{M, c->d, c->h, Tl, Tbuf, buf_t0, rope_t0, cos, sin, w->b_proj,
                     qr, kraw, kself, vraw, glogx, sig, c->ctx_mod == DM_CTX_FUSION, v_gain(c, w), vpre};
  // bf16, whole 256-row / 256-column tiles: 256 x 256 blocks (four 128 x 128 wave tiles,
  // two direct-to-LDS stages); otherwise 128 x 128 with wave tiles spanning whole heads
  if constexpr (sizeof(T) == 2) {
    if (!small_tiles && M % 256 == 0 && (nseg * c->d) % 256 == 0 && c->d % 64 == 0) {
      launch_gemm<T, 256, 256, 2, 2, -2>(sa, sb, M, nseg * c->d, c->d, epi, s, PROF_PROJ);
      return;
    }
  }
  if (M <= 64) {
    // a decode step's few rows: 64-row blocks, one head wide (twice the blocks of 128 x 128)
    if constexpr (DH == 64)
      launch_gemm_auto<T, 64, 64, 2, 2, 3, 4>(sa, sb, M, nseg * c->d, c->d, epi, s, PROF_PROJ);
    else
      launch_gemm_auto<T, 64, 128, 2, 2, 3, 4>(sa, sb, M, nseg * c->d, c->d, epi, s, PROF_PROJ);
    return;
  }
  if constexpr (DH == 64)
    launch_gemm_auto<T, 128, 128, 2, 2, 3, 4>(sa, sb, M, nseg * c->d, c->d, epi, s, PROF_PROJ);
  else
    launch_gemm_auto<T, 128, 128, 4, 1, 3, 4>(sa, sb, M, nseg * c->d, c->d, epi, s, PROF_PROJ);
}

template <typename T, int DH>
void run_proj(const dm_config* c, const dm_packed* w, const T* xhat, int M, int Tl, int Tbuf, int buf_t0,
              int rope_t0, const float* cos, const float* sin, T* qr, T* kraw, T* kself, T* vraw, T* vpre,
              T* glogx, T* sig, hipStream_t s, const int* pos_dev = nullptr, int pos_cap = 0) {
  run_proj_src<T, DH>(c, w, SrcRows<T>{xhat, c->d, M}, M, Tl, Tbuf, buf_t0, rope_t0, cos, sin, qr, kraw, kself, vraw,
                      vpre, glogx, sig, s, false, pos_dev, pos_cap);
}

template <typename T>
void run_proj_dispatch(const dm_config* c, const dm_packed* w, const T* xhat, int M, int Tl, int Tbuf,
                       int buf_t0, int rope_t0, const float* cos, const float* sin, T* qr, T* kraw, T* kself,
                       T* vraw, T* vpre, T* glogx, T* sig, hipStream_t s) {
  if (c->dh == 64)
    run_proj<T, 64>(c, w, xhat, M, Tl, Tbuf, buf_t0, rope_t0, cos, sin, qr, kraw, kself, vraw, vpre, glogx, sig, s);
  else
    run_proj<T, 128>(c, w, xhat, M, Tl, Tbuf, buf_t0, rope_t0, cos, sin, qr, kraw, kself, vraw, vpre, glogx, sig,
                     s);
}

// Split partials of the next cell's committed prefix that one fused GEMM 2 + attention launch
// computes as extra blocks (splits s0 .. s0 + ns - 1 of ca)
template <typename T> struct AheadComm {
  CommArgs<T> ca;
  int s0 = 0, ns = 0;
};

// One sweep's refine: sweep GEMM 1 (+ GEMM 2 for the mult family) with the blend
// epilogues, writing the refined rows to (Kout, Vout).
template <typename T, int DH>
void run_refine(const dm_config* c, const dm_packed* w, const CellGeom& g, int N, const T* o, const float* ssq,
                const T* kraw, const T* vraw, const T* glogx, const T* sig, const float* cos,
                const float* sin, T* Kout, T* Vout, long out_stride, int out_row0, T* vin, T* gvu,
                T* save1, T* save2, hipStream_t s, const AttendArgs<T>* next_attend = nullptr,
                bool wide = false, const AheadComm<T>* ahead = nullptr) {
  const T* normw = (const T*)w->norm_ctx_w;
  SrcRowsRs<T> sa{o, c->d, N, ssq, c->h, 1.0f / (float)c->d, c->rms_eps};
  SrcRows<T> sb{(const T*)w->w_sweep, c->d, 4 * c->d};
  const bool linear = c->ctx_mod == DM_CTX_LINEAR;
  const float* kgain = kctx_gain(c, w);
  const float* vgain = vctx_gain(c, w);
  if (kgain != nullptr || (linear && vgain != nullptr)) {
    // a norm of GEMM 1's k_ctx or (linear) v_ctx columns: blocks of one head's 2 DH packed columns
    constexpr int NG = DH / 32;
    EpiSweep1<T, DH, NG> e1{g, N, c->ctx_mod, c->mult_res_lambda, kraw, vraw, glogx, sig, cos, sin, o, normw,
                            Kout, Vout, out_stride, out_row0, vin, gvu, save1, kgain, linear ? vgain : nullptr};
    if constexpr (DH == 64)
      launch_gemm_auto<T, 64, 2 * DH, 2, 2, SW1_STAGES, 4>(sa, sb, N, 4 * c->d, c->d, e1, s, PROF_SWEEP1);
    else
      launch_gemm_auto<T, 64, 2 * DH, 1, 4, SW1_STAGES, 2>(sa, sb, N, 4 * c->d, c->d, e1, s, PROF_SWEEP1);
  } else if (wide && DM_GROUPED_WIDE_SW1) {
    // 64 x 128 blocks (two column groups each): a quarter less LDS traffic per MFMA and half the
    // o re-reads, for launches that have blocks to spare (the layer-batched forward)
    EpiSweep1<T, DH, 2> e1{g, N, c->ctx_mod, c->mult_res_lambda, kraw, vraw, glogx, sig, cos, sin, o, normw,
                           Kout, Vout, out_stride, out_row0, vin, gvu, save1};
    launch_gemm_auto<T, 64, 128, 2, 2, SW1_STAGES, 4>(sa, sb, N, 4 * c->d, c->d, e1, s, PROF_SWEEP1);
  } else if (g.pos_dev != nullptr) {
    // a decode step at a device position: RoPE row and output row read from device memory
    EpiSweep1<T, DH, 1, true> e1{g, N, c->ctx_mod, c->mult_res_lambda, kraw, vraw, glogx, sig, cos, sin, o, normw,
                                 Kout, Vout, out_stride, out_row0, vin, gvu, save1};
    launch_gemm_auto<T, 64, 64, 2, 2, SW1_STAGES, 4>(sa, sb, N, 4 * c->d, c->d, e1, s, PROF_SWEEP1);
  } else if (sizeof(T) == 2 && DM_SW1_EIGHT_WAVES && launch_log() == nullptr) {
    // bf16: 64 x 128 blocks of eight waves (each 256-thread half one 64-column group; d is a
    // multiple of 128, so the direct-to-LDS k-loop always applies): the two column groups share
    // the block's o rows, so a k-step moves 24 KB into a CU's LDS instead of the 32 KB of two
    // 64 x 64 blocks, still with eight waves per CU; the same per-element k order
    if constexpr (sizeof(T) == 2) {
      EpiSweep1<T, DH, 2, false, true> e1{g, N, c->ctx_mod, c->mult_res_lambda, kraw, vraw, glogx, sig, cos, sin, o,
                                          normw, Kout, Vout, out_stride, out_row0, vin, gvu, save1};
      launch_gemm<T, 64, 128, 2, 4, -SW1_STAGES>(sa, sb, N, 4 * c->d, c->d, e1, s, PROF_SWEEP1);
    }
  } else {
    EpiSweep1<T, DH> e1{g, N, c->ctx_mod, c->mult_res_lambda, kraw, vraw, glogx, sig, cos, sin, o, normw,
                        Kout, Vout, out_stride, out_row0, vin, gvu, save1};
    launch_gemm_auto<T, 64, 64, 2, 2, SW1_STAGES, 4>(sa, sb, N, 4 * c->d, c->d, e1, s, PROF_SWEEP1);
  }
  if (!linear && next_attend != nullptr) {
    // GEMM 2 fused with the next sweep's attention (64-row cells; the clamp and the v_ctx norm
    // are in its epilogue)
    SrcRows<T> av{vin, c->d, N};
    SrcRows<T> bv{(const T*)w->w_vctx, c->d, c->d};
    EpiSweep2Head<T, DH> e2{g, N, vraw, glogx, gvu, Vout, out_stride, out_row0, save2, vgain};
    if (launch_log() != nullptr) {
      record_launch<Sweep2AttendBody<T, DH>>(dim3(c->h, N / CMAX), dim3(256),
                                             typename Sweep2AttendBody<T, DH>::Args{av, bv, c->d, e2, *next_attend});
      return;
    }
    uint64_t* ts;
    const int idx = prof_launch_begin(PROF_SWEEP2, true, ts);
    if (ahead != nullptr && ahead->ns > 0) {
      const int nfused = c->h * (N / CMAX);
      launch_timed(idx, k_sweep2_attend_comm<T, DH>, dim3(nfused + ahead->ns * c->B * c->h), dim3(256), 0, s, av,
                   bv, c->d, e2, *next_attend, ahead->ca, nfused, ahead->s0, ts);
    } else {
      launch_timed(idx, k_sweep2_attend<T, DH>, dim3(c->h, N / CMAX), dim3(256), 0, s, av, bv, c->d, e2,
                   *next_attend, ts);
    }
    return;
  }
  if (!linear && vgain != nullptr) {
    // v_ctx norm: 64 x DH blocks hold whole heads (the clamp runs in the same epilogue)
    SrcRows<T> av{vin, c->d, N};
    SrcRows<T> bv{(const T*)w->w_vctx, c->d, c->d};
    EpiSweep2Head<T, DH> e2{g, N, vraw, glogx, gvu, Vout, out_stride, out_row0, save2, vgain};
    constexpr int S2 = SW2_STAGES > 0 ? SW2_STAGES : 3;
    launch_gemm_auto<T, 64, DH, 4, 1, S2, 4>(av, bv, N, c->d, c->d, e2, s, PROF_SWEEP2);
    return;
  }
  if (!linear) {
    SrcRows<T> av{vin, c->d, N};
    SrcRows<T> bv{(const T*)w->w_vctx, c->d, c->d};
    if (g.pos_dev != nullptr) {   // device position (see GEMM 1)
      EpiSweep2<T, DH, true> e2{g, N, vraw, glogx, gvu, Vout, out_stride, out_row0, save2};
      if constexpr (SW2_STAGES > 0)
        launch_gemm_auto<T, 64, 32, 4, 1, SW2_STAGES, 8>(av, bv, N, c->d, c->d, e2, s, PROF_SWEEP2);
      else
        launch_gemm<T, 64, 32, 4, 1, 8>(av, bv, N, c->d, c->d, e2, s, PROF_SWEEP2);
    } else {
      EpiSweep2<T, DH> e2{g, N, vraw, glogx, gvu, Vout, out_stride, out_row0, save2};
      if constexpr (SW2_STAGES > 0)
        launch_gemm_auto<T, 64, 32, 4, 1, SW2_STAGES, 8>(av, bv, N, c->d, c->d, e2, s, PROF_SWEEP2);
      else
        launch_gemm<T, 64, 32, 4, 1, 8>(av, bv, N, c->d, c->d, e2, s, PROF_SWEEP2);
    }
  }
  // v'' entry-norm clamp of the refined value rows (v_clamp_tau > 0 only)
  if (g.v_clamp_tau > 0.f) {
    const dim3 grid(cdiv((long)N * c->h, 4));
    if (launch_log() != nullptr)
      record_launch<ClampBody<T, DH>>(grid, dim3(256),
                                      typename ClampBody<T, DH>::Args{g, Vout, out_stride, out_row0, N, g.v_clamp_tau});
    else
      hipLaunchKernelGGL((k_clamp_v<T, DH>), grid, dim3(256), 0, s, g, Vout, out_stride, out_row0, N, g.v_clamp_tau);
  }
}

// Committed accumulator of a cell: split partials over its committed keys but the last ones
// (comm_prev_lo), merged by the first sweep's attention, which adds those last keys itself.
template <typename T, int DH>
int run_comm(const CellGeom& g, const T* qr, const T* Kc, const T* Vc, float scale, const CellWs& ws,
             hipStream_t s) {
  const int kstart = comm_kstart(g.pos0, g.window);
  const int prev_lo = comm_prev_lo(g.pos0, kstart);
  const CommPlan cp = comm_plan(prev_lo - kstart, g.B * g.h);
  const int BH = g.B * g.h;
  CommArgs<T> ca{g, qr, Kc, Vc, cp.split_len, scale, ws.Ap, ws.Zp, ws.Mp};
  ca.nsplit = cp.nsplit;
  ca.kstart = kstart;
  ca.kend = prev_lo;
  if (launch_log() != nullptr) {
    // recorded even without a committed prefix (grid x 0), so that every chunk of a layer
    // records the same launch sequence
    record_launch<CommBody<T, DH>>(dim3(cp.nsplit, BH), dim3(256), ca);
    return cp.nsplit;
  }
  if (cp.nsplit == 0) return 0;
  launch_k(PROF_COMM, k_comm_partial<T, DH>, dim3(cp.nsplit, BH), dim3(256), 0, s, ca);
  return cp.nsplit;
}

// Where a cell without saved state keeps its intra rows: by default the chunk's own cache rows
// [pos0, pos0 + cc) (refined in place, the last sweep leaving the final rows there); a caller
// that holds the committed prefix apart from the new rows (chunk_cell_forward's K_comm / V_comm)
// gives a separate row buffer.
template <typename T> struct CellRows {
  T* K = nullptr; T* V = nullptr;   // nullptr: the cache rows
  long stride = 0;                  // elements between (b, h) row blocks
  int row0 = 0;                     // row of chunk row 0
  int rope_t0 = -1;                 // RoPE table row of chunk row 0 (-1: pos0)
};

// One chunk cell [pos0, pos0+cc) of the layer: n_sweeps Jacobi sweeps against the
// committed rows [0, pos0) of the cache. Without `sv` the sweeps refine the
// chunk's rows in place (the cache rows, or `rows`) and the last sweep leaves the final rows
// there; with `sv` every sweep's rows and state are kept in sv (cache rows untouched).
// Layer loops hand committed-prefix work from one cell to the next: own_nsplit >= 0 says the
// previous cell's launches already computed this cell's split partials (that many); next_pos0 >= 0
// names the next cell (next_cc rows), whose split partials this cell computes inside its fused
// GEMM 2 + attention launches where it has them. Returns how many it computed (-1: none, the next
// cell runs its own). The partials are the same either way: same plan, same kernel body.
template <typename T, int DH>
int run_cell(const dm_config* c, const dm_packed* w, const dm_layer_bufs* L, const float* cos,
             const float* sin, int pos0, int cc, int n_sweeps, int buf_t0, int Tbuf, T* Kc, T* Vc,
             int cache_T, T* ocat, float* o_last, const CellWs& ws, const CellSave<T>* sv, hipStream_t s,
             const CellRows<T>& rows = CellRows<T>{}, bool wide = false, int own_nsplit = -1, int next_pos0 = -1,
             int next_cc = 0) {
  CellGeom g{c->B, cc, c->d, c->h, DH, pos0, buf_t0, Tbuf, cache_T};
  g.kmod_cols = c->kmod_vraw_heads * DH;
  g.kmod_mode = c->kmod_mode;
  g.v_clamp_tau = c->v_clamp_tau;
  g.rope_t0 = rows.rope_t0;
  g.window = window_of(c);
  T* Kr = rows.K ? rows.K : Kc;
  T* Vr = rows.K ? rows.V : Vc;
  const long rows_stride = rows.K ? rows.stride : (long)cache_T * DH;
  const int rows_row0 = rows.K ? rows.row0 : pos0;
  const int BH = c->B * c->h;
  const int N = c->B * cc;
  const size_t NS = (size_t)N, d = c->d;   // per-sweep row stride of the saved arrays
  const float scale = 1.0f / sqrtf((float)DH);
  const T* qr = (const T*)L->qr;
  const T* kself = (const T*)L->kself;
  const T* vraw = (const T*)L->vraw;
  const T* kraw = (const T*)L->kraw;
  const int nsplit = own_nsplit >= 0 ? own_nsplit : run_comm<T, DH>(g, qr, Kc, Vc, scale, ws, s);
  const int prev_lo = comm_prev_lo(pos0, comm_kstart(pos0, g.window));
  const bool committed = pos0 > comm_kstart(pos0, g.window);
  const long cache_stride = (long)cache_T * DH, ws_stride = (long)CMAX * DH;
  const size_t slot = (size_t)BH * CMAX * DH;

  // sweep s + 1's attention runs inside sweep s's GEMM 2 launch (mult family, whole 64-row
  // chunks) when B*h gives that kernel enough blocks, or when forced by the flags
  const bool fuse = c->ctx_mod != DM_CTX_LINEAR && cc == CMAX && !(c->flags & DM_FLAG_UNFUSED_ATTEND) &&
                    ((c->flags & DM_FLAG_FUSED_ATTEND) || BH >= 128);
  // the next cell's split partials, spread over this cell's fused GEMM 2 + attention launches
  // (sweeps 0 .. K-2: one block per (b, h), CUs to spare; as extra blocks of the plain 64 x 32 GEMM 2
  // launches, which fill the chip, they cost more than their own launch); they read only keys
  // before this cell (the next cell's last 64 committed keys are its own attention's)
  auto hosts = [&](int sw) { return fuse && sw < n_sweeps - 1; };
  int n_hosts = 0;
  for (int sw = 0; sw < n_sweeps; ++sw) n_hosts += hosts(sw) ? 1 : 0;
  AheadComm<T> ahead;
  int handed = -1;
  if (next_pos0 >= 0 && n_hosts > 0 && launch_log() == nullptr) {
    CellGeom gn = g;
    gn.pos0 = next_pos0;
    gn.c = next_cc;
    gn.buf_t0 = buf_t0 + (next_pos0 - pos0);
    const int kst = comm_kstart(next_pos0, g.window), plo = comm_prev_lo(next_pos0, kst);
    const CommPlan cp = comm_plan(plo - kst, BH);
    if (plo <= pos0) {
      ahead.ca = CommArgs<T>{gn, qr, Kc, Vc, cp.split_len, scale, ws.Ap, ws.Zp, ws.Mp};
      ahead.ca.nsplit = cp.nsplit;
      ahead.ca.kstart = kst;
      ahead.ca.kend = plo;
      handed = cp.nsplit;
    }
  }
  auto ahead_for = [&](int sw) -> const AheadComm<T>* {
    if (handed <= 0 || !hosts(sw)) return nullptr;
    int j = 0;   // this launch's index among the hosting ones
    for (int u = 0; u < sw; ++u) j += hosts(u) ? 1 : 0;
    ahead.s0 = handed * j / n_hosts;
    ahead.ns = handed * (j + 1) / n_hosts - ahead.s0;
    return &ahead;
  };
  // intra rows read by sweep sw (= the rows written by sweep sw - 1)
  auto rows_in = [&](int sw, const T*& Kin, const T*& Vin, long& in_stride, int& in_row0) {
    if (sw == 0) { Kin = kself; Vin = vraw; in_stride = (long)Tbuf * DH; in_row0 = buf_t0; }
    else if (sv) { Kin = sv->Kin + sw * slot; Vin = sv->Vin + sw * slot; in_stride = ws_stride; in_row0 = 0; }
    else { Kin = Kr; Vin = Vr; in_stride = rows_stride; in_row0 = rows_row0; }
  };
  auto attend_args = [&](int sw) {
    const bool last = sw == n_sweeps - 1;
    const T* Kin; const T* Vin; long in_stride; int in_row0;
    rows_in(sw, Kin, Vin, in_stride, in_row0);
    T* o = sv ? sv->o + sw * NS * d : (T*)ws.o;
    float* ssq = sv ? sv->ssq + sw * NS * c->h : ws.ssq;
    return AttendArgs<T>{g, qr, kself, vraw, Kin, Vin, in_stride, in_row0,
                         sw == 0 ? nsplit : 0, ws.Ap, ws.Zp, ws.Mp, ws.A, ws.Z, ws.M,
                         scale, o, ssq, last ? ocat : nullptr, last ? o_last : nullptr,
                         sv ? sv->stat_m + sw * (size_t)BH * CMAX : nullptr,
                         sv ? sv->stat_z + sw * (size_t)BH * CMAX : nullptr,
                         sw > 0 && committed ? 1 : 0, Kc, Vc, sw == 0 ? prev_lo : pos0};
  };

  for (int sw = 0; sw < n_sweeps; ++sw) {
    const bool last = sw == n_sweeps - 1;
    // rows written by this sweep's refine
    T* Kout; T* Vout; long out_stride; int out_row0;
    if (sv && !(last && sv->last_to_cache)) { Kout = sv->Kin + (sw + 1) * slot; Vout = sv->Vin + (sw + 1) * slot; out_stride = ws_stride; out_row0 = 0; }
    else if (sv) { Kout = Kc; Vout = Vc; out_stride = cache_stride; out_row0 = pos0; }
    else { Kout = Kr; Vout = Vr; out_stride = rows_stride; out_row0 = rows_row0; }

    T* o = sv ? sv->o + sw * NS * d : (T*)ws.o;
    float* ssq = sv ? sv->ssq + sw * NS * c->h : ws.ssq;
    if (sw == 0 || !fuse) {   // else the previous sweep's GEMM 2 launch ran it
      const AttendArgs<T> aa = attend_args(sw);
      // 16-row waves; the (b, h) blocks split by query rows until there are >= 256 blocks
      if (launch_log() != nullptr) {
        if (BH >= 256) record_launch<AttendBody<T, DH, 4>>(dim3(BH, 1), dim3(256), aa);
        else if (BH >= 128) record_launch<AttendBody<T, DH, 2>>(dim3(BH, 2), dim3(128), aa);
        else record_launch<AttendBody<T, DH, 1>>(dim3(BH, 4), dim3(64), aa);
      } else if (BH >= 256) launch_k(PROF_ATTEND, k_attend<T, DH, 4>, dim3(BH, 1), dim3(256), 0, s, aa);
      else if (BH >= 128) launch_k(PROF_ATTEND, k_attend<T, DH, 2>, dim3(BH, 2), dim3(128), 0, s, aa);
      else launch_k(PROF_ATTEND, k_attend<T, DH, 1>, dim3(BH, 4), dim3(64), 0, s, aa);
    }
    T* vin = sv ? sv->vin + sw * NS * d : (T*)ws.vin;
    const AttendArgs<T> next = attend_args(last ? sw : sw + 1);
    run_refine<T, DH>(c, w, g, N, o, ssq, kraw, vraw, (const T*)L->glogx, (const T*)L->sig, cos, sin, Kout, Vout,
                      out_stride, out_row0, vin, (T*)ws.gvu, sv ? sv->save1 + sw * NS * 4 * d : nullptr,
                      sv ? sv->save2 + sw * NS * d : nullptr, s, (fuse && !last) ? &next : nullptr, wide,
                      ahead_for(sw));
  }
  return handed;
}

template <typename T>
int run_cell_dispatch(const dm_config* c, const dm_packed* w, const dm_layer_bufs* L, const float* cos,
                      const float* sin, int pos0, int cc, int n_sweeps, int buf_t0, int Tbuf, void* Kc,
                      void* Vc, int cache_T, void* ocat, float* o_last, const CellWs& ws,
                      const CellSave<T>* sv, hipStream_t s, const CellRows<T>& rows = CellRows<T>{},
                      int own_nsplit = -1, int next_pos0 = -1, int next_cc = 0) {
  if (c->dh == 64)
    return run_cell<T, 64>(c, w, L, cos, sin, pos0, cc, n_sweeps, buf_t0, Tbuf, (T*)Kc, (T*)Vc, cache_T, (T*)ocat,
                           o_last, ws, sv, s, rows, false, own_nsplit, next_pos0, next_cc);
  return run_cell<T, 128>(c, w, L, cos, sin, pos0, cc, n_sweeps, buf_t0, Tbuf, (T*)Kc, (T*)Vc, cache_T, (T*)ocat,
                          o_last, ws, sv, s, rows, false, own_nsplit, next_pos0, next_cc);
}

inline int check_bufs(const dm_config* c, const dm_layer_bufs* L) {
  DM_REQUIRE(L != nullptr, DM_ERR_INVALID, "null layer buffers");
  DM_REQUIRE(L->T > 0, DM_ERR_INVALID, "layer buffer T=%d", L->T);
  DM_REQUIRE(L->qr && L->kraw && L->kself && L->vraw && L->glogx, DM_ERR_INVALID, "null layer buffer");
  DM_REQUIRE(aligned16(L->qr) && aligned16(L->kraw) && aligned16(L->kself) && aligned16(L->vraw),
             DM_ERR_INVALID, "layer buffers must be 16-byte aligned");
  DM_REQUIRE(c->ctx_mod == DM_CTX_LINEAR || L->sig != nullptr, DM_ERR_INVALID,
             "ctx_mod mult/mult_res needs the sig buffer");
  return DM_OK;
}

inline int check_packed(const dm_config* c, const dm_packed* w) {
  DM_REQUIRE(w != nullptr, DM_ERR_INVALID, "null packed weights");
  DM_REQUIRE(w->w_proj && w->b_proj && w->w_sweep && w->norm_ctx_w, DM_ERR_INVALID, "null packed weight");
  DM_REQUIRE(c->ctx_mod == DM_CTX_LINEAR || w->w_vctx, DM_ERR_INVALID, "mult family needs w_vctx");
  DM_REQUIRE(c->norms == 0 || w->gains, DM_ERR_INVALID, "the head norms need the packed gains");
  DM_REQUIRE(aligned16(w->w_proj) && aligned16(w->w_sweep) && aligned16(w->norm_ctx_w) &&
                 (w->w_vctx == nullptr || aligned16(w->w_vctx)),
             DM_ERR_INVALID, "packed weights must be 16-byte aligned");
  return DM_OK;
}

}  // namespace dm
