// libdm_hip.so — the backward entry points of the C ABI (include/dm_abi.h):
// reverse-scan layer backward, reading every cell's sweep states from the
// forward's tape or rebuilding them by exact per-cell recompute.
//
// Never allocates device memory and never synchronizes: every buffer is carved
// from the caller's workspace; all launches go to the caller's stream.
#include <initializer_list>
#include <utility>
#include <vector>

#include "dm_block.h"
#include "dm_bwd.h"
#include "dm_fwd_host.h"

namespace dm {

template <typename T> struct BwdWs {
  // layer accumulators (fp32)
  float *dq, *dkraw, *dkself, *dvraw;   // [B, h, T, dh]
  CellRow* cellrow;                     // [T] the cell of each layer row (written by the attention VJP)
  float *dsig;                          // [B, T, d]
  float *docat;                         // [B, T, d] = dy . W_O
  float *dnw;                           // [NSLOT, d] norm_ctx.weight partials
  // one cell
  CellWs fws;                           // forward scratch of the recompute
  CellSave<T> sv;                       // every sweep's state
  float *lamdv, *gw, *rowdot;           // [N, d], [N, d], [N, d / DU_EPI_TN]
  float *du_part;                       // [DU_SPLIT, N, d] split-K slices of du
  // committed-prefix VJP: per-row state from the attention VJP, key-side partial sums
  float *Grow, *Drow, *Mrow;            // [B*h, T, dh], [B*h, T], [B*h, T]
  T* Gb;                                // [B*h, T, dh] G in the storage dtype once complete (the
                                        // committed VJPs' MFMA operand)
  float *sdss;                          // [B*h, T] the self column's dS summed over a cell's sweeps
  int* klim;                            // [T]
  float *dKp, *dVp;                     // [comm_nsq(B*h), B*h, CMAX, dh]
  // weight grads of the sweeps, one GEMM per layer: the cells' transposed operands
  // stacked row-major, [Rp, 4d | d] with Rp >= sum over cells of K*B*c (rounded to 64);
  // a cell's sweeps write their dctx / dv_ctx rows in place, u and v_in are added per cell
  T *dctxL, *uL, *dvcL, *vinL;
  long Rp;
  float* kpart;                         // [KSPLIT_ELEMS(d)] split-K partials
  // layer close
  T* dproj;                             // [B*T, nproj*d]
  float* dxhat;                         // [B*T, d]
  float *dWp, *dWs;                     // packed weight-grad staging [nproj*d, d], [4d, d]
  float* colpart;                       // [max(NCHUNK, projection VJP chunks), 3d] column partials
  // head norms: per-row partials of the k_gain / ctx_gain grads [B*T, h], and the v_gain grad's
  // per-chunk partials [projection VJP chunks, h] (nullptr when that norm is off); the projection
  // VJP writes B*T / PROJ_ROWS * proj_rows_in_flight(d) chunks
  float *dkg, *dvg, *vgpart;
  size_t bytes;
};

constexpr int NSLOT_TM = 16;      // rows per norm_ctx-weight partial slot (k_du_epi block rows)
constexpr int DU_SPLIT = DM_DU_SPLIT;   // split-K slices of the du GEMM
constexpr int DV_BN = 64;               // dv_in GEMM block columns beside the du slices (64 x DV_BN blocks)
constexpr int DUF_BM = 32;              // block rows of du's last slice with the RMS-VJP epilogue (DUF_BM x 64)
constexpr int DUF_STAGES = 3;           // its direct-to-LDS stages
constexpr int NCHUNK = 64;        // row chunks of the column sums
// fp32 elements of the split-K partial buffer of the weight-grad GEMMs ([S, M, N], N = d): eight
// slices of the 6d x d projection product
constexpr long KSPLIT_ELEMS(long d) { return 48 * d * d; }

template <typename T>
BwdWs<T> carve_bwd(const dm_config* c, int T_, int cache_T, int kmax, void* base) {
  BwdWs<T> w{};
  const size_t B = c->B, d = c->d, h = c->h, dh = c->dh, e = sizeof(T);
  const size_t BT = B * T_, BH = B * h, N = B * CMAX;
  const size_t nproj = c->ctx_mod == DM_CTX_LINEAR ? 5 : 6;
  Carver cv(base);
  w.dq = cv.take<float>(BT * d * 4);
  w.dkraw = cv.take<float>(BT * d * 4);
  w.dkself = cv.take<float>(BT * d * 4);
  w.dvraw = cv.take<float>(BT * d * 4);
  w.cellrow = cv.take<CellRow>((size_t)T_ * sizeof(CellRow));
  w.dsig = cv.take<float>(BT * d * 4);
  w.docat = cv.take<float>(BT * d * 4);
  w.dnw = cv.take<float>(cdiv(N, NSLOT_TM) * d * 4);
  w.fws = carve_cell(c, cache_T, cv.base ? cv.base + cv.off : nullptr);
  cv.off += align256(w.fws.bytes);
  w.sv = carve_save<T>(c, N, kmax, false, false, cv);
  w.lamdv = cv.take<float>(N * d * 4);
  w.gw = cv.take<float>(N * d * 4);
  w.rowdot = cv.take<float>(N * (d / DU_EPI_TN) * 4);
  w.du_part = cv.take<float>(DU_SPLIT * N * d * 4);
  w.Grow = cv.take<float>(BT * d * 4);
  w.Gb = cv.take<T>(BT * d * e);
  w.Drow = cv.take<float>(BH * T_ * 4);
  w.Mrow = cv.take<float>(BH * T_ * 4);
  w.sdss = cv.take<float>(BH * T_ * 4);
  w.klim = cv.take<int>(T_ * 4);
  w.dKp = cv.take<float>(comm_nsq((int)BH) * BH * CMAX * dh * 4);
  w.dVp = cv.take<float>(comm_nsq((int)BH) * BH * CMAX * dh * 4);
  w.Rp = (long)cdiv((long)kmax * B * T_, 64) * 64;
  w.dctxL = cv.take<T>(w.Rp * 4 * d * e);
  w.uL = cv.take<T>(w.Rp * d * e);
  w.dvcL = cv.take<T>(w.Rp * d * e);
  w.vinL = cv.take<T>(w.Rp * d * e);
  w.kpart = cv.take<float>(KSPLIT_ELEMS((long)d) * 4);
  // the attn_norm weight partials [B*T, d] fp32 reuse dproj once it is consumed
  w.dproj = cv.take<T>(std::max(BT * nproj * d * e, BT * d * 4));
  w.dxhat = cv.take<float>(BT * d * 4);
  w.dWp = cv.take<float>(nproj * d * d * 4);
  w.dWs = cv.take<float>(4 * d * d * 4);
  const long pparts = cdiv(BT, PROJ_ROWS) * proj_rows_in_flight((int)d);   // projection VJP partial chunks
  w.colpart = cv.take<float>((size_t)std::max<long>(NCHUNK, pparts) * 3 * d * 4);
  w.dkg = (c->norms & DM_NORM_K_CTX) ? cv.take<float>(BT * h * 4) : nullptr;
  w.dvg = (c->norms & DM_NORM_V_CTX) ? cv.take<float>(BT * h * 4) : nullptr;
  w.vgpart = (c->norms & DM_NORM_V) ? cv.take<float>((size_t)pparts * h * 4) : nullptr;
  w.bytes = cv.off;
  return w;
}

// zero several fp32 arrays in one launch (array i in grid row i)
inline void fill0_list(std::initializer_list<std::pair<float*, size_t>> arrs, hipStream_t s) {
  FillList fl{};
  size_t most = 0;
  for (const auto& a : arrs) {
    if (a.second == 0) continue;
    fl.p[fl.n_arr] = a.first;
    fl.n[fl.n_arr] = (long)a.second;
    ++fl.n_arr;
    most = std::max(most, a.second);
  }
  if (fl.n_arr == 0) return;
  const int blocks = (int)std::min<size_t>((most / 4 + 255) / 256, 1024);
  hipLaunchKernelGGL(k_fill_list, dim3(blocks, fl.n_arr), dim3(256), 0, s, fl);
}

// out[chunk] column sums of a [M, ncols] fp32 matrix, added into dst[0..ncols)
inline void colsum_add(const float* src, int M, int ncols, float* part, float* dst, hipStream_t s) {
  const int rpc = cdiv(M, NCHUNK);
  hipLaunchKernelGGL(k_colsum_partial, dim3(cdiv(ncols, 256), NCHUNK), dim3(256), 0, s, M, ncols, rpc, src, part);
  hipLaunchKernelGGL(k_sum_rows_add, dim3(cdiv(ncols, 64)), dim3(256), 0, s, NCHUNK, ncols, ncols, part, dst,
                     (float*)nullptr, (float*)nullptr, ncols);
}

inline void unpack(const std::vector<UnpackSeg>& segs, int ncols, const float* src, hipStream_t s) {
  for (size_t i0 = 0; i0 < segs.size(); i0 += UNPACK_MAX_SEG) {
    UnpackArgs a{};
    a.nseg = (int)std::min<size_t>(UNPACK_MAX_SEG, segs.size() - i0);
    int rows = 0;
    for (int i = 0; i < a.nseg; ++i) { a.seg[i] = segs[i0 + i]; rows += a.seg[i].nrows; }
    a.ncols = ncols;
    a.src = src;
    hipLaunchKernelGGL(k_unpack_add, dim3(rows), dim3(256), 0, s, a);
  }
}

// C [M, N] (+)= A^T . B for row-major A [K, M], B [K, N] (the weight-grad products
// sum over rows): the operands are read K-major straight from the row-major buffers
// (bf16 with whole tiles: direct-to-LDS k-loop with transposed-view fragment loads);
// split-K over enough slices to give every CU a block, the slices stored into `part`
// and summed into C in a fixed order.
template <typename T>
void gemm_tn(const T* A, long lda, const T* Bm, long ldb, float* C, int M, int N, int K, int accumulate,
             float* part, hipStream_t s) {
  const bool dma = sizeof(T) == 2 && K % 64 == 0 && M % 128 == 0 && N % 128 == 0;
  const bool big = dma && M % 256 == 0 && N % 256 == 0;
  const long blocks = big ? (long)(M / 256) * (N / 256) : (long)cdiv(M, 128) * cdiv(N, 128);
  int S = 1;
  if (big) {
    // one 256 x 256 block per CU: a launch takes ceil(blocks S / 256) rounds of K / S each; take
    // the fewest slices within 10% of the fewest rounds per unit of k (e.g. 384 tiles: 2 slices,
    // 3 rounds of half the k instead of 2 rounds of all of it)
    long num = cdiv(blocks, 256), den = 1;
    for (int s2 = 2; s2 <= 16; s2 *= 2) {
      if ((K / 64) % s2 != 0 || (long)s2 * M * N > KSPLIT_ELEMS((long)N)) break;
      const long r = cdiv(blocks * s2, 256);
      if (r * den * 10 < num * s2 * 9) {
        num = r;
        den = s2;
      }
    }
    S = (int)den;
  } else {
    while (K % 64 == 0 && S < 16 && blocks * S * 2 < 1025 && (long)S * 2 * M * N <= KSPLIT_ELEMS((long)N) &&
           (K / 64) % (S * 2) == 0)
      S *= 2;
  }
  SrcKMajor<T> sa{A, lda, M}, sb{Bm, ldb, N};
  sa.kmax = K;
  sb.kmax = K;
  if (S == 1) {
    EpiStoreF32 ep{M, N, accumulate, C};
    launch_gemm_kk<T>(sa, sb, M, N, K, ep, s);
    return;
  }
  EpiStoreTileF32 ep{M, N, part, (long)M * N};
  if constexpr (sizeof(T) == 2) {
    if (big) launch_gemm_splitk<T, 256, 256, 2, 2, -KK_STAGES>(sa, sb, M, N, K, S, ep, s);
    else if (dma) launch_gemm_splitk<T, 128, 128, 2, 2, -3>(sa, sb, M, N, K, S, ep, s);
    else launch_gemm_splitk<T, 128, 128, 2, 2, 4>(sa, sb, M, N, K, S, ep, s);
  } else {
    launch_gemm_splitk<T, 128, 128, 2, 2, 4>(sa, sb, M, N, K, S, ep, s);
  }
  const long n = (long)M * N;
  if (n % 4 == 0 && reinterpret_cast<uintptr_t>(C) % 16 == 0 && reinterpret_cast<uintptr_t>(part) % 16 == 0 &&
      (S == 2 || S == 4 || S == 8 || S == 16)) {
    const long n4 = n / 4;
    const dim3 g4(cdiv(n4, 256));
    const float4* p4 = reinterpret_cast<const float4*>(part);
    float4* c4 = reinterpret_cast<float4*>(C);
    if (S == 2) hipLaunchKernelGGL(k_sum_splits4<2>, g4, dim3(256), 0, s, n4, p4, c4, accumulate);
    else if (S == 4) hipLaunchKernelGGL(k_sum_splits4<4>, g4, dim3(256), 0, s, n4, p4, c4, accumulate);
    else if (S == 8) hipLaunchKernelGGL(k_sum_splits4<8>, g4, dim3(256), 0, s, n4, p4, c4, accumulate);
    else hipLaunchKernelGGL(k_sum_splits4<16>, g4, dim3(256), 0, s, n4, p4, c4, accumulate);
  } else {
    hipLaunchKernelGGL(k_sum_splits, dim3(cdiv(n, 256)), dim3(256), 0, s, S, n, (const float*)part, C, accumulate);
  }
}

// ---- the SwiGLU MLP sublayer's entry points and weight grads ----------------------------------
struct MlpWs {
  float* kpart;      // split-K partials of the two weight-grad products
  float* stage;      // [2H, d] dw13 in w13's row order
  float* dwa_part;   // [ceil(M / RMSN_ROWS), d] mlp_norm weight partials
  float* colpart;    // [NCHUNK, d]
  size_t bytes;
};
inline size_t mlp_kpart_elems(long d, long H) {
  // gemm_tn's largest split (<= 16 slices, <= KSPLIT_ELEMS(N) elements) of dW2 [d, H] and dw13 [2H, d]
  return (size_t)std::max(std::min(16 * d * H, KSPLIT_ELEMS(H)), std::min(16 * 2 * H * d, KSPLIT_ELEMS(d)));
}
inline MlpWs carve_mlp(int M, int d, int H, void* base) {
  MlpWs w{};
  Carver cv(base);
  w.kpart = cv.take<float>(mlp_kpart_elems(d, H) * 4);
  w.stage = cv.take<float>((size_t)2 * H * d * 4);
  w.dwa_part = cv.take<float>((size_t)cdiv(M, RMSN_ROWS) * d * 4);
  w.colpart = cv.take<float>((size_t)NCHUNK * d * 4);
  w.bytes = cv.off;
  return w;
}
// the weight grads over all M rows (after every row's VJP): dW2 += dz^T mid, dw13 = dab^T h unpacked
// into W1 / W3, the mlp_norm weight from the per-8-row partials (in dwa_part)
template <typename T>
void mlp_wgrad(const dm_mlp_bufs* mb, const T* dz, int M, int d, int H, const dm_mlp_grads* g, const MlpWs& ws,
               hipStream_t s) {
  gemm_tn<T>(dz, d, (const T*)mb->mid, H, g->w2, d, H, M, 1, ws.kpart, s);
  gemm_tn<T>((const T*)mb->dab, 2L * H, (const T*)mb->h, d, ws.stage, 2 * H, d, M, 0, ws.kpart, s);
  hipLaunchKernelGGL(k_unpack_w13, dim3(2 * H), dim3(256), 0, s, (const float*)ws.stage, H, d, g->w1, g->w3);
  colsum_add(ws.dwa_part, cdiv(M, RMSN_ROWS), d, ws.colpart, g->norm_w, s);
}

// The backward of one layer in three parts, as the reference's fused engine splits it
// (FusedSweepCell.layer_blockmlp_bwd / cell_backward / layer_close, fused_sweep.py:1557-1959):
//   bwd_begin  zero the layer accumulators; W_O VJP (do_cat = dy . W_O, dW_O += dy^T o_cat)
//   bwd_cell   one cell, the cells last first: its sweep states (tape or exact recompute), then its
//              sweeps backward; the weight-grad operands of its rows are stacked in the workspace
//   bwd_end    the sweep weight grads (one GEMM per weight over every cell's stacked rows), the
//              projection VJP, the attn_norm VJP and dx
// The committed prefix a cell reads gets its grads one of two ways. Layer path (dm_layer_bwd): a
// cell's final rows receive, right before its sweeps, the sum over every later row's committed
// attention (k_comm_dkv from the per-row G / Dbar, complete once the later cells are done; no fp32
// grad cache) and the query side runs once per layer. Grad-cache path (dm_cell_bwd, the
// reference's protocol, engines/wavescan/engine/backward.py:92-123): the cell takes its own rows'
// grads from the caller's fp32 cache dK_gc / dV_gc, and right after its sweeps ADDS the grads of
// the committed rows it read into dK_gc / dV_gc[:, :, :pos0] and its query side into dq.
struct GradCache {
  float* dK = nullptr;   // [B, h, cache_T, dh] fp32, or nullptr: layer path
  float* dV = nullptr;
};

template <typename T, int DH>
void bwd_begin(const dm_config* c, const dm_packed* w, const T* dy, const T* ocat, int T_, const dm_grads* gr,
               const BwdWs<T>& ws, hipStream_t s) {
  const int B = c->B, d = c->d, BT = B * T_;
  fill0_list({{ws.dq, (size_t)BT * d},
              {ws.sdss, (size_t)BT * c->h},
              {ws.dkraw, (size_t)BT * d},
              {ws.dkself, (size_t)BT * d},
              {ws.dvraw, (size_t)BT * d},
              {reinterpret_cast<float*>(ws.cellrow), (size_t)T_ * sizeof(CellRow) / 4},
              {ws.dsig, (size_t)BT * d},
              {ws.dnw, (size_t)cdiv(B * CMAX, NSLOT_TM) * d},
              {ws.dWs, (size_t)4 * d * d},
              {ws.dkg, ws.dkg ? (size_t)BT * c->h : 0},
              {ws.dvg, ws.dvg ? (size_t)BT * c->h : 0}},
             s);
  // W_O: do_cat = dy . W_O ; dW_O += dy^T . ocat
  EpiStoreTileF32 ep{BT, d, ws.docat, 0};
  launch_gemm_big<T>(SrcRows<T>{dy, d, BT}, SrcRows<T>{(const T*)w->wo_t, d, d}, BT, d, d, ep, s);
  gemm_tn<T>(dy, d, ocat, d, gr->wo, d, d, BT, 1, ws.kpart, s);
}

// the stacked v_in of every cell: the tape's (saved by the forward in the backward's cell order)
// or the workspace's (written by the recompute)
template <typename T>
T* stacked_vin(const char* tape, const size_t* tape_off, int n_cells, const BwdWs<T>& ws) {
  return tape != nullptr ? (T*)(const_cast<char*>(tape) + tape_off[n_cells]) : ws.vinL;
}

// rms: tape cells' o rows to normalise after the cell loop (nullptr: now)
// What one call of a layer's reverse scan leaves for the next (cell ci - 1): far_done, that cell's
// key-side committed-VJP splits 1 .. nsq-1 were computed inside this call's attention-VJP launches
// (only split 0 is left); comm_nsplit >= 0, its exact recompute's committed-prefix split partials
// were computed inside this call's recompute (run_cell's handoff), that many.
struct CellHandoff {
  bool far_done = false;
  int comm_nsplit = -1;
};

template <typename T, int DH>
void bwd_cell(const dm_config* c, const dm_packed* w, const float* cos, const float* sin, const dm_layer_bufs* L,
              const int32_t* sched, int n_cells, int ci, const T* Kc, const T* Vc, int cache_T, const char* tape,
              const size_t* tape_off, const GradCache& gc, const BwdWs<T>& ws, std::vector<RmsSeg>* rms,
              hipStream_t s, CellHandoff* ho = nullptr) {
  const bool far_done = ho != nullptr && ho->far_done;
  const int B = c->B, d = c->d, h = c->h, T_ = L->T, BH = B * h;
  const bool mult = c->ctx_mod != DM_CTX_LINEAR;
  const float scale = 1.0f / sqrtf((float)DH);
  const float inv_d = 1.0f / (float)d;
  const T* qr = (const T*)L->qr;
  const T* kself = (const T*)L->kself;
  const T* vraw = (const T*)L->vraw;
  const T* kraw = (const T*)L->kraw;
  const size_t slot = (size_t)BH * CMAX * DH;
  const size_t lds_attn = AttnBwdCfg<T, DH>::LDS_ELEMS * sizeof(T);
  const size_t lds_attn_bwd = AttnBwdCfg<T, DH>::BWD_LDS_BYTES;
  T* vinS = stacked_vin<T>(tape, tape_off, n_cells, ws);
  const int t_end = sched[3 * (n_cells - 1)] + sched[3 * (n_cells - 1) + 1];   // rows of the schedule
  const long coff = vin_row(c, sched, n_cells, ci);   // rows of the cells after this one in the stacks

  const int pos0 = sched[3 * ci], cc = sched[3 * ci + 1], K = sched[3 * ci + 2];
  const int N = B * cc;
  const size_t NS = (size_t)N;
  CellGeom g{B, cc, d, h, DH, pos0, pos0, T_, cache_T};
  g.window = window_of(c);
  g.kmod_cols = c->kmod_vraw_heads * DH;
  g.kmod_mode = c->kmod_mode;
  g.v_clamp_tau = c->v_clamp_tau;
  // every sweep's state of the cell: saved by the forward, or an exact recompute
  CellSave<T> sv = ws.sv;
  const float* Mx;
  if (tape != nullptr) {
    Carver cv(const_cast<char*>(tape) + tape_off[ci]);
    sv = carve_save<T>(c, NS, K, true, pos0 > 0, cv);
    if (mult) sv.vin = vinS + coff * d;
    Mx = sv.Mx;
  } else {
    if (mult) sv.vin = vinS + coff * d;   // the recompute writes v_in into the stacked rows
    // in a layer's reverse scan the recompute also computes the next cell's (ci - 1) committed-prefix
    // partials inside its fused launches, as a layer's forward does for the cell after
    const int own = ho != nullptr ? ho->comm_nsplit : -1;
    const int handed = run_cell<T, DH>(c, w, L, cos, sin, pos0, cc, K, pos0, T_, (T*)Kc, (T*)Vc, cache_T, nullptr,
                                       nullptr, ws.fws, &sv, s, CellRows<T>{}, false, own,
                                       ho != nullptr && ci > 0 ? sched[3 * (ci - 1)] : -1,
                                       ho != nullptr && ci > 0 ? sched[3 * (ci - 1) + 1] : 0);
    if (ho != nullptr) ho->comm_nsplit = handed;
    Mx = pos0 > 0 ? ws.fws.M : nullptr;
  }
  // grads of the cell's final rows: layer path, the committed-prefix attention of every later
  // row (their G / Dbar / row max are in place: those cells are done), in comm_nsq partial slots;
  // grad-cache path, the cache rows [pos0, pos0 + cc)
  const float* dKn;
  const float* dVn;
  long dn_stride, dn_psum;
  int dn_row0;
  if (gc.dK == nullptr) {
    CommKeyArgs<T> ka{B, h, T_, cache_T, pos0, cc, pos0 + cc, t_end, qr, Kc, Vc, ws.Gb, ws.Drow, ws.Mrow,
                      scale, ws.dKp, ws.dVp};
    ka.window = window_of(c);
    ka.nsq = comm_nsq(BH);
    const int nlaunch = far_done ? 1 : ka.nsq;
    if (launch_log() != nullptr)
      record_launch<CommDkvBody<T, DH>>(dim3(nlaunch, BH), dim3(256), ka, (unsigned)lds_attn);
    else
      hipLaunchKernelGGL((k_comm_dkv<T, DH>), dim3(nlaunch, BH), dim3(256), lds_attn, s, ka);
    dKn = ws.dKp; dVn = ws.dVp; dn_stride = (long)CMAX * DH; dn_row0 = 0; dn_psum = (long)BH * CMAX * DH;
  } else {
    dKn = gc.dK; dVn = gc.dV; dn_stride = (long)cache_T * DH; dn_row0 = pos0; dn_psum = 0;
  }
  // The cell before this one (ci - 1): its key-side committed-VJP splits 1 .. nsq-1 read query rows
  // from pos0 + 64 on, all of them complete (the cells after this one; this cell's rows are its
  // split 0), so this cell's attention-VJP launches take them as extra blocks (head_dim 64: those
  // launches leave a third of the CUs' block slots free; in a layer's own launches only).
  CommKeyArgs<T> kprev{};
  int host_splits = 0;
  if constexpr (DH == 64) {
    if (gc.dK == nullptr && launch_log() == nullptr && ci > 0 && t_end > pos0 + 64) {
      kprev = CommKeyArgs<T>{B, h, T_, cache_T, sched[3 * (ci - 1)], sched[3 * (ci - 1) + 1], pos0, t_end, qr, Kc, Vc,
                             ws.Gb, ws.Drow, ws.Mrow, scale, ws.dKp, ws.dVp};
      kprev.window = window_of(c);
      kprev.nsq = comm_nsq(BH);
      host_splits = kprev.nsq - 1;
    }
  }
  // this cell's rows of the stacked weight-grad operands
  T* dctx = ws.dctxL + coff * 4 * d;
  T* dvc = ws.dvcL + coff * d;
  // refine VJP arguments of sweep sw (the grads of its refined rows: given by the caller)
  auto refine_args = [&](int sw) {
    return RefineBwdArgs<T>{g, N, c->ctx_mod, dKn, dVn, dn_stride, dn_row0, dn_psum,
                            sv.save1 + sw * NS * 4 * d, mult ? sv.save2 + sw * NS * d : nullptr, (const T*)L->glogx, kraw,
                            vraw, cos, sin, dctx + sw * NS * 4 * d, dvc + sw * NS * d, ws.dkraw,
                            ws.dvraw, kctx_gain(c, w), vctx_gain(c, w), ws.dkg, ws.dvg};
  };
  for (int sw = K - 1; sw >= 0; --sw) {
    // refine VJP of sweep sw: the last sweep's from the final-row grads above, in its own launch;
    // the others run inside the attention VJP of the sweep after them (below)
    if (sw == K - 1) {
      const RefineBwdArgs<T> ra = refine_args(sw);
      const dim3 rgrid(cdiv((long)N * d / 8, 256));
      if (launch_log() != nullptr) {
        if (gc.dK == nullptr && comm_nsq(BH) == 8) record_launch<RefineBwdBody<T, DH, 8>>(rgrid, dim3(256), ra);
        else if (gc.dK == nullptr) record_launch<RefineBwdBody<T, DH, 4>>(rgrid, dim3(256), ra);
        else launch_log()->unsupported = true;
      } else if (gc.dK == nullptr) {
        if (comm_nsq(BH) == 8) hipLaunchKernelGGL((k_refine_bwd<T, DH, 8>), rgrid, dim3(256), 0, s, ra);
        else hipLaunchKernelGGL((k_refine_bwd<T, DH, 4>), rgrid, dim3(256), 0, s, ra);
      } else {
        hipLaunchKernelGGL((k_refine_bwd<T, DH, 1>), rgrid, dim3(256), 0, s, ra);
      }
    }
    // du = dctx . W_sweep (+ lam dv_in) in DU_SPLIT split-K slices of d columns, then the RMS-VJP
    // inputs. Mult family: slice 2 is dctx's v_map columns, which the dv_in GEMM's epilogue writes
    // (dv_in = dv_ctx . W_vctx), so dv_in and the other slices run as one launch and slice 2 follows
    // with the RMS-VJP inputs in its epilogue (EpiDuFinal): two launches where dv_in, du and du_epi
    // took three. Linear: all slices, then k_du_epi.
    static_assert(DU_SPLIT == 4, "slice 2 of the du GEMM is the v_map column block");
    const SrcRows<T> da{dctx + sw * NS * 4 * d, 4 * d, N}, db{(const T*)w->w_sweep_t, 4 * d, d};
    const typename DuEpiBody<T, DU_SPLIT>::Args ea{N, d, h, inv_d, c->rms_eps, (const float*)ws.du_part,
                                                   mult ? (const float*)ws.lamdv : nullptr,
                                                   (const T*)(sv.o + sw * NS * d),
                                                   (const float*)(sv.ssq + sw * NS * h), (const T*)w->norm_ctx_w,
                                                   ws.gw, ws.rowdot, ws.dnw};
    EpiStoreTileF32 ep{N, d, ws.du_part, (long)N * d};
    if (mult) {
      const SrcRows<T> av{dvc + sw * NS * d, d, N}, bv{(const T*)w->w_vctx_t, d, d};
      const SrcRows<T> da2{dctx + sw * NS * 4 * d + 2 * d, 4 * d, N}, db2{(const T*)w->w_sweep_t + 2 * d, 4 * d, d};
      const EpiDuFinal<T, DU_SPLIT, 2, DUF_BM == 32> efp{N, d, h, inv_d, c->rms_eps, ea.part, ea.lamdv, ea.o, ea.ssq,
                                                         ea.normw, ea.gw, ea.rowdot, ea.dnw};
      bool grouped = false;
      if constexpr (sizeof(T) == 2) {
        if (launch_log() != nullptr) {
          // the layer-batched launch has blocks to spare: du's slices 0, 1, 3 in 128 x 128 tiles
          // (half the LDS traffic per product; every element's k order is the same, so the results
          // are too)
          grouped = true;
          using PDu = GemmPart<T, 128, 128, 2, 2, -3, SrcRows<T>, SrcRows<T>, EpiStoreTileF32>;
          using PVin = GemmPart<T, 64, 32, 4, 1, -SW2_STAGES, SrcRows<T>, SrcRows<T>, EpiVinBwd<T, 32>>;
          const EpiVinBwd<T, 32> ev{g, N, c->ctx_mod, c->mult_res_lambda, sv.save1 + sw * NS * 4 * d,
                                    (const T*)L->sig, dctx + sw * NS * 4 * d, ws.dsig, ws.lamdv};
          // dv_in and du's slices 0, 1, 3 as launches of their own (in one launch every dv_in block
          // would hold the du blocks' LDS), then slice 2 as on the layer path
          const PDu pdu{da, db, d, ep, d / 128, cdiv(N, 128), DU_SPLIT - 1, 2};
          const PVin pvin{av, bv, d, ev, d / 32, cdiv(N, 64), 1, -1};
          record_launch<GemmPartBody<PVin>>(dim3(pvin.gx * pvin.gy * pvin.nz), dim3(256), {pvin});
          record_launch<GemmPartBody<PDu>>(dim3(pdu.gx * pdu.gy * pdu.nz), dim3(256), {pdu});
          launch_gemm<T, DUF_BM, 64, 2, 2, -DUF_STAGES>(da2, db2, N, d, d, efp, s);
        }
      }
      if (!grouped) {
        constexpr int DD = sizeof(T) == 2 ? -DU_STAGES : 4;
        using PDu = GemmPart<T, 64, 64, 2, 2, DD, SrcRows<T>, SrcRows<T>, EpiStoreTileF32>;
        using PVin = GemmPart<T, 64, DV_BN, 2, 2, DD, SrcRows<T>, SrcRows<T>, EpiVinBwd<T, DV_BN>>;
        const EpiVinBwd<T, DV_BN> ev{g, N, c->ctx_mod, c->mult_res_lambda, sv.save1 + sw * NS * 4 * d,
                                     (const T*)L->sig, dctx + sw * NS * 4 * d, ws.dsig, ws.lamdv};
        launch_gemm_pair(PDu{da, db, d, ep, d / 64, cdiv(N, 64), DU_SPLIT - 1, 2},
                         PVin{av, bv, d, ev, d / DV_BN, cdiv(N, 64), 1, -1}, s);
        launch_gemm<T, DUF_BM, 64, 2, 2, sizeof(T) == 2 ? -DUF_STAGES : 4>(da2, db2, N, d, d, efp, s);
      }
    } else {
      if (sizeof(T) == 2 && launch_log() != nullptr)
        launch_gemm_splitk<T, 128, 128, 2, 2, sizeof(T) == 2 ? -3 : 4>(da, db, N, d, 4 * d, DU_SPLIT, ep, s);
      else
        launch_gemm_splitk<T, 64, 64, 2, 2, sizeof(T) == 2 ? -DU_STAGES : 4>(da, db, N, d, 4 * d, DU_SPLIT, ep, s);
      const dim3 egrid(cdiv(N, 16), d / DU_EPI_TN);
      if (launch_log() != nullptr)
        record_launch<DuEpiBody<T, DU_SPLIT>>(egrid, dim3(256), ea);
      else
        hipLaunchKernelGGL((k_du_epi<T, DU_SPLIT>), egrid, dim3(256), 0, s, ea.M, ea.d, ea.h, ea.inv_d, ea.eps, ea.part,
                           ea.lamdv, ea.o, ea.ssq, ea.normw, ea.gw, ea.rowdot, ea.dnw);
    }
    // attention VJP of sweep sw
    {
      const T* Kin; const T* Vin; long in_stride; int in_row0;
      if (sw == 0) { Kin = kself; Vin = vraw; in_stride = (long)T_ * DH; in_row0 = pos0; }
      else { Kin = sv.Kin + sw * slot; Vin = sv.Vin + sw * slot; in_stride = (long)CMAX * DH; in_row0 = 0; }
      AttnBwdArgs<T> aa{g, qr, kself, vraw, Kin, Vin, in_stride, in_row0, sv.o + sw * NS * d,
                        sv.ssq + sw * NS * h, ws.gw, ws.rowdot, d / DU_EPI_TN,
                        sw == K - 1 ? ws.docat : nullptr, sv.stat_m + sw * (size_t)BH * CMAX,
                        sv.stat_z + sw * (size_t)BH * CMAX, Mx, ws.Grow, ws.Drow, ws.Mrow, ws.klim,
                        ws.cellrow, K, (int)coff, sw == K - 1 ? 1 : 0,
                        scale, inv_d, c->rms_eps, ws.dkself, ws.dvraw, ws.dq, ws.sdss, sw >= 1 ? 1 : 0,
                        sw >= 1 ? refine_args(sw - 1) : RefineBwdArgs<T>{}};
      aa.Gb = sw == 0 ? ws.Gb : nullptr;
      // this launch's share of the cell before's hosted splits (launch j = K - 1 - sw of K)
      const int j = K - 1 - sw, h0 = 1 + host_splits * j / K, h1 = 1 + host_splits * (j + 1) / K;
      if (launch_log() != nullptr) {
        record_launch<AttnBwdBody<T, DH>>(dim3(ATTN_BWD_ROLES, BH), dim3(256), aa, (unsigned)lds_attn_bwd);
      } else if (h1 > h0) {
        kprev.s0 = h0;
        hipLaunchKernelGGL((k_attn_bwd_dkv<T, DH>), dim3((ATTN_BWD_ROLES + h1 - h0) * BH), dim3(256), lds_attn_bwd, s,
                           aa, kprev, BH);
      } else {
        hipLaunchKernelGGL((k_attn_bwd<T, DH>), dim3(ATTN_BWD_ROLES, BH), dim3(256), lds_attn_bwd, s, aa);
      }
    }
  }
  // the other operand of dW_sweep = dctx^T u: this cell's K*N rows of u = RMSNorm(o)
  // (dW_vctx = dv_ctx^T v_in reads the stacked v_in as it is). On the layer path the tape's cells
  // are normalised after the cell loop, RMS_MAX_SEG cells per launch; a recomputed cell's o is
  // overwritten by the next cell, and a per-cell call has no later batch: those now.
  const int rows = K * N;
  if (tape != nullptr && rms != nullptr) {
    rms->push_back(RmsSeg{sv.o, sv.ssq, coff, rows});
  } else if (launch_log() != nullptr) {
    record_launch<RmsRowsUBody<T>>(dim3(cdiv(rows, 4)), dim3(256),
                                   typename RmsRowsUBody<T>::Args{(const T*)sv.o, rows, d, (const float*)sv.ssq, h,
                                                                  (const T*)w->norm_ctx_w, inv_d, c->rms_eps,
                                                                  ws.uL + coff * d});
  } else {
    hipLaunchKernelGGL(k_rms_rows<T>, dim3(cdiv(rows, 4)), dim3(256), 0, s, (const T*)sv.o, rows, d,
                       (const float*)sv.ssq, h, (const T*)w->norm_ctx_w, inv_d, c->rms_eps, ws.uL + coff * d);
  }
  // grad-cache path: the committed rows [0, pos0) this cell read get their grads now, key side
  // into the cache, query side into dq
  if (gc.dK != nullptr && pos0 > 0 && launch_log() != nullptr) launch_log()->unsupported = true;
  else if (gc.dK != nullptr && pos0 > 0) {
    CommKeyArgs<T> ka{B, h, T_, cache_T, pos0, 0, pos0, pos0 + cc, qr, Kc, Vc, ws.Gb, ws.Drow, ws.Mrow,
                      scale, nullptr, nullptr, gc.dK, gc.dV};
    ka.window = window_of(c);
    hipLaunchKernelGGL((k_comm_dkv<T, DH>), dim3(cdiv(pos0, 64), BH), dim3(256), lds_attn, s, ka);
    CommQueryArgs<T> qa{B, h, T_, cache_T, pos0 + cc, ws.klim, qr, Kc, Vc, ws.Gb, ws.Drow, ws.Mrow, scale, ws.dq,
                        pos0};
    qa.window = window_of(c);
    hipLaunchKernelGGL((k_comm_dq<T, DH>), dim3(BH, cdiv(cc, 64)), dim3(256), lds_attn, s, qa);
  }
  if (ho != nullptr) ho->far_done = host_splits > 0;
}

template <typename T, int DH>
void unpack_grads(const dm_config* c, const dm_grads* gr, const BwdWs<T>& ws, hipStream_t s);

template <typename T, int DH>
void bwd_end(const dm_config* c, const dm_packed* w, const T* x, const T* dy, T* dx, const float* cos,
             const float* sin, const dm_layer_bufs* L, const int32_t* sched, int n_cells, const T* Kc, const T* Vc,
             int cache_T, const char* tape, const size_t* tape_off, bool layer_path, const std::vector<RmsSeg>& rms,
             const dm_grads* gr, const BwdWs<T>& ws, hipStream_t s) {
  const int B = c->B, d = c->d, h = c->h, T_ = L->T, BT = B * T_, BH = B * h;
  const bool mult = c->ctx_mod != DM_CTX_LINEAR;
  const int nproj = mult ? 6 : 5;
  const bool norm = w->attn_norm_w != nullptr;
  const bool residual = !(c->flags & DM_FLAG_NO_RESIDUAL);
  const float scale = 1.0f / sqrtf((float)DH);
  const float inv_d = 1.0f / (float)d;
  const T* qr = (const T*)L->qr;
  const size_t lds_attn = AttnBwdCfg<T, DH>::LDS_ELEMS * sizeof(T);
  T* vinS = stacked_vin<T>(tape, tape_off, n_cells, ws);
  const int t_end = sched[3 * (n_cells - 1)] + sched[3 * (n_cells - 1) + 1];
  const long coff = vin_row(c, sched, n_cells, -1);   // every cell's rows
  for (size_t i0 = 0; i0 < rms.size(); i0 += RMS_MAX_SEG) {
    RmsSegs ra{};
    ra.nseg = (int)std::min<size_t>(RMS_MAX_SEG, rms.size() - i0);
    int most = 0;
    for (int i = 0; i < ra.nseg; ++i) {
      ra.seg[i] = rms[i0 + i];
      most = std::max(most, ra.seg[i].rows);
    }
    hipLaunchKernelGGL(k_rms_rows_multi<T>, dim3(cdiv(most, 4), ra.nseg), dim3(256), 0, s, ra, d, h,
                       (const T*)w->norm_ctx_w, inv_d, c->rms_eps, ws.uL);
  }
  {   // the layer's sweep weight grads, one GEMM each over all cells' stacked rows
    // (zero rows up to a whole k-tile)
    const int Kp = (int)(cdiv(coff, 64) * 64);
    if (Kp > coff) {
      // fp32 words of the padding rows: rows * cols * sizeof(T) bytes, a whole number of words
      // since d is a multiple of 128 (the byte count is formed before dividing: an odd row
      // count of bf16 rows would otherwise round a row away)
      auto words = [&](size_t cols) { return (size_t)(Kp - coff) * cols * sizeof(T) / 4; };
      fill0_list({{reinterpret_cast<float*>(ws.dctxL + coff * 4 * d), words(4 * (size_t)d)},
                  {reinterpret_cast<float*>(ws.uL + coff * d), words(d)},
                  {reinterpret_cast<float*>(ws.dvcL + coff * d), words(d)},
                  {reinterpret_cast<float*>(vinS + coff * d), mult ? words(d) : 0}},
                 s);
    }
    gemm_tn<T>(ws.dctxL, 4 * d, ws.uL, d, ws.dWs, 4 * d, d, Kp, 1, ws.kpart, s);
    if (mult) gemm_tn<T>(ws.dvcL, d, vinS, d, gr->w_vctx, d, d, Kp, 1, ws.kpart, s);
  }

  // committed-prefix VJP, query side (layer path): every row with a committed prefix, into dq
  if (layer_path) {
    CommQueryArgs<T> qa{B, h, T_, cache_T, t_end, ws.klim, qr, Kc, Vc, ws.Gb, ws.Drow, ws.Mrow, scale, ws.dq};
    qa.window = window_of(c);
    hipLaunchKernelGGL((k_comm_dq<T, DH>), dim3(BH, cdiv(t_end, 64)), dim3(256), lds_attn, s, qa);
  }
  // ---- projection VJP
  // (+ the bias grads' column partials: sums of the gate logits' grads (b_gk | b_gv) and of
  // dsig sig (1 - sig) (b_vgate) over each block's rows)
  const int pchunks = cdiv(BT, PROJ_ROWS);
  const bool fusion = c->ctx_mod == DM_CTX_FUSION;
  hipLaunchKernelGGL((k_proj_bwd<T, DH>), dim3(proj_grid_x(d), pchunks), dim3(256), 0, s, BT, T_, d, h, nproj,
                     fusion ? 1 : 0,
                     (const float*)ws.dq, (const float*)ws.dkraw, (const float*)ws.dkself, (const float*)ws.dvraw,
                     (const T*)ws.dctxL, (const CellRow*)ws.cellrow, B, (const float*)ws.dsig,
                     (const T*)L->sig, cos, sin, ws.dproj,
                     ws.colpart, (const T*)L->vpre, v_gain(c, w), ws.vgpart, (const float*)ws.sdss, qr,
                     (const T*)L->kself, scale, RowMap{}, PROJ_ROWS_OUT | PROJ_PARTIALS);
  hipLaunchKernelGGL(k_sum_rows_add, dim3(cdiv(3 * d, 64)), dim3(256), 0, s, pchunks * proj_rows_in_flight(d), 3 * d, 3 * d,
                     (const float*)ws.colpart, gr->b_gk, gr->b_gv, (mult && !fusion) ? gr->b_vgate : nullptr, d);
  // the head norms' gains: sums over rows of the partials
  if (ws.vgpart)
    hipLaunchKernelGGL(k_sum_rows_add, dim3(cdiv(h, 64)), dim3(256), 0, s, pchunks * proj_rows_in_flight(d), h, h,
                       (const float*)ws.vgpart,
                       gr->v_gain, (float*)nullptr, (float*)nullptr, h);
  if (ws.dkg) colsum_add(ws.dkg, BT, h, ws.colpart, gr->k_gain, s);
  if (ws.dvg) colsum_add(ws.dvg, BT, h, ws.colpart, gr->ctx_gain, s);
  const T* xhat = norm ? (const T*)L->xhat : x;
  // dW_proj = d_proj^T . xhat (packed rows), dxhat = d_proj . W_proj
  gemm_tn<T>(ws.dproj, (long)nproj * d, xhat, d, ws.dWp, nproj * d, d, BT, 0, ws.kpart, s);
  {
    EpiStoreTileF32 ep{BT, d, ws.dxhat, 0};
    launch_gemm_big<T>(SrcRows<T>{ws.dproj, (long)nproj * d, BT},
                                      SrcRows<T>{(const T*)w->w_proj_t, (long)nproj * d, d}, BT, d, nproj * d, ep, s);
  }
  unpack_grads<T, DH>(c, gr, ws, s);
  // norm_ctx.weight
  colsum_add(ws.dnw, cdiv(B * CMAX, NSLOT_TM), d, ws.colpart, gr->norm_ctx_w, s);
  // attn_norm VJP + residual
  if (norm) {
    float* dwa_part = reinterpret_cast<float*>(ws.dproj);
    hipLaunchKernelGGL(k_rmsnorm_bwd<T>, dim3(cdiv(BT, RMSN_ROWS)), dim3(256), 4 * d * sizeof(float), s, BT, d,
                       c->rms_eps, residual ? 1 : 0, x, (const T*)w->attn_norm_w, (const float*)ws.dxhat, dy, dx,
                       dwa_part, RowMap{}, 3);
    colsum_add(dwa_part, cdiv(BT, RMSN_ROWS), d, ws.colpart, gr->attn_norm_w, s);
  } else {
    hipLaunchKernelGGL(k_dx_plain<T>, dim3(std::min(cdiv((long)BT * d, 256), 4096)), dim3(256), 0, s,
                       (long)BT * d, residual ? 1 : 0, (const float*)ws.dxhat, dy, dx);
  }
}

// the packed weight grads (dWp, dWs) added into the reference layout
template <typename T, int DH>
void unpack_grads(const dm_config* c, const dm_grads* gr, const BwdWs<T>& ws, hipStream_t s) {
  const int d = c->d, h = c->h;
  const bool mult = c->ctx_mod != DM_CTX_LINEAR;
  const bool fusion = c->ctx_mod == DM_CTX_FUSION;
  {
    std::vector<UnpackSeg> u;
    u.push_back(UnpackSeg{gr->wq, d, 0, d, 0, 0});
    u.push_back(UnpackSeg{gr->wk, d, 0, d, d, 0});
    u.push_back(UnpackSeg{gr->wv, d, 0, d, 2 * d, 0});
    u.push_back(UnpackSeg{gr->w_gk, 2 * d, 0, d, 3 * d, 0});
    u.push_back(UnpackSeg{gr->w_gv, 2 * d, 0, d, 4 * d, 0});
    if (fusion) u.push_back(UnpackSeg{gr->v_pre, 2 * d, 0, d, 5 * d, 0});   // x-half of v_pre
    else if (mult) u.push_back(UnpackSeg{gr->v_gate, d, 0, d, 5 * d, 0});
    unpack(u, d, ws.dWp, s);
    u.clear();
    for (int hd = 0; hd < h; ++hd)
      for (int q = 0; q < DH / 32; ++q) {
        const int base = 2 * DH * hd + 64 * q, r0 = hd * DH + 16 * q, r1 = r0 + DH / 2;
        u.push_back(UnpackSeg{gr->w_kctx + (size_t)r0 * d, d, 0, 16, base, 0});
        u.push_back(UnpackSeg{gr->w_kctx + (size_t)r1 * d, d, 0, 16, base + 16, 0});
        u.push_back(UnpackSeg{gr->w_gk + (size_t)r0 * 2 * d, 2 * d, d, 16, base + 32, 0});
        u.push_back(UnpackSeg{gr->w_gk + (size_t)r1 * 2 * d, 2 * d, d, 16, base + 48, 0});
      }
    if (mult) {
      if (fusion) u.push_back(UnpackSeg{gr->v_pre, 2 * d, d, d, 2 * d, 0});   // u-half of v_pre
      else u.push_back(UnpackSeg{gr->v_map, d, 0, d, 2 * d, 0});
      u.push_back(UnpackSeg{gr->w_gv, 2 * d, d, d, 3 * d, 0});
    } else {
      for (int hd = 0; hd < h; ++hd)
        for (int q = 0; q < DH / 32; ++q) {
          const int base = 2 * d + 2 * DH * hd + 64 * q, r0 = hd * DH + 32 * q;
          u.push_back(UnpackSeg{gr->w_vctx + (size_t)r0 * d, d, 0, 32, base, 0});
          u.push_back(UnpackSeg{gr->w_gv + (size_t)r0 * 2 * d, 2 * d, d, 32, base + 32, 0});
        }
    }
    unpack(u, d, ws.dWs, s);
  }
}

// ---- the layer-batched (wavefront) backward of a stack ---------------------------------------
// Per layer and cell the same kernels as bwd_begin / bwd_cell / bwd_end, restricted to the cell's
// rows: the cell's do_cat rows, its sweeps, then the tail that makes its dx rows final (the
// committed-prefix query VJP of its rows, the projection VJP rows, dxhat, the attn_norm VJP with
// the residual). A layer's sums over all rows (weight grads, bias / gain / norm-weight partials)
// run once its last cell (cell 0) is done.

constexpr int PROJ_ROWS_CHUNK = 8;   // rows per block of a cell's projection VJP rows (no partials)

template <typename T, int DH>
void record_bwd_chunk(const dm_config* c, const dm_stack_bwd_layer& ly, const float* cos, const float* sin,
                      const int32_t* sched, int n_cells, int ci, int cache_T, const size_t* toff, const BwdWs<T>& ws,
                      std::vector<RmsSeg>* rms) {
  const dm_packed* w = ly.w;
  const dm_layer_bufs* L = ly.bufs;
  const int B = c->B, d = c->d, h = c->h, T_ = L->T, BH = B * h;
  const int pos0 = sched[3 * ci], cc = sched[3 * ci + 1];
  const int N = B * cc, lc = log2_exact(cc);
  const RowMap map{lc, T_, pos0};
  const int nproj = c->ctx_mod == DM_CTX_LINEAR ? 5 : 6;
  const T* dy = (const T*)ly.dy;
  const T* Kc = (const T*)ly.K_cache;
  const T* Vc = (const T*)ly.V_cache;
  // the block tail: the cell's rows of the MLP VJP, dz -> dy (the attention sublayer's output grad)
  if (ly.mlp_w != nullptr)
    mlp_bwd_rows<T>(ly.mlp_w, (const T*)ly.mlp_y, (const T*)ly.dz, (T*)ly.dy, ly.mlp_bufs, N, d, ly.mlp_H,
                    c->rms_eps, lc, T_, pos0, 1, nullptr, nullptr);
  // do_cat rows of the cell: dy . W_O
  {
    EpiStoreTileF32 ep{N, d, ws.docat, 0, map};
    launch_gemm_auto<T, 64, 64, 2, 2, 3, 4>(SrcChunkRows<T>{dy, d, N, lc, T_, pos0},
                                            SrcRows<T>{(const T*)w->wo_t, d, d}, N, d, d, ep, nullptr);
  }
  bwd_cell<T, DH>(c, w, cos, sin, L, sched, n_cells, ci, Kc, Vc, cache_T, (const char*)ly.tape, toff, GradCache{}, ws,
                  rms, nullptr);
  // committed-prefix VJP, query side, of the cell's rows
  const size_t lds_attn = AttnBwdCfg<T, DH>::LDS_ELEMS * sizeof(T);
  const float scale = 1.0f / sqrtf((float)DH);
  CommQueryArgs<T> qa{B, h, T_, cache_T, pos0 + cc, ws.klim, (const T*)L->qr, Kc, Vc, ws.Gb, ws.Drow, ws.Mrow,
                      scale, ws.dq, pos0};
  qa.window = window_of(c);
  record_launch<CommDqBody<T, DH>>(dim3(BH, cdiv(cc, 64)), dim3(256), qa, (unsigned)lds_attn);
  // projection VJP of the cell's rows (the column partials come with the layer's close)
  typename ProjBwdBody<T, DH>::Args pa{N, T_, d, h, nproj, c->ctx_mod == DM_CTX_FUSION ? 1 : 0, ws.dq, ws.dkraw,
                                       ws.dkself, ws.dvraw, ws.dctxL, ws.cellrow, B, ws.dsig, (const T*)L->sig, cos, sin,
                                       ws.dproj,
                                       ws.colpart, (const T*)L->vpre, v_gain(c, w), ws.vgpart, ws.sdss,
                                       (const T*)L->qr, (const T*)L->kself, scale, map, PROJ_ROWS_OUT,
                                       PROJ_ROWS_CHUNK};
  record_launch<ProjBwdBody<T, DH>>(dim3(proj_grid_x(d), cdiv(N, PROJ_ROWS_CHUNK)), dim3(256), pa);
  // dxhat rows = d_proj rows . W_proj
  {
    EpiStoreTileF32 ex{N, d, ws.dxhat, 0, map};
    launch_gemm_auto<T, 64, 64, 2, 2, 3, 4>(SrcChunkRows<T>{ws.dproj, (long)nproj * d, N, lc, T_, pos0},
                                            SrcRows<T>{(const T*)w->w_proj_t, (long)nproj * d, d}, N, d, nproj * d,
                                            ex, nullptr);
  }
  // attn_norm VJP + residual: the cell's dx rows (the norm weight's partials with the close)
  typename RmsnormBwdBody<T>::Args ra{N, d, c->rms_eps, (c->flags & DM_FLAG_NO_RESIDUAL) ? 0 : 1, (const T*)ly.x,
                                      (const T*)w->attn_norm_w, ws.dxhat, dy, (T*)ly.dx, nullptr, map, 1};
  record_launch<RmsnormBwdBody<T>>(dim3(cdiv(N, RMSN_ROWS)), dim3(256), ra, (unsigned)(4 * d * sizeof(float)));
}

// The layer's close once every cell is done (direct launches): the sweep weight grads, dW_O, the
// column sums of the bias / gain / norm-weight partials, dW_proj, the unpack into the reference
// layout — bwd_begin's and bwd_end's all-row work, in bwd_end's order.
template <typename T, int DH>
void bwd_stack_close(const dm_config* c, const dm_stack_bwd_layer& ly, const float* cos, const float* sin,
                     const int32_t* sched, int n_cells, const size_t* toff, const std::vector<RmsSeg>& rms,
                     const BwdWs<T>& ws, hipStream_t s) {
  const dm_packed* w = ly.w;
  const dm_layer_bufs* L = ly.bufs;
  const dm_grads* gr = ly.grads;
  const int B = c->B, d = c->d, h = c->h, T_ = L->T, BT = B * T_;
  const bool mult = c->ctx_mod != DM_CTX_LINEAR;
  const int nproj = mult ? 6 : 5;
  const float inv_d = 1.0f / (float)d;
  T* vinS = stacked_vin<T>((const char*)ly.tape, toff, n_cells, ws);
  const long coff = vin_row(c, sched, n_cells, -1);
  gemm_tn<T>((const T*)ly.dy, d, (const T*)ly.ocat, d, gr->wo, d, d, BT, 1, ws.kpart, s);
  for (size_t i0 = 0; i0 < rms.size(); i0 += RMS_MAX_SEG) {
    RmsSegs ra{};
    ra.nseg = (int)std::min<size_t>(RMS_MAX_SEG, rms.size() - i0);
    int most = 0;
    for (int i = 0; i < ra.nseg; ++i) {
      ra.seg[i] = rms[i0 + i];
      most = std::max(most, ra.seg[i].rows);
    }
    hipLaunchKernelGGL(k_rms_rows_multi<T>, dim3(cdiv(most, 4), ra.nseg), dim3(256), 0, s, ra, d, h,
                       (const T*)w->norm_ctx_w, inv_d, c->rms_eps, ws.uL);
  }
  {
    const int Kp = (int)(cdiv(coff, 64) * 64);
    if (Kp > coff) {
      auto words = [&](size_t cols) { return (size_t)(Kp - coff) * cols * sizeof(T) / 4; };
      fill0_list({{reinterpret_cast<float*>(ws.dctxL + coff * 4 * d), words(4 * (size_t)d)},
                  {reinterpret_cast<float*>(ws.uL + coff * d), words(d)},
                  {reinterpret_cast<float*>(ws.dvcL + coff * d), words(d)},
                  {reinterpret_cast<float*>(vinS + coff * d), mult ? words(d) : 0}},
                 s);
    }
    gemm_tn<T>(ws.dctxL, 4 * d, ws.uL, d, ws.dWs, 4 * d, d, Kp, 1, ws.kpart, s);
    if (mult) gemm_tn<T>(ws.dvcL, d, vinS, d, gr->w_vctx, d, d, Kp, 1, ws.kpart, s);
  }
  const int pchunks = cdiv(BT, PROJ_ROWS);
  const bool fusion = c->ctx_mod == DM_CTX_FUSION;
  hipLaunchKernelGGL((k_proj_bwd<T, DH>), dim3(proj_grid_x(d), pchunks), dim3(256), 0, s, BT, T_, d, h, nproj,
                     fusion ? 1 : 0, (const float*)ws.dq, (const float*)ws.dkraw, (const float*)ws.dkself,
                     (const float*)ws.dvraw, (const T*)ws.dctxL, (const CellRow*)ws.cellrow, c->B,
                     (const float*)ws.dsig, (const T*)L->sig, cos,
                     sin, ws.dproj, ws.colpart, (const T*)L->vpre, v_gain(c, w), ws.vgpart, (const float*)ws.sdss,
                     (const T*)L->qr, (const T*)L->kself, 1.0f / sqrtf((float)DH), RowMap{}, PROJ_PARTIALS);
  hipLaunchKernelGGL(k_sum_rows_add, dim3(cdiv(3 * d, 64)), dim3(256), 0, s, pchunks * proj_rows_in_flight(d), 3 * d, 3 * d,
                     (const float*)ws.colpart, gr->b_gk, gr->b_gv, (mult && !fusion) ? gr->b_vgate : nullptr, d);
  if (ws.vgpart)
    hipLaunchKernelGGL(k_sum_rows_add, dim3(cdiv(h, 64)), dim3(256), 0, s, pchunks * proj_rows_in_flight(d), h, h,
                       (const float*)ws.vgpart,
                       gr->v_gain, (float*)nullptr, (float*)nullptr, h);
  if (ws.dkg) colsum_add(ws.dkg, BT, h, ws.colpart, gr->k_gain, s);
  if (ws.dvg) colsum_add(ws.dvg, BT, h, ws.colpart, gr->ctx_gain, s);
  gemm_tn<T>(ws.dproj, (long)nproj * d, (const T*)L->xhat, d, ws.dWp, nproj * d, d, BT, 0, ws.kpart, s);
  unpack_grads<T, DH>(c, gr, ws, s);
  colsum_add(ws.dnw, cdiv(B * CMAX, NSLOT_TM), d, ws.colpart, gr->norm_ctx_w, s);
  float* dwa_part = reinterpret_cast<float*>(ws.dproj);
  hipLaunchKernelGGL(k_rmsnorm_bwd<T>, dim3(cdiv(BT, RMSN_ROWS)), dim3(256), 4 * d * sizeof(float), s, BT, d,
                     c->rms_eps, 0, (const T*)ly.x, (const T*)w->attn_norm_w, (const float*)ws.dxhat, (const T*)nullptr,
                     (T*)nullptr, dwa_part, RowMap{}, 2);
  colsum_add(dwa_part, cdiv(BT, RMSN_ROWS), d, ws.colpart, gr->attn_norm_w, s);
  if (ly.mlp_w != nullptr) {
    // the block tail's sums over all rows: the mlp_norm weight partials, then the weight grads
    const MlpWs mw = carve_mlp(BT, d, ly.mlp_H, ly.mlp_workspace);
    hipLaunchKernelGGL(k_rmsnorm_bwd<T>, dim3(cdiv(BT, RMSN_ROWS)), dim3(256), 4 * d * sizeof(float), s, BT, d,
                       c->rms_eps, 0, (const T*)ly.mlp_y, (const T*)ly.mlp_w->norm_w,
                       (const float*)ly.mlp_bufs->dh, (const T*)nullptr, (T*)nullptr, mw.dwa_part, RowMap{}, 2);
    mlp_wgrad<T>(ly.mlp_bufs, (const T*)ly.dz, BT, d, ly.mlp_H, ly.mlp_grads, mw, s);
  }
}

// which part of the layer backward an entry point runs
enum BwdPart { BWD_LAYER = 0, BWD_BEGIN = 1, BWD_CELL = 2, BWD_END = 3 };
struct BwdCall {
  int part;
  const void* x; const void* dy; void* dx; const void* ocat;
  const float* cos; const float* sin; const dm_layer_bufs* L;
  const int32_t* sched; int n_cells; int cell;
  const void* Kc; const void* Vc; int cache_T;
  const void* tape; size_t tape_bytes;
  GradCache gc;
  const dm_grads* g;
  void* workspace; int kmax;
};

template <typename T>
int bwd_dispatch(const dm_config* c, const dm_packed* w, const BwdCall& a, hipStream_t s) {
  std::vector<size_t> off;
  if (a.tape != nullptr) {
    off = tape_offsets<T>(c, a.sched, a.n_cells);
    DM_REQUIRE(a.tape_bytes >= off[a.n_cells + 1], DM_ERR_WORKSPACE, "tape %zu < %zu bytes", a.tape_bytes,
               off[a.n_cells + 1]);
    DM_REQUIRE(aligned16(a.tape), DM_ERR_INVALID, "tape must be 16-byte aligned");
  }
  const BwdWs<T> ws = carve_bwd<T>(c, a.L->T, a.cache_T, a.kmax, a.workspace);
  const char* tape = (const char*)a.tape;
  const size_t* to = a.tape ? off.data() : nullptr;
  const T* Kc = (const T*)a.Kc;
  const T* Vc = (const T*)a.Vc;
  auto run = [&](auto dh_tag) {
    constexpr int DH = decltype(dh_tag)::value;
    std::vector<RmsSeg> rms;
    if (a.part == BWD_LAYER) {
      ProfScope whole(PROF_BWD, s);
      bwd_begin<T, DH>(c, w, (const T*)a.dy, (const T*)a.ocat, a.L->T, a.g, ws, s);
      CellHandoff ho;   // work each cell's launches do for the cell before it
      for (int ci = a.n_cells - 1; ci >= 0; --ci)
        bwd_cell<T, DH>(c, w, a.cos, a.sin, a.L, a.sched, a.n_cells, ci, Kc, Vc, a.cache_T, tape, to, GradCache{}, ws,
                        &rms, s, &ho);
      bwd_end<T, DH>(c, w, (const T*)a.x, (const T*)a.dy, (T*)a.dx, a.cos, a.sin, a.L, a.sched, a.n_cells, Kc, Vc,
                     a.cache_T, tape, to, true, rms, a.g, ws, s);
    } else if (a.part == BWD_BEGIN) {
      bwd_begin<T, DH>(c, w, (const T*)a.dy, (const T*)a.ocat, a.L->T, a.g, ws, s);
    } else if (a.part == BWD_CELL) {
      bwd_cell<T, DH>(c, w, a.cos, a.sin, a.L, a.sched, a.n_cells, a.cell, Kc, Vc, a.cache_T, tape, to, a.gc, ws,
                      nullptr, s);
    } else {
      bwd_end<T, DH>(c, w, (const T*)a.x, (const T*)a.dy, (T*)a.dx, a.cos, a.sin, a.L, a.sched, a.n_cells, Kc, Vc,
                     a.cache_T, tape, to, false, rms, a.g, ws, s);
    }
    return DM_OK;
  };
  return c->dh == 64 ? run(std::integral_constant<int, 64>{}) : run(std::integral_constant<int, 128>{});
}

}  // namespace dm

using namespace dm;

extern "C" {

size_t dm_layer_bwd_workspace_bytes(const dm_config* c, int32_t T, int32_t cache_T, int32_t max_sweeps) {
  if (check_cfg(c) != DM_OK || T <= 0 || cache_T < T || max_sweeps <= 0) return 0;
  return c->dtype == DM_BF16 ? carve_bwd<bf16>(c, T, cache_T, max_sweeps, nullptr).bytes
                             : carve_bwd<float>(c, T, cache_T, max_sweeps, nullptr).bytes;
}

}  // extern "C"

namespace dm {
// Checks shared by the backward entry points; kmax = the most sweeps of any cell (the workspace
// layout depends on it, so every part of one layer's backward is given the same schedule).
int check_bwd_common(const dm_config* c, const dm_packed* w, const dm_layer_bufs* L, const int32_t* sched,
                     int n_cells, int cache_T, void* workspace, size_t workspace_bytes, int* kmax) {
  int rc = check_cfg(c);
  if (rc) return rc;
  if ((rc = check_packed(c, w)) || (rc = check_bufs(c, L))) return rc;
  const bool mult = c->ctx_mod != DM_CTX_LINEAR;
  DM_REQUIRE(w->w_proj_t && w->w_sweep_t && w->wo_t && (!mult || w->w_vctx_t), DM_ERR_INVALID,
             "the backward needs the transposed packed weights");
  if ((rc = dm_check_schedule(sched, n_cells, L->T))) return rc;
  DM_REQUIRE(L->T <= cache_T, DM_ERR_INVALID, "T=%d > cache_T=%d", L->T, cache_T);
  {   // the attention VJP keeps Q, K, V and dO of a 64-row block in LDS
    const size_t lds = c->dtype == DM_BF16
                           ? (c->dh == 64 ? AttnBwdCfg<bf16, 64>::LDS_ELEMS : AttnBwdCfg<bf16, 128>::LDS_ELEMS) * 2
                           : (c->dh == 64 ? AttnBwdCfg<float, 64>::LDS_ELEMS : AttnBwdCfg<float, 128>::LDS_ELEMS) * 4;
    int dev = 0, lim = 0;
    DM_HIP(hipGetDevice(&dev));
    DM_HIP(hipDeviceGetAttribute(&lim, hipDeviceAttributeMaxSharedMemoryPerBlock, dev));
    DM_REQUIRE(lds + 1024 <= (size_t)lim, DM_ERR_UNSUPPORTED,
               "backward attention block needs %zu bytes of LDS, device allows %d (fp32 head_dim 128)", lds, lim);
  }
  int km = 0;
  for (int i = 0; i < n_cells; ++i) km = std::max(km, (int)sched[3 * i + 2]);
  const size_t need = dm_layer_bwd_workspace_bytes(c, L->T, cache_T, km);
  DM_REQUIRE(workspace && workspace_bytes >= need, DM_ERR_WORKSPACE, "workspace %zu < %zu bytes", workspace_bytes,
             need);
  *kmax = km;
  return DM_OK;
}

int check_grads(const dm_config* c, const dm_packed* w, const dm_layer_bufs* L, const dm_grads* g) {
  const bool mult = c->ctx_mod != DM_CTX_LINEAR;
  DM_REQUIRE(g != nullptr, DM_ERR_INVALID, "null gradient buffers");
  DM_REQUIRE(g->wq && g->wk && g->wv && g->wo && g->w_kctx && g->w_vctx && g->w_gk && g->w_gv && g->b_gk &&
                 g->b_gv && g->norm_ctx_w,
             DM_ERR_INVALID, "null gradient buffer");
  DM_REQUIRE(!mult || c->ctx_mod == DM_CTX_FUSION || (g->v_gate && g->b_vgate && g->v_map), DM_ERR_INVALID,
             "mult family needs v_gate/v_map grads");
  DM_REQUIRE(c->ctx_mod != DM_CTX_FUSION || g->v_pre, DM_ERR_INVALID, "ctx_mod fusion needs the v_pre grad");
  DM_REQUIRE(w->attn_norm_w == nullptr || (g->attn_norm_w && L->xhat), DM_ERR_INVALID,
             "attn_norm needs its gradient buffer and bufs->xhat");
  DM_REQUIRE(!(c->norms & DM_NORM_K_CTX) || g->k_gain, DM_ERR_INVALID, "k_ctx norm needs the k_gain grad");
  DM_REQUIRE(!(c->norms & DM_NORM_V_CTX) || g->ctx_gain, DM_ERR_INVALID, "v_ctx norm needs the ctx_gain grad");
  DM_REQUIRE(!(c->norms & DM_NORM_V) || (g->v_gain && L->vpre), DM_ERR_INVALID,
             "v_norm needs the v_gain grad and bufs->vpre");
  return DM_OK;
}

int run_bwd(const dm_config* c, const dm_packed* w, const BwdCall& call, void* stream) {
  hipStream_t s = S(stream);
  const int rc = c->dtype == DM_BF16 ? bwd_dispatch<bf16>(c, w, call, s) : bwd_dispatch<float>(c, w, call, s);
  if (rc) return rc;
  DM_HIP(hipGetLastError());
  return DM_OK;
}
// The layer-batched backward: checks, then (bytes != nullptr) the plan size, or the run: the
// accumulators of every layer zeroed, then per step the grouped launches of every active layer's
// cell and the close of each layer whose cell 0 that step finished.
int run_stack_bwd(const dm_config* c, int nl, const dm_stack_bwd_layer* layers, const float* cos, const float* sin,
                  const int32_t* sched, int n_cells, int cache_T, void* plan, size_t plan_bytes, int build,
                  void* stream, size_t* bytes) {
  DM_REQUIRE(nl >= 1 && layers != nullptr, DM_ERR_INVALID, "n_layers=%d", nl);
  int kmax = 0;
  for (int l = 0; l < nl; ++l) {
    const dm_stack_bwd_layer& ly = layers[l];
    int rc = check_bwd_common(c, ly.w, ly.bufs, sched, n_cells, cache_T, ly.workspace, ly.workspace_bytes, &kmax);
    if (rc) return rc;
    if ((rc = check_grads(c, ly.w, ly.bufs, ly.grads))) return rc;
    DM_REQUIRE(ly.x && ly.dy && ly.dx && ly.K_cache && ly.V_cache && ly.ocat, DM_ERR_INVALID,
               "layer %d: null backward argument", l);
    DM_REQUIRE(ly.w->attn_norm_w != nullptr, DM_ERR_UNSUPPORTED, "the layer-batched backward needs attn_norm");
    DM_REQUIRE(ly.bufs->T == layers[0].bufs->T, DM_ERR_INVALID, "layer %d: T differs", l);
    DM_REQUIRE((ly.tape != nullptr) == (layers[0].tape != nullptr), DM_ERR_INVALID,
               "layer %d: all layers with a tape or none", l);
    if (ly.mlp_w != nullptr) {
      if ((rc = check_mlp(c->dtype, ly.mlp_w, ly.mlp_bufs, c->B * ly.bufs->T, c->d, ly.mlp_H)) ||
          (rc = check_mlp_bwd(ly.mlp_bufs, ly.mlp_grads)))
        return rc;
      DM_REQUIRE(ly.dz && ly.mlp_y && ly.dz != ly.dy, DM_ERR_INVALID, "layer %d: the block tail needs dz, mlp_y "
                 "and a dy buffer of its own", l);
      DM_REQUIRE(ly.mlp_workspace && aligned16(ly.mlp_workspace) &&
                     ly.mlp_workspace_bytes >= carve_mlp(c->B * ly.bufs->T, c->d, ly.mlp_H, nullptr).bytes,
                 DM_ERR_WORKSPACE, "layer %d: MLP workspace %zu bytes too small", l, ly.mlp_workspace_bytes);
    }
  }
  for (int i = 0; i < n_cells; ++i)
    DM_REQUIRE(sched[3 * i + 1] == sched[1] && sched[3 * i + 2] == sched[2], DM_ERR_UNSUPPORTED,
               "the layer-batched backward needs equal cells");
  DM_REQUIRE(log2_exact(sched[1]) >= 0, DM_ERR_UNSUPPORTED, "cell length %d is not a power of two", sched[1]);
  hipStream_t s = S(stream);
  auto run = [&](auto tt, auto dh_tag) -> int {
    using T = decltype(tt);
    constexpr int DH = decltype(dh_tag)::value;
    std::vector<size_t> toff;
    const bool tape = layers[0].tape != nullptr;
    if (tape) {
      toff = tape_offsets<T>(c, sched, n_cells);
      for (int l = 0; l < nl; ++l)
        DM_REQUIRE(layers[l].tape_bytes >= toff[n_cells + 1] && aligned16(layers[l].tape), DM_ERR_WORKSPACE,
                   "layer %d: tape %zu < %zu bytes", l, layers[l].tape_bytes, toff[n_cells + 1]);
    }
    const size_t* to = tape ? toff.data() : nullptr;
    std::vector<BwdWs<T>> ws;
    for (int l = 0; l < nl; ++l) ws.push_back(carve_bwd<T>(c, layers[l].bufs->T, cache_T, kmax, layers[l].workspace));
    std::vector<std::vector<RmsSeg>> rms(nl);
    std::vector<GroupedLaunch> prog;
    std::vector<unsigned char> tab;
    size_t off = 0;
    std::vector<LaunchLog> logs;
    // layer l takes cell n_cells - 1 - (t - (nl - 1 - l)) at step t (the top layer first)
    for (int t = 0; t < n_cells + nl - 1; ++t) {
      const int la = std::max(0, nl - 1 - t), lb = std::min(nl - 1, nl - 1 - t + n_cells - 1);
      logs.assign(lb - la + 1, LaunchLog{});
      for (int l = lb; l >= la; --l) {
        const int ci = n_cells - 1 - (t - (nl - 1 - l));
        launch_log() = &logs[lb - l];
        record_bwd_chunk<T, DH>(c, layers[l], cos, sin, sched, n_cells, ci, cache_T, to, ws[l],
                                tape ? &rms[l] : nullptr);
        launch_log() = nullptr;
      }
      const int rc = merge_step(t, logs, prog, (build && bytes == nullptr) ? &tab : nullptr, off);
      if (rc) return rc;
      for (int l = lb; l >= la; --l)
        if (n_cells - 1 - (t - (nl - 1 - l)) == 0) prog.push_back(GroupedLaunch{nullptr, dim3(), dim3(), 0, 0, l});
    }
    if (bytes != nullptr) {
      *bytes = off;
      return DM_OK;
    }
    DM_REQUIRE(plan_bytes >= off, DM_ERR_WORKSPACE, "plan %zu < %zu bytes", plan_bytes, off);
    if (build) {
      const int wrc = write_plan(plan, tab.data(), off, S(stream));
      if (wrc) return wrc;
    }
    // every layer's accumulators (as bwd_begin)
    for (int l = 0; l < nl; ++l) {
      const BwdWs<T>& w = ws[l];
      const size_t BT = (size_t)c->B * layers[l].bufs->T, d = c->d;
      fill0_list({{w.dq, BT * d},
                  {w.sdss, BT * c->h},
                  {w.dkraw, BT * d},
                  {w.dkself, BT * d},
                  {w.dvraw, BT * d},
                  {reinterpret_cast<float*>(w.cellrow), (size_t)layers[l].bufs->T * sizeof(CellRow) / 4},
                  {w.dsig, BT * d},
                  {w.dnw, (size_t)cdiv(c->B * CMAX, NSLOT_TM) * d},
                  {w.dWs, 4 * d * d},
                  {w.dkg, w.dkg ? BT * c->h : 0},
                  {w.dvg, w.dvg ? BT * c->h : 0}},
                 s);
    }
    for (const GroupedLaunch& g : prog) {
      if (g.layer_end >= 0) {
        const int l = g.layer_end;
        bwd_stack_close<T, DH>(c, layers[l], cos, sin, sched, n_cells, to, rms[l], ws[l], s);
      } else {
        const int rc = issue_grouped(g, plan, s);
        if (rc) return rc;
      }
    }
    DM_HIP(hipGetLastError());
    return DM_OK;
  };
  if (c->dtype == DM_BF16)
    return c->dh == 64 ? run(bf16{}, std::integral_constant<int, 64>{}) : run(bf16{}, std::integral_constant<int, 128>{});
  return c->dh == 64 ? run(float{}, std::integral_constant<int, 64>{}) : run(float{}, std::integral_constant<int, 128>{});
}

}  // namespace dm

extern "C" {

int dm_layer_bwd(const dm_config* c, const dm_packed* w, const void* x, const void* dy, void* dx,
                 const float* cos, const float* sin, const dm_layer_bufs* L, const int32_t* sched,
                 int32_t n_cells, const void* K_cache, const void* V_cache, int32_t cache_T, const void* ocat,
                 const void* tape, size_t tape_bytes, const dm_grads* g, void* workspace, size_t workspace_bytes,
                 void* stream) {
  int kmax = 0;
  int rc = check_bwd_common(c, w, L, sched, n_cells, cache_T, workspace, workspace_bytes, &kmax);
  if (rc) return rc;
  DM_REQUIRE(x && dy && dx && cos && sin && K_cache && V_cache && ocat, DM_ERR_INVALID, "null backward argument");
  if ((rc = check_grads(c, w, L, g))) return rc;
  BwdCall call{BWD_LAYER, x, dy, dx, ocat, cos, sin, L, sched, n_cells, 0, K_cache, V_cache, cache_T, tape,
               tape_bytes, GradCache{}, g, workspace, kmax};
  return run_bwd(c, w, call, stream);
}

int dm_layer_bwd_begin(const dm_config* c, const dm_packed* w, const void* dy, const void* ocat,
                       const dm_layer_bufs* L, const int32_t* sched, int32_t n_cells, int32_t cache_T,
                       const dm_grads* g, void* workspace, size_t workspace_bytes, void* stream) {
  int kmax = 0;
  int rc = check_bwd_common(c, w, L, sched, n_cells, cache_T, workspace, workspace_bytes, &kmax);
  if (rc) return rc;
  DM_REQUIRE(dy && ocat, DM_ERR_INVALID, "null dy / ocat");
  if ((rc = check_grads(c, w, L, g))) return rc;
  BwdCall call{BWD_BEGIN, nullptr, dy, nullptr, ocat, nullptr, nullptr, L, sched, n_cells, 0, nullptr, nullptr,
               cache_T, nullptr, 0, GradCache{}, g, workspace, kmax};
  return run_bwd(c, w, call, stream);
}

int dm_cell_bwd(const dm_config* c, const dm_packed* w, const dm_layer_bufs* L, const float* cos, const float* sin,
                const dm_cell_bwd_args* a, void* stream) {
  DM_REQUIRE(a != nullptr, DM_ERR_INVALID, "null cell backward arguments");
  int kmax = 0;
  int rc = check_bwd_common(c, w, L, a->sched, a->n_cells, a->cache_T, a->workspace, a->workspace_bytes, &kmax);
  if (rc) return rc;
  DM_REQUIRE(a->cell >= 0 && a->cell < a->n_cells, DM_ERR_INVALID, "cell %d of %d", a->cell, a->n_cells);
  DM_REQUIRE(cos && sin && a->K_cache && a->V_cache && a->dK_gc && a->dV_gc, DM_ERR_INVALID,
             "null cell backward argument");
  DM_REQUIRE(aligned16(a->K_cache) && aligned16(a->V_cache) && aligned16(a->dK_gc) && aligned16(a->dV_gc),
             DM_ERR_INVALID, "caches must be 16-byte aligned");
  BwdCall call{BWD_CELL, nullptr, nullptr, nullptr, nullptr, cos, sin, L, a->sched, a->n_cells, a->cell, a->K_cache,
               a->V_cache, a->cache_T, a->tape, a->tape_bytes, GradCache{a->dK_gc, a->dV_gc}, nullptr,
               a->workspace, kmax};
  return run_bwd(c, w, call, stream);
}

size_t dm_stack_bwd_plan_bytes(const dm_config* c, int32_t n_layers, const dm_stack_bwd_layer* layers,
                               const int32_t* sched, int32_t n_cells, int32_t cache_T) {
  size_t bytes = 0;
  if (run_stack_bwd(c, n_layers, layers, nullptr, nullptr, sched, n_cells, cache_T, nullptr, 0, 0, nullptr, &bytes))
    return 0;
  return bytes;
}

int dm_stack_bwd(const dm_config* c, int32_t n_layers, const dm_stack_bwd_layer* layers, const float* cos,
                 const float* sin, const int32_t* sched, int32_t n_cells, int32_t cache_T, void* plan,
                 size_t plan_bytes, int32_t build, void* stream) {
  if (const int crc = check_cfg(c)) return crc;
  DM_REQUIRE(cos && sin, DM_ERR_INVALID, "null rope tables");
  DM_REQUIRE(plan != nullptr && (reinterpret_cast<uintptr_t>(plan) & 255) == 0, DM_ERR_INVALID,
             "plan must be non-null and 256-byte aligned");
  DM_REQUIRE(n_layers >= 1 && layers != nullptr && sched != nullptr && n_cells >= 1, DM_ERR_INVALID,
             "n_layers=%d n_cells=%d", n_layers, n_cells);
  ArgSig sig;
  sig.val(*c); sig.val(n_layers); sig.val(cos); sig.val(sin); sig.val(n_cells); sig.val(cache_T);
  sig.val(plan_bytes); sig.add(sched, sizeof(int32_t) * 3 * (size_t)n_cells);
  for (int l = 0; l < n_layers; ++l) {
    const dm_stack_bwd_layer& ly = layers[l];
    DM_REQUIRE(ly.w && ly.bufs && ly.grads, DM_ERR_INVALID, "layer %d: null weights, buffers or grads", l);
    sig.val(*ly.w); sig.bufs(ly.bufs); sig.val(*ly.grads);
    sig.val(ly.x); sig.val(ly.dy); sig.val(ly.dx); sig.val(ly.K_cache); sig.val(ly.V_cache); sig.val(ly.ocat);
    sig.val(ly.tape); sig.val(ly.tape_bytes); sig.val(ly.workspace); sig.val(ly.workspace_bytes);
    sig.val(ly.mlp_w); sig.val(ly.dz); sig.val(ly.mlp_y); sig.val(ly.mlp_H); sig.val(ly.mlp_workspace);
    sig.val(ly.mlp_workspace_bytes);
    if (ly.mlp_w != nullptr) { sig.val(*ly.mlp_w); sig.val(*ly.mlp_bufs); sig.val(*ly.mlp_grads); }
  }
  if (!build)
    DM_REQUIRE(plan_sig_matches(plan, sig.h), DM_ERR_INVALID,
               "plan %p was not written for these arguments (call once with build != 0)", plan);
  else
    plan_sig_forget(plan);
  const int rc = run_stack_bwd(c, n_layers, layers, cos, sin, sched, n_cells, cache_T, plan, plan_bytes, build,
                               stream, nullptr);
  if (rc == DM_OK && build) plan_sig_store(plan, sig.h);
  return rc;
}

int dm_layer_bwd_end(const dm_config* c, const dm_packed* w, const void* x, const void* dy, void* dx,
                     const float* cos, const float* sin, const dm_layer_bufs* L, const int32_t* sched,
                     int32_t n_cells, const void* K_cache, const void* V_cache, int32_t cache_T, const void* tape,
                     size_t tape_bytes, const dm_grads* g, void* workspace, size_t workspace_bytes, void* stream) {
  int kmax = 0;
  int rc = check_bwd_common(c, w, L, sched, n_cells, cache_T, workspace, workspace_bytes, &kmax);
  if (rc) return rc;
  DM_REQUIRE(x && dy && dx && cos && sin && K_cache && V_cache, DM_ERR_INVALID, "null backward argument");
  if ((rc = check_grads(c, w, L, g))) return rc;
  BwdCall call{BWD_END, x, dy, dx, nullptr, cos, sin, L, sched, n_cells, 0, K_cache, V_cache, cache_T, tape,
               tape_bytes, GradCache{}, g, workspace, kmax};
  return run_bwd(c, w, call, stream);
}


int dm_pack_mlp(int32_t dtype, const void* w1, const void* w3, const void* w2, const void* norm_w, int32_t d,
                int32_t H, const dm_mlp_packed* out, void* stream) {
  DM_REQUIRE(dtype == DM_F32 || dtype == DM_BF16, DM_ERR_INVALID, "dtype %d", dtype);
  DM_REQUIRE(d > 0 && H > 0 && d % 128 == 0 && H % 128 == 0, DM_ERR_INVALID, "MLP d=%d H=%d (multiples of 128)", d, H);
  DM_REQUIRE(w1 && w3 && w2 && norm_w && out, DM_ERR_INVALID, "null MLP weight");
  DM_REQUIRE(out->w13 && out->w2 && out->w13_t && out->w2_t && out->norm_w, DM_ERR_INVALID, "null packed MLP output");
  hipStream_t s = S(stream);
  const int e = (int)esz(dtype);
  // w13: W1 / W3 rows interleaved in groups of MLP_GROUP
  std::vector<PackSeg> segs;
  for (int g = 0; g < H / MLP_GROUP; ++g) {
    segs.push_back(PackSeg{(const char*)w1 + (size_t)g * MLP_GROUP * d * e, d, 0, MLP_GROUP, 2 * MLP_GROUP * g, 0});
    segs.push_back(PackSeg{(const char*)w3 + (size_t)g * MLP_GROUP * d * e, d, 0, MLP_GROUP,
                           2 * MLP_GROUP * g + MLP_GROUP, 0});
  }
  for (size_t i0 = 0; i0 < segs.size(); i0 += PACK_MAX_SEG) {
    PackArgs a{};
    a.nseg = (int)std::min<size_t>(PACK_MAX_SEG, segs.size() - i0);
    int rows = 0;
    for (int i = 0; i < a.nseg; ++i) { a.seg[i] = segs[i0 + i]; rows += a.seg[i].nrows; }
    a.ncols = d;
    a.esz = e;
    a.dst = out->w13;
    hipLaunchKernelGGL(k_pack, dim3(rows), dim3(256), 0, s, a);
  }
  DM_HIP(hipMemcpyAsync(out->w2, w2, (size_t)d * H * e, hipMemcpyDeviceToDevice, s));
  DM_HIP(hipMemcpyAsync(out->norm_w, norm_w, (size_t)d * e, hipMemcpyDeviceToDevice, s));
  auto tr = [&](const void* src, void* dst, int rows, int cols) {
    dim3 grid(cdiv(cols, 64), cdiv(rows, 64));
    if (dtype == DM_BF16)
      hipLaunchKernelGGL(k_transpose<bf16>, grid, dim3(256), 0, s, (const bf16*)src, (bf16*)dst, rows, cols);
    else
      hipLaunchKernelGGL(k_transpose<float>, grid, dim3(256), 0, s, (const float*)src, (float*)dst, rows, cols);
  };
  tr(out->w13, out->w13_t, 2 * H, d);
  tr(w2, out->w2_t, d, H);
  DM_HIP(hipGetLastError());
  return DM_OK;
}

int dm_mlp_fwd(int32_t dtype, const dm_mlp_packed* w, const void* y, void* z, const dm_mlp_bufs* bufs, int32_t M,
               int32_t d, int32_t H, float eps, void* stream) {
  int rc = check_mlp(dtype, w, bufs, M, d, H);
  if (rc) return rc;
  DM_REQUIRE(y && z && y != z && aligned16(y) && aligned16(z), DM_ERR_INVALID, "y, z: distinct, 16-byte aligned");
  hipStream_t s = S(stream);
  if (dtype == DM_BF16) mlp_fwd_rows<bf16>(w, (const bf16*)y, (bf16*)z, bufs, M, d, H, eps, -1, 0, 0, s);
  else mlp_fwd_rows<float>(w, (const float*)y, (float*)z, bufs, M, d, H, eps, -1, 0, 0, s);
  DM_HIP(hipGetLastError());
  return DM_OK;
}

size_t dm_mlp_workspace_bytes(int32_t dtype, int32_t M, int32_t d, int32_t H) {
  if ((dtype != DM_F32 && dtype != DM_BF16) || M <= 0 || d <= 0 || H <= 0 || d % 128 || H % 128) return 0;
  return carve_mlp(M, d, H, nullptr).bytes;
}

int dm_mlp_bwd(int32_t dtype, const dm_mlp_packed* w, const void* y, const void* dz, void* dy,
               const dm_mlp_bufs* bufs, const dm_mlp_grads* g, int32_t M, int32_t d, int32_t H, float eps,
               void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_mlp(dtype, w, bufs, M, d, H);
  if (rc || (rc = check_mlp_bwd(bufs, g))) return rc;
  DM_REQUIRE(y && dz && dy && dz != dy && aligned16(y) && aligned16(dz) && aligned16(dy), DM_ERR_INVALID,
             "y, dz, dy: 16-byte aligned, dy not aliasing dz");
  const MlpWs ws = carve_mlp(M, d, H, workspace);
  DM_REQUIRE(workspace && aligned16(workspace) && workspace_bytes >= ws.bytes, DM_ERR_WORKSPACE,
             "MLP workspace %zu < %zu bytes", workspace_bytes, ws.bytes);
  hipStream_t s = S(stream);
  if (dtype == DM_BF16) {
    mlp_bwd_rows<bf16>(w, (const bf16*)y, (const bf16*)dz, (bf16*)dy, bufs, M, d, H, eps, -1, 0, 0, 3, ws.dwa_part, s);
    mlp_wgrad<bf16>(bufs, (const bf16*)dz, M, d, H, g, ws, s);
  } else {
    mlp_bwd_rows<float>(w, (const float*)y, (const float*)dz, (float*)dy, bufs, M, d, H, eps, -1, 0, 0, 3,
                        ws.dwa_part, s);
    mlp_wgrad<float>(bufs, (const float*)dz, M, d, H, g, ws, s);
  }
  DM_HIP(hipGetLastError());
  return DM_OK;
}

}  // extern "C"
