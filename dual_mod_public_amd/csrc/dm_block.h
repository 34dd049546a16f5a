// The SwiGLU MLP sublayer of a Block (models/dualmod/model.py:102-112, 127-128) on the library's
// GEMM tiles: z = y + W2 (silu(W1 h) * W3 h), h = RMSNorm_mlp(y), and its VJP. One launch sequence
// serves the layer-by-layer trunk (all rows at once) and the layer-batched stack (one cell's rows,
// recorded into grouped launches): every product's per-element k order is fixed by K alone, so both
// give the same bits.
//
// Packed weights: w13 [2H, d] holds W1 and W3 rows interleaved in groups of 32 (group g: W1 rows
// 32g..32g+31, then W3 rows 32g..32g+31), so a 64-column block of h . w13^T holds the gate and the
// up product of the same 32 hidden units and the SwiGLU runs in the GEMM's epilogue.
//   forward   h = RMSNorm(y) rows; ab = h . w13^T with mid = silu(a) * b in the epilogue;
//             z = y + mid . W2^T (the residual epilogue)
//   backward  dab = the SwiGLU VJP in the epilogue of dm = dz . W2; dh = dab . w13; dy = dz +
//             RMSNorm VJP(dh); the weight grads sum over all rows once (dW2 = dz^T mid,
//             dw13 = dab^T h, unpacked into W1 / W3), as the attention's
#pragma once

#include "dm_bwd.h"
#include "dm_host.h"

namespace dm {

constexpr int MLP_GROUP = 32;   // hidden units per packed group of w13

// GEMM 1 epilogue: the raw products a | b (rounded to the storage dtype, as the reference's autocast
// linears) into ab, and mid = silu(a) * b into mid, silu(a) rounded before the product (the
// reference's two bf16 elementwise ops). Block tiles of whole 64-column groups.
template <typename T> struct EpiSwiGLU {
  static constexpr int TILE_ROWS = 64;
  int M, H;
  T* __restrict__ ab;     // [rows, 2H]
  T* __restrict__ mid;    // [rows, H]
  RowMap map = RowMap{};
  struct TilePre {};
  DM_DEV TilePre tile_prefetch(int, int) const { return TilePre{}; }
  template <int TR, int BN, int LDT>
  DM_DEV void tile_apply(const float* tile, int m0, int n0, const float*, const TilePre&, int) const {
    static_assert(BN % 64 == 0, "whole 64-column groups");
    constexpr int IPR = BN / 16;   // items of 8 hidden units per row
#pragma unroll 1
    for (int it = threadIdx.x; it < TR * IPR; it += 256) {
      const int r = it / IPR, q = it % IPR, gg = q >> 2, u0 = 8 * (q & 3);
      const int m = m0 + r;
      if (m >= M) continue;
      const float* tr = tile + r * LDT + 64 * gg;
      float a[8], b[8], o[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        a[i] = stored<T>(tr[u0 + i]);
        b[i] = stored<T>(tr[32 + u0 + i]);
        o[i] = stored<T>(a[i] * sigmoidf_(a[i])) * b[i];
      }
      const long row = map(m);
      T* abr = ab + row * 2 * H + n0 + 64 * gg;
      store_vec<T, 8>(abr + u0, a);
      store_vec<T, 8>(abr + 32 + u0, b);
      store_vec<T, 8>(mid + row * H + n0 / 2 + 32 * gg + u0, o);
    }
  }
};

// GEMM 3 epilogue: acc = dm = dz . W2 for hidden units n0..; with a, b from ab,
//   da = dm b silu'(a), silu'(a) = s (1 + a (1 - s)), s = sigma(a);  db = dm silu(a)
// into dab (w13's row order). Block tiles of whole 32-unit groups.
template <typename T> struct EpiSwiGLUBwd {
  static constexpr int TILE_ROWS = 64;
  int M, H;
  const T* __restrict__ ab;   // [rows, 2H]
  T* __restrict__ dab;        // [rows, 2H]
  RowMap map = RowMap{};
  struct TilePre {};
  DM_DEV TilePre tile_prefetch(int, int) const { return TilePre{}; }
  // a chunk's a, b runs, loaded before the chunk before it is applied
  static constexpr int MAXI = 8;   // items per thread and chunk
  struct ChunkPre {
    Raw8<T> a[MAXI], b[MAXI];
  };
  template <int TR, int BN> struct Shape {
    static constexpr int IPR = BN / 8, NI = TR * IPR / 256;   // items of 8 hidden units per row
    static_assert(BN % MLP_GROUP == 0, "whole 32-unit groups");
    static_assert((TR * IPR) % 256 == 0 && NI <= MAXI, "whole items per thread");
  };
  DM_DEV long item_col(int u) const { return 2L * MLP_GROUP * (u / MLP_GROUP) + u % MLP_GROUP; }
  template <int TR, int BN> DM_DEV ChunkPre chunk_prefetch(int m0, int n0) const {
    using S = Shape<TR, BN>;
    ChunkPre cp;
#pragma unroll
    for (int i = 0; i < S::NI; ++i) {
      const int it = threadIdx.x + 256 * i, r = it / S::IPR, u = n0 + 8 * (it % S::IPR);
      const T* p = ab + map(min(m0 + r, M - 1)) * 2 * H + item_col(u);
      cp.a[i] = ld8_global(p);
      cp.b[i] = ld8_global(p + MLP_GROUP);
    }
    return cp;
  }
  template <int TR, int BN, int LDT>
  DM_DEV void tile_apply(const float* tile, int m0, int n0, const float*, const TilePre&, int,
                         const ChunkPre& cp) const {
    using S = Shape<TR, BN>;
#pragma unroll
    for (int i = 0; i < S::NI; ++i) {
      const int it = threadIdx.x + 256 * i, r = it / S::IPR, u = n0 + 8 * (it % S::IPR);
      const int m = m0 + r;
      if (m >= M) continue;
      const long row = map(m);
      const long col = item_col(u);
      float a[8], b[8], dm[8], da[8], db[8];
      unpack8<T>(cp.a[i], a);
      unpack8<T>(cp.b[i], b);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        dm[i] = tile[r * LDT + (u - n0) + i];
        const float s = sigmoidf_(a[i]);
        da[i] = dm[i] * b[i] * s * (1.f + a[i] * (1.f - s));
        db[i] = dm[i] * stored<T>(a[i] * s);
      }
      store_vec<T, 8>(dab + row * 2 * H + col, da);
      store_vec<T, 8>(dab + row * 2 * H + col + MLP_GROUP, db);
    }
  }
};

// dW13 [2H, d] (fp32, w13's row order) added into the reference layout: W1 / W3 [H, d]
static __global__ __launch_bounds__(256) void k_unpack_w13(const float* __restrict__ src, int H, int d,
                                                           float* __restrict__ g1, float* __restrict__ g3) {
  const int p = blockIdx.x;   // packed row
  const int grp = p / (2 * MLP_GROUP), w = p % (2 * MLP_GROUP);
  float* dst = (w < MLP_GROUP ? g1 : g3) + (long)(MLP_GROUP * grp + (w % MLP_GROUP)) * d;
  const float* sr = src + (long)p * d;
  for (int j = threadIdx.x; j < d; j += 256) dst[j] += sr[j];
}

// The forward of M rows: rows of the [B, T, .] buffers given by (lc, Tr, pos0) of one chunk (lc >= 0:
// the recorded stack launches) or all rows in order (lc < 0, M = B T). Both take the large tiles
// (256 x 256 where M and N allow: a chunk's B c rows are one or two row tiles, and a layer-batched
// launch has blocks to spare).
template <typename T>
void mlp_fwd_rows(const dm_mlp_packed* w, const T* y, T* z, const dm_mlp_bufs* mb, int M, int d, int H, float eps,
                  int lc, int Tr, int pos0, hipStream_t s) {
  const RowMap map = lc >= 0 ? RowMap{lc, Tr, pos0} : RowMap{};
  T* h = (T*)mb->h;
  T* ab = (T*)mb->ab;
  T* mid = (T*)mb->mid;
  EpiSwiGLU<T> e1{M, H, ab, mid, map};
  EpiResidual<T> e2{M, d, y, z, map};
  const SrcRows<T> w13{(const T*)w->w13, d, 2 * H}, w2{(const T*)w->w2, H, d};
  if (lc >= 0) {
    record_launch<RmsRowsBody<T>>(dim3(cdiv(M, 4)), dim3(256),
                                  typename RmsRowsBody<T>::Args{y, (const T*)w->norm_w, h, M, d, eps, map});
    launch_gemm_big<T>(SrcChunkRows<T>{h, d, M, lc, Tr, pos0}, w13, M, 2 * H, d, e1, s);
    launch_gemm_big<T>(SrcChunkRows<T>{mid, H, M, lc, Tr, pos0}, w2, M, d, H, e2, s);
    return;
  }
  hipLaunchKernelGGL(k_rmsnorm_rows<T>, dim3(cdiv(M, 4)), dim3(256), 0, s, y, (const T*)w->norm_w, h, M, d, eps);
  launch_gemm_big<T>(SrcRows<T>{h, d, M}, w13, M, 2 * H, d, e1, s);
  launch_gemm_big<T>(SrcRows<T>{mid, H, M}, w2, M, d, H, e2, s);
}

// The VJP rows of the same M rows: dab (GEMM 3's epilogue), dh, then dy = dz + RMSNorm VJP(dh)
// (rmsnorm_bwd flags: 1 dy rows, 2 the norm weight's partials into dwa_part, one row per 8 rows).
template <typename T>
void mlp_bwd_rows(const dm_mlp_packed* w, const T* y, const T* dz, T* dy, const dm_mlp_bufs* mb, int M, int d, int H,
                  float eps, int lc, int Tr, int pos0, int flags, float* dwa_part, hipStream_t s) {
  const RowMap map = lc >= 0 ? RowMap{lc, Tr, pos0} : RowMap{};
  const T* ab = (const T*)mb->ab;
  T* dab = (T*)mb->dab;
  EpiSwiGLUBwd<T> e3{M, H, ab, dab, map};
  EpiStoreTileF32 e4{M, d, mb->dh, 0, map};
  const SrcRows<T> w2t{(const T*)w->w2_t, d, H}, w13t{(const T*)w->w13_t, 2 * H, d};
  typename RmsnormBwdBody<T>::Args ra{M, d, eps, 1, y, (const T*)w->norm_w, mb->dh, dz, dy, dwa_part, map, flags};
  const unsigned lds = (unsigned)(4 * d * sizeof(float));
  if (lc >= 0) {
    launch_gemm_big<T>(SrcChunkRows<T>{dz, d, M, lc, Tr, pos0}, w2t, M, H, d, e3, s);
    launch_gemm_big<T>(SrcChunkRows<T>{dab, 2 * H, M, lc, Tr, pos0}, w13t, M, d, 2 * H, e4, s);
    record_launch<RmsnormBwdBody<T>>(dim3(cdiv(M, RMSN_ROWS)), dim3(256), ra, lds);
    return;
  }
  launch_gemm_big<T>(SrcRows<T>{dz, d, M}, w2t, M, H, d, e3, s);
  launch_gemm_big<T>(SrcRows<T>{dab, 2 * H, M}, w13t, M, d, 2 * H, e4, s);
  hipLaunchKernelGGL(k_rmsnorm_bwd<T>, dim3(cdiv(M, RMSN_ROWS)), dim3(256), lds, s, ra.M, ra.d, ra.eps, ra.residual,
                     ra.x, ra.w, ra.dxhat, ra.dy, ra.dx, ra.dwa_part, ra.map, ra.flags);
}

// argument checks of the MLP entry points and of the stacks' block tails
inline int check_mlp(int dtype, const dm_mlp_packed* w, const dm_mlp_bufs* mb, int M, int d, int H) {
  DM_REQUIRE(dtype == DM_F32 || dtype == DM_BF16, DM_ERR_INVALID, "dtype %d", dtype);
  DM_REQUIRE(M > 0 && d > 0 && H > 0 && d % 128 == 0 && H % 128 == 0, DM_ERR_INVALID,
             "MLP M=%d d=%d H=%d (d and H multiples of 128)", M, d, H);
  DM_REQUIRE(w && w->w13 && w->w2 && w->w13_t && w->w2_t && w->norm_w, DM_ERR_INVALID, "null packed MLP weight");
  DM_REQUIRE(mb && mb->h && mb->ab && mb->mid, DM_ERR_INVALID, "null MLP buffer");
  DM_REQUIRE(aligned16(w->w13) && aligned16(w->w2) && aligned16(w->w13_t) && aligned16(w->w2_t) && aligned16(mb->h) &&
                 aligned16(mb->ab) && aligned16(mb->mid),
             DM_ERR_INVALID, "MLP weights and buffers must be 16-byte aligned");
  return DM_OK;
}
inline int check_mlp_bwd(const dm_mlp_bufs* mb, const dm_mlp_grads* g) {
  DM_REQUIRE(mb->dab && mb->dh && aligned16(mb->dab) && aligned16(mb->dh), DM_ERR_INVALID,
             "the MLP backward needs 16-byte aligned dab and dh buffers");
  DM_REQUIRE(g && g->w1 && g->w3 && g->w2 && g->norm_w, DM_ERR_INVALID, "null MLP gradient");
  return DM_OK;
}

}  // namespace dm
