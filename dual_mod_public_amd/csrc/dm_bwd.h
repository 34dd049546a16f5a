// Kernels of the reverse-scan backward
// (engines/wavescan/cells/fused_sweep.py:1557-1850 semantics, own design).
//
// Per cell, sweeps run in reverse. For sweep s with its saved (or recomputed) state:
//   k_refine_bwd  VJP of the blend/gate/RoPE epilogue of the sweep-s refine:
//                 grads of the refined rows -> dctx (packed GEMM-1 column order),
//                 dv_ctx, and the layer accumulators dkraw / dvraw
//   EpiVinBwd     epilogue of dv_in = dv_ctx . W_vctx: tanh / sigmoid VJP of v_in
//   k_du_epi      after the split-K GEMM du = dctx . W_sweep (+ lam dv_in): g = du * w_ctx,
//                 per-row partial <g, o> for the RMS VJP, norm_ctx weight partials
//   k_attn_bwd    attention VJP of sweep s per (b, h): intra rows (strict lower)
//                 + raw self column; accumulates the committed part's G, Dbar
// The committed-prefix part of every sweep is one VJP per row (k_comm_dkv, k_comm_dq):
//   sum_s dS_comm^s = E o (G V^T - Dbar),  E = exp(S - m_comm),
//   G = sum_s alpha_s dO_s, Dbar = sum_s alpha_s D_s, alpha_s = exp(m_comm - M_s) / Z_s,
// which is exact because the committed scores are the same in every sweep.
#pragma once

#include "dm_kernels.h"

namespace dm {

// ---------------------------------------------------------------------------
// small helpers
// ---------------------------------------------------------------------------
// zero up to FILL_MAX fp32 arrays, array blockIdx.y; 16-byte stores where the array allows
constexpr int FILL_MAX = 12;
struct FillList {
  float* p[FILL_MAX];
  long n[FILL_MAX];
  int n_arr;
};
static __global__ __launch_bounds__(256) void k_fill_list(FillList fl) {
  float* __restrict__ p = fl.p[blockIdx.y];
  const long n = fl.n[blockIdx.y];
  const long stride = (long)gridDim.x * 256;
  const long i0 = blockIdx.x * 256L + threadIdx.x;
  if ((reinterpret_cast<uintptr_t>(p) & 15) == 0) {
    for (long i = i0; 4 * i + 3 < n; i += stride) *reinterpret_cast<floatx4*>(p + 4 * i) = zero4();
    for (long j = (n / 4) * 4 + i0; j < n; j += stride) p[j] = 0.f;
  } else {
    for (long i = i0; i < n; i += stride) p[i] = 0.f;
  }
}

// C-layout MFMA product for one wave: acc[t] += X[16 rows, KD] . Y[16 t + (0..15), KD]^T,
// X and Y row-major in LDS with leading dimensions ldx / ldy (K contiguous).
template <typename T, int KD, int NT>
DM_DEV void wave_mma(const T* X, int ldx, const T* Y, int ldy, floatx4 (&acc)[NT]) {
  using MF = Mfma<T>;
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int k = 0; k < KD; k += MF::KSTEP) {
    const typename MF::frag a = MF::load(X + (lane & 15) * ldx + k + (lane >> 4) * MF::KPL);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const typename MF::frag b = MF::load(Y + (16 * t + (lane & 15)) * ldy + k + (lane >> 4) * MF::KPL);
      acc[t] = MF::mma(a, b, acc[t]);
    }
  }
}

// The same with the B operand read from the transposed view of a row-major LDS
// matrix Z [KD rows][ldz]: acc[t] += X[16 rows, KD] . Z[:, 16 t + (0..15)] (no
// transposed copy of Z is staged).
// X is the calling wave's own LDS staging, written by its lanes just before: LDS operations
// of one wave complete in order, and the wave barriers keep the compiler from moving these
// reads above those writes, or the wave's next writes of X above these reads.
template <typename T, int KD, int NT>
DM_DEV void wave_mma_bt(const T* X, int ldx, const T* Z, int ldz, floatx4 (&acc)[NT]) {
  using MF = Mfma<T>;
  const int lane = threadIdx.x & 63;
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int k = 0; k < KD; k += MF::KSTEP) {
    const typename MF::frag a = MF::load(X + (lane & 15) * ldx + k + (lane >> 4) * MF::KPL);
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = MF::mma(a, MF::load_tr(Z + (long)k * ldz + 16 * t, ldz), acc[t]);
  }
  __builtin_amdgcn_wave_barrier();
}

// The cell of a layer row, for the backward's per-row sums over a cell's sweeps: its first
// row pos0, length c, sweeps K, and the row of the weight-grad stacks (dctx) that holds its
// sweep 0, batch element 0, cell row 0 (sweep s, element b, cell row p at row0 + s B c + b c + p).
// K = 0: the row is in no cell.
struct CellRow {
  int pos0, c, K, row0;
};

// packed GEMM-1 column of the k_ctx / g_k(u) quads (see EpiSweep1)
template <int DH> DM_DEV int col_k(int hd, int jj, int part) {
  return hd * 2 * DH + 64 * (jj / 16) + 16 * part + (jj % 16);
}
// linear ctx_mod: packed column of v_ctx element e of head hd (g_v(u) at +32)
template <int DH> DM_DEV int col_vlin(int d, int hd, int e) {
  return 2 * d + hd * 2 * DH + 64 * (e / 32) + (e % 32);
}

// ---------------------------------------------------------------------------
// refine VJP of one sweep (attention.py:314-387 backward). One item = (row m, head hd,
// 4 consecutive RoPE pairs jj..jj+3): K pairs (jj + i, jj + i + DH/2), V elements likewise.
// The DH / 8 items of a (row, head) are consecutive lanes, which reduce the head-wide sums of
// the k_ctx / v_ctx norms and of the v'' clamp.
// ---------------------------------------------------------------------------
template <typename T> struct RefineBwdArgs {
  CellGeom g;
  int N, ctx_mod;
  const float* dK; const float* dV;    // grads of the refined rows (rotated K, V): the sum of
  long dk_stride; int dk_row0;         //   NS slices psum_stride apart, (b,h) at bh*dk_stride,
  long psum_stride;                    //   chunk row p at row dk_row0 + p (standalone kernel)
  const T* save1;                      // [N, 4d] raw GEMM-1 outputs of this sweep (storage dtype)
  const T* save2;                      // [N, d] raw v_ctx (mult family)
  const T* glogx; const T* kraw; const T* vraw;
  const float* cos; const float* sin;
  T* dctx;                             // [N, 4d] (packed columns; v_map columns written by EpiVinBwd)
  T* dvc;                              // [N, d] dv_ctx (mult family)
  float* dkraw; float* dvraw;          // layer accumulators (+=). The gate logits' grads dl go
                                       //   to dctx only: the projection VJP sums them per row
  // k_ctx / v_ctx norms (attention.py:238-269): gains [h] (nullptr = off) and the gains'
  // per-row gradient partials [B*Tbuf, h] (+=)
  const float* kgain = nullptr; const float* vgain = nullptr;
  float* dkg = nullptr; float* dvg = nullptr;
};

// the grads of one item's refined values: K at columns jj.. (a) and jj + DH/2.. (b), V likewise
struct RefineGrad4 {
  float ka[4], kb[4], va[4], vb[4];
};

template <typename T> DM_DEV void ld4(const T* p, float* out) {
  if constexpr (sizeof(T) == 2) unpack4<T>(ld_global<typename Raw4<T>::type>(p), out);
  else unpackf4(ld_global<floatx4>(p), out);
}

// The gathered inputs of one item (the loads, issued together before any math)
struct RefineIn {
  float cs[4], sn[4], kx1[4], kx2[4], gu1[4], gu2[4], gx1[4], gx2[4], gxv1[4], gxv2[4];
  float kr1[4], kr2[4], vr1[4], vr2[4], vx1[4], vx2[4], gvu1[4], gvu2[4];
  float okr1[4], okr2[4], ovr1[4], ovr2[4];
};

template <typename T, int DH>
DM_DEV RefineIn refine_gather(const RefineBwdArgs<T>& a, int m, int hd, int jj) {
  const CellGeom& g = a.g;
  const int d = g.d, h = g.h;
  const int b = m / g.c, p = m - b * g.c;
  const int t = g.buf_t0 + p, pos = rope_row(g, p);
  const long lrow = (((long)b * h + hd) * g.Tbuf + t) * DH + jj;
  const long xrow = (long)b * g.Tbuf + t;
  const T* S1 = a.save1 + (long)m * 4 * d;
  const T* gxr = a.glogx + xrow * 2 * d;
  const int c1 = hd * DH + jj, c2 = c1 + DH / 2;
  RefineIn in;
  ld4<float>(a.cos + (long)pos * (DH / 2) + jj, in.cs);
  ld4<float>(a.sin + (long)pos * (DH / 2) + jj, in.sn);
  ld4<T>(S1 + col_k<DH>(hd, jj, 0), in.kx1);
  ld4<T>(S1 + col_k<DH>(hd, jj, 1), in.kx2);
  ld4<T>(S1 + col_k<DH>(hd, jj, 2), in.gu1);
  ld4<T>(S1 + col_k<DH>(hd, jj, 3), in.gu2);
  ld4<T>(gxr + c1, in.gx1);
  ld4<T>(gxr + c2, in.gx2);
  ld4<T>(gxr + d + c1, in.gxv1);
  ld4<T>(gxr + d + c2, in.gxv2);
  ld4<T>(a.kraw + lrow, in.kr1);
  ld4<T>(a.kraw + lrow + DH / 2, in.kr2);
  ld4<T>(a.vraw + lrow, in.vr1);
  ld4<T>(a.vraw + lrow + DH / 2, in.vr2);
  if (a.ctx_mod == 0) {
    const int cv1 = col_vlin<DH>(d, hd, jj), cv2 = col_vlin<DH>(d, hd, jj + DH / 2);
    ld4<T>(S1 + cv1, in.vx1);
    ld4<T>(S1 + cv2, in.vx2);
    ld4<T>(S1 + cv1 + 32, in.gvu1);
    ld4<T>(S1 + cv2 + 32, in.gvu2);
  } else {
    ld4<T>(a.save2 + (long)m * d + c1, in.vx1);
    ld4<T>(a.save2 + (long)m * d + c2, in.vx2);
    ld4<T>(S1 + 3 * d + c1, in.gvu1);
    ld4<T>(S1 + 3 * d + c2, in.gvu2);
  }
  // the accumulators' current values, loaded with the inputs (one memory round trip)
  ld4<float>(a.dkraw + lrow, in.okr1);
  ld4<float>(a.dkraw + lrow + DH / 2, in.okr2);
  ld4<float>(a.dvraw + lrow, in.ovr1);
  ld4<float>(a.dvraw + lrow + DH / 2, in.ovr2);
  return in;
}

template <typename T, int DH>
DM_DEV void refine_apply(const RefineBwdArgs<T>& a, int m, int hd, int jj, const RefineIn& in,
                         const RefineGrad4& gr) {
  constexpr int L = DH / 8;   // lanes per (row, head)
  const CellGeom& g = a.g;
  const int d = g.d, h = g.h;
  const int b = m / g.c, p = m - b * g.c;
  const int t = g.buf_t0 + p;
  const long lrow = (((long)b * h + hd) * g.Tbuf + t) * DH + jj;
  const long xrow = (long)b * g.Tbuf + t;
  const int c1 = hd * DH + jj, c2 = c1 + DH / 2;
  // k_ctx / v_ctx as the blends took them: raw (kx, vx), or normed, (x r) gain from and to
  // stored values, r over the head's L lanes
  float kc1[4], kc2[4], vc1[4], vc2[4];
  float rk = 0.f, gk = 0.f, rv = 0.f, gvn = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) { kc1[i] = in.kx1[i]; kc2[i] = in.kx2[i]; vc1[i] = in.vx1[i]; vc2[i] = in.vx2[i]; }
  if (a.kgain != nullptr) {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) ss += in.kx1[i] * in.kx1[i] + in.kx2[i] * in.kx2[i];
    rk = head_norm_r(group_sum<L>(ss), 1.0f / DH);
    gk = a.kgain[hd];
#pragma unroll
    for (int i = 0; i < 4; ++i) { kc1[i] = stored<T>((in.kx1[i] * rk) * gk); kc2[i] = stored<T>((in.kx2[i] * rk) * gk); }
  }
  if (a.vgain != nullptr) {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) ss += in.vx1[i] * in.vx1[i] + in.vx2[i] * in.vx2[i];
    rv = head_norm_r(group_sum<L>(ss), 1.0f / DH);
    gvn = a.vgain[hd];
#pragma unroll
    for (int i = 0; i < 4; ++i) { vc1[i] = stored<T>((in.vx1[i] * rv) * gvn); vc2[i] = stored<T>((in.vx2[i] * rv) * gvn); }
  }
  // ---- key: unrotate, then the convex blend k'' = g k_raw + (1 - g) k_ctx
  float dkc1[4], dkc2[4], dl1[4], dl2[4], nk1[4], nk2[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float dk1 = gr.ka[i] * in.cs[i] + gr.kb[i] * in.sn[i], dk2 = -gr.ka[i] * in.sn[i] + gr.kb[i] * in.cs[i];
    const float g1 = sigmoidf_(in.gx1[i] + in.gu1[i]), g2 = sigmoidf_(in.gx2[i] + in.gu2[i]);
    dl1[i] = dk1 * (in.kr1[i] - kc1[i]) * g1 * (1.f - g1);
    dl2[i] = dk2 * (in.kr2[i] - kc2[i]) * g2 * (1.f - g2);
    dkc1[i] = dk1 * (1.f - g1);
    dkc2[i] = dk2 * (1.f - g2);
    nk1[i] = in.okr1[i] + dk1 * g1;
    nk2[i] = in.okr2[i] + dk2 * g2;
  }
  if (a.kgain != nullptr) {
    // norm VJP: dx = gain (r dy - r^3 x <dy, x> / DH); d gain += r <dy, x> (this row's partial)
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) s += dkc1[i] * in.kx1[i] + dkc2[i] * in.kx2[i];
    const float sk = group_sum<L>(s);
    const float r3 = rk * rk * rk * sk * (1.0f / DH);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      dkc1[i] = gk * (rk * dkc1[i] - r3 * in.kx1[i]);
      dkc2[i] = gk * (rk * dkc2[i] - r3 * in.kx2[i]);
    }
    if (jj == 0) a.dkg[xrow * h + hd] += rk * sk;
  }
  // ---- value: v'' = g_v v_raw + (1 - g_v) v_ctx; kmod heads (attention.py:362-384):
  // raw v'' = v_raw (or tanh(v_raw)) takes no gate or v_ctx grad; gated_norm blends with
  // v_ctx = 0 (live gate, no v_ctx grad)
  float dv1[4], dv2[4], gv1[4], gv2[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    dv1[i] = gr.va[i];
    dv2[i] = gr.vb[i];
    gv1[i] = sigmoidf_(in.gxv1[i] + in.gvu1[i]);
    gv2[i] = sigmoidf_(in.gxv2[i] + in.gvu2[i]);
  }
  if (g.v_clamp_tau > 0.f) {
    // VJP of the norm clamp v = v'' min(1, tau / ||v''||) (attention.py:389-402): outside the
    // radius dv'' = (tau / n) (dv - v'' <v'', dv> / n^2), n = ||v''||, else dv'' = dv
    float p1[4], p2[4], ss = 0.f, dt = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      p1[i] = value_blend(g, c1 + i, gv1[i], in.vr1[i], vc1[i]);
      p2[i] = value_blend(g, c2 + i, gv2[i], in.vr2[i], vc2[i]);
      ss += p1[i] * p1[i] + p2[i] * p2[i];
      dt += p1[i] * dv1[i] + p2[i] * dv2[i];
    }
    ss = group_sum<L>(ss);
    dt = group_sum<L>(dt);
    const float n = sqrtf(ss);
    if (n > g.v_clamp_tau) {
      const float sc = g.v_clamp_tau / n, k = dt / ss;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        dv1[i] = sc * (dv1[i] - p1[i] * k);
        dv2[i] = sc * (dv2[i] - p2[i] * k);
      }
    }
  }
  float dlv1[4], dlv2[4], dvc1[4], dvc2[4], nv1[4], nv2[4];
  const bool kmod = c1 < g.kmod_cols;   // whole heads: uniform over the item
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float dvr1, dvr2;
    if (kmod) {
      const bool gated = g.kmod_mode == DM_KMOD_GATED_NORM;
      dlv1[i] = gated ? dv1[i] * in.vr1[i] * gv1[i] * (1.f - gv1[i]) : 0.f;
      dlv2[i] = gated ? dv2[i] * in.vr2[i] * gv2[i] * (1.f - gv2[i]) : 0.f;
      dvc1[i] = 0.f;
      dvc2[i] = 0.f;
      if (gated) { dvr1 = dv1[i] * gv1[i]; dvr2 = dv2[i] * gv2[i]; }
      else if (g.kmod_mode == DM_KMOD_RAW_TANH) {
        const float t1 = tanhf_(in.vr1[i]), t2 = tanhf_(in.vr2[i]);
        dvr1 = dv1[i] * (1.f - t1 * t1);
        dvr2 = dv2[i] * (1.f - t2 * t2);
      } else { dvr1 = dv1[i]; dvr2 = dv2[i]; }
    } else {
      dlv1[i] = dv1[i] * (in.vr1[i] - vc1[i]) * gv1[i] * (1.f - gv1[i]);
      dlv2[i] = dv2[i] * (in.vr2[i] - vc2[i]) * gv2[i] * (1.f - gv2[i]);
      dvc1[i] = dv1[i] * (1.f - gv1[i]);
      dvc2[i] = dv2[i] * (1.f - gv2[i]);
      dvr1 = dv1[i] * gv1[i];
      dvr2 = dv2[i] * gv2[i];
    }
    nv1[i] = in.ovr1[i] + dvr1;
    nv2[i] = in.ovr2[i] + dvr2;
  }
  if (a.vgain != nullptr) {   // v_ctx norm VJP, as the key's (kmod heads: dvc = 0, so zero)
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) s += dvc1[i] * in.vx1[i] + dvc2[i] * in.vx2[i];
    const float sv = group_sum<L>(s);
    const float r3 = rv * rv * rv * sv * (1.0f / DH);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      dvc1[i] = gvn * (rv * dvc1[i] - r3 * in.vx1[i]);
      dvc2[i] = gvn * (rv * dvc2[i] - r3 * in.vx2[i]);
    }
    if (jj == 0) a.dvg[xrow * h + hd] += rv * sv;
  }
  // ---- stores
  T* D = a.dctx + (long)m * 4 * d;
  st4<T>(D + col_k<DH>(hd, jj, 0), dkc1);
  st4<T>(D + col_k<DH>(hd, jj, 1), dkc2);
  st4<T>(D + col_k<DH>(hd, jj, 2), dl1);
  st4<T>(D + col_k<DH>(hd, jj, 3), dl2);
  if (a.ctx_mod == 0) {
    const int cv1 = col_vlin<DH>(d, hd, jj), cv2 = col_vlin<DH>(d, hd, jj + DH / 2);
    st4<T>(D + cv1, dvc1);
    st4<T>(D + cv2, dvc2);
    st4<T>(D + cv1 + 32, dlv1);
    st4<T>(D + cv2 + 32, dlv2);
  } else {
    st4<T>(a.dvc + (long)m * d + c1, dvc1);
    st4<T>(a.dvc + (long)m * d + c2, dvc2);
    st4<T>(D + 3 * d + c1, dlv1);
    st4<T>(D + 3 * d + c2, dlv2);
  }
  st4<float>(a.dkraw + lrow, nk1);
  st4<float>(a.dkraw + lrow + DH / 2, nk2);
  st4<float>(a.dvraw + lrow, nv1);
  st4<float>(a.dvraw + lrow + DH / 2, nv2);
}


template <typename T, int DH>
DM_DEV void refine_vjp4(const RefineBwdArgs<T>& a, int m, int hd, int jj, const RefineGrad4& gr) {
  const RefineIn in = refine_gather<T, DH>(a, m, hd, jj);
  refine_apply<T, DH>(a, m, hd, jj, in, gr);
}

// The refine VJP as its own launch (the first reverse sweep of a cell, whose grads come from
// the committed-prefix VJP or the grad cache): one thread per item, the grads read from the NS
// slices.
template <typename T, int DH, int NS>
DM_DEV void refine_bwd_body(const RefineBwdArgs<T>& a) {
  constexpr int Q = DH / 8;   // items per (row, head)
  const int per_row = a.g.d / 8;
  const int idx = blockIdx.x * 256 + threadIdx.x;
  if (idx >= a.N * per_row) return;   // whole (row, head) lane groups: Q divides 256 and per_row
  const int m = idx / per_row, rem = idx - m * per_row;
  const int hd = rem / Q, jj = 4 * (rem - hd * Q);
  const int b = m / a.g.c, p = m - b * a.g.c;
  const long drow = ((long)b * a.g.h + hd) * a.dk_stride + (long)(a.dk_row0 + p) * DH + jj;
  RefineGrad4 gr;
  float t0[4], t1[4], t2[4], t3[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) { gr.ka[i] = 0.f; gr.kb[i] = 0.f; gr.va[i] = 0.f; gr.vb[i] = 0.f; }
#pragma unroll
  for (int q = 0; q < NS; ++q) {
    const long o = q * a.psum_stride + drow;
    ld4<float>(a.dK + o, t0);
    ld4<float>(a.dK + o + DH / 2, t1);
    ld4<float>(a.dV + o, t2);
    ld4<float>(a.dV + o + DH / 2, t3);
#pragma unroll
    for (int i = 0; i < 4; ++i) { gr.ka[i] += t0[i]; gr.kb[i] += t1[i]; gr.va[i] += t2[i]; gr.vb[i] += t3[i]; }
  }
  refine_vjp4<T, DH>(a, m, hd, jj, gr);
}

template <typename T, int DH, int NS>
static __global__ __launch_bounds__(256) void k_refine_bwd(RefineBwdArgs<T> a) {
  refine_bwd_body<T, DH, NS>(a);
}

// ---------------------------------------------------------------------------
// dv_in = dv_ctx . W_vctx epilogue (mult family): v_in = lam u + sig tanh(vm)
//   dsig += dv_in tanh(vm); dctx[:, 2d + j] = dv_in sig (1 - tanh^2); lamdv = lam dv_in
//   (fusion, v_in = u + silu(z), z = px + vm: dsig and dctx[:, 2d + j] += dv_in silu'(z), lamdv = dv_in)
// ---------------------------------------------------------------------------
template <typename T, int BN = 32> struct EpiVinBwd {
  CellGeom g;
  int M, ctx_mod;
  float lam;
  const T* __restrict__ save1;       // [N, 4d]
  const T* __restrict__ sig;         // [B, Tbuf, d]
  T* __restrict__ dctx;              // [N, 4d]
  float* __restrict__ dsig;          // layer accumulator [B, Tbuf, d]
  float* __restrict__ lamdv;         // [N, d]
  // Block tile 64 x BN: thread t owns row t / 4 and, in each 32-column group q, columns
  // 32 q + 8 (t % 4) .. + 7; its inputs (and the dsig values it will add to) are gathered
  // before the k-loop.
  static constexpr int NQ = BN / 32;
  struct TilePre {
    Raw8<T> sg[NQ];
    floatx4 ds[NQ][2];
    Raw8<T> vm[NQ];
  };
  // vector-memory load instructions tile_prefetch issues (Raw8 = one 16-byte load in bf16, two in
  // fp32: 16-byte loads, which the compiler cannot merge into fewer)
  static constexpr int LATE_GATHERS = NQ * (2 + 2 * (int)(sizeof(T) / 2));
  DM_DEV TilePre tile_prefetch(int m0, int n0) const {
    const int r = threadIdx.x >> 2, c0 = n0 + 8 * (threadIdx.x & 3);
    const int d = g.d;
    const int m = min(m0 + r, M - 1);
    const int b = m / g.c;
    const long xrow = (long)b * g.Tbuf + g.buf_t0 + m - b * g.c;
    TilePre pr;
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int col = c0 + 32 * q;
      pr.sg[q] = ld8_global(sig + xrow * d + col);
#pragma unroll
      for (int k = 0; k < 2; ++k) pr.ds[q][k] = ld_global<floatx4>(dsig + xrow * d + col + 4 * k);
      pr.vm[q] = ld8_global(save1 + (long)m * 4 * d + 2 * d + col);
    }
    return pr;
  }
  template <int BM, int BN_, int LDT>
  DM_DEV void tile_apply(const float* tile, int m0, int n0, const float*, const TilePre& pr, int) const {
    static_assert(BM == 64 && BN_ == BN, "dv_in GEMM block tile is 64 x BN");
    const int r = threadIdx.x >> 2, d = g.d;
    const int m = m0 + r;
    float dv[NQ][8], sg[NQ][8], ds[NQ][8], vm[NQ][8];
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int c0 = 32 * q + 8 * (threadIdx.x & 3);
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        unpackf4(*reinterpret_cast<const floatx4*>(tile + r * LDT + c0 + 4 * k), dv[q] + 4 * k);
        unpackf4(pr.ds[q][k], ds[q] + 4 * k);
      }
      unpack8<T>(pr.sg[q], sg[q]);
      unpack8<T>(pr.vm[q], vm[q]);
    }
    if (m >= M) return;
#pragma unroll
    for (int q = 0; q < NQ; ++q) { settle(sg[q]); settle(ds[q]); settle(vm[q]); }   // all loads before any store
    const int b = m / g.c;
    const long xrow = (long)b * g.Tbuf + g.buf_t0 + m - b * g.c;
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int col = n0 + 32 * q + 8 * (threadIdx.x & 3);
      float dso[8], dc[8], lv[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if (ctx_mod == 3) {   // fusion: v_in = u + silu(z), z = px + vm; silu' = s (1 + z (1 - s))
          const float z = sg[q][i] + vm[q][i], s = sigmoidf_(z);
          const float dz = dv[q][i] * s * (1.f + z * (1.f - s));
          dso[i] = ds[q][i] + dz;
          dc[i] = dz;
          lv[i] = dv[q][i];
        } else {
          const float th = tanhf_(vm[q][i]);
          dso[i] = ds[q][i] + dv[q][i] * th;
          dc[i] = dv[q][i] * sg[q][i] * (1.f - th * th);
          lv[i] = ctx_mod == 1 ? lam * dv[q][i] : 0.f;
        }
      }
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        *reinterpret_cast<floatx4*>(dsig + xrow * d + col + 4 * k) = floatx4{dso[4 * k], dso[4 * k + 1], dso[4 * k + 2], dso[4 * k + 3]};
        *reinterpret_cast<floatx4*>(lamdv + (long)m * d + col + 4 * k) = floatx4{lv[4 * k], lv[4 * k + 1], lv[4 * k + 2], lv[4 * k + 3]};
      }
      store_vec<T, 8>(dctx + (long)m * 4 * d + 2 * d + col, dc);
    }
  }
};

// ---------------------------------------------------------------------------
// RMS-VJP inputs from the split-K slices of du = dctx . W_sweep (+ lam dv_in):
//   gw = du * w (fp32), rowdot[m, chunk] = sum over the chunk's DU_EPI_TN columns of gw * o,
//   dnw[m / 16][col] += sum over the 16 rows of du * o * r   (norm_ctx.weight)
// One block per (16 rows, 64 columns): wave q takes rows 4q..4q+3, lane = column.
// Slices are summed in order z = 0..S-1; every load is issued before the first add.
// ---------------------------------------------------------------------------
constexpr int DU_EPI_TN = 64;
template <typename T, int S>
DM_DEV void du_epi_body(int M, int d, int h, float inv_d, float eps,
                        const float* __restrict__ part,
                        const float* __restrict__ lamdv, const T* __restrict__ o,
                        const float* __restrict__ ssq, const T* __restrict__ normw,
                        float* __restrict__ gw, float* __restrict__ rowdot,
                        float* __restrict__ dnw){
  __shared__ float cs[4][DU_EPI_TN];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int m0 = blockIdx.x * 16 + 4 * wave, col = blockIdx.y * DU_EPI_TN + lane;
  const long n = (long)M * d;
  float pv[S][4], lv[4], ov[4], ss[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = min(m0 + i, M - 1);
    const long idx = (long)m * d + col;
#pragma unroll
    for (int z = 0; z < S; ++z) pv[z][i] = part[z * n + idx];
    lv[i] = lamdv != nullptr ? lamdv[idx] : 0.f;
    ov[i] = to_f(o[idx]);
    // the row's h partial sums of squares, split over the wave's lanes
    ss[i] = lane < h ? ssq[(long)m * h + lane] : 0.f;
  }
  const float w = to_f(normw[col]);
  const float dn_old = wave == 0 ? dnw[(long)blockIdx.x * d + col] : 0.f;
  float dn = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = m0 + i;
    float du = pv[0][i];
#pragma unroll
    for (int z = 1; z < S; ++z) du += pv[z][i];
    du += lv[i];
    const float r = rsqrtf(wave_sum(ss[i]) * inv_d + eps);
    const float g = du * w;
    const float dot = wave_sum(g * ov[i]);
    if (m < M) {
      gw[(long)m * d + col] = g;
      dn += du * ov[i] * r;
      if (lane == 0) rowdot[(long)m * (d / DU_EPI_TN) + blockIdx.y] = dot;
    }
  }
  cs[wave][lane] = dn;
  __syncthreads();
  if (wave == 0) dnw[(long)blockIdx.x * d + col] = dn_old + (cs[0][lane] + cs[1][lane] + cs[2][lane] + cs[3][lane]);
}

// The RMS-VJP inputs of du_epi_body as the tile epilogue of the GEMM of slice ZS (its accumulators
// stand for that slice; the other slices come from part), so the last du launch computes them and
// no separate pass over the slices is needed: du = slices summed in order z = 0..S-1, + lam dv_in;
// gw = du * w; rowdot[m, chunk] = the row's sum of gw * o over a 64-column chunk; dnw[slot][col] +=
// the sum over the slot's 16 rows, in row order, of du * o * r. Each thread takes 8 consecutive
// columns of a row and the 8 threads of a 64-column chunk are 8 consecutive lanes: the row's sums
// (of its head sums of squares, of gw * o) are a fixed xor-tree over those lanes, so every block
// width gives the same bits.
template <typename T, int S, int ZS, bool PRE = false> struct EpiDuFinal {
  static constexpr int TILE_ROWS = 32;
  static constexpr int CPT = 8, LPC = DU_EPI_TN / CPT;   // columns per thread, lanes per 64-column chunk
  static constexpr int NSS = MAX_HEADS / LPC;            // head-sum loads per thread
  // PRE (32 x 64 block tiles: each thread one row of 8 columns, one pass): the row's inputs are
  // gathered with the k-loop's last stage. The exact count of their load instructions (16-byte
  // loads and the head sums' dwords, which the compiler cannot merge):
  static constexpr int LATE_GATHERS = PRE ? 2 * (S - 1) + 2 + 2 * (int)(sizeof(T) / 2) + NSS : 0;
  int M, d, h;
  float inv_d, eps;
  const float* __restrict__ part;    // [S, M, d] split-K slices (slice ZS, this GEMM's, not read)
  const float* __restrict__ lamdv;   // [M, d]
  const T* __restrict__ o;           // [M, d]
  const float* __restrict__ ssq;     // [M, h]
  const T* __restrict__ normw;       // [d]
  float* __restrict__ gw;
  float* __restrict__ rowdot;
  float* __restrict__ dnw;
  struct TilePre {
    floatx4 pv[PRE ? S - 1 : 1][2], lv[2];
    Raw8<T> ov, wv;
    float ss[NSS];
  };
  DM_DEV TilePre tile_prefetch(int m0, int n0) const {
    TilePre pr;
    if constexpr (PRE) {
      const int t = threadIdx.x, pt = t % (64 / CPT) , r = t / (64 / CPT);
      const int mc = min(m0 + r, M - 1), col = n0 + pt * CPT;
      const long n = (long)M * d, idx = (long)mc * d + col;
      int zi = 0;
#pragma unroll
      for (int z = 0; z < S; ++z) {
        if (z == ZS) continue;
        pr.pv[zi][0] = ld_global<floatx4>(part + z * n + idx);
        pr.pv[zi][1] = ld_global<floatx4>(part + z * n + idx + 4);
        ++zi;
      }
      pr.lv[0] = ld_global<floatx4>(lamdv + idx);
      pr.lv[1] = ld_global<floatx4>(lamdv + idx + 4);
      pr.ov = ld8_global(o + idx);
      pr.wv = ld8_global(normw + col);
#pragma unroll
      for (int i = 0; i < NSS; ++i) pr.ss[i] = ssq[(long)mc * h + min(pt % LPC + i * LPC, h - 1)];
    }
    return pr;
  }
  template <int TR, int BN, int LDT>
  DM_DEV void tile_apply(const float* tile_in, int m0, int n0, const float*, const TilePre& pr, int) const {
    constexpr int P = BN / CPT, RPP = 256 / P;       // threads per row, rows per pass
    static_assert(BN % DU_EPI_TN == 0 && 256 % P == 0 && TR % RPP == 0 && TR % 16 == 0, "tile shape");
    static_assert(!PRE || (BN == 64 && TR == 32), "the gathered inputs cover one 32 x 64 pass");
    static_assert(MAX_HEADS % LPC == 0, "head sums split over a chunk's lanes");
    float* tile = const_cast<float*>(tile_in);  // the block's own LDS chunk: reused for du o r
    const int t = threadIdx.x, pt = t % P;
    const int c0 = pt * CPT, col = n0 + c0;
    const long n = (long)M * d;
    float wv[CPT];
    if constexpr (PRE) unpack8<T>(pr.wv, wv);
    else load_vec<T, CPT>(normw + col, wv);
#pragma unroll 1
    for (int r = t / P; r < TR; r += RPP) {
      const int m = m0 + r, mc = min(m, M - 1);
      const long idx = (long)mc * d + col;
      float pv[S][CPT], lv[CPT], ov[CPT], ssv[NSS];
      if constexpr (PRE) {
        int zi = 0;
#pragma unroll
        for (int z = 0; z < S; ++z) {
          if (z == ZS) continue;
          unpackf4(pr.pv[zi][0], pv[z]);
          unpackf4(pr.pv[zi][1], pv[z] + 4);
          ++zi;
        }
        unpackf4(pr.lv[0], lv);
        unpackf4(pr.lv[1], lv + 4);
        unpack8<T>(pr.ov, ov);
#pragma unroll
        for (int i = 0; i < NSS; ++i) ssv[i] = pr.ss[i];
      } else {
#pragma unroll
        for (int z = 0; z < S; ++z)
          if (z != ZS) load_vec<float, CPT>(part + z * n + idx, pv[z]);
        load_vec<float, CPT>(lamdv + idx, lv);
        load_vec<T, CPT>(o + idx, ov);
#pragma unroll
        for (int i = 0; i < NSS; ++i) ssv[i] = ssq[(long)mc * h + min(pt % LPC + i * LPC, h - 1)];
      }
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < NSS; ++i) ss += (pt % LPC + i * LPC < h) ? ssv[i] : 0.f;
#pragma unroll
      for (int j = 0; j < CPT; ++j) pv[ZS][j] = tile[r * LDT + c0 + j];
#pragma unroll
      for (int x = 1; x < LPC; x <<= 1) ss += __shfl_xor(ss, x, 64);
      const float rr = rsqrtf(ss * inv_d + eps);
      float g[CPT], dot = 0.f;
#pragma unroll
      for (int j = 0; j < CPT; ++j) {
        float du = pv[0][j];
#pragma unroll
        for (int z = 1; z < S; ++z) du += pv[z][j];
        du += lv[j];
        g[j] = du * wv[j];
        dot += g[j] * ov[j];
        tile[r * LDT + c0 + j] = m < M ? du * ov[j] * rr : 0.f;
      }
#pragma unroll
      for (int x = 1; x < LPC; x <<= 1) dot += __shfl_xor(dot, x, 64);
      if (m < M) {
        store_vec<float, CPT>(gw + (long)m * d + col, g);
        if (pt % LPC == 0) rowdot[(long)m * (d / DU_EPI_TN) + col / DU_EPI_TN] = dot;
      }
    }
    __syncthreads();
    // norm_ctx-weight partials: one thread per (16-row slot, column)
#pragma unroll 1
    for (int it = t; it < (TR / 16) * BN; it += 256) {
      const int sl = it / BN, cc = it % BN;
      if (m0 + 16 * sl >= M) continue;
      float sum = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) sum += tile[(16 * sl + i) * LDT + cc];
      float* dst = dnw + (long)((m0 + 16 * sl) / 16) * d + n0 + cc;
      *dst = *dst + sum;
    }
  }
};

template <typename T, int S>
static __global__ __launch_bounds__(256) void k_du_epi(int M, int d, int h, float inv_d, float eps,
                                                       const float* __restrict__ part,
                                                       const float* __restrict__ lamdv, const T* __restrict__ o,
                                                       const float* __restrict__ ssq, const T* __restrict__ normw,
                                                       float* __restrict__ gw, float* __restrict__ rowdot,
                                                       float* __restrict__ dnw) {
  du_epi_body<T, S>(M, d, h, inv_d, eps, part, lamdv, o, ssq, normw, gw, rowdot, dnw);
}


// ---------------------------------------------------------------------------
// attention VJP of one sweep, ATTN_BWD_ROLES blocks per (b, h), 4 waves x 16 rows each:
// role 0 the query-major half (dQ, the committed grads G / Dbar, the self column's dS
// summed into sdss), roles 1 and 2 the key-major half for one half of the keys each (dK, dV,
// the self column's dvraw, the refine VJP of those rows). Each block writes its own rows, so
// the blocks run concurrently.
// ---------------------------------------------------------------------------
template <typename T> struct AttnBwdArgs {
  CellGeom g;
  const T* qr; const T* kself; const T* vraw;          // layer buffers
  const T* Kin; const T* Vin; long in_stride; int in_row0;   // intra rows read by this sweep
  const T* o; const float* ssq;                        // this sweep's o [N, d], ssq [N, h]
  const float* gw; const float* rowdot; int nrd;       // RMS VJP inputs (k_du_epi)
  const float* docat;                                  // [B, Tbuf, d] upstream grad of o_cat, or nullptr
  const float* stat_m; const float* stat_z;            // [B*h, c] final row max / sum of the sweep
  const float* Mx;                                     // committed row max [B*h, c] or nullptr
  float* G; float* Dbar;                               // committed grads per layer-buffer row
  float* Mrow; int* klim;                              //   [B*h, Tbuf, DH], [B*h, Tbuf]; row max [B*h, Tbuf],
                                                       //   committed prefix length [Tbuf] (first sweep)
  CellRow* cellrow; int stack_K, stack_row0;          // [Tbuf] this cell's rows (first sweep), K, stack row
  int first;                                           // first reverse sweep: G / Dbar are written, else +=
  float scale, inv_d, eps;
  float* dkself; float* dvraw; float* dq;              // layer accumulators [B, h, Tbuf, DH] (+=)
  // [B*h, Tbuf] (+=): the self column's dS summed over the sweeps. Its dq and dkself terms,
  // scale dS_self k_self and scale dS_self q, have the same k_self / q in every sweep, so the
  // projection VJP applies them once from this sum (no per-sweep dq / dkself round trip).
  float* sdss;
  // sweep >= 1 (fuse_refine): the grads of the intra rows are those of the previous sweep's
  // refined rows; the key-major blocks run that sweep's refine VJP on them (ref). Sweep 0:
  // the intra rows are the raw rows, their grads go to dkself / dvraw.
  int fuse_refine;
  RefineBwdArgs<T> ref;
  // the cell's last reverse sweep: G is complete after it; the query-major blocks also store it
  // rounded to the storage dtype, the committed VJPs' MFMA operand (nullptr: other sweeps)
  T* Gb = nullptr;
};

constexpr int ATTN_BWD_ROLES = 3;   // blocks per (b, h) of the attention VJP (grid x)

template <typename T, int DH> struct AttnBwdCfg {
  static constexpr int PAD = 16 / (int)sizeof(T);
  static constexpr int LDE = DH + PAD;     // rows over head_dim
  static constexpr int LDI = 64 + PAD;     // rows over the 64 queries / keys
  // four [64][LDE] row-major tiles (Q, K, V, dO or G) + a per-wave stage [4][16][LDI]
  static constexpr int LDS_ELEMS = 4 * 64 * LDE + 4 * 16 * LDI;
  // k_attn_bwd: + the self column's dv_raw terms of the block's 32 key rows, fp32 [32][DH], where
  // that fits the 160 KB of LDS (all but fp32 at head_dim 128)
  static constexpr size_t PD_BYTES = 32 * DH * 4;
  static constexpr bool PD_LDS = (size_t)LDS_ELEMS * sizeof(T) + PD_BYTES <= 160 * 1024;
  static constexpr size_t BWD_LDS_BYTES = (size_t)LDS_ELEMS * sizeof(T) + (PD_LDS ? PD_BYTES : 0);
};

// L: the block's linear id in its grid of ATTN_BWD_ROLES x BH blocks
template <typename T, int DH>
DM_DEV void attn_bwd_body(const AttnBwdArgs<T>& a, int L, int nbh) {
  using C = AttnBwdCfg<T, DH>;
  constexpr int LDE = C::LDE, LDI = C::LDI, NDT = DH / 16;
  extern __shared__ __attribute__((aligned(16))) char smem_raw[];
  T* Qs = reinterpret_cast<T*>(smem_raw);
  T* Ks = Qs + 64 * LDE;
  T* Vs = Ks + 64 * LDE;
  T* dOs = Vs + 64 * LDE;
  T* Wst = dOs + 64 * LDE;
  __shared__ float sM[64], sZ[64], sD[64];

  const CellGeom& g = a.g;
  // Three blocks per (b, h): role 0 the query-major half, roles 1 and 2 the key-major half for
  // keys [0, 32) and [32, 64) (each stages every row, computes its keys' dK / dV and runs their
  // refine VJP). The roles of one (b, h) read the same inputs, so they get blocks on the same XCD
  // (blocks go round-robin over the 8 XCDs by linear id, x fastest): in each run of 24 linear
  // ids, ids k, k + 8 and k + 16 are the roles of one (b, h); a last partial run takes them in
  // turn.
  int role, bh;
  {
    const int full = (nbh / 8) * 8 * ATTN_BWD_ROLES;
    if (L < full) {
      role = (L % (8 * ATTN_BWD_ROLES)) >> 3;
      bh = 8 * (L / (8 * ATTN_BWD_ROLES)) + (L & 7);
    } else {
      role = (L - full) % ATTN_BWD_ROLES;
      bh = full / ATTN_BWD_ROLES + (L - full) / ATTN_BWD_ROLES;
    }
  }
  const int kh = role - 1;   // key roles: the key half (rows 32 kh .. 32 kh + 31)
  const int b = bh / g.h, hh = bh - b * g.h;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g4 = lane >> 4, lc = lane & 15;
  const int d = g.d, c = g.c;
  const int wl = intra_wlim(g.window);   // intra keys at most wl rows before the query
  const long lrow0 = (long)bh * g.Tbuf + g.buf_t0;
  // the wave's own 16 rows of staging: written and read by that wave only (LDS
  // operations of one wave complete in order, so no workgroup barrier is needed)
  T* W = Wst + wave * 16 * LDI;

  // ---- phase 1: 4 threads per row i build dO, D, stage Q / K / V / dO, self column
  {
    constexpr int EPT = DH / 4;          // elements per thread
    const int i = tid >> 2, part = tid & 3, e0 = part * EPT;
    const bool ok = i < c;
    const int ic = ok ? i : 0;
    const long n = (long)b * c + ic;                      // row of the sweep arrays
    float q[EPT], kv[EPT], vv[EPT], ks[EPT], vr[EPT], ov[EPT], gwv[EPT], dc[EPT];
    load_vec<T, EPT>(a.qr + (lrow0 + ic) * DH + e0, q);
    // a key role reads K / V rows (its keys) and the raw self pair (its rows' self column) of its
    // own key half only; a wave's 16 rows lie in one half, so this is uniform over the wave
    const bool own = role == 0 || (i >> 5) == kh;
    if (own) {
      load_vec<T, EPT>(a.Kin + (long)bh * a.in_stride + (long)(a.in_row0 + ic) * DH + e0, kv);
      load_vec<T, EPT>(a.Vin + (long)bh * a.in_stride + (long)(a.in_row0 + ic) * DH + e0, vv);
      load_vec<T, EPT>(a.kself + (lrow0 + ic) * DH + e0, ks);
      load_vec<T, EPT>(a.vraw + (lrow0 + ic) * DH + e0, vr);
    } else {
#pragma unroll
      for (int e = 0; e < EPT; ++e) { kv[e] = 0.f; vv[e] = 0.f; ks[e] = 0.f; vr[e] = 0.f; }
    }
    load_vec<T, EPT>(a.o + n * d + hh * DH + e0, ov);
    load_vec<float, EPT>(a.gw + n * d + hh * DH + e0, gwv);
    if (a.docat != nullptr) {
      load_vec<float, EPT>(a.docat + ((long)b * g.Tbuf + g.buf_t0 + ic) * d + hh * DH + e0, dc);
    } else {
#pragma unroll
      for (int e = 0; e < EPT; ++e) dc[e] = 0.f;
    }
    // the accumulators' current values, loaded with the inputs (one memory round trip)
    const long lr = (lrow0 + ic) * DH + e0;
    float acc1[EPT], gold[EPT];
    float dbold = 0.f, mx = 0.f, sdold = 0.f;
    if (role == 0) {
      sdold = a.sdss[lrow0 + ic];
      if (a.Mx != nullptr) {
        mx = a.Mx[(long)bh * c + ic];
        load_vec<float, EPT>(a.G + lr, gold);
        dbold = a.Dbar[lrow0 + ic];
      }
    } else if ((i >> 5) == kh && !(C::PD_LDS && a.fuse_refine)) {
      load_vec<float, EPT>(a.dvraw + lr, acc1);
    }
    float ss = 0.f, dot = 0.f;
    if ((g.h & 15) == 0 && (a.nrd & 15) == 0) {   // 16-byte loads: a quarter of the load instructions
      ss = sum_quads<MAX_HEADS / 16>(a.ssq + n * g.h, part, g.h);
      dot = sum_quads<MAX_ROWDOT / 16>(a.rowdot + n * a.nrd, part, a.nrd);
    } else {
      ss = sum_strided<MAX_HEADS / 4>(a.ssq + n * g.h, part, g.h, 4);
      dot = sum_strided<MAX_ROWDOT / 4>(a.rowdot + n * a.nrd, part, a.nrd, 4);
    }
    ss += __shfl_xor(ss, 1, 64); ss += __shfl_xor(ss, 2, 64);
    dot += __shfl_xor(dot, 1, 64); dot += __shfl_xor(dot, 2, 64);
    const float r = rsqrtf(ss * a.inv_d + a.eps);
    const float c3 = r * r * r * a.inv_d * dot;
    const float Mi = ok ? a.stat_m[(long)bh * c + i] : 0.f;
    const float Zi = ok ? a.stat_z[(long)bh * c + i] : 1.f;
    float dO[EPT], Dp = 0.f, sq = 0.f, dov = 0.f;
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      dO[e] = ok ? r * gwv[e] - ov[e] * c3 + dc[e] : 0.f;
      dO[e] = to_f(from_f<T>(dO[e]));    // the value the MFMA products use
      Dp += dO[e] * ov[e];
      sq += q[e] * ks[e];
      dov += dO[e] * vr[e];
    }
    Dp += __shfl_xor(Dp, 1, 64); Dp += __shfl_xor(Dp, 2, 64);
    sq += __shfl_xor(sq, 1, 64); sq += __shfl_xor(sq, 2, 64);
    dov += __shfl_xor(dov, 1, 64); dov += __shfl_xor(dov, 2, 64);
    // raw self column: p_self = exp(s_self - M) / Z, dS_self = p_self (dO.v_raw - D)
    const float ps = ok ? __expf(sq * a.scale - Mi) / Zi : 0.f;
    const float dss = ps * (dov - Dp);
    if (part == 0) { sM[i] = Mi; sZ[i] = Zi; sD[i] = Dp; }
    // committed part: alpha = exp(m_comm - M) / Z
    if (role == 0 && a.Mx != nullptr && ok) {
      const float alpha = __expf(mx - Mi) / Zi;
      float gn[EPT];
#pragma unroll
      for (int e = 0; e < EPT; ++e) gn[e] = (a.first ? 0.f : gold[e]) + alpha * dO[e];
      store_vec<float, EPT>(a.G + lr, gn);
      if (a.Gb != nullptr) store_vec<T, EPT>(a.Gb + lr, gn);
      if (part == 0) {
        a.Dbar[lrow0 + i] = (a.first ? 0.f : dbold) + alpha * Dp;
        if (a.first) a.Mrow[lrow0 + i] = mx;
      }
    }
    if (role == 0 && a.first && bh == 0 && part == 0 && ok) {
      a.klim[g.buf_t0 + i] = g.pos0;
      a.cellrow[g.buf_t0 + i] = CellRow{g.pos0, c, a.stack_K, a.stack_row0};
    }
    if (ok) {
      if (role == 0) {
        if (part == 0) a.sdss[lrow0 + i] = sdold + dss;
      } else if ((i >> 5) == kh) {
        if (C::PD_LDS && a.fuse_refine) {
          // the refine VJP of these rows adds to the same dv_raw rows: it takes this term from
          // LDS, so dv_raw is read (early, with its other inputs) and written once
          float* pd = reinterpret_cast<float*>(smem_raw + (size_t)C::LDS_ELEMS * sizeof(T)) + (i - 32 * kh) * DH + e0;
#pragma unroll
          for (int e = 0; e < EPT; ++e) pd[e] = ps * dO[e];
        } else {
#pragma unroll
          for (int e = 0; e < EPT; ++e) acc1[e] += ps * dO[e];
          store_vec<float, EPT>(a.dvraw + lr, acc1);
        }
      }
    } else {
#pragma unroll
      for (int e = 0; e < EPT; ++e) { q[e] = 0.f; kv[e] = 0.f; vv[e] = 0.f; }
    }
    store_vec<T, EPT>(Qs + i * LDE + e0, q);
    store_vec<T, EPT>(Ks + i * LDE + e0, kv);
    store_vec<T, EPT>(Vs + i * LDE + e0, vv);
    store_vec<T, EPT>(dOs + i * LDE + e0, dO);
  }
  __syncthreads();

  // ---- phase 2: query-major (rows i = 16 wave + ..): dS, then dQ = dS . K
  if (role == 0) {
    float dqo[4][NDT];   // dq rows after phase 1, loaded before the products
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int ic = min(16 * wave + 4 * g4 + r, c - 1);
#pragma unroll
      for (int t = 0; t < NDT; ++t) dqo[r][t] = a.dq[(lrow0 + ic) * DH + 16 * t + lc];
    }
    floatx4 S[4], dP[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) { S[t] = zero4(); dP[t] = zero4(); }
    wave_mma<T, DH, 4>(Qs + 16 * wave * LDE, LDE, Ks, LDE, S);
    wave_mma<T, DH, 4>(dOs + 16 * wave * LDE, LDE, Vs, LDE, dP);
    // exponentials for every element, then masked (a masked exponential would
    // become a branch); 1 / Z once per row
    float Mr[4], rZ[4], Dr[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = 16 * wave + 4 * g4 + r;
      Mr[r] = sM[i]; rZ[r] = 1.f / sZ[i]; Dr[r] = sD[i];
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int il = 4 * g4 + r, i = 16 * wave + il;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int j = 16 * t + lc;
        const float e = __expf(S[t][r] * a.scale - Mr[r]) * rZ[r];
        W[il * LDI + j] = from_f<T>((j < i && i - j <= wl && i < c ? e : 0.f) * (dP[t][r] - Dr[r]));
      }
    }
    floatx4 dQ[NDT];
#pragma unroll
    for (int t = 0; t < NDT; ++t) dQ[t] = zero4();
    wave_mma_bt<T, 64, NDT>(W, LDI, Ks, LDE, dQ);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = 16 * wave + 4 * g4 + r;
      if (i >= c) continue;
#pragma unroll
      for (int t = 0; t < NDT; ++t) a.dq[(lrow0 + i) * DH + 16 * t + lc] = dqo[r][t] + a.scale * dQ[t][r];
    }
  }
  // ---- phase 3: key-major (rows j = 16 wave + ..): P^T, dS^T -> dV = P^T dO, dK = dS^T Q.
  // The block's key half is waves 2 kh and 2 kh + 1 (wave-uniform); the other two waves only
  // take part in the barriers and the refine items.
  else {
    const bool mine = (wave >> 1) == kh;
    // sweep >= 1: the thread's first refine item's inputs (the forward state and the dk_raw /
    // dv_raw accumulators, whose phase-1 writes, if any, are behind the barrier above), gathered
    // before the products so their latency overlaps them
    constexpr int Q = DH / 8;
    const int n_items = a.fuse_refine ? max(0, min(c - 32 * kh, 32)) * Q : 0;
    RefineIn in0;
    if (tid < n_items) in0 = refine_gather<T, DH>(a.ref, b * c + 32 * kh + tid / Q, hh, 4 * (tid % Q));
    // sweep 0: the dkself rows and the dvraw rows after phase 1, loaded before the products
    float dko[4][NDT], dvo[4][NDT];
    if (!a.fuse_refine && mine) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int jc = min(16 * wave + 4 * g4 + r, c - 1);
#pragma unroll
        for (int t = 0; t < NDT; ++t) {
          dko[r][t] = a.dkself[(lrow0 + jc) * DH + 16 * t + lc];
          dvo[r][t] = a.dvraw[(lrow0 + jc) * DH + 16 * t + lc];
        }
      }
    }
    floatx4 dV[NDT], dK[NDT];
#pragma unroll
    for (int t = 0; t < NDT; ++t) { dV[t] = zero4(); dK[t] = zero4(); }
    if (mine) {
      floatx4 St[4], dPt[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) { St[t] = zero4(); dPt[t] = zero4(); }
      wave_mma<T, DH, 4>(Ks + 16 * wave * LDE, LDE, Qs, LDE, St);
      wave_mma<T, DH, 4>(Vs + 16 * wave * LDE, LDE, dOs, LDE, dPt);
      float Mq[4], rZq[4], Dq[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int i = 16 * t + lc;
        Mq[t] = sM[i]; rZq[t] = 1.f / sZ[i]; Dq[t] = sD[i];
      }
      float Pt[4][4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int i = 16 * t + lc;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int j = 16 * wave + 4 * g4 + r;
          const float e = __expf(St[t][r] * a.scale - Mq[t]) * rZq[t];
          Pt[t][r] = (j < i && i - j <= wl && i < c) ? e : 0.f;
          W[(4 * g4 + r) * LDI + i] = from_f<T>(Pt[t][r]);
        }
      }
      wave_mma_bt<T, 64, NDT>(W, LDI, dOs, LDE, dV);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int i = 16 * t + lc;
#pragma unroll
        for (int r = 0; r < 4; ++r) W[(4 * g4 + r) * LDI + i] = from_f<T>(Pt[t][r] * (dPt[t][r] - Dq[t]));
      }
      wave_mma_bt<T, 64, NDT>(W, LDI, Qs, LDE, dK);
    }
    if (a.fuse_refine) {
      // the grads stay on chip: staged in LDS over the Q / K / V / dO tiles once every wave is
      // done with them, then one refine item (row, 4 RoPE pairs) per thread at a time
      constexpr int LDF = DH + 4;
      static_assert(2 * 64 * LDF * 4 <= C::LDS_ELEMS * (int)sizeof(T), "grad staging fits the tiles");
      float* dKs = reinterpret_cast<float*>(smem_raw);
      float* dVs = dKs + 64 * LDF;
      __syncthreads();
      if (mine) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int j = 16 * wave + 4 * g4 + r;
#pragma unroll
          for (int t = 0; t < NDT; ++t) {
            dKs[j * LDF + 16 * t + lc] = a.scale * dK[t][r];
            dVs[j * LDF + 16 * t + lc] = dV[t][r];
          }
        }
      }
      __syncthreads();
      // Items it = tid + 256 k over the block's key rows: row 32 kh + it / Q, pairs 4 (it % Q);
      // a row's items are Q consecutive lanes. One item per thread at a time: with two in
      // flight the kernel needs more than 256 registers a lane and a CU holds one block
      // instead of two. The first item's inputs were gathered before the products.
      const float* pds = reinterpret_cast<const float*>(smem_raw + (size_t)C::LDS_ELEMS * sizeof(T));
      auto apply = [&](int it, RefineIn& in) {
        const int j = 32 * kh + it / Q, jj = 4 * (it % Q);
        const float* kr = dKs + j * LDF + jj;
        const float* vr = dVs + j * LDF + jj;
        RefineGrad4 gr;
        unpackf4(*reinterpret_cast<const floatx4*>(kr), gr.ka);
        unpackf4(*reinterpret_cast<const floatx4*>(kr + DH / 2), gr.kb);
        unpackf4(*reinterpret_cast<const floatx4*>(vr), gr.va);
        unpackf4(*reinterpret_cast<const floatx4*>(vr + DH / 2), gr.vb);
        if constexpr (C::PD_LDS) {   // the self column's dv_raw term of the row (phase 1)
          const float* pd = pds + (j - 32 * kh) * DH + jj;
          float p1[4], p2[4];
          unpackf4(*reinterpret_cast<const floatx4*>(pd), p1);
          unpackf4(*reinterpret_cast<const floatx4*>(pd + DH / 2), p2);
#pragma unroll
          for (int e = 0; e < 4; ++e) { in.ovr1[e] += p1[e]; in.ovr2[e] += p2[e]; }
        }
        refine_apply<T, DH>(a.ref, b * c + j, hh, jj, in, gr);
      };
      if (tid < n_items) apply(tid, in0);
      for (int it = tid + 256; it < n_items; it += 256) {
        RefineIn in = refine_gather<T, DH>(a.ref, b * c + 32 * kh + it / Q, hh, 4 * (it % Q));
        apply(it, in);
      }
      return;
    }
    if (!mine) return;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int j = 16 * wave + 4 * g4 + r;
      if (j >= c) continue;
#pragma unroll
      for (int t = 0; t < NDT; ++t) {
        const int e = 16 * t + lc;
        a.dkself[(lrow0 + j) * DH + e] = dko[r][t] + a.scale * dK[t][r];
        a.dvraw[(lrow0 + j) * DH + e] = dvo[r][t] + dV[t][r];
      }
    }
  }
}

// head_dim 64: at most 256 registers a lane, two blocks per CU
template <typename T, int DH>
static __global__ __launch_bounds__(256, DH == 64 ? 2 : 1) void k_attn_bwd(AttnBwdArgs<T> a) {
  attn_bwd_body<T, DH>(a, (int)blockIdx.x + ATTN_BWD_ROLES * (int)blockIdx.y, (int)gridDim.y);
}

// ---------------------------------------------------------------------------
// committed-prefix VJP. Every query row i of a cell at pos0 > 0 attends the
// committed keys j < klim_i = pos0 with E_ij = exp(scale q_i . k_j - Mx_i) and
//   dS_ij = E_ij (G_i . v_j - Dbar_i),
//   dq_i += scale sum_j dS_ij k_j,  dK_j += scale sum_i dS_ij q_i,  dV_j += sum_i E_ij G_i,
// with G_i, Dbar_i, Mx_i kept per row by the attention VJP. The key side runs per
// key cell right before that cell's sweep VJP (its rows are in the prefix of every
// later row, so the sum is complete and is written once); the query side runs
// once per layer after every cell.
// ---------------------------------------------------------------------------
// query splits of the key side (partial slots summed by k_refine_bwd): 8 when B*h leaves the 4-split
// grid at one block per CU (64 heads: 256 blocks), else 4
inline int comm_nsq(int BH) { return BH <= 64 ? 8 : 4; }

template <typename T> struct CommKeyArgs {
  int B, h, Tbuf, cache_T;
  int k0, kc;                                  // key cell: cache rows [k0, k0 + kc)
  int q_lo, q_hi;                              // query rows [q_lo, q_hi) of the layer buffers
  const T* qr; const T* Kc; const T* Vc;       // layer buffer q_r; the cache rows
  const T* Gb; const float* Dbar; const float* Mx;   // per layer-buffer row (see AttnBwdArgs; G complete,
                                                     // in the storage dtype)
  float scale;
  float* dKp; float* dVp;                      // [nsq, B*h, CMAX, DH] partial sums per split
  // grad-cache form (dKg != nullptr): block x takes keys [64 x, min(64 x + 64, k0)) of the committed
  // prefix [0, k0) against every query row [q_lo, q_hi) and ADDS into the fp32 grad cache
  // dKg / dVg [B*h, cache_T, DH] (engines/wavescan/engine/backward.py:116-119)
  float* dKg = nullptr; float* dVg = nullptr;
  int window = 0;   // local_window W: query row i reads keys >= i - W + 1 (0: none)
  int nsq = 4;      // query splits (comm_nsq)
  int s0 = 0;       // split of block x = 0 (a launch may cover some splits only)
};

// One block per (query split s, b, h). Split 0 takes the first 64-row query tile (the rows right
// after the key cell: the last to be complete in the reverse scan), split s >= 1 the tiles
// s, s + (nsq - 1), .. (the rest, complete a cell earlier): a layer's backward can compute those
// while the cell before is still running. Wave w owns keys 16w .. 16w + 15 of the cell
// (key-major products, as in k_attn_bwd). In the grad-cache form one block per (64-key tile,
// b, h) takes every query tile.
template <typename T, int DH>
DM_DEV void comm_dkv_body(const CommKeyArgs<T>& a, int bx, int bh) {
  using C = AttnBwdCfg<T, DH>;
  constexpr int LDE = C::LDE, LDI = C::LDI, NDT = DH / 16;
  extern __shared__ __attribute__((aligned(16))) char smem_raw[];
  T* Ks = reinterpret_cast<T*>(smem_raw);
  T* Vs = Ks + 64 * LDE;
  T* Qs = Vs + 64 * LDE;
  T* Gs = Qs + 64 * LDE;
  T* Wst = Gs + 64 * LDE;
  __shared__ float sM[64], sD[64];

  const bool gcache = a.dKg != nullptr;   // uniform
  const int s = gcache ? 0 : a.s0 + bx;
  const int k0 = gcache ? 64 * bx : a.k0;
  const int kc = gcache ? min(64, a.k0 - k0) : a.kc;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g4 = lane >> 4, lc = lane & 15;
  // the wave's own 16 rows of staging (LDS operations of one wave complete in order)
  T* W = Wst + wave * 16 * LDI;
  const long qrow0 = (long)bh * a.Tbuf;
  constexpr int EPT = DH / 4;
  constexpr int VT = 16 / (int)sizeof(T), NW = EPT / VT;   // 16-byte words per thread and row
  const int ri = tid >> 2, re0 = (tid & 3) * EPT;
  // with a window, query rows past k0 + kc + W - 2 see none of these keys
  const int q_hi = a.window > 0 ? max(a.q_lo, min(a.q_hi, k0 + kc + a.window - 1)) : a.q_hi;
  const int ntile = (q_hi - a.q_lo + 63) / 64;
  const int step = gcache ? 1 : (s == 0 ? ntile : a.nsq - 1);   // query tiles of this block: s, s + step, ..
  const int wlim = a.window > 0 ? a.window - 1 : (1 << 30);   // largest query - key distance read

  // the cell's keys and values, row-wise (A operands of the key-major products)
  {
    const bool ok = ri < kc;
    const long row = ((long)bh * a.cache_T + k0 + (ok ? ri : 0)) * DH + re0;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      *reinterpret_cast<uint4*>(Ks + ri * LDE + re0 + w * VT) =
          keep_if(*reinterpret_cast<const uint4*>(a.Kc + row + w * VT), ok);
      *reinterpret_cast<uint4*>(Vs + ri * LDE + re0 + w * VT) =
          keep_if(*reinterpret_cast<const uint4*>(a.Vc + row + w * VT), ok);
    }
  }
  // query tile rows: q, G (raw words), row max, Dbar into registers, then LDS; rows
  // past the end are zeroed when staged (a select on a loaded value right after
  // its load would make the compiler wait for the load there)
  uint4 qv[NW], gw[NW];
  float mv, dv;
  bool tok = false;
  auto load_tile = [&](int t) {
    const int i0 = a.q_lo + 64 * t;
    tok = ri < q_hi - i0;
    const long r = qrow0 + i0 + (tok ? ri : 0);
#pragma unroll
    for (int w = 0; w < NW; ++w) qv[w] = *reinterpret_cast<const uint4*>(a.qr + r * DH + re0 + w * VT);
#pragma unroll
    for (int w = 0; w < NW; ++w) gw[w] = *reinterpret_cast<const uint4*>(a.Gb + r * DH + re0 + w * VT);
    mv = a.Mx[r];
    dv = a.Dbar[r];
  };
  floatx4 dK[NDT], dV[NDT];
#pragma unroll
  for (int t = 0; t < NDT; ++t) { dK[t] = zero4(); dV[t] = zero4(); }
  if (s < ntile) load_tile(s);
  for (int t = s; t < ntile; t += step) {
    const int nq = min(64, q_hi - (a.q_lo + 64 * t));
    const int dqk = a.q_lo + 64 * t - k0;   // query row i - key row j = dqk + i - j
    __syncthreads();   // the previous tile's readers are done (first pass: publishes K / V)
#pragma unroll
    for (int w = 0; w < NW; ++w) *reinterpret_cast<uint4*>(Qs + ri * LDE + re0 + w * VT) = keep_if(qv[w], tok);
#pragma unroll
    for (int w = 0; w < NW; ++w) *reinterpret_cast<uint4*>(Gs + ri * LDE + re0 + w * VT) = keep_if(gw[w], tok);
    if ((tid & 3) == 0) { sM[ri] = tok ? mv : 0.f; sD[ri] = tok ? dv : 0.f; }
    __syncthreads();
    if (t + step < ntile) load_tile(t + step);
    // key-major: E^T, dS^T (rows j = 16 wave + .., columns i = queries) -> dV += E^T G, dK += dS^T Q
    floatx4 St[4], dPt[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) { St[u] = zero4(); dPt[u] = zero4(); }
    wave_mma<T, DH, 4>(Ks + 16 * wave * LDE, LDE, Qs, LDE, St);
    wave_mma<T, DH, 4>(Vs + 16 * wave * LDE, LDE, Gs, LDE, dPt);
    // the row values are read before the exponentials, which are computed for every
    // element and then masked (a masked exponential with its LDS read would become
    // a branch that waits for that read)
    float mq[4], dq[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) { mq[u] = sM[16 * u + lc]; dq[u] = sD[16 * u + lc]; }
    float Et[4][4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = 16 * u + lc;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int j = 16 * wave + 4 * g4 + r;
        const float e = __expf(St[u][r] * a.scale - mq[u]);
        Et[u][r] = (j < kc && i < nq && dqk + i - j <= wlim) ? e : 0.f;
        W[(4 * g4 + r) * LDI + i] = from_f<T>(Et[u][r]);
      }
    }
    wave_mma_bt<T, 64, NDT>(W, LDI, Gs, LDE, dV);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = 16 * u + lc;
#pragma unroll
      for (int r = 0; r < 4; ++r) W[(4 * g4 + r) * LDI + i] = from_f<T>(Et[u][r] * (dPt[u][r] - dq[u]));
    }
    wave_mma_bt<T, 64, NDT>(W, LDI, Qs, LDE, dK);
  }
  if (gcache) {
    // add into the grad cache rows of the tile: every current value loaded first
    const long grow = (long)bh * a.cache_T + k0;
    float ok_[4][NDT], ov_[4][NDT];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int jc = min(16 * wave + 4 * g4 + r, kc - 1);
#pragma unroll
      for (int t = 0; t < NDT; ++t) {
        ok_[r][t] = a.dKg[(grow + jc) * DH + 16 * t + lc];
        ov_[r][t] = a.dVg[(grow + jc) * DH + 16 * t + lc];
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int j = 16 * wave + 4 * g4 + r;
      if (j >= kc) continue;
#pragma unroll
      for (int t = 0; t < NDT; ++t) {
        a.dKg[(grow + j) * DH + 16 * t + lc] = ok_[r][t] + a.scale * dK[t][r];
        a.dVg[(grow + j) * DH + 16 * t + lc] = ov_[r][t] + dV[t][r];
      }
    }
    return;
  }
  const long slot = ((long)s * a.B * a.h + bh) * CMAX;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int j = 16 * wave + 4 * g4 + r;
    if (j >= kc) continue;
#pragma unroll
    for (int t = 0; t < NDT; ++t) {
      a.dKp[(slot + j) * DH + 16 * t + lc] = a.scale * dK[t][r];
      a.dVp[(slot + j) * DH + 16 * t + lc] = dV[t][r];
    }
  }
}

template <typename T, int DH>
static __global__ __launch_bounds__(256) void k_comm_dkv(CommKeyArgs<T> a) {
  comm_dkv_body<T, DH>(a, blockIdx.x, blockIdx.y);
}

// The attention VJP launch (ATTN_BWD_ROLES x nbh blocks) with some key-side committed-VJP splits
// of the cell before this one as extra blocks (ka.s0 .., nbh blocks each; one dynamic LDS object)
template <typename T, int DH>
static __global__ __launch_bounds__(256, DH == 64 ? 2 : 1) void k_attn_bwd_dkv(AttnBwdArgs<T> a, CommKeyArgs<T> ka,
                                                                             int nbh) {
  const int L = blockIdx.x, na = ATTN_BWD_ROLES * nbh;
  if (L < na) attn_bwd_body<T, DH>(a, L, nbh);
  else comm_dkv_body<T, DH>(ka, (L - na) / nbh, (L - na) % nbh);
}

template <typename T> struct CommQueryArgs {
  int B, h, Tbuf, cache_T, nrows;              // query rows [row0, nrows)
  const int* klim;                             // [Tbuf] committed prefix length of each row (0: none)
  const T* qr; const T* Kc; const T* Vc;
  const T* Gb; const float* Dbar; const float* Mx;   // per layer-buffer row (see CommKeyArgs)
  float scale;
  float* dq;                                   // [B*h, Tbuf, DH] (+=)
  int row0 = 0;                                // first query row (a multiple of 64 or one cell's start)
  int window = 0;                              // local_window W: row i reads keys >= i - W + 1 (0: none)
};

// One block per (b, h, 64-row query tile), the tiles with the longest prefixes
// first; wave w owns query rows 16w .. 16w + 15 (query-major products).
template <typename T, int DH>
DM_DEV void comm_dq_body(const CommQueryArgs<T>& a) {
  using C = AttnBwdCfg<T, DH>;
  constexpr int LDE = C::LDE, LDI = C::LDI, NDT = DH / 16;
  extern __shared__ __attribute__((aligned(16))) char smem_raw[];
  T* Qs = reinterpret_cast<T*>(smem_raw);
  T* Gs = Qs + 64 * LDE;
  T* Ks = Gs + 64 * LDE;
  T* Vs = Ks + 64 * LDE;
  T* Wst = Vs + 64 * LDE;
  __shared__ float sM[64], sD[64];
  __shared__ int sL[64];

  const int bh = blockIdx.x;
  const int i0 = a.row0 + 64 * ((int)gridDim.y - 1 - (int)blockIdx.y);
  const int nq = min(64, a.nrows - i0);
  const int k_end = a.klim[i0 + nq - 1];   // the prefix lengths do not decrease along the rows
  if (k_end <= 0) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g4 = lane >> 4, lc = lane & 15;
  T* W = Wst + wave * 16 * LDI;   // the wave's own rows (LDS operations of one wave complete in order)
  const long qrow0 = (long)bh * a.Tbuf + i0;
  const T* Kb = a.Kc + (long)bh * a.cache_T * DH;
  const T* Vb = a.Vc + (long)bh * a.cache_T * DH;
  constexpr int EPT = DH / 4;
  constexpr int VT = 16 / (int)sizeof(T), NW = EPT / VT;
  const int ri = tid >> 2, re0 = (tid & 3) * EPT;
  {
    const bool ok = ri < nq;
    const long r = qrow0 + (ok ? ri : 0);
    uint4 gg[NW];
#pragma unroll
    for (int w = 0; w < NW; ++w) gg[w] = *reinterpret_cast<const uint4*>(a.Gb + r * DH + re0 + w * VT);
#pragma unroll
    for (int w = 0; w < NW; ++w)
      *reinterpret_cast<uint4*>(Qs + ri * LDE + re0 + w * VT) =
          keep_if(*reinterpret_cast<const uint4*>(a.qr + r * DH + re0 + w * VT), ok);
    const int L = ok ? a.klim[i0 + ri] : 0;
    // no committed prefix (or past the end): contributes nothing
#pragma unroll
    for (int w = 0; w < NW; ++w) *reinterpret_cast<uint4*>(Gs + ri * LDE + re0 + w * VT) = keep_if(gg[w], L != 0);
    if ((tid & 3) == 0) {
      sM[ri] = L > 0 ? a.Mx[r] : 0.f;
      sD[ri] = L > 0 ? a.Dbar[r] : 0.f;
      sL[ri] = L;
    }
  }
  floatx4 dQ[NDT];
#pragma unroll
  for (int t = 0; t < NDT; ++t) dQ[t] = zero4();
  // the lane's rows' prefix length, row max and Dbar, read once (published by the
  // first tile's barrier)
  int lq[4] = {0, 0, 0, 0};
  float mq[4], dq[4];
  // the next key tile in registers (raw words; rows past the end zeroed when staged)
  uint4 kv[NW], vv[NW];
  auto load_keys = [&](int k0) {
    const int j = min(ri, k_end - k0 - 1);
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      kv[w] = *reinterpret_cast<const uint4*>(Kb + (long)(k0 + j) * DH + re0 + w * VT);
      vv[w] = *reinterpret_cast<const uint4*>(Vb + (long)(k0 + j) * DH + re0 + w * VT);
    }
  };
  // with a window the tile's first row reads keys from i0 - W + 1 on (later rows masked below)
  const int k_lo = a.window > 0 ? max(0, i0 - a.window + 1) : 0;
  const int wlim = a.window > 0 ? a.window - 1 : (1 << 30);
  load_keys(k_lo);
  for (int k0 = k_lo; k0 < k_end; k0 += 64) {
    const bool kok = ri < k_end - k0;
    __syncthreads();   // the previous tile's readers are done (first pass: publishes Q / G)
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      *reinterpret_cast<uint4*>(Ks + ri * LDE + re0 + w * VT) = keep_if(kv[w], kok);
      *reinterpret_cast<uint4*>(Vs + ri * LDE + re0 + w * VT) = keep_if(vv[w], kok);
    }
    __syncthreads();
    if (k0 == k_lo) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 16 * wave + 4 * g4 + r;
        lq[r] = sL[i]; mq[r] = sM[i]; dq[r] = sD[i];
      }
    }
    if (k0 + 64 < k_end) load_keys(k0 + 64);
    floatx4 S[4], dP[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) { S[t] = zero4(); dP[t] = zero4(); }
    wave_mma<T, DH, 4>(Qs + 16 * wave * LDE, LDE, Ks, LDE, S);
    wave_mma<T, DH, 4>(Gs + 16 * wave * LDE, LDE, Vs, LDE, dP);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int il = 4 * g4 + r;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int j = k0 + 16 * t + lc;
        const float e = __expf(S[t][r] * a.scale - mq[r]);
        const bool keep = j < lq[r] && i0 + 16 * wave + il - j <= wlim;
        W[il * LDI + 16 * t + lc] = from_f<T>((keep ? e : 0.f) * (dP[t][r] - dq[r]));
      }
    }
    wave_mma_bt<T, 64, NDT>(W, LDI, Ks, LDE, dQ);
  }
  // dq rows: every current value loaded first, then the sums stored
  float old[4][NDT];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int ic = min(16 * wave + 4 * g4 + r, nq - 1);
#pragma unroll
    for (int t = 0; t < NDT; ++t) old[r][t] = a.dq[(qrow0 + ic) * DH + 16 * t + lc];
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int i = 16 * wave + 4 * g4 + r;
    if (i >= nq || lq[r] == 0) continue;
#pragma unroll
    for (int t = 0; t < NDT; ++t) a.dq[(qrow0 + i) * DH + 16 * t + lc] = old[r][t] + a.scale * dQ[t][r];
  }
}

template <typename T, int DH>
static __global__ __launch_bounds__(256) void k_comm_dq(CommQueryArgs<T> a) {
  comm_dq_body<T, DH>(a);
}

// ---------------------------------------------------------------------------
// projection VJP inputs: d_proj [B*T, nproj*d] in the w_proj row order
//   q: unrotate(dq_r + scale S k_self); k: dkraw + unrotate(dkself + scale S q_r), S = sdss (the
//   self column's dS summed over the sweeps); v: dvraw; gate x-halves: the row's gate-logit
//   grads summed over its cell's sweeps (their dctx columns);
//   v_gate: dsig * sig * (1 - sig)
// and the bias gradients' column partials over the block's rows:
//   bpart[chunk][0, d) = sum of the key gate's (b_gk), [d, 2d) the value gate's (b_gv),
//   [2d, 3d) = sum dsig sig (1 - sig) (b_vgate).
// With the v_norm (vgain != nullptr) dvraw is the grad of the normed value: the v columns get
// its VJP, from the kept pre-norm values vpre, and vgpart[chunk][head] the v_gain partials.
// One thread per item: head hd, RoPE pairs jj .. jj + 3 (jj a multiple of 4) and their partners
// jj + DH/2 .. + 3, with 4-wide loads and stores. A row has d / 8 items; a block runs
// proj_rows_in_flight(d) rows at a time (row lane sub = thread / (d / 8)), or, from d = 2048 up,
// 256 items of one row (grid.x = d / 2048). rpb rows per block, each row's loads issued before
// its stores. Column partials: one chunk per (block row, row lane), chunk blockIdx.y * rif + sub.
// ---------------------------------------------------------------------------
constexpr int PROJ_ROWS = 32;
DM_HOST_DEV inline int proj_rows_in_flight(int d) { return d / 8 >= 256 ? 1 : 256 / (d / 8); }
DM_HOST_DEV inline int proj_grid_x(int d) { return d / 8 > 256 ? (d / 8 + 255) / 256 : 1; }
// map: row m of this launch -> layer row (one chunk's rows, or the identity); flags: PROJ_ROWS_OUT
// writes the dproj rows, PROJ_PARTIALS the column partials
constexpr int PROJ_ROWS_OUT = 1, PROJ_PARTIALS = 2;
template <typename T, int DH>
DM_DEV void proj_bwd_body(int M, int T_, int d, int h, int nproj, int fusion, const float* __restrict__ dq,
                          const float* __restrict__ dkraw, const float* __restrict__ dkself,
                          const float* __restrict__ dvraw, const T* __restrict__ dctxL,
                          const CellRow* __restrict__ cellrow, int B, const float* __restrict__ dsig,
                          const T* __restrict__ sig, const float* __restrict__ cos,
                          const float* __restrict__ sin, T* __restrict__ dproj, float* __restrict__ bpart,
                          const T* __restrict__ vpre, const float* __restrict__ vgain,
                          float* __restrict__ vgpart, const float* __restrict__ sdss,
                          const T* __restrict__ qr, const T* __restrict__ kself, float scale, RowMap map,
                          int flags, int rpb) {
  constexpr int Q = DH / 8;   // items per head (consecutive lanes)
  const int ipr = d / 8, rif = proj_rows_in_flight(d);
  const int sub = ipr >= 256 ? 0 : (int)threadIdx.x / ipr;
  const int item = ipr >= 256 ? (int)(blockIdx.x * 256 + threadIdx.x) : (int)threadIdx.x - sub * ipr;
  if (sub >= rif || item >= ipr) return;   // whole heads (ipr is a multiple of Q)
  const int hd = item / Q, jj = 4 * (item - hd * Q);
  const int c1 = hd * DH + jj, c2 = c1 + DH / 2;
  const int ck1 = col_k<DH>(hd, jj, 2), ck2 = col_k<DH>(hd, jj, 3);
  const int cv1 = nproj == 5 ? col_vlin<DH>(d, hd, jj) + 32 : 3 * d + c1;
  const int cv2 = nproj == 5 ? col_vlin<DH>(d, hd, jj + DH / 2) + 32 : 3 * d + c2;
  const int r0 = blockIdx.y * rpb, r1 = min(r0 + rpb, M);
  float bg[4][4] = {}, bv[2][4] = {}, vg = 0.f;
  const float gvn = vgain != nullptr ? vgain[hd] : 0.f;
  for (int mi = r0 + sub; mi < r1; mi += rif) {
    const long m = map(mi);
    const int b = (int)(m / T_), t = (int)(m - (long)b * T_);
    const long hr = (((long)b * h + hd) * T_ + t) * DH + jj;
    float cs[4], sn[4], q1[4], q2[4], s1[4], s2[4], k1[4], k2[4], v1[4], v2[4];
    ld4<float>(cos + (long)t * (DH / 2) + jj, cs);
    ld4<float>(sin + (long)t * (DH / 2) + jj, sn);
    ld4<float>(dq + hr, q1);
    ld4<float>(dq + hr + DH / 2, q2);
    ld4<float>(dkself + hr, s1);
    ld4<float>(dkself + hr + DH / 2, s2);
    ld4<float>(dkraw + hr, k1);
    ld4<float>(dkraw + hr + DH / 2, k2);
    ld4<float>(dvraw + hr, v1);
    ld4<float>(dvraw + hr + DH / 2, v2);
    // the gate logits' x-half grads: the sum of the row's dl columns in the stacked dctx rows
    // of its cell's sweeps, last sweep first (the order their VJPs ran)
    float g[4][4] = {};
    {
      const CellRow cr = cellrow[t];
      const long step = (long)B * cr.c * 4 * d;
      const T* R = dctxL + ((long)cr.row0 + (long)b * cr.c + (t - cr.pos0)) * 4 * d;
      for (int sw = cr.K - 1; sw >= 0; --sw) {
        const T* Rs = R + sw * step;
        float x[4][4];
        ld4<T>(Rs + ck1, x[0]);
        ld4<T>(Rs + ck2, x[1]);
        ld4<T>(Rs + cv1, x[2]);
        ld4<T>(Rs + cv2, x[3]);
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
          for (int i = 0; i < 4; ++i) g[u][i] += x[u][i];
      }
    }
    if (vgain != nullptr) {   // v_norm VJP over the head's Q lanes (a whole lane group)
      float x1[4], x2[4], ss = 0.f, sv = 0.f;
      ld4<T>(vpre + hr, x1);
      ld4<T>(vpre + hr + DH / 2, x2);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        ss += x1[i] * x1[i] + x2[i] * x2[i];
        sv += v1[i] * x1[i] + v2[i] * x2[i];
      }
      const float r = head_norm_r(group_sum<Q>(ss), 1.0f / DH);
      sv = group_sum<Q>(sv);
      const float r3 = r * r * r * sv * (1.0f / DH);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v1[i] = gvn * (r * v1[i] - r3 * x1[i]);
        v2[i] = gvn * (r * v2[i] - r3 * x2[i]);
      }
      if (jj == 0) vg += r * sv;
    }
    float z1[4] = {}, z2[4] = {};
    if (nproj == 6) {
      float sg1[4], sg2[4], ds1[4], ds2[4];
      ld4<T>(sig + m * d + c1, sg1);
      ld4<T>(sig + m * d + c2, sg2);
      ld4<float>(dsig + m * d + c1, ds1);
      ld4<float>(dsig + m * d + c2, ds2);
      // fusion: dsig already holds the grad of the raw pre-activation (no sigmoid, no bias)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        z1[i] = fusion ? ds1[i] : ds1[i] * sg1[i] * (1.f - sg1[i]);
        z2[i] = fusion ? ds2[i] : ds2[i] * sg2[i] * (1.f - sg2[i]);
      }
    }
    if (flags & PROJ_ROWS_OUT) {
      // the self column's terms: dq += scale S k_self, dk_self += scale S q (both rotated)
      const float S = scale * sdss[((long)b * h + hd) * T_ + t];
      float ks1[4], ks2[4], qa[4], qb[4];
      ld4<T>(kself + hr, ks1);
      ld4<T>(kself + hr + DH / 2, ks2);
      ld4<T>(qr + hr, qa);
      ld4<T>(qr + hr + DH / 2, qb);
      float o[12][4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float dq1 = q1[i] + S * ks1[i], dq2 = q2[i] + S * ks2[i];
        const float ds1 = s1[i] + S * qa[i], ds2 = s2[i] + S * qb[i];
        o[0][i] = dq1 * cs[i] + dq2 * sn[i];
        o[1][i] = -dq1 * sn[i] + dq2 * cs[i];
        o[2][i] = k1[i] + ds1 * cs[i] + ds2 * sn[i];
        o[3][i] = k2[i] - ds1 * sn[i] + ds2 * cs[i];
        o[4][i] = v1[i];
        o[5][i] = v2[i];
        o[6][i] = g[0][i];
        o[7][i] = g[1][i];
        o[8][i] = g[2][i];
        o[9][i] = g[3][i];
        o[10][i] = z1[i];
        o[11][i] = z2[i];
      }
      T* D = dproj + m * nproj * d;
#pragma unroll
      for (int p = 0; p < 6; ++p) {
        if (p == 5 && nproj != 6) break;
        st4<T>(D + p * d + c1, o[2 * p]);
        st4<T>(D + p * d + c2, o[2 * p + 1]);
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int u = 0; u < 4; ++u) bg[u][i] += g[u][i];
      bv[0][i] += z1[i];
      bv[1][i] += z2[i];
    }
  }
  if (!(flags & PROJ_PARTIALS)) return;
  const int chunk = blockIdx.y * rif + sub;
  float* P = bpart + (long)chunk * 3 * d;
  st4<float>(P + c1, bg[0]);
  st4<float>(P + c2, bg[1]);
  st4<float>(P + d + c1, bg[2]);
  st4<float>(P + d + c2, bg[3]);
  st4<float>(P + 2 * d + c1, bv[0]);
  st4<float>(P + 2 * d + c2, bv[1]);
  if (vgain != nullptr && jj == 0) vgpart[(long)chunk * h + hd] = vg;
}

template <typename T, int DH>
static __global__ __launch_bounds__(256) void k_proj_bwd(int M, int T_, int d, int h, int nproj, int fusion,
                                                         const float* __restrict__ dq, const float* __restrict__ dkraw,
                                                         const float* __restrict__ dkself,
                                                         const float* __restrict__ dvraw,
                                                         const T* __restrict__ dctxL,
                                                         const CellRow* __restrict__ cellrow, int B,
                                                         const float* __restrict__ dsig, const T* __restrict__ sig,
                                                         const float* __restrict__ cos, const float* __restrict__ sin,
                                                         T* __restrict__ dproj, float* __restrict__ bpart,
                                                         const T* __restrict__ vpre, const float* __restrict__ vgain,
                                                         float* __restrict__ vgpart, const float* __restrict__ sdss,
                                                         const T* __restrict__ qr, const T* __restrict__ kself,
                                                         float scale, RowMap map, int flags) {
  proj_bwd_body<T, DH>(M, T_, d, h, nproj, fusion, dq, dkraw, dkself, dvraw, dctxL, cellrow, B, dsig, sig, cos, sin,
                       dproj, bpart,
                       vpre, vgain, vgpart, sdss, qr, kself, scale, map, flags, PROJ_ROWS);
}

template <typename T, int DH> struct ProjBwdBody {
  static constexpr int THREADS = 256;
  struct Args {
    int M, T_, d, h, nproj, fusion;
    const float *dq, *dkraw, *dkself, *dvraw;
    const T* dctxL;
    const CellRow* cellrow;
    int B;
    const float* dsig;
    const T* sig;
    const float *cos, *sin;
    T* dproj;
    float* bpart;
    const T* vpre;
    const float* vgain;
    float* vgpart;
    const float* sdss;
    const T *qr, *kself;
    float scale;
    RowMap map;
    int flags;
    int rpb;   // rows per block (PROJ_ROWS when the block partials are written)
  };
  static DM_DEV void run(const Args& a, int, int) {
    proj_bwd_body<T, DH>(a.M, a.T_, a.d, a.h, a.nproj, a.fusion, a.dq, a.dkraw, a.dkself, a.dvraw, a.dctxL, a.cellrow,
                         a.B, a.dsig,
                         a.sig, a.cos, a.sin, a.dproj, a.bpart, a.vpre, a.vgain, a.vgpart, a.sdss, a.qr, a.kself,
                         a.scale, a.map, a.flags, a.rpb);
  }
};

// Column sums of a row-major fp32 matrix [M, ncols], stage 1: part[chunk][col]
static __global__ __launch_bounds__(256) void k_colsum_partial(int M, int ncols, int rows_per_chunk,
                                                        const float* __restrict__ src, float* __restrict__ part) {
  const int col = blockIdx.x * 256 + threadIdx.x;
  if (col >= ncols) return;
  const int r0 = blockIdx.y * rows_per_chunk, r1 = min(r0 + rows_per_chunk, M);
  float s = 0.f;
  for (int m0 = r0; m0 < r1; m0 += 8) {   // eight rows' loads in flight at a time
    float v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = src[(long)min(m0 + k, r1 - 1) * ncols + col];
#pragma unroll
    for (int k = 0; k < 8; ++k) s += (m0 + k < r1) ? v[k] : 0.f;
  }
  part[(long)blockIdx.y * ncols + col] = s;
}

// out[col] += sum_chunk part[chunk * ld + col], col < ncols
// C[i] (+)= sum_z part[z * n + i], z = 0..S-1 in order (split-K slices)
static __global__ __launch_bounds__(256) void k_sum_splits(int S, long n, const float* __restrict__ part,
                                                           float* __restrict__ C, int accumulate) {
  const long i = blockIdx.x * 256L + threadIdx.x;
  if (i >= n) return;
  float v = 0.f;
  for (int z = 0; z < S; ++z) v += part[(long)z * n + i];
  C[i] = accumulate ? C[i] + v : v;
}

// k_sum_splits on 4 consecutive elements per thread, the S slices' loads all in flight (the same
// per-element order: 0 + slice 0 + slice 1 + ...)
template <int S>
static __global__ __launch_bounds__(256) void k_sum_splits4(long n4, const float4* __restrict__ part,
                                                            float4* __restrict__ C, int accumulate) {
  const long i = blockIdx.x * 256L + threadIdx.x;
  if (i >= n4) return;
  float4 p[S];
#pragma unroll
  for (int z = 0; z < S; ++z) p[z] = part[(long)z * n4 + i];
  float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int z = 0; z < S; ++z) {
    v.x += p[z].x;
    v.y += p[z].y;
    v.z += p[z].z;
    v.w += p[z].w;
  }
  if (accumulate) {
    const float4 c = C[i];
    v = make_float4(c.x + v.x, c.y + v.y, c.z + v.z, c.w + v.w);
  }
  C[i] = v;
}

static __global__ __launch_bounds__(256) void k_sum_rows_add(int nchunk, int ncols, int ld, const float* __restrict__ part,
                                                      float* __restrict__ out0, float* __restrict__ out1,
                                                      float* __restrict__ out2, int seg) {
  // out_i[c] += sum_k part[k * ld + i * seg + c]: 64 columns per block, four row
  // groups (rows rg, rg + 4, ..) whose sums are added in LDS; eight loads in flight
  __shared__ float red[4][64];
  const int lane = threadIdx.x & 63, rg = threadIdx.x >> 6;
  const int col = blockIdx.x * 64 + lane;
  const int cc = min(col, ncols - 1);
  float s = 0.f;
  for (int k0 = rg; k0 < nchunk; k0 += 32) {
    float v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = part[(long)min(k0 + 4 * k, nchunk - 1) * ld + cc];
#pragma unroll
    for (int k = 0; k < 8; ++k) s += (k0 + 4 * k < nchunk) ? v[k] : 0.f;
  }
  red[rg][lane] = s;
  __syncthreads();
  if (rg == 0 && col < ncols) {
    const int i = col / seg, c = col - i * seg;
    float* out = i == 0 ? out0 : (i == 1 ? out1 : out2);
    if (out != nullptr) out[c] += red[0][lane] + red[1][lane] + red[2][lane] + red[3][lane];
  }
}

// ---------------------------------------------------------------------------
// attn_norm VJP (attention.py:74-83) with the block residual, one wave per row,
// RMSN_ROWS rows per block:
//   dx = dy + r w dxhat - x r^3 / d <w dxhat, x>;
//   dwa_part[block][j] = sum over the block's rows of dxhat x r (the norm weight's
//   gradient, summed over the blocks afterwards); each wave accumulates its rows in
//   its own LDS row, the four are added at the end.
// ---------------------------------------------------------------------------
constexpr int RMSN_ROWS = 8;
// map: row m of this launch -> layer row; flags: 1 writes dx, 2 the weight-grad partials
template <typename T>
DM_DEV void rmsnorm_bwd_body(int M, int d, float eps, int residual, const T* __restrict__ x,
                             const T* __restrict__ w, const float* __restrict__ dxhat, const T* __restrict__ dy,
                             T* __restrict__ dx, float* __restrict__ dwa_part, RowMap map, int flags) {
  extern __shared__ float acc_lds[];   // [4][d]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float* acc = acc_lds + (long)wave * d;
  // each lane owns runs of 8 consecutive columns (16-byte loads of bf16; d is a multiple of 8)
  constexpr int V = 8;
  for (int j = lane; j < d; j += 64) acc[j] = 0.f;
  const int r0 = blockIdx.x * RMSN_ROWS, r1 = min(r0 + RMSN_ROWS, M);
  for (int mi = r0 + wave; mi < r1; mi += 4) {
    const long m = map(mi);
    const T* xr = x + m * d;
    const float* gr = dxhat + m * d;
    float ss = 0.f, dot = 0.f;
    for (int j0 = lane * V; j0 < d; j0 += 64 * V) {
      float xv[V], wv[V], gv[V];
      unpack8<T>(ld8_global(xr + j0), xv);
      unpack8<T>(ld8_global(w + j0), wv);
      unpackf4(ld_global<floatx4>(gr + j0), gv);
      unpackf4(ld_global<floatx4>(gr + j0 + 4), gv + 4);
#pragma unroll
      for (int i = 0; i < V; ++i) {
        ss += xv[i] * xv[i];
        dot += wv[i] * gv[i] * xv[i];
      }
    }
    ss = wave_sum(ss);
    dot = wave_sum(dot);
    const float r = rsqrtf(ss / (float)d + eps);
    const float c3 = r * r * r / (float)d * dot;
    for (int j0 = lane * V; j0 < d; j0 += 64 * V) {
      float xv[V], wv[V], gv[V], yv[V], o[V];
      unpack8<T>(ld8_global(xr + j0), xv);
      unpack8<T>(ld8_global(w + j0), wv);
      unpackf4(ld_global<floatx4>(gr + j0), gv);
      unpackf4(ld_global<floatx4>(gr + j0 + 4), gv + 4);
      if ((flags & 1) && residual) unpack8<T>(ld8_global(dy + m * d + j0), yv);
      else
#pragma unroll
        for (int i = 0; i < V; ++i) yv[i] = 0.f;
      float* ar = acc + j0;
      floatx4 a0 = *reinterpret_cast<floatx4*>(ar), a1 = *reinterpret_cast<floatx4*>(ar + 4);
#pragma unroll
      for (int i = 0; i < V; ++i) {
        o[i] = r * wv[i] * gv[i] - xv[i] * c3 + yv[i];
        const float t = gv[i] * xv[i] * r;
        if (i < 4) a0[i] += t;
        else a1[i - 4] += t;
      }
      *reinterpret_cast<floatx4*>(ar) = a0;
      *reinterpret_cast<floatx4*>(ar + 4) = a1;
      if (flags & 1) st8<T>(dx + m * d + j0, o);
    }
  }
  if (!(flags & 2)) return;
  __syncthreads();
  for (int j = threadIdx.x; j < d; j += 256)
    dwa_part[(long)blockIdx.x * d + j] = acc_lds[j] + acc_lds[d + j] + acc_lds[2 * d + j] + acc_lds[3 * d + j];
}

template <typename T>
static __global__ __launch_bounds__(256) void k_rmsnorm_bwd(int M, int d, float eps, int residual,
                                                     const T* __restrict__ x, const T* __restrict__ w,
                                                     const float* __restrict__ dxhat, const T* __restrict__ dy,
                                                     T* __restrict__ dx, float* __restrict__ dwa_part, RowMap map,
                                                     int flags) {
  rmsnorm_bwd_body<T>(M, d, eps, residual, x, w, dxhat, dy, dx, dwa_part, map, flags);
}

template <typename T> struct RmsnormBwdBody {
  static constexpr int THREADS = 256;
  struct Args {
    int M, d;
    float eps;
    int residual;
    const T *x, *w;
    const float* dxhat;
    const T* dy;
    T* dx;
    float* dwa_part;
    RowMap map;
    int flags;
  };
  static DM_DEV void run(const Args& a, int, int) {
    rmsnorm_bwd_body<T>(a.M, a.d, a.eps, a.residual, a.x, a.w, a.dxhat, a.dy, a.dx, a.dwa_part, a.map, a.flags);
  }
};

// dx = dy + dxhat (no attn_norm) or dx = dxhat (no residual either)
template <typename T>
static __global__ __launch_bounds__(256) void k_dx_plain(long n, int residual, const float* __restrict__ dxhat,
                                                  const T* __restrict__ dy, T* __restrict__ dx) {
  for (long i = blockIdx.x * 256L + threadIdx.x; i < n; i += (long)gridDim.x * 256)
    dx[i] = from_f<T>(dxhat[i] + (residual ? to_f(dy[i]) : 0.f));
}

// ---------------------------------------------------------------------------
// unpack: ref[dst rows] (+)= packed[src rows] (fp32), the inverse of k_pack
// ---------------------------------------------------------------------------
struct UnpackSeg {
  float* dst;
  long dst_ld;     // elements between destination rows
  int dst_col;     // first destination column
  int nrows;
  int src_row;     // first packed row
  int pad_;
};
constexpr int UNPACK_MAX_SEG = 48;
struct UnpackArgs {
  UnpackSeg seg[UNPACK_MAX_SEG];
  int nseg;
  int ncols;
  const float* src;
};

static __global__ __launch_bounds__(256) void k_unpack_add(UnpackArgs a) {
  const int row = blockIdx.x;
  int s = 0, acc = 0;
  while (s < a.nseg && row >= acc + a.seg[s].nrows) { acc += a.seg[s].nrows; ++s; }
  const UnpackSeg& sg = a.seg[s];
  const int r = row - acc;
  const float* src = a.src + (long)(sg.src_row + r) * a.ncols;
  float* dst = sg.dst + (long)r * sg.dst_ld + sg.dst_col;
  for (int j0 = 0; j0 < a.ncols; j0 += 4 * 256) {   // four elements' loads before their stores
    float sv[4], dv[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int j = min(j0 + k * 256 + (int)threadIdx.x, a.ncols - 1);
      sv[k] = src[j];
      dv[k] = dst[j];
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int j = j0 + k * 256 + threadIdx.x;
      if (j < a.ncols) dst[j] = dv[k] + sv[k];
    }
  }
}

// ---- grouped-launch bodies of the backward's per-cell kernels (the layer-batched backward) ----
template <typename T, int DH, int NS> struct RefineBwdBody {
  static constexpr int THREADS = 256;
  using Args = RefineBwdArgs<T>;
  static DM_DEV void run(const Args& a, int, int) { refine_bwd_body<T, DH, NS>(a); }
};
template <typename T, int S> struct DuEpiBody {
  static constexpr int THREADS = 256;
  struct Args {
    int M, d, h;
    float inv_d, eps;
    const float *part, *lamdv;
    const T* o;
    const float* ssq;
    const T* normw;
    float *gw, *rowdot, *dnw;
  };
  static DM_DEV void run(const Args& a, int, int) {
    du_epi_body<T, S>(a.M, a.d, a.h, a.inv_d, a.eps, a.part, a.lamdv, a.o, a.ssq, a.normw, a.gw, a.rowdot, a.dnw);
  }
};
template <typename T, int DH> struct AttnBwdBody {
  static constexpr int THREADS = 256;
  static constexpr int MIN_WAVES = DH == 64 ? 2 : 1;
  using Args = AttnBwdArgs<T>;
  static DM_DEV void run(const Args& a, int bx, int by) {
    attn_bwd_body<T, DH>(a, bx + ATTN_BWD_ROLES * by, (int)gridDim.y);
  }
};
template <typename T, int DH> struct CommDkvBody {
  static constexpr int THREADS = 256;
  using Args = CommKeyArgs<T>;
  static DM_DEV void run(const Args& a, int bx, int by) { comm_dkv_body<T, DH>(a, bx, by); }
};
template <typename T, int DH> struct CommDqBody {
  static constexpr int THREADS = 256;
  using Args = CommQueryArgs<T>;
  static DM_DEV void run(const Args& a, int, int) { comm_dq_body<T, DH>(a); }
};

}  // namespace dm
