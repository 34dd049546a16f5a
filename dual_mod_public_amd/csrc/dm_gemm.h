// MFMA GEMM mainloop: C[BM x BN] = A[BM x K] . B[BN x K]^T  (both K-contiguous).
//
// 256 threads = 4 waves arranged WM x WN; each wave owns a (BM/WM) x (BN/WN)
// sub-tile made of 16x16 MFMA tiles. A and B k-tiles are staged through LDS
// (one buffer, next tile prefetched into registers while the current one
// feeds the MFMAs). After the k-loop the fp32 accumulators are written to an
// LDS tile so the epilogue can read any (row, col) pattern it needs (RoPE
// pairs, gate/candidate column pairs, per-head reductions).
#pragma once

#include "dm_common.h"

namespace dm {

template <typename T> struct GemmTraits {
  static constexpr int BK = (sizeof(T) == 2) ? 64 : 32;   // k per LDS tile
  static constexpr int PAD = 16 / (int)sizeof(T);          // 16-byte row pad
  static constexpr int VEC = 16 / (int)sizeof(T);          // elems per 16 B
  static constexpr int LDK = BK + PAD;
};

// ---- A-operand loaders: 16 bytes of row m, columns [k, k+VEC) -------------
template <typename T> struct ALoadPlain {
  const T* A;
  long lda;
  int M;
  DM_DEV void prepare(int, float*) const {}
  DM_DEV uint4 load(int m, int k, const float*) const {
    if (m >= M) return uint4{0u, 0u, 0u, 0u};
    return *reinterpret_cast<const uint4*>(A + (long)m * lda + k);
  }
};

// u = o * rs[m] * w[k]: RMSNorm applied on the fly to an fp32 row-major
// matrix o [M, ldo]; rs is computed per tile row from per-head partial sums
// of squares ssq [M, nparts] (rs = rsqrt(sum/d + eps)).
template <typename T, int BM> struct ALoadRms {
  const float* o;
  long ldo;
  const float* ssq;
  int nparts;
  const T* w;
  int M;
  int d;
  float eps;
  DM_DEV void prepare(int m0, float* rs_lds) const {
    for (int i = threadIdx.x; i < BM; i += blockDim.x) {
      int m = m0 + i;
      float s = 0.f;
      if (m < M)
        for (int p = 0; p < nparts; ++p) s += ssq[(long)m * nparts + p];
      rs_lds[i] = rsqrtf(s / (float)d + eps);
    }
  }
  DM_DEV uint4 load(int m, int k, const float* rs_lds_rel) const {
    constexpr int V = GemmTraits<T>::VEC;
    float f[V];
    if (m >= M) {
#pragma unroll
      for (int j = 0; j < V; ++j) f[j] = 0.f;
    } else {
      const float r = rs_lds_rel[0];
      const float* src = o + (long)m * ldo + k;
      float wf[V];
      unpack16<T>(*reinterpret_cast<const uint4*>(w + k), wf);
#pragma unroll
      for (int j = 0; j < V; j += 4) {
        float4 v = *reinterpret_cast<const float4*>(src + j);
        f[j] = v.x * r * wf[j];
        f[j + 1] = v.y * r * wf[j + 1];
        f[j + 2] = v.z * r * wf[j + 2];
        f[j + 3] = v.w * r * wf[j + 3];
      }
    }
    return pack16<T>(f);
  }
};

template <typename T, int BM, int BN>
constexpr int gemm_lds_bytes() {
  constexpr int ab = (BM + BN) * GemmTraits<T>::LDK * (int)sizeof(T);
  constexpr int c = BM * (BN + 4) * 4;
  constexpr int body = ab > c ? ab : c;
  return body + BM * 4;   // + per-row scale scratch
}

// Runs the k-loop for the tile at (m0, n0) and leaves the fp32 result in
// Cs[BM][BN+4] (LDS). Must be called by all 256 threads.
template <typename T, int BM, int BN, int WM, int WN, class AL>
DM_DEV void gemm_tile(const AL& al, const T* __restrict__ Bw, long ldb, int K, int m0,
                      int n0, char* smem, float*& Cs_out) {
  using Tr = GemmTraits<T>;
  using MF = Mfma<T>;
  constexpr int BK = Tr::BK, LDK = Tr::LDK, VEC = Tr::VEC;
  constexpr int TM = BM / WM, TN = BN / WN, FM = TM / 16, FN = TN / 16;
  constexpr int VPR = BK / VEC;                 // 16-byte vectors per tile row
  constexpr int NA = BM * VPR / 256, NB = BN * VPR / 256;
  static_assert(WM * WN == 4, "4 waves");
  static_assert(BM * VPR % 256 == 0 && BN * VPR % 256 == 0, "tile/threads");
  static_assert(TM % 16 == 0 && TN % 16 == 0, "wave tile");

  T* As = reinterpret_cast<T*>(smem);
  T* Bs = As + BM * LDK;
  float* Cs = reinterpret_cast<float*>(smem);
  float* rs = reinterpret_cast<float*>(smem + (gemm_lds_bytes<T, BM, BN>() - BM * 4));

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  al.prepare(m0, rs);
  __syncthreads();

  floatx4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = zero4();

  uint4 ra[NA], rb[NB];
  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      int v = tid + i * 256;
      int r = v / VPR, kc = (v % VPR) * VEC;
      ra[i] = al.load(m0 + r, k0 + kc, rs + r);
    }
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      int v = tid + i * 256;
      int r = v / VPR, kc = (v % VPR) * VEC;
      rb[i] = *reinterpret_cast<const uint4*>(Bw + (long)(n0 + r) * ldb + k0 + kc);
    }
  };
  auto sstore = [&]() {
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      int v = tid + i * 256;
      int r = v / VPR, kc = (v % VPR) * VEC;
      *reinterpret_cast<uint4*>(As + r * LDK + kc) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      int v = tid + i * 256;
      int r = v / VPR, kc = (v % VPR) * VEC;
      *reinterpret_cast<uint4*>(Bs + r * LDK + kc) = rb[i];
    }
  };

  const int nk = K / BK;
  gload(0);
  sstore();
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    if (kt + 1 < nk) gload((kt + 1) * BK);
#pragma unroll
    for (int kk = 0; kk < BK; kk += MF::KSTEP) {
      typename MF::frag af[FM], bfr[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i)
        af[i] = MF::load(As + (wm * TM + i * 16 + (lane & 15)) * LDK + kk + (lane >> 4) * MF::KPL);
#pragma unroll
      for (int j = 0; j < FN; ++j)
        bfr[j] = MF::load(Bs + (wn * TN + j * 16 + (lane & 15)) * LDK + kk + (lane >> 4) * MF::KPL);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = MF::mma(af[i], bfr[j], acc[i][j]);
    }
    __syncthreads();
    if (kt + 1 < nk) {
      sstore();
      __syncthreads();
    }
  }
  // accumulators -> LDS tile (aliases As/Bs; the loop ended on a barrier)
  constexpr int LDC = BN + 4;
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        Cs[(wm * TM + i * 16 + 4 * (lane >> 4) + r) * LDC + wn * TN + j * 16 + (lane & 15)] =
            acc[i][j][r];
  __syncthreads();
  Cs_out = Cs;
}

// Generic kernel: tile -> epilogue functor epi(Cs, LDC, m0, n0).
template <typename T, int BM, int BN, int WM, int WN, class AL, class EPI>
__global__ __launch_bounds__(256) void k_gemm(AL al, const T* __restrict__ Bw, long ldb, int K,
                                              EPI epi) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  float* Cs;
  gemm_tile<T, BM, BN, WM, WN, AL>(al, Bw, ldb, K, m0, n0, smem, Cs);
  epi(Cs, BN + 4, m0, n0);
}

}  // namespace dm
