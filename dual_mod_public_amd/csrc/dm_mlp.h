// The Block's SwiGLU MLP on a decode step's few rows (models/dualmod/model.py:102-112:
// w2(silu(w1 x) * w3 x)), for M <= 64 rows: two weight-streaming kernels.
//
// With one token per sequence the products are M x d times d x H: the weights are read once and
// nothing else is large, so each kernel is bound by how fast it streams its weight rows. Up to four
// 16 x 16 MFMA tiles hold the M rows (rows >= M are zero) against 16 weight rows; the waves of a
// block split k and their partial tiles are summed through LDS in a fixed order (deterministic,
// no atomics). The weights are K-contiguous rows ([H, d] for w1 / w3, [d, H] for w2), so a lane's
// 8-element fragment is one 16-byte load.
#pragma once

#include <type_traits>

#include "dm_common.h"

namespace dm {

constexpr int MLP_ROWS = 64;   // rows per call: up to four 16-row MFMA tiles

// act[M, H] = silu(x W1^T) * (x W3^T): block = 16 columns of H, 4 waves each a quarter of d
// (d a multiple of 128); x [M, d], RT = ceil(M / 16) row tiles.
template <typename T, int RT>
__global__ __launch_bounds__(256) void k_swiglu_up(const T* __restrict__ x, const T* __restrict__ w1,
                                                   const T* __restrict__ w3, T* __restrict__ act, int M, int d,
                                                   int H) {
  using MF = Mfma<T>;
  __shared__ float red[2][4][RT * 256];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n0 = blockIdx.x * 16, r = lane & 15, kq = 8 * (lane >> 4);
  const int kw = d / 4, k0 = wave * kw;
  const T* xa[RT];
  bool live[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    live[rt] = 16 * rt + r < M;
    xa[rt] = x + (long)min(16 * rt + r, M - 1) * d + k0 + kq;
  }
  const T* p1 = w1 + (long)(n0 + r) * d + k0 + kq;
  const T* p3 = w3 + (long)(n0 + r) * d + k0 + kq;
  floatx4 g[RT], u[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) { g[rt] = zero4(); u[rt] = zero4(); }
#pragma unroll 8
  for (int k = 0; k < kw; k += 32) {
    const typename MF::frag b1 = __builtin_bit_cast(typename MF::frag, *reinterpret_cast<const uint4*>(p1 + k));
    const typename MF::frag b3 = __builtin_bit_cast(typename MF::frag, *reinterpret_cast<const uint4*>(p3 + k));
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const typename MF::frag af =
          __builtin_bit_cast(typename MF::frag, keep_if(*reinterpret_cast<const uint4*>(xa[rt] + k), live[rt]));
      g[rt] = MF::mma(af, b1, g[rt]);
      u[rt] = MF::mma(af, b3, u[rt]);
    }
  }
  // lane holds rows 16 rt + 4 (lane / 16) + q, column lane % 16 of the tile
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int e = rt * 256 + (4 * (lane >> 4) + q) * 16 + r;
      red[0][wave][e] = g[rt][q];
      red[1][wave][e] = u[rt][q];
    }
  __syncthreads();
#pragma unroll
  for (int e = threadIdx.x; e < RT * 256; e += 256) {
    const int i = e >> 4, j = e & 15;
    if (i < M) {
      const float G = ((red[0][0][e] + red[0][1][e]) + red[0][2][e]) + red[0][3][e];
      const float U = ((red[1][0][e] + red[1][1][e]) + red[1][2][e]) + red[1][3][e];
      act[(long)i * H + n0 + j] = from_f<T>(G * sigmoidf_(G) * U);
    }
  }
}

// out[M, d] = act[M, H] W2^T: block = 16 columns of d, 8 waves taking the 32-wide k steps of H
// round robin (H a multiple of 32).
template <typename T, int RT>
__global__ __launch_bounds__(512) void k_swiglu_down(const T* __restrict__ act, const T* __restrict__ w2,
                                                     T* __restrict__ out, int M, int d, int H) {
  using MF = Mfma<T>;
  __shared__ float red[8][RT * 256];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n0 = blockIdx.x * 16, r = lane & 15, kq = 8 * (lane >> 4);
  const T* aa[RT];
  bool live[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    live[rt] = 16 * rt + r < M;
    aa[rt] = act + (long)min(16 * rt + r, M - 1) * H + kq;
  }
  const T* pw = w2 + (long)(n0 + r) * H + kq;
  floatx4 acc[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) acc[rt] = zero4();
  const int nst = H / 32;
#pragma unroll 4
  for (int s = wave; s < nst; s += 8) {
    const typename MF::frag b = __builtin_bit_cast(typename MF::frag, *reinterpret_cast<const uint4*>(pw + 32 * s));
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const uint4 a = keep_if(*reinterpret_cast<const uint4*>(aa[rt] + 32 * s), live[rt]);
      acc[rt] = MF::mma(__builtin_bit_cast(typename MF::frag, a), b, acc[rt]);
    }
  }
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int q = 0; q < 4; ++q) red[wave][rt * 256 + (4 * (lane >> 4) + q) * 16 + r] = acc[rt][q];
  __syncthreads();
  for (int e = threadIdx.x; e < RT * 256; e += 512) {
    const int i = e >> 4, j = e & 15;
    if (i < M) {
      float v = 0.f;
#pragma unroll
      for (int w = 0; w < 8; ++w) v += red[w][e];
      out[(long)i * d + n0 + j] = from_f<T>(v);
    }
  }
}

// out[M, N] = a[M, K] W^T for M <= MLP_ROWS bf16 rows, W [N, K] K-contiguous (N a multiple of 16,
// K of 32): k_swiglu_down's weight-streaming product (the MLP's down projection, a decode step's W_O)
template <typename T>
void launch_rows_wt(const T* a, const T* W, T* out, int M, int N, int K, hipStream_t s) {
  auto run = [&](auto rt) {
    constexpr int RT = decltype(rt)::value;
    hipLaunchKernelGGL((k_swiglu_down<T, RT>), dim3(N / 16), dim3(512), 0, s, a, W, out, M, N, K);
  };
  const int rts = (M + 15) / 16;
  if (rts == 1) run(std::integral_constant<int, 1>{});
  else if (rts == 2) run(std::integral_constant<int, 2>{});
  else if (rts == 3) run(std::integral_constant<int, 3>{});
  else run(std::integral_constant<int, 4>{});
}

}  // namespace dm
