// MFMA GEMM core: C[BM x BN] = A[BM x K] . B[BN x K]^T with fp32 accumulation.
//
// 256 threads = 4 waves arranged WM x WN; each wave owns a (BM/WM) x (BN/WN)
// sub-tile of 16x16 MFMA tiles, kept in registers. Two k-loops, chosen by the
// template parameter D:
//  * D > 0 (register ring): operands are staged through two LDS buffers (one
//    barrier per k-tile) and fed from a ring of D register stages, so the global
//    loads of k-tile kt+D are in flight while tiles kt..kt+D-1 are consumed;
//  * D < 0 (bf16, K-contiguous sources, K a multiple of 64): -D LDS stages filled
//    straight from global memory (global_load_lds_dwordx4, no register round trip),
//    rows of 128 bytes with the 16-byte chunks XOR-swizzled by row so the MFMA
//    fragment reads are bank-conflict free; tiles kt+1..kt-D-1 in flight.
// The small-M sweep GEMMs (M = B*c rows) have little compute per k-tile and are
// otherwise bound by load latency.
//
// Operand sources describe a logical row-major [rows x K] operand:
//   SrcRows   element (r, k) at p[r*ld + k]   (K contiguous; 16-byte vector loads along k)
//   SrcRowsRs SrcRows plus per-row RMS scales staged in LDS for the epilogue
//   SrcKMajor element (r, k) at p[k*ld + r]   (rows contiguous; vectors along r,
//                                              transposed on the way into LDS)
// After the k-loop the epilogue functor receives the wave's accumulators:
// lane l holds rows 16i + 4(l>>4) + q (q = 0..3) of column 16j + (l & 15) of the
// wave tile, so head-aligned wave tiles keep RoPE pairs and gate/candidate
// columns in one lane.
#pragma once

#include <type_traits>

#include "dm_common.h"
#include "dm_group.h"

namespace dm {

template <typename T> struct GemmTraits {
  static constexpr int BK = (sizeof(T) == 2) ? 64 : 32;   // k per LDS tile
  static constexpr int PAD = 16 / (int)sizeof(T);          // 16-byte row pad
  static constexpr int VEC = 16 / (int)sizeof(T);          // elements per 16 B
  static constexpr int LDK = BK + PAD;
};

DM_DEV uint4 zero_u4() { return uint4{0u, 0u, 0u, 0u}; }

// Row-major operand loads clamp the row instead of branching: a load under a
// divergent branch makes the compiler wait for every outstanding load at the join,
// which would drain the prefetch ring each k-tile. Rows past the end (a partial
// last tile) then repeat the last row; they only feed output rows >= M, which no
// epilogue stores.

template <typename T> struct SrcRows {
  static constexpr bool KMAJOR = false;
  const T* __restrict__ p;
  long ld;
  int rows;   // valid rows (global index bound)
  DM_DEV const T* ptr(int r, int k) const { return p + (long)min(r, rows - 1) * ld + k; }
  DM_DEV uint4 load(int r, int k) const { return *reinterpret_cast<const uint4*>(ptr(r, k)); }
  DM_DEV uint4 xform(uint4 v, int, int, const float*, int) const { return v; }
};

// Row-major operand whose rows are the rows of one chunk of every batch element of a
// [B, T, ld] tensor: row r = b * c + p is tensor row b * T + pos0 + p (c a power of two).
template <typename T> struct SrcChunkRows {
  static constexpr bool KMAJOR = false;
  const T* __restrict__ p;
  long ld;
  int rows;         // B * c
  int lc, Tr, pos0;  // log2(c), rows per batch element of the tensor, chunk start
  DM_DEV const T* ptr(int r, int k) const {
    r = min(r, rows - 1);
    return p + ((long)(r >> lc) * Tr + pos0 + (r & ((1 << lc) - 1))) * ld + k;
  }
  DM_DEV uint4 load(int r, int k) const { return *reinterpret_cast<const uint4*>(ptr(r, k)); }
  DM_DEV uint4 xform(uint4 v, int, int, const float*, int) const { return v; }
};

constexpr int RMS_MAXR = 128;     // row-scale slots in LDS (>= BM of any row-scaled GEMM)
constexpr int RMS_MAXK = 4096;    // largest d_model the row scales are built for

// Row-major operand whose rows carry an RMS scale for the epilogue:
// rs[r] = rsqrt(sum_p ssq[r, p] * inv_d + eps) is staged in LDS before the k-loop
// (prepare_load issues the ssq loads ahead of the operand ring, prepare_store
// writes LDS) and handed to the epilogue. The operand itself is loaded unchanged:
// RMSNorm(o) . W^T = rs * (o . (W diag(w))^T) with the norm weight w folded into
// the packed weights.
template <typename T> struct SrcRowsRs {
  static constexpr bool KMAJOR = false;
  const T* __restrict__ p;           // o [rows, ld]
  long ld;
  int rows;
  const float* __restrict__ ssq;     // [rows, nparts] partial sums of squares
  int nparts;
  float inv_d, eps;
  struct Pre {
    float v[MAX_HEADS / 2];   // the loaded partials (summed in prepare_store, so no wait here)
  };
  // 256 / R adjacent threads per row split its nparts (<= MAX_HEADS) partial sums
  template <int R> static constexpr int prepare_loads() { return MAX_HEADS / (256 / R); }
  template <int R> DM_DEV Pre prepare_load(int r0, int) const {
    constexpr int P = 256 / R, Q = MAX_HEADS / P;
    static_assert(256 % R == 0 && P >= 2 && P <= 8, "rows per block");
    const int r = min(r0 + (int)threadIdx.x / P, rows - 1), part = threadIdx.x % P;
    const float* row = ssq + (long)r * nparts;
    Pre pr;
#pragma unroll
    for (int i = 0; i < Q; ++i) pr.v[i] = row[min(part + i * P, nparts - 1)];
    return pr;
  }
  template <int R> DM_DEV void prepare_store(const Pre& pr, float* rs_lds, T*, int) const {
    constexpr int P = 256 / R, Q = MAX_HEADS / P;
    const int part = threadIdx.x % P;
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < Q; ++i) s += part + i * P < nparts ? pr.v[i] : 0.f;
#pragma unroll
    for (int o = 1; o < P; o <<= 1) s += __shfl_xor(s, o, 64);
    if (threadIdx.x % P == 0) rs_lds[threadIdx.x / P] = rsqrtf(s * inv_d + eps);
  }
  DM_DEV const T* ptr(int r, int k) const { return p + (long)min(r, rows - 1) * ld + k; }
  DM_DEV uint4 load(int r, int k) const { return *reinterpret_cast<const uint4*>(ptr(r, k)); }
  DM_DEV uint4 xform(uint4 v, int, int, const float*, int) const { return v; }
};

template <typename T> struct SrcKMajor {
  static constexpr bool KMAJOR = true;
  const T* __restrict__ p;   // element (r, k) at p[k*ld + r]
  long ld;
  int rows;
  int kmax = 0x7fffffff;     // k >= kmax reads as zero (K not a multiple of the k-tile)
  DM_DEV uint4 load(int r, int k) const {   // VEC consecutive rows r.. at column k
    return (r < rows && k < kmax) ? *reinterpret_cast<const uint4*>(p + (long)k * ld + r) : zero_u4();
  }
  // direct-to-LDS path (whole tiles in range, K a multiple of the k-tile): row r of k-row k
  DM_DEV const T* ptr_k(int k, int r) const { return p + (long)k * ld + r; }
  DM_DEV uint4 xform(uint4 v, int, int, const float*, int) const { return v; }
};

template <class S> struct requires_prepare { static constexpr bool value = false; };
template <typename T> struct requires_prepare<SrcRowsRs<T>> { static constexpr bool value = true; };
struct NoPre {};
template <class S> struct PrepOf { using type = NoPre; };
// vector-memory loads of a source's prepare_load (row scales), 0 for plain sources
template <class S, int BM> constexpr int prepare_loads_of() {
  if constexpr (requires_prepare<S>::value) return S::template prepare_loads<BM>();
  else return 0;
}
template <typename T> struct PrepOf<SrcRowsRs<T>> { using type = typename SrcRowsRs<T>::Pre; };

// Tile epilogues: an EPI with a member type TilePre gathers its global inputs with
// pre = epi.tile_prefetch(m0, n0) before the k-loop (the loads complete under it),
// then sees the block's whole output tile, staged in LDS as fp32 rows of BN + 4
// floats: epi.tile_apply<BM, BN, LDT>(tile, m0, n0, rs, pre), rs = the block's row
// scales. Each thread then owns runs of consecutive columns (16-byte loads and
// stores) instead of the MFMA fragment layout's one column per lane. Otherwise
// epi(acc, row0, col0, rs) is called on each wave's fragments.
// An EPI with a static TILE_ROWS < BM sees the tile in chunks of TILE_ROWS rows
// (tile_apply<TILE_ROWS, BN, LDT>(tile, m0 + chunk origin, ...)), so that blocks too
// large for one LDS tile still store whole rows.
template <class E, class = void> struct has_tile_epi { static constexpr bool value = false; };
template <class E> struct has_tile_epi<E, std::void_t<typename E::TilePre>> { static constexpr bool value = true; };
template <class E, class = void> struct tile_rows_of { static constexpr int value = 1 << 30; };
// An EPI with a static LATE_GATHERS = the exact number of vector-memory load instructions its
// tile_prefetch issues gets them issued late in the direct-to-LDS k-loop (gemm_mainloop_dma).
template <class E, class = void> struct late_gathers_of { static constexpr int value = 0; };
template <class E> struct late_gathers_of<E, std::void_t<decltype(E::LATE_GATHERS)>> {
  static constexpr int value = E::LATE_GATHERS;
};
template <class E> struct tile_rows_of<E, std::void_t<decltype(E::TILE_ROWS)>> { static constexpr int value = E::TILE_ROWS; };
// A tile EPI with a member type ChunkPre: chunk_prefetch<TR, BN>(chunk m0, n0) gathers a chunk's
// inputs, issued for chunk c + 1 before chunk c is applied (tile_apply(..., cp) takes them)
template <class E, class = void> struct has_chunk_pre { static constexpr bool value = false; };
template <class E> struct has_chunk_pre<E, std::void_t<typename E::ChunkPre>> { static constexpr bool value = true; };
template <class E, class = void> struct EPI_ChunkPre { typedef char type; };
template <class E> struct EPI_ChunkPre<E, std::void_t<typename E::ChunkPre>> { typedef typename E::ChunkPre type; };

// k-rows per stage of the K-major direct-to-LDS k-loop: 32 for 256 x 256 blocks with
// at least 4 stages (four 32 KB stages keep three in flight), else 64
template <int BM, int BN, int S>
constexpr int kk_stage_k() { return BM * BN >= 65536 && S >= 4 ? 32 : 64; }

// operand stages, then the row scales
template <typename T, int BM, int BN, int D, bool KM = false>
constexpr int gemm_stage_bytes() {
  if constexpr (D > 0) return 2 * (BM + BN) * GemmTraits<T>::LDK * (int)sizeof(T);
  else if constexpr (KM) return (-D) * kk_stage_k<BM, BN, -D>() * (BM + BN) * 2;
  else return (-D) * (BM + BN) * 128;
}
template <typename T, int BM, int BN, int D, bool RMS, bool KM = false>
constexpr int gemm_lds_bytes() {
  return gemm_stage_bytes<T, BM, BN, D, KM>() + (RMS ? RMS_MAXR * 4 : BM * 4);
}

// Wave tile geometry of a (BM, BN, WM, WN) block.
template <int BM, int BN, int WM, int WN> struct WaveTile {
  static constexpr int TM = BM / WM, TN = BN / WN, FM = TM / 16, FN = TN / 16;
  static_assert(WM * WN == 4 || WM * WN == 8, "4 or 8 waves per block");
  static_assert(TM % 16 == 0 && TN % 16 == 0, "wave tile must be whole 16x16 MFMA tiles");
};

// The k-loop. acc must be zero-initialised by the caller (or hold a C to add to).
// Reduces k in [kbase, kbase + K).
template <typename T, int BM, int BN, int WM, int WN, int D, class SA, class SB>
DM_DEV void gemm_mainloop(const SA& sa, const SB& sb, int K, int m0, int n0, char* smem,
                          floatx4 (&acc)[WaveTile<BM, BN, WM, WN>::FM][WaveTile<BM, BN, WM, WN>::FN],
                          int kbase) {
  using Tr = GemmTraits<T>;
  using MF = Mfma<T>;
  using WT = WaveTile<BM, BN, WM, WN>;
  static_assert(WM * WN == 4, "register-ring k-loop: 4 waves");
  constexpr int BK = Tr::BK, LDK = Tr::LDK, VEC = Tr::VEC;
  constexpr int FM = WT::FM, FN = WT::FN, TM = WT::TM, TN = WT::TN;
  constexpr int NA = BM * BK / VEC / 256, NB = BN * BK / VEC / 256;
  static_assert(BM * BK / VEC % 256 == 0 && BN * BK / VEC % 256 == 0, "tile/threads");

  T* buf[2];
  buf[0] = reinterpret_cast<T*>(smem);
  buf[1] = buf[0] + (BM + BN) * LDK;
  float* rs_lds = reinterpret_cast<float*>(smem + 2 * (BM + BN) * LDK * sizeof(T));

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  // per-operand vector coordinates (fixed over k-tiles)
  auto coordA = [&](int i, int& r, int& kc) {
    const int v = tid + i * 256;
    if constexpr (SA::KMAJOR) { r = (v % (BM / VEC)) * VEC; kc = v / (BM / VEC); }
    else { r = v / (BK / VEC); kc = (v % (BK / VEC)) * VEC; }
  };
  auto coordB = [&](int i, int& r, int& kc) {
    const int v = tid + i * 256;
    if constexpr (SB::KMAJOR) { r = (v % (BN / VEC)) * VEC; kc = v / (BN / VEC); }
    else { r = v / (BK / VEC); kc = (v % (BK / VEC)) * VEC; }
  };

  uint4 ra[D][NA], rb[D][NB];
  auto gload = [&](int kt, uint4 (&xa)[NA], uint4 (&xb)[NB]) {
    const int k0 = kbase + kt * BK;
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      int r, kc;
      coordA(i, r, kc);
      xa[i] = sa.load(m0 + r, k0 + kc);
    }
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      int r, kc;
      coordB(i, r, kc);
      xb[i] = sb.load(n0 + r, k0 + kc);
    }
  };
  auto sstore = [&](int kt, T* dst, const uint4 (&xa)[NA], const uint4 (&xb)[NB]) {
    const int k0 = kbase + kt * BK;
    T* As = dst;
    T* Bs = dst + BM * LDK;
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      int r, kc;
      coordA(i, r, kc);
      const uint4 v = sa.xform(xa[i], r, k0 + kc, rs_lds, m0);
      if constexpr (SA::KMAJOR) {
        const T* e = reinterpret_cast<const T*>(&v);
#pragma unroll
        for (int j = 0; j < VEC; ++j) As[(r + j) * LDK + kc] = e[j];
      } else {
        *reinterpret_cast<uint4*>(As + r * LDK + kc) = v;
      }
    }
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      int r, kc;
      coordB(i, r, kc);
      const uint4 v = xb[i];
      if constexpr (SB::KMAJOR) {
        const T* e = reinterpret_cast<const T*>(&v);
#pragma unroll
        for (int j = 0; j < VEC; ++j) Bs[(r + j) * LDK + kc] = e[j];
      } else {
        *reinterpret_cast<uint4*>(Bs + r * LDK + kc) = v;
      }
    }
  };
  auto compute = [&](const T* src) {
    const T* As = src;
    const T* Bs = src + BM * LDK;
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
  };

  const int nk = (K + BK - 1) / BK;   // a partial last tile needs k-bounded sources
  if (nk >= D && nk % D == 0) {
    // Software pipeline with no data-dependent branches around the loads: the
    // steady state always prefetches tile kt + D (it exists), the last D tiles run
    // unrolled without prefetch. The waitcnt before each LDS store then only waits
    // for the oldest ring slot.
#pragma unroll
    for (int s = 0; s < D; ++s) gload(s, ra[s], rb[s]);
    sstore(0, buf[0], ra[0], rb[0]);
    __syncthreads();
    for (int kt0 = 0; kt0 < nk - D; kt0 += D) {
#pragma unroll
      for (int j = 0; j < D; ++j) {
        const int kt = kt0 + j;
        gload(kt + D, ra[j], rb[j]);
        compute(buf[j & 1]);
        sstore(kt + 1, buf[(j + 1) & 1], ra[(j + 1) % D], rb[(j + 1) % D]);
        __syncthreads();
      }
    }
#pragma unroll
    for (int j = 0; j < D; ++j) {
      const int kt = nk - D + j;
      compute(buf[j & 1]);
      if (j + 1 < D) sstore(kt + 1, buf[(j + 1) & 1], ra[(j + 1) % D], rb[(j + 1) % D]);
      __syncthreads();
    }
  } else {
    // short or ragged K: one tile at a time
    for (int kt = 0; kt < nk; ++kt) {
      gload(kt, ra[0], rb[0]);
      sstore(kt, buf[0], ra[0], rb[0]);
      __syncthreads();
      compute(buf[0]);
      __syncthreads();
    }
  }
}

// s_waitcnt vmcnt(n) lgkmcnt(0) (gfx9 encoding: vmcnt in [3:0] and [15:14], expcnt
// [6:4] left at 7 = no wait, lgkmcnt [11:8])
template <int N> DM_DEV void wait_vm_lgkm0() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));
}

typedef __attribute__((address_space(3))) void lds_void_t;

// The direct-to-LDS k-loop (D = -S < 0). Stage layout: BM then BN rows of 64 bf16
// (128 bytes, no padding); 16-byte chunk c of row r is stored at chunk c ^ (r & 7).
// One global_load_lds_dwordx4 per wave fills 8 rows (lane l: row l/8, stored chunk
// l%8), each wave issues BM/32 + BN/32 of them per k-tile. Per k-tile: wait for
// this wave's loads of tile kt (vmcnt), barrier (everyone's landed, and stage
// (kt-1)%S is free), issue tile kt+S-1 into it, compute on stage kt%S.
struct NoLate {
  DM_DEV void operator()() const {}
};

// G > 0: late(), which issues exactly G vector-memory loads (the epilogue's gathers), is
// called right after the last stage is issued, and the waits that follow leave those G
// loads outstanding (vector loads complete in issue order, so they would otherwise gate
// the next stage's wait); before the k-loop they would gate its first wait instead.
template <typename T, int BM, int BN, int WM, int WN, int S, int G = 0, class SA, class SB, class LATE = NoLate>
DM_DEV void gemm_mainloop_dma(const SA& sa, const SB& sb, int K, int m0, int n0, char* smem,
                              floatx4 (&acc)[WaveTile<BM, BN, WM, WN>::FM][WaveTile<BM, BN, WM, WN>::FN],
                              int kbase, const LATE& late = LATE{}) {
  static_assert(sizeof(T) == 2 && !SA::KMAJOR && !SB::KMAJOR, "direct-to-LDS path: bf16, K-contiguous");
  static_assert(S >= 2 && BM % 32 == 0 && BN % 32 == 0, "stages / tile rows");
  using MF = Mfma<T>;
  using WT = WaveTile<BM, BN, WM, WN>;
  constexpr int FM = WT::FM, FN = WT::FN, TM = WT::TM, TN = WT::TN;
  constexpr int STAGE = (BM + BN) * 128;
  // wave load instructions per tile: each fills 8 rows of 128 bytes, the block's waves in turn
  constexpr int NWV = WM * WN, LA = BM / (8 * NWV), LB = BN / (8 * NWV), L = LA + LB;
  static_assert(LA >= 1 && LB >= 1 && LA * 8 * NWV == BM && LB * 8 * NWV == BN, "whole 8-row loads per wave");
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int lrow = lane >> 3, lchunk = (lane & 7) ^ lrow;   // rows of an 8-row group start at multiples of 8

  auto issue = [&](int kt, int st) {
    char* base = smem + st * STAGE;
    const int k = kbase + kt * 64 + lchunk * 8;
#pragma unroll
    for (int i = 0; i < LA; ++i) {
      const int r = (wave * LA + i) * 8;
      __builtin_amdgcn_global_load_lds((const void*)sa.ptr(m0 + r + lrow, k), (lds_void_t*)(base + r * 128), 16,
                                       0, 0);
    }
#pragma unroll
    for (int i = 0; i < LB; ++i) {
      const int r = (wave * LB + i) * 8;
      __builtin_amdgcn_global_load_lds((const void*)sb.ptr(n0 + r + lrow, k),
                                       (lds_void_t*)(base + (BM + r) * 128), 16, 0, 0);
    }
  };
  // Both k-halves' fragments are read first, then the MFMAs run: the reads of the second half
  // overlap the first half's MFMAs, and each MFMA waits only for its own operands (LDS reads
  // complete in order). Left to itself the scheduler sinks every A fragment read to just before
  // its MFMAs, reusing one register quad, which exposes the LDS latency FM times per half.
  auto compute = [&](const char* As) {
    const char* Bs = As + BM * 128;
    typename MF::frag af[2][FM], bfr[2][FN];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int r = wm * TM + i * 16 + (lane & 15);
        af[kk][i] = *reinterpret_cast<const typename MF::frag*>(As + r * 128 +
                                                                 (((kk * 4 + (lane >> 4)) ^ (r & 7)) << 4));
      }
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int r = wn * TN + j * 16 + (lane & 15);
        bfr[kk][j] = *reinterpret_cast<const typename MF::frag*>(Bs + r * 128 +
                                                                  (((kk * 4 + (lane >> 4)) ^ (r & 7)) << 4));
      }
    }
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = MF::mma(af[kk][i], bfr[kk][j], acc[i][j]);
    if constexpr (FM * FN >= 16) {
      // the first half's reads; the second half's one per MFMA of the first half; the rest
      // (at most 15 LDS reads are outstanding when an MFMA has to wait for its operands: the
      // wait counter's range)
      __builtin_amdgcn_sched_group_barrier(0x100, FM + FN, 0);
#pragma unroll
      for (int q = 0; q < FM + FN; ++q) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 2 * FM * FN - (FM + FN), 0);
    }
  };

  static_assert(G >= 0 && 2 * L + G < 64, "vmcnt range");
  const int nk = K / 64;
#pragma unroll
  for (int st = 0; st < S - 1; ++st)
    if (st < nk) issue(st, st);
  // one k-tile: wait for this wave's loads of tile kt (lg: the G late loads, issued after
  // every stage, may stay outstanding), barrier, issue tile kt + S - 1, compute on tile kt
  auto step = [&](int kt, bool lg, bool with_late) {
    // tiles issued after kt and possibly outstanding: min(S-2, nk-1-kt)
    const int after = min(S - 2, nk - 1 - kt);
    if constexpr (S >= 4) {
      if (after >= 2) { if (lg) wait_vm_lgkm0<2 * L + G>(); else wait_vm_lgkm0<2 * L>(); }
      else if (after == 1) { if (lg) wait_vm_lgkm0<L + G>(); else wait_vm_lgkm0<L>(); }
      else { if (lg) wait_vm_lgkm0<G>(); else wait_vm_lgkm0<0>(); }
    } else if constexpr (S == 3) {
      if (after >= 1) { if (lg) wait_vm_lgkm0<L + G>(); else wait_vm_lgkm0<L>(); }
      else { if (lg) wait_vm_lgkm0<G>(); else wait_vm_lgkm0<0>(); }
    } else {
      if (lg) wait_vm_lgkm0<G>(); else wait_vm_lgkm0<0>();
    }
    __builtin_amdgcn_s_barrier();
    if (kt + S - 1 < nk) issue(kt + S - 1, (kt + S - 1) % S);
    if constexpr (G > 0)
      if (with_late) late();
    compute(smem + (kt % S) * STAGE);
  };
  if constexpr (G > 0) {
    // the late loads go out with the last stage (iteration nk - S), or after the prologue;
    // that iteration is peeled so the loads sit in straight-line code between the loops
    const int kg = nk - S;
    if (kg < 0) {
      late();
      for (int kt = 0; kt < nk; ++kt) step(kt, true, false);
    } else {
      for (int kt = 0; kt < kg; ++kt) step(kt, false, false);
      step(kg, false, true);
      for (int kt = kg + 1; kt < nk; ++kt) step(kt, true, false);
    }
  } else {
    for (int kt = 0; kt < nk; ++kt) step(kt, false, false);
  }
  // every wave is done reading the stages before the epilogue may reuse LDS
  __syncthreads();
}

// The direct-to-LDS k-loop for K-major operands (bf16, both operands K-major: the
// weight-grad products C = A^T B summed over rows). A stage holds KS k-rows
// (kk_stage_k) of the block's BM (then BN) columns, BM * 2 bytes per k-row, its 16-byte chunk c stored
// at chunk c ^ kk_swz<BM * 2>(k); one global_load_lds_dwordx4 per wave fills 1 KB (1024 /
// (BM * 2) k-rows). MFMA fragments (8 consecutive k of one column per lane) come
// from two ds_read_b64_tr_b16 each: in a 16-lane group, lane s names the 8 bytes
// at k-row 8g + s / 4 (+ 4), columns 4 (s % 4) .. + 3 of the fragment's 16 columns,
// and receives that 4 x 16 block's column s.
//
// The swizzle: LDS serves a ds_read_b64_tr_b16 in two passes of 32 lanes over 64 four-byte
// banks (256 bytes), so the 32-byte column pieces of the 8 k-rows one pass names (8 g + 0..3
// for g = 0, 1; then 2, 3) must fill the 256 bytes without overlap. k-rows of 256 bytes or more
// all start at bank 0: the piece moves by 2 (k & 3) chunks within a 128-byte half and by 8
// chunks (the other half) for k-rows 8 apart. 128-byte k-rows pair up in a 256-byte span (odd
// k-rows in the upper half): the piece moves by 2 ((k >> 1) & 1) + 4 ((k >> 3) & 1). Measured on
// gfx950 with SQ_LDS_BANK_CONFLICT: 2.0 conflict cycles per read with 2 (k & 3) alone, 0 with these.
template <int ROW> DM_DEV int kk_swz(int kr) {
  static_assert(ROW == 128 || ROW == 256 || ROW == 512, "k-row bytes");
  if constexpr (ROW == 128) return 2 * ((kr >> 1) & 1) + 4 * ((kr >> 3) & 1);
  else return (2 * (kr & 3)) ^ (8 * ((kr >> 3) & 1));
}
template <int ROW> DM_DEV bf16x8 frag_kmajor(const char* stage, int k0, int c0) {
  const int lane = threadIdx.x & 63, g = lane >> 4, s = lane & 15;
  const int kr = k0 + 8 * g + (s >> 2);
  const int col = c0 + 4 * (s & 3);
  const char* p = stage + kr * ROW + ((((col >> 3) ^ kk_swz<ROW>(kr)) << 4) | ((col & 7) << 1));
  const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
  const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p + 4 * ROW));
  return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

template <typename T, int BM, int BN, int WM, int WN, int S, class SA, class SB>
DM_DEV void gemm_mainloop_dma_kk(const SA& sa, const SB& sb, int K, int m0, int n0, char* smem,
                                 floatx4 (&acc)[WaveTile<BM, BN, WM, WN>::FM][WaveTile<BM, BN, WM, WN>::FN],
                                 int kbase) {
  static_assert(sizeof(T) == 2 && SA::KMAJOR && SB::KMAJOR, "K-major direct-to-LDS path: bf16, both K-major");
  static_assert(S >= 2 && (BM == 64 || BM == 128 || BM == 256) && (BN == 64 || BN == 128 || BN == 256),
                "stages / tile columns");
  using MF = Mfma<T>;
  using WT = WaveTile<BM, BN, WM, WN>;
  static_assert(WM * WN == 4, "K-major k-loop: 4 waves");
  constexpr int FM = WT::FM, FN = WT::FN, TM = WT::TM, TN = WT::TN;
  constexpr int KS = kk_stage_k<BM, BN, S>();             // k-rows per stage
  constexpr int ROWA = BM * 2, ROWB = BN * 2;              // bytes per k-row
  constexpr int STAGE = KS * (ROWA + ROWB);
  constexpr int RPA = 1024 / ROWA, RPB = 1024 / ROWB;      // k-rows per wave load instruction
  static_assert(KS % (4 * RPA) == 0 && KS % (4 * RPB) == 0, "whole wave loads per stage");
  constexpr int LA = KS / RPA / 4, LB = KS / RPB / 4, L = LA + LB;
  constexpr int CPA = ROWA / 16, CPB = ROWB / 16;          // 16-byte chunks per k-row
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  auto issue = [&](int kt, int st) {
    char* base = smem + st * STAGE;
    const int k = kbase + kt * KS;
#pragma unroll
    for (int i = 0; i < LA; ++i) {
      const int r0 = (wave * LA + i) * RPA, r = r0 + lane / CPA;
      const int c = (lane % CPA) ^ kk_swz<ROWA>(r);
      __builtin_amdgcn_global_load_lds((const void*)sa.ptr_k(k + r, m0 + 8 * c), (lds_void_t*)(base + r0 * ROWA),
                                       16, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < LB; ++i) {
      const int r0 = (wave * LB + i) * RPB, r = r0 + lane / CPB;
      const int c = (lane % CPB) ^ kk_swz<ROWB>(r);
      __builtin_amdgcn_global_load_lds((const void*)sb.ptr_k(k + r, n0 + 8 * c),
                                       (lds_void_t*)(base + KS * ROWA + r0 * ROWB), 16, 0, 0);
    }
  };
  if constexpr (S == 2 && KS == 64 && FM * FN >= 32) {
    // Software-pipelined: the fragments of the next 32-k half are read while the MFMAs of the
    // current half run (two register sets), across the stage boundary too, so the MFMAs never
    // wait for LDS (the compiler's own interleaving of the reads and MFMAs: forced orders measured
    // slower). Per stage kt: MFMAs of half 0 with the reads of half 1; then the wait for
    // stage kt + 1's loads and for this wave's reads of stage kt, the barrier (stage kt free
    // everywhere), the loads of stage kt + 2 into it; then MFMAs of half 1 with the reads of
    // stage kt + 1's half 0. Each accumulator still sums its k in ascending order.
    typename MF::frag a0[FM], b0[FN], a1[FM], b1[FN];
    auto rd = [&](const char* st, int kk, typename MF::frag(&af)[FM], typename MF::frag(&bf)[FN]) {
#pragma unroll
      for (int i = 0; i < FM; ++i) af[i] = frag_kmajor<ROWA>(st, 32 * kk, wm * TM + 16 * i);
#pragma unroll
      for (int j = 0; j < FN; ++j) bf[j] = frag_kmajor<ROWB>(st + KS * ROWA, 32 * kk, wn * TN + 16 * j);
    };
    auto mm = [&](const typename MF::frag(&af)[FM], const typename MF::frag(&bf)[FN]) {
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = MF::mma(af[i], bf[j], acc[i][j]);
    };
    const int nk = K / KS;
    if (nk <= 0) return;
    issue(0, 0);
    if (nk > 1) {
      issue(1, 1);
      wait_vm_lgkm0<L>();
    } else {
      wait_vm_lgkm0<0>();
    }
    __builtin_amdgcn_s_barrier();
    rd(smem, 0, a0, b0);
    for (int kt = 0; kt < nk - 1; ++kt) {
      rd(smem + (kt & 1) * STAGE, 1, a1, b1);
      mm(a0, b0);
      wait_vm_lgkm0<0>();
      __builtin_amdgcn_s_barrier();
      if (kt + 2 < nk) issue(kt + 2, kt & 1);
      rd(smem + ((kt + 1) & 1) * STAGE, 0, a0, b0);
      mm(a1, b1);
    }
    rd(smem + ((nk - 1) & 1) * STAGE, 1, a1, b1);
    mm(a0, b0);
    mm(a1, b1);
    __syncthreads();
    return;
  }
  // Per 32-k step the step's fragment reads go first, then its MFMAs (the reads of one fragment
  // otherwise sink to just before its MFMAs, each exposing the LDS latency).
  auto compute = [&](const char* As) {
    const char* Bs = As + KS * ROWA;
#pragma unroll
    for (int kk = 0; kk < KS / 32; ++kk) {
      typename MF::frag af[FM], bfr[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i) af[i] = frag_kmajor<ROWA>(As, 32 * kk, wm * TM + 16 * i);
#pragma unroll
      for (int j = 0; j < FN; ++j) bfr[j] = frag_kmajor<ROWB>(Bs, 32 * kk, wn * TN + 16 * j);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = MF::mma(af[i], bfr[j], acc[i][j]);
      if constexpr (FM * FN >= 16) {
        __builtin_amdgcn_sched_group_barrier(0x100, 2 * (FM + FN), 0);
        __builtin_amdgcn_sched_group_barrier(0x008, FM * FN, 0);
      }
    }
  };

  const int nk = K / KS;
#pragma unroll
  for (int st = 0; st < S - 1; ++st)
    if (st < nk) issue(st, st);
  for (int kt = 0; kt < nk; ++kt) {
    const int after = min(S - 2, nk - 1 - kt);
    if constexpr (S >= 4) {
      if (after >= 2) wait_vm_lgkm0<2 * L>();
      else if (after == 1) wait_vm_lgkm0<L>();
      else wait_vm_lgkm0<0>();
    } else if constexpr (S == 3) {
      if (after >= 1) wait_vm_lgkm0<L>();
      else wait_vm_lgkm0<0>();
    } else {
      wait_vm_lgkm0<0>();
    }
    __builtin_amdgcn_s_barrier();
    if (kt + S - 1 < nk) issue(kt + S - 1, (kt + S - 1) % S);
    compute(smem + (kt % S) * STAGE);
  }
  __syncthreads();
}

// Generic kernel: zero accumulators, k-loop, epilogue on the wave's registers.
// epi(acc, row0, col0) with row0/col0 the global origin of the wave tile.
// Split-K launches (gridDim.z > 1) reduce k in [z*K, (z+1)*K) in block z; their
// epilogue gets the slice index z.
template <typename T, int BM, int BN, int WM, int WN, int D, class SA, class SB>
DM_DEV void gemm_kloop(const SA& sa, const SB& sb, int K, int m0, int n0, char* smem,
                       floatx4 (&acc)[WaveTile<BM, BN, WM, WN>::FM][WaveTile<BM, BN, WM, WN>::FN], int kbase) {
  if constexpr (D > 0) gemm_mainloop<T, BM, BN, WM, WN, D>(sa, sb, K, m0, n0, smem, acc, kbase);
  else if constexpr (SA::KMAJOR && SB::KMAJOR) gemm_mainloop_dma_kk<T, BM, BN, WM, WN, -D>(sa, sb, K, m0, n0, smem, acc, kbase);
  else gemm_mainloop_dma<T, BM, BN, WM, WN, -D>(sa, sb, K, m0, n0, smem, acc, kbase);
}

// LDS bytes of one block of a k_gemm configuration
template <typename T, int BM, int BN, int D, class SA, class SB>
constexpr int gemm_block_lds() {
  return gemm_lds_bytes<T, BM, BN, D, requires_prepare<SA>::value, SA::KMAJOR && SB::KMAJOR && D < 0>();
}

// One block tile (bx, by) of split-K slice bz, in the LDS at smem (gemm_block_lds bytes,
// 1024-byte aligned).
template <typename T, int BM, int BN, int WM, int WN, int D, class SA, class SB, class EPI>
DM_DEV void gemm_block_at(const SA& sa, const SB& sb, int K, const EPI& epi, int bx, int by, int bz, char* smem) {
  using WT = WaveTile<BM, BN, WM, WN>;
  constexpr bool RMS = requires_prepare<SA>::value;
  constexpr bool KM = SA::KMAJOR && SB::KMAJOR && D < 0;
  const int m0 = by * BM, n0 = bx * BN;
  static_assert(!RMS || BM <= RMS_MAXR, "row-scale slots");
  const int wave = threadIdx.x >> 6;
  const int row0 = m0 + (wave / WN) * WT::TM, col0 = n0 + (wave % WN) * WT::TN;
  const float* rs = reinterpret_cast<const float*>(smem + gemm_stage_bytes<T, BM, BN, D, KM>()) + (wave / WN) * WT::TM;
  floatx4 acc[WT::FM][WT::FN];
#pragma unroll
  for (int i = 0; i < WT::FM; ++i)
#pragma unroll
    for (int j = 0; j < WT::FN; ++j) acc[i][j] = zero4();
  // Row scales (row-scaled operands feed tile epilogues only): their inputs are
  // loaded first and the scales are staged in LDS after the k-loop, so no wait on
  // them, or on the epilogue's gathers issued after them, precedes the k-loop.
  static_assert(!RMS || has_tile_epi<EPI>::value, "row-scaled operands need a tile epilogue");
  typename PrepOf<SA>::type pre_a{};
  if constexpr (has_tile_epi<EPI>::value) {
    constexpr int TR = tile_rows_of<EPI>::value < BM ? tile_rows_of<EPI>::value : BM;   // rows per chunk
    constexpr int LDT = BN + 4;
    static_assert(BM % TR == 0 && TR % 16 == 0, "whole 16-row groups per chunk");
    static_assert(TR * LDT * 4 <= gemm_stage_bytes<T, BM, BN, D, KM>(), "output chunk fits the stages");
    typename EPI::TilePre pre;
    if constexpr (late_gathers_of<EPI>::value > 0 && D < 0 && !KM) {
      // the gathers (and row-scale loads) are issued with the k-loop's last stage
      constexpr int G = late_gathers_of<EPI>::value + prepare_loads_of<SA, BM>();
      auto late = [&]() {
        if constexpr (RMS) pre_a = sa.template prepare_load<BM>(m0, K);
        pre = epi.tile_prefetch(m0, n0);
      };
      gemm_mainloop_dma<T, BM, BN, WM, WN, -D, G>(sa, sb, K, m0, n0, smem, acc, bz * K, late);
    } else {
      if constexpr (RMS) pre_a = sa.template prepare_load<BM>(m0, K);
      pre = epi.tile_prefetch(m0, n0);
      gemm_kloop<T, BM, BN, WM, WN, D>(sa, sb, K, m0, n0, smem, acc, bz * K);
    }
    // the k-loop ends with a barrier: the stages are free for the output tile
    float* tile = reinterpret_cast<float*>(smem);
    const float* rs_lds = reinterpret_cast<const float*>(smem + gemm_stage_bytes<T, BM, BN, D, KM>());
    const int lane = threadIdx.x & 63;
    constexpr int NCP = has_chunk_pre<EPI>::value ? 2 : 0;
    typename EPI_ChunkPre<EPI>::type cp[2];
    if constexpr (NCP > 0) cp[0] = epi.template chunk_prefetch<TR, BN>(m0, n0);
#pragma unroll
    for (int c = 0; c < BM / TR; ++c) {
      if (c > 0) __syncthreads();   // the previous chunk has been read
#pragma unroll
      for (int i = 0; i < WT::FM; ++i) {
        if ((row0 - m0 + 16 * i) / TR != c) continue;   // wave-uniform
#pragma unroll
        for (int j = 0; j < WT::FN; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q)
            tile[(row0 - m0 - c * TR + 16 * i + 4 * (lane >> 4) + q) * LDT + col0 - n0 + 16 * j + (lane & 15)] =
                acc[i][j][q];
      }
      if constexpr (RMS)
        if (c == 0) sa.template prepare_store<BM>(pre_a, const_cast<float*>(rs_lds), nullptr, K);
      __syncthreads();
      if constexpr (NCP > 0) {
        if (c + 1 < BM / TR) cp[(c + 1) & 1] = epi.template chunk_prefetch<TR, BN>(m0 + (c + 1) * TR, n0);
        epi.template tile_apply<TR, BN, LDT>(tile, m0 + c * TR, n0, rs_lds + c * TR, pre, bz, cp[c & 1]);
      } else {
        epi.template tile_apply<TR, BN, LDT>(tile, m0 + c * TR, n0, rs_lds + c * TR, pre, bz);
      }
    }
  } else {
    gemm_kloop<T, BM, BN, WM, WN, D>(sa, sb, K, m0, n0, smem, acc, bz * K);
    epi(acc, row0, col0, rs, bz);
  }
}

template <typename T, int BM, int BN, int WM, int WN, int D, class SA, class SB, class EPI>
DM_DEV void gemm_block(const SA& sa, const SB& sb, int K, const EPI& epi, int bx, int by, int bz) {
  __shared__ __attribute__((aligned(1024))) char smem[gemm_block_lds<T, BM, BN, D, SA, SB>()];
  gemm_block_at<T, BM, BN, WM, WN, D, SA, SB, EPI>(sa, sb, K, epi, bx, by, bz, smem);
}

template <typename T, int BM, int BN, int WM, int WN, int D, class SA, class SB, class EPI>
__global__ __launch_bounds__(64 * WM * WN) void k_gemm(SA sa, SB sb, int K, EPI epi, uint64_t* prof_ts) {
  const uint64_t t0 = prof_begin(prof_ts);
  // Blocks are dispatched round-robin over the 8 XCDs (each with its own L2). For
  // the K-major (weight-grad) products every XCD gets a contiguous range of tiles
  // instead (x fastest, then y, then the split-K slice), so tiles that share operand
  // columns at the same k share an L2.
  int bx = blockIdx.x, by = blockIdx.y, bz = blockIdx.z;
  if constexpr (SA::KMAJOR && SB::KMAJOR && D < 0) {
    const int gx = gridDim.x, gy = gridDim.y, nb = gx * gy * (int)gridDim.z;
    if (nb % 8 == 0) {
      const int L = bx + gx * (by + gy * bz);
      const int t = (L % 8) * (nb / 8) + L / 8;
      bx = t % gx;
      by = (t / gx) % gy;
      bz = t / (gx * gy);
    }
  }
  gemm_block<T, BM, BN, WM, WN, D, SA, SB, EPI>(sa, sb, K, epi, bx, by, bz);
  prof_end(prof_ts, t0);
}

// a split-K k_gemm as a grouped-launch body: slice z of S in grid rows [z * mt, (z + 1) * mt)
template <typename T, int BM, int BN, int WM, int WN, int D, class SA, class SB, class EPI>
struct SplitGemmBody {
  static constexpr int THREADS = 256;
  struct Args {
    SA sa;
    SB sb;
    int K;   // per slice
    EPI epi;
    int mt;  // row tiles
  };
  static DM_DEV void run(const Args& a, int bx, int by) {
    gemm_block<T, BM, BN, WM, WN, D, SA, SB, EPI>(a.sa, a.sb, a.K, a.epi, bx, by % a.mt, by / a.mt);
  }
};

// k_gemm as a grouped-launch body (one split-K slice)
template <typename T, int BM, int BN, int WM, int WN, int D, class SA, class SB, class EPI>
struct GemmBody {
  static constexpr int THREADS = 256;
  struct Args {
    SA sa;
    SB sb;
    int K;
    EPI epi;
  };
  static DM_DEV void run(const Args& a, int bx, int by) {
    gemm_block<T, BM, BN, WM, WN, D, SA, SB, EPI>(a.sa, a.sb, a.K, a.epi, bx, by, 0);
  }
};

// Two independent GEMMs in one launch (blocks [0, P1 blocks) the first, the rest the second),
// sharing one LDS allocation: a GemmPart is one k_gemm configuration over a grid of
// (gx, gy) tiles and nz split-K slices (slice skip_z >= 0 left out: its K range is another
// launch's).
template <typename T, int BM_, int BN_, int WM, int WN, int D, class SA, class SB, class EPI>
struct GemmPart {
  static constexpr int LDS = gemm_block_lds<T, BM_, BN_, D, SA, SB>();
  SA sa;
  SB sb;
  int K;   // per slice
  EPI epi;
  int gx, gy, nz, skip_z;
  DM_DEV int blocks() const { return gx * gy * nz; }
  DM_DEV void run(int L, char* smem) const {
    const int bx = L % gx, by = (L / gx) % gy, zi = L / (gx * gy);
    const int bz = (skip_z >= 0 && zi >= skip_z) ? zi + 1 : zi;
    gemm_block_at<T, BM_, BN_, WM, WN, D, SA, SB, EPI>(sa, sb, K, epi, bx, by, bz, smem);
  }
};
template <class P1, class P2> struct GemmPairBody {
  static constexpr int THREADS = 256;
  static constexpr int LDS = P1::LDS > P2::LDS ? P1::LDS : P2::LDS;
  struct Args {
    P1 p1;
    P2 p2;
  };
  static DM_DEV void run(const Args& a, int bx, int) {
    __shared__ __attribute__((aligned(1024))) char smem[LDS];
    const int n1 = a.p1.blocks();
    if (bx < n1) a.p1.run(bx, smem);
    else a.p2.run(bx - n1, smem);
  }
};
// one GemmPart as a grouped-launch body (its own LDS size)
template <class P> struct GemmPartBody {
  static constexpr int THREADS = 256;
  struct Args {
    P p;
  };
  static DM_DEV void run(const Args& a, int bx, int) {
    __shared__ __attribute__((aligned(1024))) char smem[P::LDS];
    a.p.run(bx, smem);
  }
};
template <class P1, class P2>
__global__ __launch_bounds__(256) void k_gemm_pair(typename GemmPairBody<P1, P2>::Args a) {
  GemmPairBody<P1, P2>::run(a, (int)blockIdx.x, 0);
}

}  // namespace dm
