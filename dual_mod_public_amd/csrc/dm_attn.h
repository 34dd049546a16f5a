// Flash-style attention tiles on MFMA for the DM cell.
//
// One workgroup = 4 waves = 64 query rows of one (batch, head); wave w owns
// rows 16w..16w+15. Keys stream through LDS in tiles of 64: K row-major
// (B-operand of S = Q K^T), V transposed (B-operand of O += P V), P staged
// per wave (A-operand). Row max / row sum reductions run inside the 16-lane
// groups that hold one output row (shuffle xor 1..8); the per-lane partial
// row sums are combined only once, at the end.
//
// Lane layout of every 16x16 fp32 tile: lane l holds rows 4*(l>>4)+r (r=0..3)
// of column (l & 15).
#pragma once

#include "dm_common.h"

namespace dm {

constexpr float NEG_INF = -__builtin_huge_valf();

template <typename T, int DH> struct AttnCfg {
  using MF = Mfma<T>;
  static constexpr int KT = 64;                     // keys per tile
  static constexpr int PAD = 16 / (int)sizeof(T);
  static constexpr int LDK = DH + PAD;              // Ks row stride
  static constexpr int LDP = KT + PAD;              // Ps row stride (keys)
  static constexpr int NDT = DH / 16;               // 16-wide output column tiles
  static constexpr int NKS = DH / MF::KSTEP;        // k-steps over head_dim
  static constexpr int NPS = KT / MF::KSTEP;        // k-steps over keys
  static constexpr int VEC = 16 / (int)sizeof(T);   // elements per 16-byte load
  static constexpr int LDS_ELEMS = 2 * KT * LDK + 4 * 16 * LDP;   // Ks, Vs [key][dh] + per-wave P
};

template <typename T, int DH> struct FlashState {
  floatx4 O[DH / 16];   // O[dt][r]: row 4g+r, col (lane&15)+16dt
  float m[4];           // running row max (uniform across the 16-lane group)
  float z[4];           // per-lane partial row sum
};

template <typename T, int DH>
DM_DEV void flash_init(FlashState<T, DH>& st) {
#pragma unroll
  for (int dt = 0; dt < DH / 16; ++dt) st.O[dt] = zero4();
#pragma unroll
  for (int r = 0; r < 4; ++r) { st.m[r] = NEG_INF; st.z[r] = 0.f; }
}

// Query fragments for rows qrow = 16*wave + (lane&15): A-operand of S = Q K^T.
template <typename T, int DH>
DM_DEV void load_q_frags(const T* qrow_ptr, bool valid, typename Mfma<T>::frag* qf) {
  using C = AttnCfg<T, DH>;
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int ks = 0; ks < C::NKS; ++ks) {
    if (valid) {
      qf[ks] = Mfma<T>::load(qrow_ptr + ks * Mfma<T>::KSTEP + (lane >> 4) * Mfma<T>::KPL);
    } else {
      float z[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      qf[ks] = Mfma<T>::from_floats(z);
    }
  }
}

// One key tile held in registers (global -> registers -> LDS, so the next tile's
// loads can be in flight while the current tile is used). Consecutive lanes take
// consecutive 16-byte chunks of a row (whole rows per load instruction).
template <typename T, int DH, int NT = 256> struct KVRegs {
  static constexpr int VPR = DH / AttnCfg<T, DH>::VEC;             // 16-byte vectors per row
  static constexpr int NV = AttnCfg<T, DH>::KT * VPR / NT;         // vectors per thread (NT threads)
  uint4 k[NV], v[NV];
  int nvalid;                                                      // keys [0, nvalid) of the tile
};

// Load keys [0, nvalid) of a tile; rows >= nvalid become zeros when stored (so
// 0-probability columns multiply zeros). The mask is applied at the store, not
// here: an operation on a loaded value right after its load would make the
// compiler wait for the load there, and the next tile's loads would no longer
// overlap the current tile's work.
template <typename T, int DH, int NT = 256>
DM_DEV void load_kv(const T* __restrict__ Kg, const T* __restrict__ Vg, long row_stride, int nvalid,
                    KVRegs<T, DH, NT>& r) {
  using R = KVRegs<T, DH, NT>;
  r.nvalid = nvalid;
#pragma unroll
  for (int i = 0; i < R::NV; ++i) {
    const int v = threadIdx.x + NT * i;
    const int k = v / R::VPR, c0 = (v % R::VPR) * AttnCfg<T, DH>::VEC;
    const long off = (long)(k < nvalid ? k : 0) * row_stride + c0;
    r.k[i] = *reinterpret_cast<const uint4*>(Kg + off);
    r.v[i] = *reinterpret_cast<const uint4*>(Vg + off);
  }
}

// K rows only (the V rows are already in LDS)
template <typename T, int DH, int NT = 256>
DM_DEV void load_k(const T* __restrict__ Kg, long row_stride, int nvalid, KVRegs<T, DH, NT>& r) {
  using R = KVRegs<T, DH, NT>;
  r.nvalid = nvalid;
#pragma unroll
  for (int i = 0; i < R::NV; ++i) {
    const int v = threadIdx.x + NT * i;
    const int k = v / R::VPR, c0 = (v % R::VPR) * AttnCfg<T, DH>::VEC;
    r.k[i] = *reinterpret_cast<const uint4*>(Kg + (long)(k < nvalid ? k : 0) * row_stride + c0);
  }
}
template <typename T, int DH, int NT = 256>
DM_DEV void store_k(const KVRegs<T, DH, NT>& r, T* Ks) {
  using C = AttnCfg<T, DH>;
  using R = KVRegs<T, DH, NT>;
#pragma unroll
  for (int i = 0; i < R::NV; ++i) {
    const int v = threadIdx.x + NT * i;
    const int k = v / R::VPR, c0 = (v % R::VPR) * C::VEC;
    *reinterpret_cast<uint4*>(Ks + k * C::LDK + c0) = keep_if(r.k[i], k < r.nvalid);
  }
}

// K rows -> Ks [key][dh], V rows -> Vs [key][dh] (P V reads V through the
// transposed-view fragment loads).
template <typename T, int DH, int NT = 256>
DM_DEV void store_kv(const KVRegs<T, DH, NT>& r, T* Ks, T* Vs) {
  using C = AttnCfg<T, DH>;
  using R = KVRegs<T, DH, NT>;
#pragma unroll
  for (int i = 0; i < R::NV; ++i) {
    const int v = threadIdx.x + NT * i;
    const int k = v / R::VPR, c0 = (v % R::VPR) * C::VEC;
    const bool ok = k < r.nvalid;
    *reinterpret_cast<uint4*>(Ks + k * C::LDK + c0) = keep_if(r.k[i], ok);
    *reinterpret_cast<uint4*>(Vs + k * C::LDK + c0) = keep_if(r.v[i], ok);
  }
}

// One 64-key tile: S = Q K^T * scale, mask, online softmax update, O += P V.
// mask(q, key) -> true if the score is kept; q is the wave-relative row + 16*wave.
template <typename T, int DH, class MASK>
DM_DEV void flash_tile(const typename Mfma<T>::frag* qf, const T* Ks, const T* Vs, T* Pw,
                       float scale, const MASK& keep, FlashState<T, DH>& st) {
  using C = AttnCfg<T, DH>;
  using MF = Mfma<T>;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, col = lane & 15;

  floatx4 S[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    S[t] = zero4();
#pragma unroll
    for (int ks = 0; ks < C::NKS; ++ks) {
      typename MF::frag kf = MF::load(Ks + (col + 16 * t) * C::LDK + ks * MF::KSTEP + g * MF::KPL);
      S[t] = MF::mma(qf[ks], kf, S[t]);
    }
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int q = 16 * wave + 4 * g + r;
    float mx = NEG_INF;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      float s = S[t][r] * scale;
      if (!keep(q, col + 16 * t)) s = NEG_INF;
      S[t][r] = s;
      mx = fmaxf(mx, s);
    }
    mx = group16_max(mx);
    const float mnew = fmaxf(st.m[r], mx);
    const float alpha = (st.m[r] == NEG_INF) ? 0.f : __expf(st.m[r] - mnew);
    st.m[r] = mnew;
    st.z[r] *= alpha;
#pragma unroll
    for (int dt = 0; dt < C::NDT; ++dt) st.O[dt][r] *= alpha;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const float p = (S[t][r] == NEG_INF) ? 0.f : __expf(S[t][r] - mnew);
      st.z[r] += p;
      Pw[(4 * g + r) * C::LDP + col + 16 * t] = from_f<T>(p);
    }
  }
  // P is the wave's own staging: LDS operations of one wave complete in order, so
  // its lanes see each other's P without a workgroup barrier; the wave barrier keeps
  // the compiler from moving the reads below above the writes above
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int kb = 0; kb < C::NPS; ++kb) {
    typename MF::frag pf = MF::load(Pw + col * C::LDP + kb * MF::KSTEP + g * MF::KPL);
#pragma unroll
    for (int dt = 0; dt < C::NDT; ++dt) {
      typename MF::frag vf = MF::load_tr(Vs + kb * MF::KSTEP * C::LDK + 16 * dt, C::LDK);
      st.O[dt] = MF::mma(pf, vf, st.O[dt]);
    }
  }
}

}  // namespace dm
