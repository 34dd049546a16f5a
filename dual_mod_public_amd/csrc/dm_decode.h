// Decode kernels: split-P streaming read of the static tape + LSE merge.
#pragma once

#include "dm_attn.h"

namespace dm {

// ---------------------------------------------------------------------------
// decode: split-P read of the tape (attention.py:283-312 over a static tape)
// grid (nsplit, B*h); keys [lo + s*L, min(lo + (s+1)*L, pos))
// ---------------------------------------------------------------------------
template <typename T> struct DecodeArgs {
  int B, h, d, tape_T, pos, lo, split_len, nsplit;
  float scale;
  const T* q;        // [B, h, 1, dh] rotated query of this step
  const T* kself;    // [B, h, 1, dh]
  const T* vself;    // [B, h, 1, dh]
  const T* Kt; const T* Vt;   // tape [B, h, tape_T, dh]
  float* part;       // [nsplit, B*h, dh + 2]: A[dh], Z, m
  float* o;          // [B, d] fp32
  float* ssq;        // [B, h]
  T* o_cat;          // [B, d] storage dtype
  uint64_t* prof_ts; // per-dispatch timing slots (nullptr: untimed)
};

template <typename T, int DH, int L>
__global__ __launch_bounds__(256) void k_decode_partial(DecodeArgs<T> a) {
  constexpr int VEC = 16 / (int)sizeof(T);
  constexpr int LPK = DH / VEC;          // lanes per key row
  constexpr int KPP = 256 / LPK;         // keys per pass
  constexpr int NP = L / KPP;            // passes
  static_assert(L % KPP == 0, "split length");
  const uint64_t t0 = prof_begin(a.prof_ts);
  __shared__ float red[4][DH + 2];
  const int s = blockIdx.x, bh = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int kslot = tid / LPK, part = tid - kslot * LPK;
  const int k_begin = a.lo + s * a.split_len;
  const int k_end = min(k_begin + a.split_len, a.pos);

  float qv[VEC];
  unpack16<T>(*reinterpret_cast<const uint4*>(a.q + (long)bh * DH + part * VEC), qv);
  const T* Kb = a.Kt + (long)bh * a.tape_T * DH + part * VEC;
  const T* Vb = a.Vt + (long)bh * a.tape_T * DH + part * VEC;

  uint4 raw[NP];
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    const int key = k_begin + i * KPP + kslot;
    raw[i] = keep_if(ld_nt(Kb + (long)(key < k_end ? key : k_begin) * DH), key < k_end);
  }
  float sc[NP];
  float mx = NEG_INF;
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    float kv[VEC];
    unpack16<T>(raw[i], kv);
    float dot = 0.f;
#pragma unroll
    for (int j = 0; j < VEC; ++j) dot += qv[j] * kv[j];
#pragma unroll
    for (int o = 1; o < LPK; o <<= 1) dot += __shfl_xor(dot, o, 64);
    const int key = k_begin + i * KPP + kslot;
    sc[i] = (key < k_end) ? dot * a.scale : NEG_INF;
    mx = fmaxf(mx, sc[i]);
  }
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    const int key = k_begin + i * KPP + kslot;
    raw[i] = keep_if(ld_nt(Vb + (long)(key < k_end ? key : k_begin) * DH), key < k_end);
  }
  // block max
#pragma unroll
  for (int o = LPK; o < 64; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  if (lane == 0) red[wave][0] = mx;
  __syncthreads();
  const float M = fmaxf(fmaxf(red[0][0], red[1][0]), fmaxf(red[2][0], red[3][0]));
  __syncthreads();
  float acc[VEC];
#pragma unroll
  for (int j = 0; j < VEC; ++j) acc[j] = 0.f;
  float z = 0.f;
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    const float p = (sc[i] == NEG_INF) ? 0.f : __expf(sc[i] - M);
    z += p;
    float vv[VEC];
    unpack16<T>(raw[i], vv);
#pragma unroll
    for (int j = 0; j < VEC; ++j) acc[j] += p * vv[j];
  }
  // reduce over key slots: lanes with equal `part` inside the wave, then waves
#pragma unroll
  for (int o = LPK; o < 64; o <<= 1) {
#pragma unroll
    for (int j = 0; j < VEC; ++j) acc[j] += __shfl_xor(acc[j], o, 64);
  }
  // z counted once per key (all LPK lanes of a key hold the same p): use part 0
  float zz = (part == 0) ? z : 0.f;
  zz = wave_sum(zz);
  if (lane < LPK) {
#pragma unroll
    for (int j = 0; j < VEC; ++j) red[wave][lane * VEC + j] = acc[j];
  }
  if (lane == 0) red[wave][DH] = zz;
  __syncthreads();
  float* out = a.part + ((long)s * (a.B * a.h) + bh) * (DH + 2);
  for (int i = tid; i < DH + 1; i += 256) out[i] = red[0][i] + red[1][i] + red[2][i] + red[3][i];
  if (tid == 0) out[DH + 1] = M;
  prof_end(a.prof_ts, t0);
}

// merge split partials + raw self column -> o, ssq, o_cat (one wave per (b, h))
template <typename T, int DH>
__global__ __launch_bounds__(64) void k_decode_merge(DecodeArgs<T> a) {
  constexpr int PER = DH / 64;
  const int bh = blockIdx.x, lane = threadIdx.x;
  const int b = bh / a.h, hh = bh - b * a.h;
  float qk = 0.f;
#pragma unroll
  for (int e = 0; e < PER; ++e)
    qk += to_f(a.q[(long)bh * DH + lane * PER + e]) * to_f(a.kself[(long)bh * DH + lane * PER + e]);
  const float ss = wave_sum(qk) * a.scale;
  float M = ss;
  for (int s = 0; s < a.nsplit; ++s) M = fmaxf(M, a.part[((long)s * (a.B * a.h) + bh) * (DH + 2) + DH + 1]);
  const float es = __expf(ss - M);
  float z = es;
  float acc[PER];
#pragma unroll
  for (int e = 0; e < PER; ++e) acc[e] = es * to_f(a.vself[(long)bh * DH + lane * PER + e]);
  for (int s = 0; s < a.nsplit; ++s) {
    const float* pp = a.part + ((long)s * (a.B * a.h) + bh) * (DH + 2);
    const float w = (pp[DH + 1] == NEG_INF) ? 0.f : __expf(pp[DH + 1] - M);
    z += w * pp[DH];
#pragma unroll
    for (int e = 0; e < PER; ++e) acc[e] += w * pp[lane * PER + e];
  }
  const float inv = 1.0f / z;
  float sq = 0.f;
#pragma unroll
  for (int e = 0; e < PER; ++e) {
    const float v = acc[e] * inv;
    sq += v * v;
    a.o[(long)b * a.d + hh * DH + lane * PER + e] = v;
    a.o_cat[(long)b * a.d + hh * DH + lane * PER + e] = from_f<T>(v);
  }
  sq = wave_sum(sq);
  if (lane == 0) a.ssq[(long)b * a.h + hh] = sq;
}

}  // namespace dm
