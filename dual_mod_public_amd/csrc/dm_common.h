// Common device helpers for the Dual-Mod CDNA4 kernels (gfx950, wave64).
//
// Storage types: float (fp32 parity runs) and __bf16 (production). All
// arithmetic that the reference keeps in fp32 islands (softmax, sigmoid,
// RMS, RoPE, blends) is fp32 here as well.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define DM_DEV __device__ __forceinline__
#define DM_HOST_DEV __host__ __device__

typedef __bf16 bf16;
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
typedef float floatx2 __attribute__((ext_vector_type(2)));

namespace dm {

constexpr int WAVE = 64;
constexpr int CMAX = 64;   // max chunk length of one cell (rows of one attention block)
constexpr int COMM_MAX_SPLITS = 8;   // committed-prefix splits of a cell's forward accumulator

DM_DEV float to_f(float x) { return x; }
DM_DEV float to_f(bf16 x) { return (float)x; }
template <typename T> DM_DEV T from_f(float x);
template <> DM_DEV float from_f<float>(float x) { return x; }
template <> DM_DEV bf16 from_f<bf16>(float x) { return (bf16)x; }

// 16-byte vector of storage elements: 8 bf16 or 4 fp32.
template <typename T> struct Vec16;
template <> struct Vec16<bf16> {
  static constexpr int N = 8;
  typedef uint4 raw;
};
template <> struct Vec16<float> {
  static constexpr int N = 4;
  typedef uint4 raw;
};

template <typename T>
DM_DEV void unpack16(const uint4& r, float* out) {
  if constexpr (sizeof(T) == 2) {
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[2 * i] = __uint_as_float(w[i] << 16);
      out[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  } else {
    out[0] = __uint_as_float(r.x);
    out[1] = __uint_as_float(r.y);
    out[2] = __uint_as_float(r.z);
    out[3] = __uint_as_float(r.w);
  }
}

template <typename T>
DM_DEV uint4 pack16(const float* in) {
  uint4 r;
  if constexpr (sizeof(T) == 2) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      bf16 lo = (bf16)in[2 * i];
      bf16 hi = (bf16)in[2 * i + 1];
      w[i] = (uint32_t)__builtin_bit_cast(uint16_t, lo) |
             ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
    }
    r.x = w[0]; r.y = w[1]; r.z = w[2]; r.w = w[3];
  } else {
    r.x = __float_as_uint(in[0]);
    r.y = __float_as_uint(in[1]);
    r.z = __float_as_uint(in[2]);
    r.w = __float_as_uint(in[3]);
  }
  return r;
}

// N consecutive elements (16-byte aligned, N a multiple of 16 / sizeof(T)) -> floats
template <typename T, int N>
DM_DEV void load_vec(const T* p, float* out) {
  constexpr int V = 16 / (int)sizeof(T);
#pragma unroll
  for (int i = 0; i < N / V; ++i) unpack16<T>(*reinterpret_cast<const uint4*>(p + i * V), out + i * V);
}
template <typename T, int N>
DM_DEV void store_vec(T* p, const float* in) {
  constexpr int V = 16 / (int)sizeof(T);
#pragma unroll
  for (int i = 0; i < N / V; ++i) *reinterpret_cast<uint4*>(p + i * V) = pack16<T>(in + i * V);
}
// store_vec with the non-temporal hint: for data no kernel of the same pass reads back (the
// forward tape), so that it does not displace reused operands from the caches
template <typename T, int N>
DM_DEV void store_vec_nt(T* p, const float* in) {
  constexpr int V = 16 / (int)sizeof(T);
  typedef unsigned int w4 __attribute__((ext_vector_type(4)));
#pragma unroll
  for (int i = 0; i < N / V; ++i) {
    const uint4 r = pack16<T>(in + i * V);
    const w4 w = {r.x, r.y, r.z, r.w};
    __builtin_nontemporal_store(w, reinterpret_cast<w4*>(p + i * V));
  }
}

// Make every value of an array available here (one wait for all of them) before the
// code that follows: on gfx9 the memory counter also counts stores, so a wait for a
// loaded value issued after some stores also waits for those stores; consuming all
// gathered values before the first store keeps store latency out of the chain.
template <int N> DM_DEV void settle(const float (&v)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i) asm volatile("" ::"v"(v[i]));
}
template <typename V> DM_DEV void settle_raw(const V& v) {
  static_assert(sizeof(V) % 4 == 0, "whole dwords");
  struct W { uint32_t w[sizeof(V) / 4]; };
  const W x = __builtin_bit_cast(W, v);
#pragma unroll
  for (int i = 0; i < (int)(sizeof(V) / 4); ++i) asm volatile("" ::"v"(x.w[i]));
}

typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// A load through a pointer into global memory, typed as such: a generic (flat) load
// would also count against the LDS counter that later LDS waits drain. V must be a
// native vector or scalar type (HIP's struct vectors copy through a generic
// reference, which loses the address space).
template <typename V, typename P> DM_DEV V ld_global(const P* p) {
  return *(const __attribute__((address_space(1))) V*)(p);
}

// 4 consecutive storage elements as one load / store: 8 bytes of bf16, 16 of fp32
template <typename T> struct Raw4 { typedef u32x4 type; };
template <> struct Raw4<bf16> { typedef u32x2 type; };
template <typename T> DM_DEV void unpack4(const typename Raw4<T>::type& r, float* out) {
  if constexpr (sizeof(T) == 2) {
    out[0] = __uint_as_float(r[0] << 16);
    out[1] = __uint_as_float(r[0] & 0xffff0000u);
    out[2] = __uint_as_float(r[1] << 16);
    out[3] = __uint_as_float(r[1] & 0xffff0000u);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = __uint_as_float(r[i]);
  }
}
template <typename T> DM_DEV void st4(T* p, const float* in) {
  if constexpr (sizeof(T) == 2) {
    uint32_t w[2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
      w[i] = (uint32_t)__builtin_bit_cast(uint16_t, (bf16)in[2 * i]) |
             ((uint32_t)__builtin_bit_cast(uint16_t, (bf16)in[2 * i + 1]) << 16);
    *reinterpret_cast<u32x2*>(p) = u32x2{w[0], w[1]};
  } else {
    *reinterpret_cast<floatx4*>(p) = floatx4{in[0], in[1], in[2], in[3]};
  }
}
// 8 consecutive storage elements: one 16-byte load of bf16, two of fp32
template <typename T> struct Raw8 {
  u32x4 v[sizeof(T) / 2];
};
template <typename T> DM_DEV Raw8<T> ld8_global(const T* p) {
  Raw8<T> r;
#pragma unroll
  for (int i = 0; i < (int)(sizeof(T) / 2); ++i) r.v[i] = ld_global<u32x4>(p + i * (16 / sizeof(T)));
  return r;
}
template <typename T> DM_DEV void unpack8(const Raw8<T>& r, float* out) {
  if constexpr (sizeof(T) == 2) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[2 * i] = __uint_as_float(r.v[0][i] << 16);
      out[2 * i + 1] = __uint_as_float(r.v[0][i] & 0xffff0000u);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = __uint_as_float(r.v[i >> 2][i & 3]);
  }
}
template <typename T> DM_DEV void st8(T* p, const float* in) {
  if constexpr (sizeof(T) == 2) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = (uint32_t)__builtin_bit_cast(uint16_t, (bf16)in[2 * i]) |
             ((uint32_t)__builtin_bit_cast(uint16_t, (bf16)in[2 * i + 1]) << 16);
    *reinterpret_cast<u32x4*>(p) = u32x4{w[0], w[1], w[2], w[3]};
  } else {
    *reinterpret_cast<floatx4*>(p) = floatx4{in[0], in[1], in[2], in[3]};
    *reinterpret_cast<floatx4*>(p + 4) = floatx4{in[4], in[5], in[6], in[7]};
  }
}
DM_DEV void unpackf4(const floatx4& v, float* out) {
#pragma unroll
  for (int i = 0; i < 4; ++i) out[i] = v[i];
}

// v if ok else 0, without a branch: the mask is made opaque to the optimizer so the
// (unconditional) load that produced v is not sunk into a divergent branch (the
// compiler then has to drain all outstanding loads at the join).
DM_DEV uint4 keep_if(uint4 v, bool ok) {
  unsigned m = ok ? 0xffffffffu : 0u;
  asm volatile("" : "+v"(m));
  v.x &= m; v.y &= m; v.z &= m; v.w &= m;
  return v;
}

// streaming 16-byte load (non-temporal hint: the data is read once)
template <typename T>
DM_DEV uint4 ld_nt(const T* p) {
  u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return uint4{v.x, v.y, v.z, v.w};
}

DM_DEV float sigmoidf_(float x) { return 1.0f / (1.0f + __expf(-x)); }

// tanh from the exponential: tanh(x) = sign(x) * (1 - e) / (1 + e), e = exp(-2|x|).
// Accurate to a few fp32 ulp away from 0; near 0 the odd Taylor series
// x - x^3/3 + 2x^5/15 is used (its error is below fp32 resolution for |x| < 2^-4).
DM_DEV float tanhf_(float x) {
  // both forms, then a select: a branch per element would diverge inside the wave (the
  // epilogues call this on every element of a tile); each input keeps the same formula
  const float ax = fabsf(x);
  const float x2 = x * x;
  const float series = x * (1.0f + x2 * (-1.0f / 3.0f + x2 * (2.0f / 15.0f)));
  const float e = __expf(-2.0f * ax);
  const float t = copysignf((1.0f - e) / (1.0f + e), x);
  return ax < 0.0625f ? series : t;
}

// the value as stored in dtype T (rounded to bf16; fp32 unchanged)
template <typename T> DM_DEV float stored(float x) { return to_f(from_f<T>(x)); }

// per-head RMS norm (attention.py:218-269): y = gain x r, r = rsqrt(sum of x^2 / dh + 1e-6)
constexpr float HEAD_NORM_EPS = 1e-6f;
DM_DEV float head_norm_r(float ss, float inv_dh) { return rsqrtf(ss * inv_dh + HEAD_NORM_EPS); }

// ---- wave reductions (full 64-lane and within 16-lane groups) ----------------
// sum over aligned groups of G consecutive lanes (G a power of two <= 64)
template <int G> DM_DEV float group_sum(float v) {
  static_assert(G >= 1 && G <= 64 && (G & (G - 1)) == 0, "lane group");
#pragma unroll
  for (int o = 1; o < G; o <<= 1) v += __shfl_xor(v, o, 64);
  return v;
}
DM_DEV float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
DM_DEV float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
// reduce across the 16 lanes that share lane>>4 (xor over the low 4 bits)
DM_DEV float group16_max(float v) {
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
DM_DEV float group16_sum(float v) {
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// ---- MFMA traits -------------------------------------------------------------
// 16x16 output tile; lane l holds D[4*(l>>4) + r][l & 15], r = 0..3.
// A fragment: row (l & 15), k-group (l >> 4); B fragment: col (l & 15), same k-group.
// bf16: v_mfma_f32_16x16x32_bf16, 8 consecutive k per lane (k = 8*(l>>4) + j).
// fp32: v_mfma_f32_16x16x4_f32, 1 k per lane (k = l >> 4).
template <typename T> struct Mfma;
template <> struct Mfma<bf16> {
  static constexpr int KSTEP = 32;   // k consumed per instruction
  static constexpr int KPL = 8;      // k elements held per lane
  typedef bf16x8 frag;
  static DM_DEV floatx4 mma(const frag& a, const frag& b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  // load KPL consecutive elements starting at p (16-byte aligned)
  static DM_DEV frag load(const bf16* p) { return *reinterpret_cast<const frag*>(p); }
  // The fragment of the transposed view of a row-major LDS matrix X (row stride ldx,
  // 8-byte aligned rows): lane l gets X[8 (l / 16) + v][l % 16], v = 0..7, i.e. the
  // B operand k = row, n = column. Two ds_read_b64_tr_b16: in each 16-lane group,
  // lane s names the 8 bytes at row (s / 4), column 4 (s % 4) of a 4 x 16 block and
  // receives that block's column s.
  static DM_DEV frag load_tr(const bf16* X, int ldx) {
    const int lane = threadIdx.x & 63, g = lane >> 4, s = lane & 15;
    const bf16* p = X + (8 * g + (s >> 2)) * ldx + 4 * (s & 3);
    const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
    const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p + 4 * ldx));
    // whole-vector casts (element-wise inserts into a bf16 vector are mis-lowered)
    const i16x8 both = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_bit_cast(frag, both);
  }
  static DM_DEV frag from_floats(const float* f) {
    frag r;
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = (bf16)f[i];
    return r;
  }
};
template <> struct Mfma<float> {
  static constexpr int KSTEP = 4;
  static constexpr int KPL = 1;
  typedef float frag;
  static DM_DEV floatx4 mma(const frag& a, const frag& b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
  static DM_DEV frag load(const float* p) { return *p; }
  // transposed view of a row-major LDS matrix X: lane l gets X[l / 16][l % 16]
  static DM_DEV frag load_tr(const float* X, int ldx) {
    const int lane = threadIdx.x & 63;
    return X[(lane >> 4) * ldx + (lane & 15)];
  }
  static DM_DEV frag from_floats(const float* f) { return f[0]; }
};

DM_DEV floatx4 zero4() { return floatx4{0.f, 0.f, 0.f, 0.f}; }

// sum of p[q] for q = q0, q0 + step, ... < n, given n <= q0 + MAXQ * step: every load
// is issued before the first add (indices clamped in bounds, excess terms masked),
// so a runtime-length reduction costs one memory latency rather than one per term.
template <int MAXQ>
DM_DEV float sum_strided(const float* __restrict__ p, int q0, int n, int step) {
  float v[MAXQ];
#pragma unroll
  for (int i = 0; i < MAXQ; ++i) v[i] = p[min(q0 + i * step, n - 1)];
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < MAXQ; ++i) s += (q0 + i * step < n) ? v[i] : 0.f;
  return s;
}

// sum of p[q] for q = 4 part + 16 j + i (i < 4, j < n / 16), n a multiple of 16 and at most 16 MAXJ:
// one 16-byte load per j, every load issued before the first add
template <int MAXJ>
DM_DEV float sum_quads(const float* __restrict__ p, int part, int n) {
  const int nj = n >> 4;
  floatx4 v[MAXJ];
#pragma unroll
  for (int j = 0; j < MAXJ; ++j) v[j] = *reinterpret_cast<const floatx4*>(p + 4 * part + 16 * min(j, nj - 1));
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < MAXJ; ++j) s += j < nj ? (v[j][0] + v[j][1]) + (v[j][2] + v[j][3]) : 0.f;
  return s;
}

// The per-row partial sums of the sweep arrays: ssq holds h <= MAX_HEADS per-head
// sums of squares per row, rowdot d / 32 <= MAX_ROWDOT partial dot products.
constexpr int MAX_HEADS = 64;
constexpr int MAX_ROWDOT = 128;

// ---- optional per-dispatch timing from the device clock ---------------------
// A timed launch gets prof_ts = [PROF_SLOTS] earliest block starts followed by
// [PROF_SLOTS] latest block ends (s_memrealtime ticks; block b folds into slot
// b % PROF_SLOTS). The kernel's span is max(end) - min(start), the interval a
// kernel-trace profiler reports. prof_ts is nullptr on every untimed launch.
constexpr int PROF_SLOTS = 1024;

DM_DEV uint64_t prof_begin(const uint64_t* prof_ts) { return prof_ts ? wall_clock64() : 0; }

DM_DEV void prof_end(uint64_t* prof_ts, uint64_t t0) {
  if (prof_ts == nullptr) return;   // uniform: a kernel argument
  __syncthreads();
  if (threadIdx.x == 0) {
    const int b = ((int)blockIdx.z * (int)gridDim.y + (int)blockIdx.y) * (int)gridDim.x + (int)blockIdx.x;
    atomicMin(reinterpret_cast<unsigned long long*>(prof_ts + b % PROF_SLOTS), (unsigned long long)t0);
    atomicMax(reinterpret_cast<unsigned long long*>(prof_ts + PROF_SLOTS + b % PROF_SLOTS),
              (unsigned long long)wall_clock64());
  }
}

}  // namespace dm
