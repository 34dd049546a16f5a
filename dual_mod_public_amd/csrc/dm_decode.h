// Decode kernels: split-P streaming read of the static tape + LSE merge.
#pragma once

#include "dm_attn.h"

namespace dm {

// ---------------------------------------------------------------------------
// decode: split-P read of the tape (attention.py:283-312 over a static tape)
// grid (nsplit, B*h); keys [lo + s*L, min(lo + (s+1)*L, pos))
// With pos_dev set, the position is read from device memory at run time (one launch
// shape serves every position, as a captured graph needs): the grid covers the whole
// tape, blocks past the position return, and (pos, lo, nsplit) follow from *pos_dev.
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
  const int* pos_dev = nullptr;   // device position (nullptr: pos / lo / nsplit above)
  int window = 0;                 // local_window (W tokens incl. self, 0 = full) for pos_dev
};

// a device position clamped into the tape (a caller's position past the tape reads and
// writes inside it instead of out of bounds)
DM_DEV int clamp_pos(int p, int tape_T) { return p < 0 ? 0 : (p >= tape_T ? tape_T - 1 : p); }
DM_DEV int window_lo(int pos, int W) { return (W > 0 && pos > W - 1) ? pos - (W - 1) : 0; }
template <typename T>
DM_DEV void dec_geometry(const DecodeArgs<T>& a, int& pos, int& lo, int& nsplit) {
  if (a.pos_dev == nullptr) {
    pos = a.pos; lo = a.lo; nsplit = a.nsplit;
    return;
  }
  pos = clamp_pos(*a.pos_dev, a.tape_T);
  lo = window_lo(pos, a.window);
  nsplit = pos > lo ? (pos - lo + a.split_len - 1) / a.split_len : 0;
}

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
  int pos, lo, nsplit;
  dec_geometry(a, pos, lo, nsplit);
  if (s >= nsplit) return;   // whole block: past the position (device-position grids only)
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int kslot = tid / LPK, part = tid - kslot * LPK;
  const int k_begin = lo + s * a.split_len;
  const int k_end = min(k_begin + a.split_len, pos);

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
  int pos, lo, nsplit;
  dec_geometry(a, pos, lo, nsplit);
  float qk = 0.f;
#pragma unroll
  for (int e = 0; e < PER; ++e)
    qk += to_f(a.q[(long)bh * DH + lane * PER + e]) * to_f(a.kself[(long)bh * DH + lane * PER + e]);
  const float ss = wave_sum(qk) * a.scale;
  float M = ss;
  for (int s = 0; s < nsplit; ++s) M = fmaxf(M, a.part[((long)s * (a.B * a.h) + bh) * (DH + 2) + DH + 1]);
  const float es = __expf(ss - M);
  float z = es;
  float acc[PER];
#pragma unroll
  for (int e = 0; e < PER; ++e) acc[e] = es * to_f(a.vself[(long)bh * DH + lane * PER + e]);
  for (int s = 0; s < nsplit; ++s) {
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

// device position: the RoPE rows of position *pos_dev -> rope[0, half) cos, rope[half, 2 half) sin
__global__ __launch_bounds__(64) void k_decode_pos_rope(const int* pos_dev, int tape_T, const float* cos,
                                                        const float* sin, int half, float* rope) {
  const int pos = clamp_pos(*pos_dev, tape_T);
  for (int i = threadIdx.x; i < half; i += 64) {
    rope[i] = cos[(long)pos * half + i];
    rope[half + i] = sin[(long)pos * half + i];
  }
}

// device position: the refined rows [B*h, DH] staged by the refine -> tape slot *pos_dev
template <typename T, int DH>
__global__ __launch_bounds__(DH) void k_decode_commit(const int* pos_dev, int tape_T, const T* Kst, const T* Vst,
                                                      T* Kt, T* Vt) {
  const int pos = clamp_pos(*pos_dev, tape_T);
  const long bh = blockIdx.x;
  const long dst = (bh * tape_T + pos) * DH + threadIdx.x;
  Kt[dst] = Kst[bh * DH + threadIdx.x];
  Vt[dst] = Vst[bh * DH + threadIdx.x];
}

// the trunk's fp32 residual stream around a decode step (models/dualmod/model.py:127-130,
// attention.py:74-83): x[r] += delta[r] (when delta), then y[r] = x[r] * rsqrt(mean(x[r]^2) + eps)
// * w (when w), in the storage dtype. One block per row; each thread re-reads only the
// elements it wrote itself.
template <typename T>
__global__ __launch_bounds__(256) void k_residual_rmsnorm(float* x, const T* delta, const float* w, T* y, int d,
                                                         float eps) {
  __shared__ float red[4];
  float* xr = x + (long)blockIdx.x * d;
  float ss = 0.f;
  for (int j = threadIdx.x; j < d; j += 256) {
    float v = xr[j];
    if (delta != nullptr) {
      v += to_f(delta[(long)blockIdx.x * d + j]);
      xr[j] = v;
    }
    ss += v * v;
  }
  if (w == nullptr) return;
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float rs = rsqrtf((red[0] + red[1] + red[2] + red[3]) / (float)d + eps);
  T* yr = y + (long)blockIdx.x * d;
  for (int j = threadIdx.x; j < d; j += 256) yr[j] = from_f<T>(xr[j] * rs * w[j]);
}

// torch.argmax's order: NaN is greater than every number (the first NaN wins), otherwise the
// larger value, the smaller index on ties. argmax_takes: a lane's scan in increasing column
// order replaces its pick only by a strictly greater value or by a first NaN.
DM_DEV bool argmax_takes(float f, float v) { return f > v || (f != f && v == v); }
DM_DEV bool argmax_better(float ov, int oi, float v, int idx) {
  const bool on = ov != ov, vn = v != v;
  if (on != vn) return on;
  if (on) return oi < idx;
  return ov > v || (ov == v && oi < idx);
}

// row argmax of x [rows, cols] (first index of the maximum; one block per row)
template <typename T>
__global__ __launch_bounds__(256) void k_argmax_rows(const T* x, long ld, int cols, int64_t* out) {
  __shared__ float bv[4];
  __shared__ int bi[4];
  const T* r = x + blockIdx.x * ld;
  float v = NEG_INF;
  int idx = 0x7fffffff;
  for (int j = threadIdx.x; j < cols; j += 256) {
    const float f = to_f(r[j]);
    if (argmax_takes(f, v)) { v = f; idx = j; }   // strided scan: this lane's first maximum
  }
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const float ov = __shfl_xor(v, o, 64);
    const int oi = __shfl_xor(idx, o, 64);
    if (argmax_better(ov, oi, v, idx)) { v = ov; idx = oi; }
  }
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) { bv[wave] = v; bi[wave] = idx; }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 4; ++w)
      if (argmax_better(bv[w], bi[w], v, idx)) { v = bv[w]; idx = bi[w]; }
    out[blockIdx.x] = idx == 0x7fffffff ? 0 : idx;
  }
}

// k_residual_rmsnorm with the row held in registers (d <= 256 NPT): every load (x, delta, w) is
// issued before the reduction and nothing is re-read; the same per-element arithmetic and the same
// order of the sums, so the same results.
template <typename T, int NPT>
__global__ __launch_bounds__(256) void k_residual_rmsnorm_reg(float* x, const T* delta, const float* w, T* y, int d,
                                                             float eps) {
  __shared__ float red[4];
  float* xr = x + (long)blockIdx.x * d;
  float v[NPT], wv[NPT];
#pragma unroll
  for (int i = 0; i < NPT; ++i) {
    const int j = threadIdx.x + 256 * i;
    const int jc = j < d ? j : 0;
    v[i] = xr[jc];
    if (delta != nullptr) v[i] += to_f(delta[(long)blockIdx.x * d + jc]);
    wv[i] = w != nullptr ? w[jc] : 0.f;
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NPT; ++i) {
    const int j = threadIdx.x + 256 * i;
    if (j < d) {
      if (delta != nullptr) xr[j] = v[i];
      ss += v[i] * v[i];
    }
  }
  if (w == nullptr) return;
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float rs = rsqrtf((red[0] + red[1] + red[2] + red[3]) / (float)d + eps);
  T* yr = y + (long)blockIdx.x * d;
#pragma unroll
  for (int i = 0; i < NPT; ++i) {
    const int j = threadIdx.x + 256 * i;
    if (j < d) yr[j] = from_f<T>(v[i] * rs * wv[i]);
  }
}

// k_argmax_rows for 16-byte aligned rows (ld a multiple of the vector width): 1024 threads per row,
// 16-byte loads. A lane visits its columns in increasing order (its vectors, then the tail columns,
// which come last in the row), so a strict > keeps its first maximum; lanes and waves then merge
// by value, the smaller index on ties; a NaN is the maximum (the first NaN wins), as torch.argmax.
template <typename T>
__global__ __launch_bounds__(1024) void k_argmax_rows_vec(const T* x, long ld, int cols, int64_t* out) {
  constexpr int VEC = 16 / (int)sizeof(T);
  __shared__ float bv[16];
  __shared__ int bi[16];
  const T* r = x + blockIdx.x * ld;
  const int nv = cols / VEC;
  float v = NEG_INF;
  int idx = 0x7fffffff;
  for (int q = threadIdx.x; q < nv; q += 1024) {
    float f[VEC];
    unpack16<T>(*reinterpret_cast<const uint4*>(r + (long)q * VEC), f);
#pragma unroll
    for (int e = 0; e < VEC; ++e)
      if (argmax_takes(f[e], v)) { v = f[e]; idx = q * VEC + e; }
  }
  for (int j = nv * VEC + threadIdx.x; j < cols; j += 1024) {
    const float f = to_f(r[j]);
    if (argmax_takes(f, v)) { v = f; idx = j; }
  }
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const float ov = __shfl_xor(v, o, 64);
    const int oi = __shfl_xor(idx, o, 64);
    if (argmax_better(ov, oi, v, idx)) { v = ov; idx = oi; }
  }
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) { bv[wave] = v; bi[wave] = idx; }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 16; ++w)
      if (argmax_better(bv[w], bi[w], v, idx)) { v = bv[w]; idx = bi[w]; }
    out[blockIdx.x] = idx == 0x7fffffff ? 0 : idx;
  }
}

}  // namespace dm
