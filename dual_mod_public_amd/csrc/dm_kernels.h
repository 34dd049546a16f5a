// Kernels of the DM forward cell and the layer projection pass.
#pragma once

#include "../../include/dm_abi.h"
#include "dm_attn.h"
#include "dm_gemm.h"

namespace dm {

// ---------------------------------------------------------------------------
// weight packing: gather rows of the reference parameters into packed buffers
// ---------------------------------------------------------------------------
struct PackSeg {
  const void* src;
  long src_ld;     // elements between source rows
  int src_col;     // first source column
  int nrows;
  int dst_row;
  int pad_;
};
constexpr int PACK_MAX_SEG = 48;
struct PackArgs {
  PackSeg seg[PACK_MAX_SEG];
  int nseg;
  int ncols;       // elements copied per row
  int esz;         // element size in bytes (2 or 4)
  void* dst;       // rows of ncols elements
};

static __global__ __launch_bounds__(256) void k_pack(PackArgs a) {
  int row = blockIdx.x;   // row index within this launch's segments (concatenated)
  int s = 0, acc = 0;
  while (s < a.nseg && row >= acc + a.seg[s].nrows) { acc += a.seg[s].nrows; ++s; }
  const PackSeg& sg = a.seg[s];
  const int sr = row - acc;
  const char* src = reinterpret_cast<const char*>(sg.src) + ((long)sr * sg.src_ld + sg.src_col) * a.esz;
  char* dst = reinterpret_cast<char*>(a.dst) + (long)(sg.dst_row + sr) * a.ncols * a.esz;
  const int nbytes = a.ncols * a.esz;
  for (int i = threadIdx.x * 2; i < nbytes; i += 512)
    *reinterpret_cast<uint16_t*>(dst + i) = *reinterpret_cast<const uint16_t*>(src + i);
}

template <typename T>
__global__ void k_to_f32(const T* __restrict__ src, float* __restrict__ dst, int n) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) dst[i] = to_f(src[i]);
}

// out [cols, rows] = in [rows, cols]^T, 64x64 tiles through LDS
template <typename T>
static __global__ __launch_bounds__(256) void k_transpose(const T* __restrict__ in, T* __restrict__ out, int rows,
                                                   int cols) {
  __shared__ T tile[64][65];
  const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
  for (int i = threadIdx.x; i < 64 * 64; i += 256) {
    const int r = i / 64, cc = i % 64;
    if (r0 + r < rows && c0 + cc < cols) tile[r][cc] = in[(long)(r0 + r) * cols + c0 + cc];
  }
  __syncthreads();
  for (int i = threadIdx.x; i < 64 * 64; i += 256) {
    const int cc = i / 64, r = i % 64;
    if (r0 + r < rows && c0 + cc < cols) out[(long)(c0 + cc) * rows + r0 + r] = tile[r][cc];
  }
}


// W[r, k] *= w[k] (in place)
template <typename T>
static __global__ __launch_bounds__(256) void k_scale_cols(T* __restrict__ W, const T* __restrict__ w, int rows,
                                                           int cols) {
  const long i = blockIdx.x * 256L + threadIdx.x;
  if (i < (long)rows * cols) W[i] = from_f<T>(to_f(W[i]) * to_f(w[i % cols]));
}

// u rows of the sweep weight grads: out[r] = o[r] * rsqrt(sum_p ssq[r, p] * inv_d + eps) * w
// (the RMSNorm the sweep GEMM applied), one wave per row, 16-byte vectors.
template <typename T>
DM_DEV void rms_rows_body(const T* __restrict__ o, int rows, int cols, const float* __restrict__ ssq, int nparts,
                          const T* __restrict__ w, float inv_d, float eps, T* __restrict__ out) {
  constexpr int V = 16 / (int)sizeof(T);
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const float rs = rsqrtf(wave_sum(lane < nparts ? ssq[(long)r * nparts + lane] : 0.f) * inv_d + eps);
  for (int c = lane * V; c < cols; c += 64 * V) {
    float f[V], wf[V];
    unpack16<T>(*reinterpret_cast<const uint4*>(o + (long)r * cols + c), f);
    unpack16<T>(*reinterpret_cast<const uint4*>(w + c), wf);
#pragma unroll
    for (int e = 0; e < V; ++e) f[e] *= rs * wf[e];
    *reinterpret_cast<uint4*>(out + (long)r * cols + c) = pack16<T>(f);
  }
}

template <typename T>
static __global__ __launch_bounds__(256) void k_rms_rows(const T* __restrict__ o, int rows, int cols,
                                                         const float* __restrict__ ssq, int nparts,
                                                         const T* __restrict__ w, float inv_d, float eps,
                                                         T* __restrict__ out) {
  rms_rows_body<T>(o, rows, cols, ssq, nparts, w, inv_d, eps, out);
}

template <typename T> struct RmsRowsUBody {
  static constexpr int THREADS = 256;
  struct Args {
    const T* o;
    int rows, cols;
    const float* ssq;
    int nparts;
    const T* w;
    float inv_d, eps;
    T* out;
  };
  static DM_DEV void run(const Args& a, int, int) {
    rms_rows_body<T>(a.o, a.rows, a.cols, a.ssq, a.nparts, a.w, a.inv_d, a.eps, a.out);
  }
};



// k_rms_rows over several row sets in one launch (set blockIdx.y): set i has `rows`
// rows o / ssq and writes output rows out_row0.. of one stacked output.
constexpr int RMS_MAX_SEG = 64;
struct RmsSeg {
  const void* o;
  const float* ssq;
  long out_row0;
  int rows;
};
struct RmsSegs {
  RmsSeg seg[RMS_MAX_SEG];
  int nseg;
};
template <typename T>
static __global__ __launch_bounds__(256) void k_rms_rows_multi(RmsSegs a, int cols, int nparts,
                                                               const T* __restrict__ w, float inv_d, float eps,
                                                               T* __restrict__ out) {
  constexpr int V = 16 / (int)sizeof(T);
  const RmsSeg& sg = a.seg[blockIdx.y];
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= sg.rows) return;
  const T* __restrict__ o = reinterpret_cast<const T*>(sg.o);
  T* __restrict__ dst = out + (sg.out_row0 + r) * (long)cols;
  const float rs = rsqrtf(wave_sum(lane < nparts ? sg.ssq[(long)r * nparts + lane] : 0.f) * inv_d + eps);
  for (int c = lane * V; c < cols; c += 64 * V) {
    float f[V], wf[V];
    unpack16<T>(*reinterpret_cast<const uint4*>(o + (long)r * cols + c), f);
    unpack16<T>(*reinterpret_cast<const uint4*>(w + c), wf);
#pragma unroll
    for (int e = 0; e < V; ++e) f[e] *= rs * wf[e];
    *reinterpret_cast<uint4*>(dst + c) = pack16<T>(f);
  }
}

// ---------------------------------------------------------------------------
// row RMSNorm (attn_norm, models/dualmod/attention.py:74-83): one wave per row
// ---------------------------------------------------------------------------
// Row m of a launch -> tensor row: the identity (lc < 0), or the rows of one chunk of every
// batch element of a [B, T, d] tensor (m = b * 2^lc + p -> b * T + pos0 + p).
struct RowMap {
  int lc = -1, T = 0, pos0 = 0;
  DM_DEV long operator()(int m) const {
    return lc < 0 ? (long)m : (long)(m >> lc) * T + pos0 + (m & ((1 << lc) - 1));
  }
};

// one wave per row
template <typename T>
DM_DEV void rmsnorm_row(const T* __restrict__ x, const T* __restrict__ w, T* __restrict__ y, long row, int d,
                        float eps) {
  const int lane = threadIdx.x & 63;
  const T* xr = x + row * d;
  float ss = 0.f;
  for (int j = lane; j < d; j += 64) {
    float v = to_f(xr[j]);
    ss += v * v;
  }
  ss = wave_sum(ss);
  const float rs = rsqrtf(ss / (float)d + eps);
  T* yr = y + row * d;
  for (int j = lane; j < d; j += 64) yr[j] = from_f<T>(to_f(xr[j]) * rs * to_f(w[j]));
}

template <typename T>
static __global__ __launch_bounds__(256) void k_rmsnorm_rows(const T* __restrict__ x, const T* __restrict__ w,
                                                      T* __restrict__ y, int M, int d, float eps) {
  const int m = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (m >= M) return;
  rmsnorm_row<T>(x, w, y, m, d, eps);
}

// the rows of one chunk (RowMap), as a grouped-launch body: grid (ceil(M / 4))
template <typename T> struct RmsRowsBody {
  static constexpr int THREADS = 256;
  struct Args {
    const T* x; const T* w; T* y;
    int M, d;
    float eps;
    RowMap map;
  };
  static DM_DEV void run(const Args& a, int bx, int) {
    const int m = bx * 4 + (threadIdx.x >> 6);
    if (m >= a.M) return;
    rmsnorm_row<T>(a.x, a.w, a.y, a.map(m), a.d, a.eps);
  }
};

// ---------------------------------------------------------------------------
// projection epilogue: xhat . [wq | wk | wv | w_gk_x | w_gv_x | v_gate]^T
// (fused_sweep.py:1403-1436 hoists; rope.py:22-33 on q and the raw key).
// A tile epilogue: the accumulators are staged in LDS, TILE_ROWS rows at a time, so the
// epilogue's registers do not compete with a 128 x 128 wave tile's. The block's columns are
// taken one head (DH columns) at a time; a head never straddles a segment (d is a multiple of
// DH). q / k / v heads: DH / 8 lanes per row, each with 4 consecutive RoPE pairs (jj, jj + DH/2);
// gate / v_gate columns: DH / 4 lanes per row, 4 consecutive columns each.
// ---------------------------------------------------------------------------
// a decode step's device position (graph replay), clamped to [0, cap) as the decode kernels do
DM_DEV int dev_position(const int* pos_dev, int cap) {
  const int p = *pos_dev;
  return p < 0 ? 0 : (p >= cap ? cap - 1 : p);
}

template <typename T, int DH, bool DEVPOS = false> struct EpiProj {
  int M, d, h;
  int Tl;        // rows per batch element in this call
  int Tbuf;      // T of the destination head buffers
  int buf_t0;    // buffer row of local row 0
  int rope_t0;   // RoPE position of local row 0
  const float* __restrict__ cos;
  const float* __restrict__ sin;
  const float* __restrict__ bias;   // [3d] fp32
  T* __restrict__ qr; T* __restrict__ kraw; T* __restrict__ kself; T* __restrict__ vraw;
  T* __restrict__ glogx; T* __restrict__ sig;   // storage dtype (as the reference's LayerBufs)
  int fusion;    // ctx_mod fusion: segment 5 is v_pre's x-half, stored as the raw pre-activation
  // v_norm (attention.py:218-234): v_raw = (x r) gain per head, x the stored projection,
  // r = rsqrt(mean x^2 + 1e-6); vgain [h] fp32 (nullptr = off); vpre keeps x (nullptr = not kept)
  const float* __restrict__ vgain = nullptr;
  T* __restrict__ vpre = nullptr;
  const int* pos_dev = nullptr;   // DEVPOS: RoPE row of local row 0 = *pos_dev clamped to [0, pos_cap)
  int pos_cap = 0;

  static constexpr int TILE_ROWS = 64;
  struct TilePre {};
  DM_DEV TilePre tile_prefetch(int, int) const { return TilePre{}; }

  template <int TR, int BN, int LDT>
  DM_DEV void tile_apply(const float* tile, int m0, int n0, const float*, const TilePre&, int) const {
    static_assert(BN % DH == 0, "whole heads per block");
    const int seg0 = n0 / d;
    if constexpr (BN > DH) {
      if ((n0 + BN - 1) / d == seg0) {   // every unit of the block in one segment (uniform)
        if (seg0 <= 1) {
          rope_block<TR, BN, LDT>(tile, m0, n0, seg0);
          return;
        }
        if (seg0 >= 3) {
          row_block<TR, BN, LDT>(tile, m0, n0, seg0);
          return;
        }
      }
    }
#pragma unroll 1
    for (int hu = 0; hu < BN / DH; ++hu) {
      const int col0 = n0 + hu * DH;
      const int seg = col0 / d, c0 = col0 - seg * d;
      if (seg <= 2) head_unit<TR, LDT>(tile + hu * DH, m0, seg, c0 / DH);
      else row_unit<TR, LDT>(tile + hu * DH, m0, seg, c0);
    }
  }

  // q (rotated), k (raw and rotated) or v (raw, or normed) of head hh for the chunk's rows
  template <int TR, int LDT>
  DM_DEV void head_unit(const float* tl, int m0, int seg, int hh) const {
    constexpr int L = DH / 8;     // lanes per row
    constexpr int RP = 256 / L;   // rows per pass
    static_assert(TR % RP == 0, "whole passes");
    const int jj = 4 * (threadIdx.x % L);
    const float gn = (seg == 2 && vgain != nullptr) ? vgain[hh] : 0.f;
#pragma unroll
    for (int pass = 0; pass < TR / RP; ++pass) {
      const int r = threadIdx.x / L + pass * RP, m = m0 + r;
      const floatx4 av = *reinterpret_cast<const floatx4*>(tl + r * LDT + jj);
      const floatx4 bv = *reinterpret_cast<const floatx4*>(tl + r * LDT + jj + DH / 2);
      float a[4] = {av.x, av.y, av.z, av.w}, b[4] = {bv.x, bv.y, bv.z, bv.w};
      float nr = 0.f;
      if (seg == 2 && vgain != nullptr) {   // the head's sum of squares over the row's L lanes
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          a[i] = stored<T>(a[i]);
          b[i] = stored<T>(b[i]);
          ss += a[i] * a[i] + b[i] * b[i];
        }
        nr = head_norm_r(group_sum<L>(ss), 1.0f / DH);
      }
      if (m >= M) continue;
      const int bb = m / Tl, t = m - bb * Tl;
      const long hrow = (((long)bb * h + hh) * Tbuf + buf_t0 + t) * DH + jj;
      if (seg <= 1) {
        const int r0 = DEVPOS ? dev_position(pos_dev, pos_cap) : rope_t0;
        const long rrow = (long)(r0 + t) * (DH / 2) + jj;
        float c[4], s[4], o1[4], o2[4];
        unpackf4(ld_global<floatx4>(cos + rrow), c);
        unpackf4(ld_global<floatx4>(sin + rrow), s);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          o1[i] = a[i] * c[i] - b[i] * s[i];
          o2[i] = b[i] * c[i] + a[i] * s[i];
        }
        if (seg == 0) {
          st4<T>(qr + hrow, o1);
          st4<T>(qr + hrow + DH / 2, o2);
        } else {
          st4<T>(kraw + hrow, a);
          st4<T>(kraw + hrow + DH / 2, b);
          st4<T>(kself + hrow, o1);
          st4<T>(kself + hrow + DH / 2, o2);
        }
      } else if (vgain != nullptr) {
        float ya[4], yb[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          ya[i] = (a[i] * nr) * gn;
          yb[i] = (b[i] * nr) * gn;
        }
        st4<T>(vraw + hrow, ya);
        st4<T>(vraw + hrow + DH / 2, yb);
        if (vpre != nullptr) {
          st4<T>(vpre + hrow, a);
          st4<T>(vpre + hrow + DH / 2, b);
        }
      } else {
        st4<T>(vraw + hrow, a);
        st4<T>(vraw + hrow + DH / 2, b);
      }
    }
  }

  // q or k of the block's BN / DH heads (one segment): the RoPE angles depend on the row and the
  // pair only, so each pass's cos / sin are loaded once for every head, all passes' before the first
  // head (head_unit's arithmetic, the same values)
  template <int TR, int BN, int LDT>
  DM_DEV void rope_block(const float* tl, int m0, int n0, int seg) const {
    constexpr int L = DH / 8, RP = 256 / L, NP = TR / RP;
    static_assert(TR % RP == 0, "whole passes");
    const int jj = 4 * (threadIdx.x % L);
    const int r0 = DEVPOS ? dev_position(pos_dev, pos_cap) : rope_t0;
    float cs[NP][4], sn[NP][4];
#pragma unroll
    for (int pass = 0; pass < NP; ++pass) {
      const int m = min(m0 + (int)threadIdx.x / L + pass * RP, M - 1);
      const int t = m - (m / Tl) * Tl;
      const long rrow = (long)(r0 + t) * (DH / 2) + jj;
      unpackf4(ld_global<floatx4>(cos + rrow), cs[pass]);
      unpackf4(ld_global<floatx4>(sin + rrow), sn[pass]);
    }
#pragma unroll 1
    for (int hu = 0; hu < BN / DH; ++hu) {
      const int hh = (n0 + hu * DH - seg * d) / DH;
      const float* tu = tl + hu * DH;
#pragma unroll
      for (int pass = 0; pass < NP; ++pass) {
        const int r = threadIdx.x / L + pass * RP, m = m0 + r;
        if (m >= M) continue;
        const floatx4 av = *reinterpret_cast<const floatx4*>(tu + r * LDT + jj);
        const floatx4 bv = *reinterpret_cast<const floatx4*>(tu + r * LDT + jj + DH / 2);
        const float a[4] = {av.x, av.y, av.z, av.w}, b[4] = {bv.x, bv.y, bv.z, bv.w};
        const int bb = m / Tl, t = m - bb * Tl;
        const long hrow = (((long)bb * h + hh) * Tbuf + buf_t0 + t) * DH + jj;
        float o1[4], o2[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          o1[i] = a[i] * cs[pass][i] - b[i] * sn[pass][i];
          o2[i] = b[i] * cs[pass][i] + a[i] * sn[pass][i];
        }
        if (seg == 0) {
          st4<T>(qr + hrow, o1);
          st4<T>(qr + hrow + DH / 2, o2);
        } else {
          st4<T>(kraw + hrow, a);
          st4<T>(kraw + hrow + DH / 2, b);
          st4<T>(kself + hrow, o1);
          st4<T>(kself + hrow + DH / 2, o2);
        }
      }
    }
  }

  // row units of the block's BN / DH column groups (one segment): every group's bias loaded
  // before the first group
  template <int TR, int BN, int LDT>
  DM_DEV void row_block(const float* tl, int m0, int n0, int seg) const {
    constexpr int NU = BN / DH, L = DH / 4;
    const int e = 4 * (threadIdx.x % L);
    float bs[NU][4];
#pragma unroll
    for (int hu = 0; hu < NU; ++hu) {
#pragma unroll
      for (int i = 0; i < 4; ++i) bs[hu][i] = 0.f;
      if (!(seg == 5 && fusion)) unpackf4(ld_global<floatx4>(bias + (seg - 3) * d + n0 + hu * DH - seg * d + e), bs[hu]);
    }
#pragma unroll 1
    for (int hu = 0; hu < NU; ++hu) row_rows<TR, LDT>(tl + hu * DH, m0, seg, n0 + hu * DH - seg * d, bs[hu]);
  }

  // gate logits (x-halves + bias) or sigma(v_gate) / fusion's raw v_pre x-half, fp32 math, stored
  // in the storage dtype
  template <int TR, int LDT>
  DM_DEV void row_unit(const float* tl, int m0, int seg, int c0) const {
    constexpr int L = DH / 4;
    const int e = 4 * (threadIdx.x % L), col = c0 + e;
    float bs[4] = {0.f, 0.f, 0.f, 0.f};
    if (!(seg == 5 && fusion)) unpackf4(ld_global<floatx4>(bias + (seg - 3) * d + col), bs);
    row_rows<TR, LDT>(tl, m0, seg, c0, bs);
  }
  template <int TR, int LDT>
  DM_DEV void row_rows(const float* tl, int m0, int seg, int c0, const float (&bs)[4]) const {
    constexpr int L = DH / 4;
    constexpr int RP = 256 / L;
    static_assert(TR % RP == 0, "whole passes");
    const int e = 4 * (threadIdx.x % L), col = c0 + e;
#pragma unroll
    for (int pass = 0; pass < TR / RP; ++pass) {
      const int r = threadIdx.x / L + pass * RP, m = m0 + r;
      if (m >= M) continue;
      const floatx4 v = *reinterpret_cast<const floatx4*>(tl + r * LDT + e);
      const int bb = m / Tl, t = m - bb * Tl;
      const long xrow = (long)bb * Tbuf + buf_t0 + t;
      float o[4] = {v.x + bs[0], v.y + bs[1], v.z + bs[2], v.w + bs[3]};
      if (seg <= 4) {
        st4<T>(glogx + xrow * 2 * d + (seg - 3) * d + col, o);
      } else {
        if (!fusion) {
#pragma unroll
          for (int i = 0; i < 4; ++i) o[i] = sigmoidf_(o[i]);
        }
        st4<T>(sig + xrow * d + col, o);
      }
    }
  }
};

// ---------------------------------------------------------------------------
// sweep geometry shared by the attention and GEMM epilogues of a cell
// ---------------------------------------------------------------------------
struct CellGeom {
  int B, c, d, h, dh;
  int pos0;        // absolute position (RoPE, cache row) of chunk row 0
  int buf_t0;      // row of chunk row 0 inside the layer buffers
  int Tbuf;        // T of the layer buffers (qr/kraw/kself/vraw/glogx/sig)
  int cache_T;     // T of the K/V cache
  int kmod_cols = 0;   // value columns [0, kmod_cols) belong to kmod heads (kmod_vraw_heads * dh)
  int kmod_mode = 0;   // dm_kmod_mode of those columns
  float v_clamp_tau = 0.f;   // v'' norm clamp radius per (row, head), 0 = off
  int rope_t0 = -1;    // RoPE table row of chunk row 0 (-1: pos0, tables indexed by position)
  int window = 0;      // local_window W (a row at position i reads keys >= i - W + 1); 0 = none
  // a decode step at a device position (graph replay): the epilogues instantiated for it read
  // the position here, clamped to [0, pos_cap), as their RoPE row and output row
  const int* pos_dev = nullptr;
  int pos_cap = 0;
};
// RoPE table row of chunk row p
DM_DEV int rope_row(const CellGeom& g, int p) { return (g.rope_t0 < 0 ? g.pos0 : g.rope_t0) + p; }

// ---------------------------------------------------------------------------
// v'' entry-norm clamp (attention.py:389-402): v <- v min(1, tau / ||v||) over each
// (row, head) of the refined value rows, in place, fp32 norm of the stored values.
// One wave per (row, head); the rows are (b, h) at bh * stride, chunk row p at row0 + p.
// ---------------------------------------------------------------------------
template <typename T, int DH>
DM_DEV void clamp_v_block(const CellGeom& g, T* __restrict__ V, long stride, int row0, int N, float tau, int bx) {
  constexpr int PER = (DH + 63) / 64;   // elements per lane
  const int lane = threadIdx.x & 63;
  const long w = bx * 4L + (threadIdx.x >> 6);   // (row m, head hd) = (w / h, w % h)
  if (w >= (long)N * g.h) return;
  const int m = (int)(w / g.h), hd = (int)(w - (long)m * g.h);
  const int b = m / g.c, p = m - b * g.c;
  T* row = V + ((long)b * g.h + hd) * stride + (long)(row0 + p) * DH;
  float v[PER], ss = 0.f;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int e = lane + 64 * i;
    v[i] = e < DH ? to_f(row[e]) : 0.f;
    ss += v[i] * v[i];
  }
  const float n = sqrtf(wave_sum(ss));
  if (n <= tau) return;   // wave-uniform: identity inside the radius
  const float sc = tau / fmaxf(n, 1e-20f);
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int e = lane + 64 * i;
    if (e < DH) row[e] = from_f<T>(v[i] * sc);
  }
}

template <typename T, int DH>
static __global__ __launch_bounds__(256) void k_clamp_v(CellGeom g, T* __restrict__ V, long stride, int row0,
                                                        int N, float tau) {
  clamp_v_block<T, DH>(g, V, stride, row0, N, tau, blockIdx.x);
}

template <typename T, int DH> struct ClampBody {
  static constexpr int THREADS = 256;
  struct Args {
    CellGeom g;
    T* V;
    long stride;
    int row0, N;
    float tau;
  };
  static DM_DEV void run(const Args& a, int bx, int) { clamp_v_block<T, DH>(a.g, a.V, a.stride, a.row0, a.N, a.tau, bx); }
};

// Value blend of column col (attention.py:362-384): v'' = g v_raw + (1 - g) v_ctx, except
// for the kmod heads: raw (v_raw, or tanh(v_raw) with the tanh bound) or, gated_norm,
// the blend with v_ctx = 0.
DM_DEV float value_blend(const CellGeom& g, int col, float gv, float vr, float vc) {
  if (col < g.kmod_cols) {
    if (g.kmod_mode == DM_KMOD_GATED_NORM) return gv * vr;
    return g.kmod_mode == DM_KMOD_RAW_TANH ? tanhf_(vr) : vr;
  }
  return gv * vr + (1.f - gv) * vc;
}

// ---------------------------------------------------------------------------
// committed-prefix accumulator (scan_cell_fwd.py:119-129): per (split, b, h),
// keys [s*L, min((s+1)*L, pos0)) -> unnormalised A [c, dh], Z [c], m [c].
// The next key tile is loaded into registers while the current one is used.
// ---------------------------------------------------------------------------
template <typename T> struct CommArgs {
  CellGeom g;
  const T* qr;
  const T* Kc;
  const T* Vc;
  int split_len;
  float scale;
  float* A;    // [nsplit, B*h, c, dh]
  float* Z;    // [nsplit, B*h, c]
  float* Mx;   // [nsplit, B*h, c]
  int nsplit = 0;   // splits of this cell (a grouped launch's grid covers the largest)
  int kstart = 0;   // first committed key of split 0 (the window's start for chunk row 0)
  int kend = 0;     // end of the keys the splits cover (the cell's last committed keys are the
                    // first sweep's attention's: AttendArgs::prev_lo)
};

struct KeyBound {
  int n;
  DM_DEV bool operator()(int, int key) const { return key < n; }
};
// intra keys of chunk row q0 + q: key < q0 + q, and at most wlim rows back (W - 1 with a
// window, a huge value without)
struct KeyStrictLower {   // q is block-relative; q0 = the block's first query row
  int q0, wlim;
  DM_DEV bool operator()(int q, int key) const { return key < q + q0 && q + q0 - key <= wlim; }
};
DM_DEV int intra_wlim(int window) { return window > 0 ? window - 1 : (1 << 30); }
// committed keys of a tile starting at position k0: key < n, and inside chunk row q's window
// (position k0 + key >= lo0 + q, lo0 = pos0 - W + 1; a very negative lo0 without a window)
struct KeyWindow {
  int n, k0, lo0;
  DM_DEV bool operator()(int q, int key) const { return key < n && k0 + key >= lo0 + q; }
};
constexpr int NO_WINDOW_LO = -(1 << 30);

// in the LDS at lds (AttnCfg<T, DH>::LDS_ELEMS elements)
template <typename T, int DH>
DM_DEV void comm_partial_block_at(const CommArgs<T>& a, int s, int bh, T* lds) {
  using C = AttnCfg<T, DH>;
  T* Ks = lds;
  T* Vs = Ks + C::KT * C::LDK;
  T* Ps = Vs + C::KT * C::LDK;
  const CellGeom& g = a.g;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int BH = g.B * g.h;
  const int k_begin = a.kstart + s * a.split_len;
  const int k_end = min(k_begin + a.split_len, a.kend);
  const int qrow = 16 * wave + (lane & 15);
  const int lo0 = g.window > 0 ? g.pos0 - g.window + 1 : NO_WINDOW_LO;

  const T* Kb = a.Kc + (long)bh * g.cache_T * DH;
  const T* Vb = a.Vc + (long)bh * g.cache_T * DH;
  KVRegs<T, DH> kv;
  if (k_begin < k_end) load_kv<T, DH>(Kb + (long)k_begin * DH, Vb + (long)k_begin * DH, DH,
                                      min(C::KT, k_end - k_begin), kv);
  typename Mfma<T>::frag qf[C::NKS];
  load_q_frags<T, DH>(a.qr + ((long)bh * g.Tbuf + g.buf_t0 + qrow) * DH, qrow < g.c, qf);
  FlashState<T, DH> st;
  flash_init(st);
  for (int k0 = k_begin; k0 < k_end; k0 += C::KT) {
    const int nv = min(C::KT, k_end - k0);
    __syncthreads();
    store_kv<T, DH>(kv, Ks, Vs);
    __syncthreads();
    const int k1 = k0 + C::KT;
    if (k1 < k_end) load_kv<T, DH>(Kb + (long)k1 * DH, Vb + (long)k1 * DH, DH, min(C::KT, k_end - k1), kv);
    flash_tile<T, DH>(qf, Ks, Vs, Ps + wave * 16 * C::LDP, a.scale, KeyWindow{nv, k0, lo0}, st);
  }
  const int g4 = lane >> 4, col = lane & 15;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int q = 16 * wave + 4 * g4 + r;
    const float z = group16_sum(st.z[r]);
    if (q < g.c) {
      const long base = ((long)s * BH + bh) * g.c + q;
      if (col == 0) {
        a.Z[base] = z;
        a.Mx[base] = st.m[r];
      }
#pragma unroll
      for (int dt = 0; dt < C::NDT; ++dt) a.A[base * DH + col + 16 * dt] = st.O[dt][r];
    }
  }
}

template <typename T, int DH>
DM_DEV void comm_partial_block(const CommArgs<T>& a, int s, int bh) {
  __shared__ __attribute__((aligned(16))) T lds[AttnCfg<T, DH>::LDS_ELEMS];
  comm_partial_block_at<T, DH>(a, s, bh, lds);
}

template <typename T, int DH>
static __global__ __launch_bounds__(256) void k_comm_partial(CommArgs<T> a) {
  comm_partial_block<T, DH>(a, blockIdx.x, blockIdx.y);
}


template <typename T, int DH> struct CommBody {
  static constexpr int THREADS = 256;
  using Args = CommArgs<T>;
  static DM_DEV void run(const Args& a, int bx, int by) {
    if (bx >= a.nsplit) return;   // uniform: past this cell's splits
    comm_partial_block<T, DH>(a, bx, by);
  }
};

// ---------------------------------------------------------------------------
// one sweep's read (scan_cell_fwd.py:63-85 / :132-149): intra rows (strict
// lower) + raw self column, merged with the committed accumulator. The first
// sweep of a cell merges the committed split partials (flash-decoding style)
// and writes the merged (A, Z, m) for the later sweeps.
// Writes o [B*c, d] in the storage dtype and per-head sums of squares of the
// stored values, ssq [B*c, h] (the norm_ctx RMS of the next GEMM).
// ---------------------------------------------------------------------------
template <typename T> struct AttendArgs {
  CellGeom g;
  const T* qr; const T* kself; const T* vraw;   // layer buffers
  const T* Kin; const T* Vin;                   // intra rows of this sweep: (b,h) at bh*in_stride,
  long in_stride; int in_row0;                  //   chunk row p at row in_row0 + p
  // The committed prefix [kstart, pos0): merged_in, the merged state A / Z / Mx of the cell's first
  // sweep (later sweeps); else the first sweep merges nsplit split partials (keys [kstart, prev_lo))
  // and its last keys [prev_lo, pos0) (cache rows Kc / Vc) and stores the merged state.
  int nsplit;                                   // split partials to merge
  const float* Ap; const float* Zp; const float* Mp;   // partials [nsplit, B*h, c, ...]
  float* A; float* Z; float* Mx;                // merged committed state [B*h, c, ...]
  float scale;
  T* o;         // [B*c, d]
  float* ssq;   // [B*c, h]
  T* ocat;      // [B, Tbuf, d] or nullptr (buffer rows buf_t0 + p)
  float* o_last;    // [B*c, d] or nullptr
  float* stat_m;    // [B*h, c] final row max (or nullptr)
  float* stat_z;    // [B*h, c] final row sum (or nullptr)
  int merged_in = 0;
  const T* Kc = nullptr;   // the committed cache rows (row stride DH, (b, h) stride g.cache_T DH)
  const T* Vc = nullptr;
  int prev_lo = 0;         // first of the last committed keys (pos0: none)
};

// The attention of query rows [q0, q0 + 16 NW) of (b, h) = bh, NW waves of 16 rows. With
// V_STAGED the block has already written the intra V rows [0, 16 NW) into Vs (the fused
// GEMM 2 + attention kernel); otherwise K and V are both loaded here.
template <typename T, int DH, int NW, bool V_STAGED>
DM_DEV void attend_rows(const AttendArgs<T>& a, int bh, int q0, T* lds) {
  using C = AttnCfg<T, DH>;
  T* Ks = lds;
  T* Vs = Ks + C::KT * C::LDK;
  T* Ps = Vs + C::KT * C::LDK;
  const CellGeom& g = a.g;
  const int b = bh / g.h, hh = bh - b * g.h;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g4 = lane >> 4, col = lane & 15;
  const int wq = q0 + 16 * wave;               // the wave's first query row
  const int qrow = wq + col;
  const long lrow0 = (long)bh * g.Tbuf + g.buf_t0;   // layer-buffer row of chunk row 0
  const int BH = g.B * g.h;

  KVRegs<T, DH, 64 * NW> kv;   // keys < the block's last row (strict lower)
  if constexpr (V_STAGED)
    load_k<T, DH, 64 * NW>(a.Kin + (long)bh * a.in_stride + (long)a.in_row0 * DH, DH, min(g.c, q0 + 16 * NW), kv);
  else
    load_kv<T, DH, 64 * NW>(a.Kin + (long)bh * a.in_stride + (long)a.in_row0 * DH,
                            a.Vin + (long)bh * a.in_stride + (long)a.in_row0 * DH, DH, min(g.c, q0 + 16 * NW), kv);
  typename Mfma<T>::frag qf[C::NKS];
  load_q_frags<T, DH>(a.qr + (lrow0 + qrow) * DH, qrow < g.c, qf);
  FlashState<T, DH> st;
  flash_init(st);
  // the cell's last committed keys (first sweep), loaded with the intra rows where the registers
  // allow (at most 8 16-byte vectors of each per thread), else right before their use
  [[maybe_unused]] const bool prev = !V_STAGED && !a.merged_in && a.prev_lo < g.pos0;
  [[maybe_unused]] KVRegs<T, DH, 64 * NW> pk;
  [[maybe_unused]] const long pb = (long)bh * g.cache_T * DH + (long)a.prev_lo * DH;
  constexpr bool PREV_EARLY = KVRegs<T, DH, 64 * NW>::NV <= 8;
  if constexpr (!V_STAGED && PREV_EARLY) {
    if (prev) load_kv<T, DH, 64 * NW>(a.Kc + pb, a.Vc + pb, DH, g.pos0 - a.prev_lo, pk);
  }
  bool store_merged = false;
  if (a.merged_in) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int q = wq + 4 * g4 + r;
      if (q < g.c) {
        const long o = (long)bh * g.c + q;
        st.m[r] = a.Mx[o];
        st.z[r] = (col == 0) ? a.Z[o] : 0.f;
#pragma unroll
        for (int dt = 0; dt < C::NDT; ++dt) st.O[dt][r] = a.A[o * DH + col + 16 * dt];
      }
    }
  } else if (a.nsplit > 0) {
    // merge the split partials: per row, every split's loads are issued before the
    // first use (indices clamped in bounds, splits >= nsplit masked)
    constexpr int MS = COMM_MAX_SPLITS;
#pragma unroll
    for (int r = 0; r < 4; ++r) {   // one row at a time (scheduling barrier below):
                                    // MS * (2 + DH/16) loads in flight
      const int qc = min(wq + 4 * g4 + r, g.c - 1);
      float ms[MS], zs[MS], as[MS][C::NDT];
#pragma unroll
      for (int s = 0; s < MS; ++s) {
        const long base = ((long)min(s, a.nsplit - 1) * BH + bh) * g.c + qc;
        ms[s] = a.Mp[base];
        zs[s] = a.Zp[base];
#pragma unroll
        for (int dt = 0; dt < C::NDT; ++dt) as[s][dt] = a.Ap[base * DH + col + 16 * dt];
      }
      float M = NEG_INF;
#pragma unroll
      for (int s = 0; s < MS; ++s) M = (s < a.nsplit) ? fmaxf(M, ms[s]) : M;
      float z = 0.f;
#pragma unroll
      for (int dt = 0; dt < C::NDT; ++dt) st.O[dt][r] = 0.f;
#pragma unroll
      for (int s = 0; s < MS; ++s) {
        const float w = (s < a.nsplit && ms[s] != NEG_INF) ? __expf(ms[s] - M) : 0.f;
        z += w * zs[s];
#pragma unroll
        for (int dt = 0; dt < C::NDT; ++dt) st.O[dt][r] += w * as[s][dt];
      }
      st.m[r] = M;
      st.z[r] = (col == 0) ? z : 0.f;   // per-lane partial sums
      __builtin_amdgcn_sched_barrier(0);
    }
    store_merged = true;
  }
  if constexpr (!V_STAGED) {
    if (prev) {
      // keys [prev_lo, pos0), inside each row's window: lo0 + q0 + q for block row q
      const int lo0 = g.window > 0 ? g.pos0 - g.window + 1 : NO_WINDOW_LO;
      if constexpr (!PREV_EARLY) load_kv<T, DH, 64 * NW>(a.Kc + pb, a.Vc + pb, DH, g.pos0 - a.prev_lo, pk);
      store_kv<T, DH, 64 * NW>(pk, Ks, Vs);
      __syncthreads();
      flash_tile<T, DH>(qf, Ks, Vs, Ps + wave * 16 * C::LDP, a.scale,
                        KeyWindow{g.pos0 - a.prev_lo, a.prev_lo, lo0 == NO_WINDOW_LO ? lo0 : lo0 + q0}, st);
      __syncthreads();   // Ks / Vs are free for the intra rows
      store_merged = true;
    }
  }
  if (store_merged) {   // the merged committed state, read by the cell's later sweeps
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int q = wq + 4 * g4 + r;
      const float zt = group16_sum(st.z[r]);
      if (q < g.c) {
        const long o = (long)bh * g.c + q;
#pragma unroll
        for (int dt = 0; dt < C::NDT; ++dt) a.A[o * DH + col + 16 * dt] = st.O[dt][r];
        if (col == 0) {
          a.Z[o] = zt;
          a.Mx[o] = st.m[r];
        }
      }
    }
  }
  // raw self column inputs, loaded before the barriers below: partial <q_r, k_self_r>
  // over this lane's PER elements, and v_raw at the lane's output columns
  constexpr int PER = DH / 16;
  float sdot[4], vself[4][C::NDT];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int qc = min(wq + 4 * g4 + r, g.c - 1);
    const T* qp = a.qr + (lrow0 + qc) * DH + col * PER;
    const T* kp = a.kself + (lrow0 + qc) * DH + col * PER;
    float dot = 0.f;
#pragma unroll
    for (int e = 0; e < PER; ++e) dot += to_f(qp[e]) * to_f(kp[e]);
    sdot[r] = dot;
    const T* vp = a.vraw + (lrow0 + qc) * DH;
#pragma unroll
    for (int dt = 0; dt < C::NDT; ++dt) vself[r][dt] = to_f(vp[col + 16 * dt]);
  }
  if constexpr (V_STAGED) store_k<T, DH, 64 * NW>(kv, Ks);
  else store_kv<T, DH, 64 * NW>(kv, Ks, Vs);
  __syncthreads();
  flash_tile<T, DH>(qf, Ks, Vs, Ps + wave * 16 * C::LDP, a.scale, KeyStrictLower{q0, intra_wlim(g.window)}, st);

  // raw self column: s_self = scale * <q_r, k_self_r> (fp32), value v_raw
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float ss = group16_sum(sdot[r]) * a.scale;
    const float mnew = fmaxf(st.m[r], ss);
    const float alpha = (st.m[r] == NEG_INF) ? 0.f : __expf(st.m[r] - mnew);
    const float es = __expf(ss - mnew);
#pragma unroll
    for (int dt = 0; dt < C::NDT; ++dt) st.O[dt][r] = st.O[dt][r] * alpha + es * vself[r][dt];
    st.z[r] = st.z[r] * alpha + (col == 0 ? es : 0.f);
    st.m[r] = mnew;
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int q = wq + 4 * g4 + r;
    const float zt = group16_sum(st.z[r]);
    const float inv = 1.0f / zt;
    float sq = 0.f;
    float ov[C::NDT];
#pragma unroll
    for (int dt = 0; dt < C::NDT; ++dt) {
      ov[dt] = to_f(from_f<T>(st.O[dt][r] * inv));   // the stored (rounded) value
      sq += ov[dt] * ov[dt];
    }
    sq = group16_sum(sq);
    if (q < g.c) {
      const long n = (long)b * g.c + q;
      T* orow = a.o + n * g.d + hh * DH;
#pragma unroll
      for (int dt = 0; dt < C::NDT; ++dt) orow[col + 16 * dt] = from_f<T>(ov[dt]);
      if (a.o_last != nullptr) {
        float* lrow = a.o_last + n * g.d + hh * DH;
#pragma unroll
        for (int dt = 0; dt < C::NDT; ++dt) lrow[col + 16 * dt] = ov[dt];
      }
      if (a.ocat != nullptr) {
        T* crow = a.ocat + ((long)b * g.Tbuf + g.buf_t0 + q) * g.d + hh * DH;
#pragma unroll
        for (int dt = 0; dt < C::NDT; ++dt) crow[col + 16 * dt] = from_f<T>(ov[dt]);
      }
      if (col == 0) {
        a.ssq[n * g.h + hh] = sq;
        if (a.stat_m != nullptr) {
          a.stat_m[(long)bh * g.c + q] = st.m[r];
          a.stat_z[(long)bh * g.c + q] = zt;
        }
      }
    }
  }
}

// NW waves per block, 16 query rows per wave: block y takes rows [16 NW y, 16 NW (y + 1)),
// so a (b, h) spreads over 4 / NW blocks (more blocks when B*h alone underfills the GPU).
template <typename T, int DH, int NW>
static __global__ __launch_bounds__(64 * NW) void k_attend(AttendArgs<T> a) {
  __shared__ __attribute__((aligned(16))) T lds[AttnCfg<T, DH>::LDS_ELEMS];
  const int q0 = 16 * NW * (int)blockIdx.y;   // the block's first query row
  if (q0 >= a.g.c) return;                     // uniform: no rows in this block
  attend_rows<T, DH, NW, false>(a, blockIdx.x, q0, lds);
}

template <typename T, int DH, int NW> struct AttendBody {
  static constexpr int THREADS = 64 * NW;
  using Args = AttendArgs<T>;
  static DM_DEV void run(const Args& a, int bx, int by) {
    __shared__ __attribute__((aligned(16))) T lds[AttnCfg<T, DH>::LDS_ELEMS];
    const int q0 = 16 * NW * by;
    if (q0 >= a.g.c) return;
    attend_rows<T, DH, NW, false>(a, bx, q0, lds);
  }
};

// ---------------------------------------------------------------------------
// sweep GEMM 1: u . W_sweep^T (u = RMSNorm_ctx(o) on the A load)
// (attention.py:314-387; fused_sweep.py:514-611, :1064-1089). W_sweep rows are
// packed in 64-row groups so that one wave's 16 x 64 tile is self-contained:
//   [0, 2d)  per head g, group q < DH/32:  k_ctx cols 16q.., k_ctx cols DH/2+16q..,
//            g_k(u) cols 16q.., g_k(u) cols DH/2+16q..  -> blend, RoPE, K rows
//   linear [2d, 4d) per head g, group q < DH/32: v_ctx cols 32q.. | g_v(u) cols 32q..
//            -> blend, V rows
//   mult   [2d, 3d) v_map(u) -> v_in = lam*u + sig * tanh(.)  (fusion: v_pre u-half ->
//          v_in = u + silu(px + .), px = v_pre x-half from the projection in the sig buffer)
//          [3d, 4d) g_v(u)   -> scratch for GEMM 2 (storage dtype, as the GEMM's raw outputs)
// save != nullptr stores the raw GEMM outputs [rows, 4d] in this packed order.
// ---------------------------------------------------------------------------
template <typename T, int DH, int NG = 1, bool DEVPOS = false, bool SPLIT = false> struct EpiSweep1 {
  CellGeom g;
  int M, ctx_mod;
  float lam;
  const T* __restrict__ kraw; const T* __restrict__ vraw;
  const T* __restrict__ glogx; const T* __restrict__ sig;   // the projection's gate inputs
  const float* __restrict__ cos; const float* __restrict__ sin;
  const T* __restrict__ o; const T* __restrict__ normw;   // u = o * rs * w for v_in's lam*u term
  T* __restrict__ Kout; T* __restrict__ Vout;             // refined rows: (b,h) at bh*out_stride,
  long out_stride; int out_row0;                          //   chunk row p at row out_row0 + p
  T* __restrict__ vin; T* __restrict__ gvu;               // v_in, g_v(u) for GEMM 2 (storage dtype)
  T* __restrict__ save;
  // Per-head norms of the GEMM outputs (attention.py:238-269), fp32 gains [h], nullptr = off:
  // kgain k_ctx (norm_kctx), vgain the linear ctx_mod's v_ctx (norm_vctx). Either needs block
  // tiles of NG = DH / 32 column groups (BN = 2 DH: one head's k_ctx / g_k(u), or v_ctx / g_v(u),
  // columns), so that the block holds whole heads.
  const float* __restrict__ kgain = nullptr;
  const float* __restrict__ vgain = nullptr;

  // Block tile 64 x 64 NG: NG packed column groups of 64. Thread t owns row t / 4 and the
  // column quad lc0 = 4 (t % 4) .. + 3 of each group's four 16-column sections, so its global
  // inputs and outputs are runs of 4 consecutive elements. With up to two groups the inputs
  // are gathered during the k-loop's last stage; with more, at the start of the epilogue.
  // SPLIT: a 512-thread block of two groups (eight waves), each 256-thread half owning one
  // group (threads t and t + 256 the same row and quad); no per-head norms.
  static_assert(!SPLIT || NG == 2, "split: two groups, one per 256-thread half");
  static constexpr int NGT = SPLIT ? 1 : NG;   // groups per thread
  DM_DEV static int trow() { return (SPLIT ? (int)(threadIdx.x & 255) : (int)threadIdx.x) >> 2; }
  DM_DEV static int tquad() { return threadIdx.x & 3; }
  DM_DEV static int tgroup() { return SPLIT ? (int)(threadIdx.x >> 8) : 0; }
  struct GroupPre {
    typename Raw4<T>::type x[4];    // K: gx_a, gx_b; linear V: gx x2; v_map: sig x4 (storage dtype)
    floatx4 f[2];                   // K: cos, sin
    typename Raw4<T>::type h[8];    // K: kraw_a, kraw_b; linear V: v_raw x2; v_map: o x4, norm weight x4
  };
  static constexpr bool LATE = NG <= 2;
  struct TilePre {
    GroupPre p[LATE ? NGT : 1];
  };
  // tile_prefetch issues exactly 14 loads per group of the thread (one per x / f / h slot,
  // unconditionally)
  static constexpr int LATE_GATHERS = LATE ? 14 * NGT : 0;
  DM_DEV TilePre tile_prefetch(int m0, int n0) const {
    TilePre pr{};
    if constexpr (LATE) {
#pragma unroll
      for (int gi = 0; gi < NGT; ++gi) pr.p[gi] = group_prefetch(m0, n0 + 64 * (gi + tgroup()));
    }
    return pr;
  }
  DM_DEV GroupPre group_prefetch(int m0, int n0) const {
    const int r = trow(), lc0 = 4 * tquad();
    const int d = g.d, h = g.h;
    const int m = min(m0 + r, M - 1);
    const int b = m / g.c, p = m - b * g.c;
    const int t = g.buf_t0 + p, pos = DEVPOS ? dev_position(g.pos_dev, g.pos_cap) + p : rope_row(g, p);
    const long xrow = (long)b * g.Tbuf + t;
    // The (block-uniform) branches only pick addresses; the loads follow them
    // unconditionally (unused slots re-read a valid address), so no loaded value
    // has to be merged, and waited for, where the branches join.
    const T* xp[4];
    const float* fp[2];
    const T* hp[8];
    const T* x0 = glogx + xrow * 2 * d;
    const T* h0 = kraw + ((long)b * h * g.Tbuf + t) * DH;
#pragma unroll
    for (int k = 0; k < 4; ++k) xp[k] = x0;
    fp[0] = cos + (long)pos * (DH / 2);
    fp[1] = sin + (long)pos * (DH / 2);
#pragma unroll
    for (int k = 0; k < 8; ++k) hp[k] = h0;
    if (n0 < 2 * d) {
      const int hd = n0 / (2 * DH), jj = 16 * ((n0 % (2 * DH)) / 64) + lc0;
      const long lrow = (((long)b * h + hd) * g.Tbuf + t) * DH + jj;
      xp[0] = x0 + hd * DH + jj;
      xp[1] = xp[0] + DH / 2;
      fp[0] += jj;
      fp[1] += jj;
      hp[0] = kraw + lrow;
      hp[1] = hp[0] + DH / 2;
    } else if (ctx_mod == 0) {
      const int cl = n0 - 2 * d;
      const int hd = cl / (2 * DH), e = 32 * ((cl % (2 * DH)) / 64) + lc0;
      const long lrow = (((long)b * h + hd) * g.Tbuf + t) * DH + e;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        xp[j] = x0 + d + hd * DH + e + 16 * j;
        hp[j] = vraw + lrow + 16 * j;
      }
    } else if (n0 < 3 * d) {
      const int c0 = n0 - 2 * d + lc0;
#pragma unroll
      for (int k = 0; k < 4; ++k) xp[k] = sig + xrow * d + c0 + 16 * k;
      if (ctx_mod == 1 || ctx_mod == 3) {   // mult_res, fusion: v_in has a u term
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          hp[k] = o + (long)m * d + c0 + 16 * k;
          hp[4 + k] = normw + c0 + 16 * k;
        }
      }
    }
    GroupPre pr;
#pragma unroll
    for (int k = 0; k < 4; ++k) pr.x[k] = ld_global<typename Raw4<T>::type>(xp[k]);
#pragma unroll
    for (int k = 0; k < 2; ++k) pr.f[k] = ld_global<floatx4>(fp[k]);
#pragma unroll
    for (int k = 0; k < 8; ++k) pr.h[k] = ld_global<typename Raw4<T>::type>(hp[k]);
    return pr;
  }

  template <int BM, int BN, int LDT>
  DM_DEV void tile_apply(const float* tile, int m0, int n0, const float* rs, const TilePre& pr, int) const {
    static_assert(BM == 64 && BN == 64 * NG, "sweep GEMM 1 block tile is NG 64 x 64 column groups");
    const float sc = rs[trow()];
    if constexpr (NG == 1) {
      group_apply<LDT>(tile, m0, n0, sc, pr.p[0], false, 0.f, 0.f);
    } else if constexpr (SPLIT) {
      group_apply<LDT>(tile + 64 * tgroup(), m0, n0 + 64 * tgroup(), sc, pr.p[0], false, 0.f, 0.f);
    } else {
      GroupPre pg[NG];
#pragma unroll
      for (int gi = 0; gi < NG; ++gi) {
        if constexpr (LATE) pg[gi] = pr.p[gi];
        else pg[gi] = group_prefetch(m0, n0 + 64 * gi);
      }
      // The block's NG groups are one head's k_ctx / g_k(u) (or linear v_ctx / g_v(u)) columns:
      // the head's norm scale r * gain from sections 0 and 1 of every group (the k_ctx, v_ctx
      // columns), over the row's 4 threads.
      const int r = trow(), lc0 = 4 * tquad();
      const int d = g.d;
      const float* gain = nullptr;
      int hd = 0;
      if (n0 < 2 * d) { gain = kgain; hd = n0 / (2 * DH); }
      else if (ctx_mod == 0) { gain = vgain; hd = (n0 - 2 * d) / (2 * DH); }
      float nr = 0.f, ng = 0.f;
      if (gain != nullptr) {
        float ss = 0.f;
#pragma unroll
        for (int gi = 0; gi < NG; ++gi)
#pragma unroll
          for (int k = 0; k < 2; ++k) {
            const floatx4 v = *reinterpret_cast<const floatx4*>(tile + r * LDT + 64 * gi + 16 * k + lc0);
            const float x0 = stored<T>(v.x * sc), x1 = stored<T>(v.y * sc);
            const float x2 = stored<T>(v.z * sc), x3 = stored<T>(v.w * sc);
            ss += x0 * x0 + x1 * x1 + x2 * x2 + x3 * x3;
          }
        ss += __shfl_xor(ss, 1, 64);
        ss += __shfl_xor(ss, 2, 64);
        nr = head_norm_r(ss, 1.0f / DH);
        ng = gain[hd];
      }
#pragma unroll
      for (int gi = 0; gi < NG; ++gi)
        group_apply<LDT>(tile + 64 * gi, m0, n0 + 64 * gi, sc, pg[gi], gain != nullptr, nr, ng);
    }
  }

  // One 64-column group of the tile (tile points at the group's first column). nrm: the group's
  // k_ctx / v_ctx columns are normed, x -> (x nr) ng, from and to stored values.
  template <int LDT>
  DM_DEV void group_apply(const float* tile, int m0, int n0, float sc, const GroupPre& pr, bool nrm, float nr,
                          float ng) const {
    const int r = trow(), lc0 = 4 * tquad();
    const int d = g.d, h = g.h;
    const int m = m0 + r;
    // the GEMM ran on o with norm_ctx.weight folded into W: u . W^T = rs * acc
    float a[4][4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const floatx4 v = *reinterpret_cast<const floatx4*>(tile + r * LDT + 16 * k + lc0);
      a[k][0] = v.x * sc; a[k][1] = v.y * sc; a[k][2] = v.z * sc; a[k][3] = v.w * sc;
    }
    // raw outputs for the tape: this thread's 16 consecutive columns of row r
    float sv[16];
    if (save != nullptr) {
      const int cs0 = 16 * tquad();
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const floatx4 v = *reinterpret_cast<const floatx4*>(tile + r * LDT + cs0 + 4 * k);
        sv[4 * k] = v.x * sc; sv[4 * k + 1] = v.y * sc; sv[4 * k + 2] = v.z * sc; sv[4 * k + 3] = v.w * sc;
      }
    }
    if (NG > 1 && nrm) {   // normed k_ctx / v_ctx (sections 0 and 1)
#pragma unroll
      for (int k = 0; k < 2; ++k)
#pragma unroll
        for (int i = 0; i < 4; ++i) a[k][i] = stored<T>((stored<T>(a[k][i]) * nr) * ng);
    }
    if (m >= M) return;
    const int b = m / g.c, p = m - b * g.c;
    const int orow0 = DEVPOS ? dev_position(g.pos_dev, g.pos_cap) : out_row0;
    if (n0 < 2 * d) {
      float gxa[4], gxb[4], cs[4], sn[4], ka[4], kb[4];
      unpack4<T>(pr.x[0], gxa); unpack4<T>(pr.x[1], gxb); unpackf4(pr.f[0], cs); unpackf4(pr.f[1], sn);
      unpack4<T>(pr.h[0], ka); unpack4<T>(pr.h[1], kb);
      settle(gxa); settle(gxb); settle(cs); settle(sn); settle(ka); settle(kb);   // all loads before any store
      if (save != nullptr) store_vec_nt<T, 16>(save + (long)m * 4 * d + n0 + 16 * tquad(), sv);
      const int hd = n0 / (2 * DH), jj = 16 * ((n0 % (2 * DH)) / 64) + lc0;
      float o1[4], o2[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float ga = sigmoidf_(gxa[i] + a[2][i]);
        const float gb = sigmoidf_(gxb[i] + a[3][i]);
        const float k1 = ga * ka[i] + (1.f - ga) * a[0][i];
        const float k2 = gb * kb[i] + (1.f - gb) * a[1][i];
        o1[i] = k1 * cs[i] - k2 * sn[i];
        o2[i] = k2 * cs[i] + k1 * sn[i];
      }
      T* crow = Kout + ((long)b * h + hd) * out_stride + (long)(orow0 + p) * DH + jj;
      st4<T>(crow, o1);
      st4<T>(crow + DH / 2, o2);
    } else if (ctx_mod == 0) {
      float gx[2][4], vr[2][4];
#pragma unroll
      for (int j = 0; j < 2; ++j) { unpack4<T>(pr.x[j], gx[j]); unpack4<T>(pr.h[j], vr[j]); settle(gx[j]); settle(vr[j]); }
      if (save != nullptr) store_vec_nt<T, 16>(save + (long)m * 4 * d + n0 + 16 * tquad(), sv);
      const int cl = n0 - 2 * d;
      const int hd = cl / (2 * DH), e = 32 * ((cl % (2 * DH)) / 64) + lc0;
      T* crow = Vout + ((long)b * h + hd) * out_stride + (long)(orow0 + p) * DH + e;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
          v[i] = value_blend(g, hd * DH + e + 16 * j + i, sigmoidf_(gx[j][i] + a[j + 2][i]), vr[j][i], a[j][i]);
        st4<T>(crow + 16 * j, v);
      }
    } else if (n0 < 3 * d) {
      float sg[4][4], ov[4][4], nw[4][4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        unpack4<T>(pr.x[k], sg[k]);
        settle(sg[k]);
        if (ctx_mod == 1 || ctx_mod == 3) {
          unpack4<T>(pr.h[k], ov[k]); unpack4<T>(pr.h[4 + k], nw[k]); settle(ov[k]); settle(nw[k]);
        }
      }
      if (save != nullptr) store_vec_nt<T, 16>(save + (long)m * 4 * d + n0 + 16 * tquad(), sv);
      const int c0 = n0 - 2 * d + lc0;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (ctx_mod == 3) {   // fusion (attention.py:341-342): u + silu(v_pre x-half + u-half)
            const float z = sg[k][i] + a[k][i];
            v[i] = ov[k][i] * sc * nw[k][i] + z * sigmoidf_(z);
          } else {
            v[i] = sg[k][i] * tanhf_(a[k][i]);
            if (ctx_mod == 1) v[i] += lam * (ov[k][i] * sc * nw[k][i]);
          }
        }
        st4<T>(vin + (long)m * d + c0 + 16 * k, v);
      }
    } else {
      if (save != nullptr) store_vec_nt<T, 16>(save + (long)m * 4 * d + n0 + 16 * tquad(), sv);
      const int c0 = n0 - 3 * d + lc0;
#pragma unroll
      for (int k = 0; k < 4; ++k) st4<T>(gvu + (long)m * d + c0 + 16 * k, a[k]);
    }
  }
};

// sweep GEMM 2 (mult family): v_ctx = v_in . w_vctx^T ->
// v'' = g_v v_raw + (1 - g_v) v_ctx -> V rows. save2 stores raw v_ctx [rows, d].
// Block tile 64 x 32: thread t owns row t / 4, columns 8 (t % 4) .. + 7 (inputs
// gathered before the k-loop).
template <typename T, int DH, bool DEVPOS = false> struct EpiSweep2 {
  CellGeom g;
  int M;
  const T* __restrict__ vraw;
  const T* __restrict__ glogx;
  const T* __restrict__ gvu;
  T* __restrict__ Vout;
  long out_stride; int out_row0;
  T* __restrict__ save2;

  struct TilePre {
    Raw8<T> gx, gu, vr;
  };
  // vector-memory load instructions tile_prefetch issues (Raw8 = one 16-byte load in bf16, two in
  // fp32: 16-byte loads, which the compiler cannot merge into fewer)
  static constexpr int LATE_GATHERS = 3 * (int)(sizeof(T) / 2);
  DM_DEV TilePre tile_prefetch(int m0, int n0) const {
    const int r = threadIdx.x >> 2, col = n0 + 8 * (threadIdx.x & 3);
    const int m = min(m0 + r, M - 1);
    const int b = m / g.c, t = g.buf_t0 + m - b * g.c;
    const int hd = col / DH, e = col - hd * DH;
    const T* gx = glogx + ((long)b * g.Tbuf + t) * 2 * g.d + g.d + col;
    const T* gu = gvu + (long)m * g.d + col;
    TilePre pr;
    pr.gx = ld8_global(gx);
    pr.gu = ld8_global(gu);
    pr.vr = ld8_global(vraw + (((long)b * g.h + hd) * g.Tbuf + t) * DH + e);
    return pr;
  }
  template <int BM, int BN, int LDT>
  DM_DEV void tile_apply(const float* tile, int m0, int n0, const float*, const TilePre& pr, int) const {
    static_assert(BM == 64 && BN == 32, "sweep GEMM 2 block tile is 64 x 32");
    const int r = threadIdx.x >> 2, c0 = 8 * (threadIdx.x & 3), col = n0 + c0;
    const int m = m0 + r;
    float a[8], gx[8], gu[8], vr[8];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      unpackf4(*reinterpret_cast<const floatx4*>(tile + r * LDT + c0 + 4 * k), a + 4 * k);
    }
    unpack8<T>(pr.gx, gx);
    unpack8<T>(pr.gu, gu);
    unpack8<T>(pr.vr, vr);
    if (m >= M) return;
    settle(gx); settle(gu); settle(vr);   // all loads before any store
    const int b = m / g.c, p = m - b * g.c;
    const int hd = col / DH, e = col - hd * DH;
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = value_blend(g, col + i, sigmoidf_(gx[i] + gu[i]), vr[i], a[i]);
    const int orow0 = DEVPOS ? dev_position(g.pos_dev, g.pos_cap) : out_row0;
    store_vec<T, 8>(Vout + ((long)b * g.h + hd) * out_stride + (long)(orow0 + p) * DH + e, v);
    if (save2 != nullptr) store_vec_nt<T, 8>(save2 + (long)m * g.d + col, a);
  }
};


// ---------------------------------------------------------------------------
// Sweep GEMM 2 of sweep s fused with the attention of sweep s + 1 (cells of c = 64 rows).
// Block (hh, b) computes v_ctx = v_in . W_vctx^T for the 64 rows of batch b (its whole
// chunk) and head hh's DH columns, blends the refined V rows (the value blend of
// EpiSweep2, plus the norm clamp: the block holds whole heads) into Vout and into the
// attention's LDS V tile, then runs sweep s + 1's attention of (b, hh): its intra V rows
// are exactly the rows this block wrote, its K rows came from sweep s's GEMM 1 (the
// previous launch). Nothing crosses blocks, one launch per sweep less.
// Epilogue layout: thread t owns row t / 4 and columns (t % 4) DH / 4 .. + DH / 4 - 1.
// As a GEMM tile epilogue (64 x DH blocks) it is GEMM 2 with whole heads per block, which the
// v_ctx norm needs.
// ---------------------------------------------------------------------------
template <typename T, int DH> struct EpiSweep2Head {
  static constexpr int CW = DH / 4;   // columns per thread
  CellGeom g;
  int M;
  const T* __restrict__ vraw;
  const T* __restrict__ glogx;
  const T* __restrict__ gvu;
  T* __restrict__ Vout;
  long out_stride; int out_row0;
  T* __restrict__ save2;
  const float* __restrict__ vgain = nullptr;   // v_ctx norm gains [h] (norm_vctx), nullptr = off
  struct TilePre {
    Raw8<T> gx[CW / 8], gu[CW / 8], vr[CW / 8];
  };
  // vector-memory load instructions tile_prefetch issues (Raw8 = one 16-byte load in bf16, two in
  // fp32: 16-byte loads, which the compiler cannot merge into fewer)
  static constexpr int LATE_GATHERS = 3 * (CW / 8) * (int)(sizeof(T) / 2);
  DM_DEV TilePre tile_prefetch(int m0, int n0) const {
    const int r = threadIdx.x >> 2, e0 = CW * (threadIdx.x & 3), col = n0 + e0;
    const int m = min(m0 + r, M - 1);
    const int b = m / g.c, t = g.buf_t0 + m - b * g.c;
    const int hd = n0 / DH;
    const T* gx = glogx + ((long)b * g.Tbuf + t) * 2 * g.d + g.d + col;
    const T* gu = gvu + (long)m * g.d + col;
    const T* vr = vraw + (((long)b * g.h + hd) * g.Tbuf + t) * DH + e0;
    TilePre pr;
#pragma unroll
    for (int k = 0; k < CW / 8; ++k) {
      pr.gx[k] = ld8_global(gx + 8 * k);
      pr.gu[k] = ld8_global(gu + 8 * k);
      pr.vr[k] = ld8_global(vr + 8 * k);
    }
    return pr;
  }
  template <int BM, int BN, int LDT>
  DM_DEV void tile_apply(const float* tile, int m0, int n0, const float*, const TilePre& pr, int) const {
    static_assert(BM == 64 && BN == DH, "GEMM 2 head tile is 64 x DH");
    apply<LDT>(tile, m0, n0, pr, nullptr, 0);
  }
  // v'' of the thread's columns into Vout (and save2 = raw v_ctx) and into vs [64][ldv] (if given)
  template <int LDT>
  DM_DEV void apply(const float* tile, int m0, int n0, const TilePre& pr, T* vs, int ldv) const {
    const int r = threadIdx.x >> 2, e0 = CW * (threadIdx.x & 3), col = n0 + e0;
    const int m = min(m0 + r, M - 1);
    float a[CW], gx[CW], gu[CW], vr[CW], v[CW];
#pragma unroll
    for (int k = 0; k < CW / 4; ++k) {
      unpackf4(*reinterpret_cast<const floatx4*>(tile + r * LDT + e0 + 4 * k), a + 4 * k);
    }
#pragma unroll
    for (int k = 0; k < CW / 8; ++k) {
      unpack8<T>(pr.gx[k], gx + 8 * k);
      unpack8<T>(pr.gu[k], gu + 8 * k);
      unpack8<T>(pr.vr[k], vr + 8 * k);
    }
    float vc[CW];   // v_ctx as the blend takes it: normed (from and to stored values) with the norm on
#pragma unroll
    for (int i = 0; i < CW; ++i) vc[i] = a[i];
    if (vgain != nullptr) {
      float sn = 0.f;
#pragma unroll
      for (int i = 0; i < CW; ++i) {
        vc[i] = stored<T>(a[i]);
        sn += vc[i] * vc[i];
      }
      sn += __shfl_xor(sn, 1, 64);
      sn += __shfl_xor(sn, 2, 64);
      const float nr = head_norm_r(sn, 1.0f / DH), ng = vgain[n0 / DH];
#pragma unroll
      for (int i = 0; i < CW; ++i) vc[i] = stored<T>((vc[i] * nr) * ng);
    }
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < CW; ++i) {
      v[i] = to_f(from_f<T>(value_blend(g, col + i, sigmoidf_(gx[i] + gu[i]), vr[i], vc[i])));   // the stored value
      ss += v[i] * v[i];
    }
    if (g.v_clamp_tau > 0.f) {   // norm clamp of the stored row (as k_clamp_v): the row's 4 threads
      ss += __shfl_xor(ss, 1, 64);
      ss += __shfl_xor(ss, 2, 64);
      const float n = sqrtf(ss);
      if (n > g.v_clamp_tau) {
        const float sc = g.v_clamp_tau / fmaxf(n, 1e-20f);
#pragma unroll
        for (int i = 0; i < CW; ++i) v[i] = to_f(from_f<T>(v[i] * sc));
      }
    }
    settle(gx); settle(gu); settle(vr);   // all loads before any store
    if (vs != nullptr) store_vec<T, CW>(vs + r * ldv + e0, v);
    if (m0 + r >= M) return;
    const int b = m / g.c, p = m - b * g.c;
    store_vec<T, CW>(Vout + ((long)b * g.h + n0 / DH) * out_stride + (long)(out_row0 + p) * DH + e0, v);
    if (save2 != nullptr) store_vec_nt<T, CW>(save2 + (long)m * g.d + col, a);
  }
};

// LDS of the fused GEMM 2 + attention block: the GEMM's stages, then the attention's tiles (one
// LDS object for both: a second __shared__ array makes the compiler guard every read of the
// direct-to-LDS stages with a full vmcnt wait, serialising the k-loop)
template <typename T, int DH> struct Sweep2AttendLds {
  static constexpr int D = sizeof(T) == 2 ? -3 : 4;
  static constexpr int GEMM = (gemm_lds_bytes<T, 64, DH, D, false>() + 15) / 16 * 16;
  static constexpr int BYTES = GEMM + AttnCfg<T, DH>::LDS_ELEMS * (int)sizeof(T);
};

template <typename T, int DH>
DM_DEV void sweep2_attend_block_at(const SrcRows<T>& sa, const SrcRows<T>& sb, int K, const EpiSweep2Head<T, DH>& epi,
                                   const AttendArgs<T>& aa, int hh, int b, char* smem) {
  constexpr int D = Sweep2AttendLds<T, DH>::D;
  constexpr int LDT = DH + 4;
  using WT = WaveTile<64, DH, 2, 2>;
  using C = AttnCfg<T, DH>;
  T* alds = reinterpret_cast<T*>(smem + Sweep2AttendLds<T, DH>::GEMM);
  static_assert(64 * LDT * 4 <= gemm_stage_bytes<T, 64, DH, D>(), "output tile fits the stages");
  const int m0 = b * 64, n0 = hh * DH;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  floatx4 acc[WT::FM][WT::FN];
#pragma unroll
  for (int i = 0; i < WT::FM; ++i)
#pragma unroll
    for (int j = 0; j < WT::FN; ++j) acc[i][j] = zero4();
  typename EpiSweep2Head<T, DH>::TilePre pre;
  if constexpr (D < 0) {   // gathers issued with the k-loop's last stage (see gemm_mainloop_dma)
    auto late = [&]() { pre = epi.tile_prefetch(m0, n0); };
    gemm_mainloop_dma<T, 64, DH, 2, 2, -D, EpiSweep2Head<T, DH>::LATE_GATHERS>(sa, sb, K, m0, n0, smem, acc, 0,
                                                                               late);
  } else {
    pre = epi.tile_prefetch(m0, n0);
    gemm_kloop<T, 64, DH, 2, 2, D>(sa, sb, K, m0, n0, smem, acc, 0);
  }
  // the k-loop ends with a barrier: the stages are free for the output tile
  float* tile = reinterpret_cast<float*>(smem);
  const int r0 = (wave / 2) * WT::TM, c0 = (wave % 2) * WT::TN;
#pragma unroll
  for (int i = 0; i < WT::FM; ++i)
#pragma unroll
    for (int j = 0; j < WT::FN; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        tile[(r0 + 16 * i + 4 * (lane >> 4) + q) * LDT + c0 + 16 * j + (lane & 15)] = acc[i][j][q];
  __syncthreads();
  epi.template apply<LDT>(tile, m0, n0, pre, alds + C::KT * C::LDK, C::LDK);
  __syncthreads();   // the V tile is complete
  attend_rows<T, DH, 4, true>(aa, b * aa.g.h + hh, 0, alds);
}

template <typename T, int DH>
DM_DEV void sweep2_attend_block(const SrcRows<T>& sa, const SrcRows<T>& sb, int K, const EpiSweep2Head<T, DH>& epi,
                                const AttendArgs<T>& aa, int hh, int b) {
  __shared__ __attribute__((aligned(1024))) char smem[Sweep2AttendLds<T, DH>::BYTES];
  sweep2_attend_block_at<T, DH>(sa, sb, K, epi, aa, hh, b, smem);
}

template <typename T, int DH>
static __global__ __launch_bounds__(256) void k_sweep2_attend(SrcRows<T> sa, SrcRows<T> sb, int K,
                                                              EpiSweep2Head<T, DH> epi, AttendArgs<T> aa,
                                                              uint64_t* prof_ts) {
  const uint64_t t0 = prof_begin(prof_ts);
  sweep2_attend_block<T, DH>(sa, sb, K, epi, aa, blockIdx.x, blockIdx.y);
  prof_end(prof_ts, t0);
}

// The same launch with the next cell's committed-prefix split partials s0 .. (ca) as extra blocks
// after the (h, rows / 64) fused ones: that launch holds one block per (b, h) and leaves CUs free,
// and those partials read only rows that are final before this cell began.
template <typename T, int DH>
static __global__ __launch_bounds__(256) void k_sweep2_attend_comm(SrcRows<T> sa, SrcRows<T> sb, int K,
                                                                   EpiSweep2Head<T, DH> epi, AttendArgs<T> aa,
                                                                   CommArgs<T> ca, int nfused, int s0,
                                                                   uint64_t* prof_ts) {
  const uint64_t t0 = prof_begin(prof_ts);
  __shared__ __attribute__((aligned(1024))) char smem[Sweep2AttendLds<T, DH>::BYTES];
  const int L = blockIdx.x;
  if (L < nfused) {
    sweep2_attend_block_at<T, DH>(sa, sb, K, epi, aa, L % aa.g.h, L / aa.g.h, smem);
  } else {
    const int BH = ca.g.B * ca.g.h, j = L - nfused;
    comm_partial_block_at<T, DH>(ca, s0 + j / BH, j % BH, reinterpret_cast<T*>(smem + Sweep2AttendLds<T, DH>::GEMM));
  }
  prof_end(prof_ts, t0);
}

template <typename T, int DH> struct Sweep2AttendBody {
  static constexpr int THREADS = 256;
  struct Args {
    SrcRows<T> sa, sb;
    int K;
    EpiSweep2Head<T, DH> epi;
    AttendArgs<T> aa;
  };
  static DM_DEV void run(const Args& a, int bx, int by) { sweep2_attend_block<T, DH>(a.sa, a.sb, a.K, a.epi, a.aa, bx, by); }
};

// y = acc (+ x): the W_O projection with the block residual, or plain nn.Linear
// y = acc + x (x nullptr: no residual), row m of the GEMM at row map(m) of both; y may alias x.
// A tile epilogue: each thread owns runs of 8 consecutive columns (16-byte bf16 loads and stores);
// the residual runs of the next 64-row chunk are loaded before the current chunk is stored.
template <typename T> struct EpiResidual {
  int M, N;
  const T* x;
  T* y;
  RowMap map = RowMap{};   // output / residual row of GEMM row m
  static constexpr int TILE_ROWS = 64;
  static constexpr int VEC = 8, MAXP = 8;   // columns per run; runs per thread and chunk
  struct TilePre {};
  DM_DEV TilePre tile_prefetch(int, int) const { return TilePre{}; }
  struct ChunkPre {
    Raw8<T> v[MAXP];
  };
  template <int TR, int BN> struct Shape {
    static constexpr int TPR = BN / VEC, RPP = 256 / TPR, NP = TR / RPP;
    static_assert(BN % VEC == 0 && 256 % TPR == 0 && TR % RPP == 0 && NP <= MAXP, "runs of a chunk");
  };
  template <int TR, int BN> DM_DEV ChunkPre chunk_prefetch(int m0, int n0) const {
    using S = Shape<TR, BN>;
    ChunkPre cp;
    if (x == nullptr) return cp;   // uniform
    const int cg = threadIdx.x % S::TPR, r0 = threadIdx.x / S::TPR;
#pragma unroll
    for (int p = 0; p < S::NP; ++p)
      cp.v[p] = ld8_global(x + map(min(m0 + r0 + p * S::RPP, M - 1)) * N + n0 + cg * VEC);
    return cp;
  }
  template <int TR, int BN, int LDT>
  DM_DEV void tile_apply(const float* tile, int m0, int n0, const float*, const TilePre&, int,
                         const ChunkPre& cp) const {
    using S = Shape<TR, BN>;
    const int cg = threadIdx.x % S::TPR, r0 = threadIdx.x / S::TPR;
#pragma unroll
    for (int p = 0; p < S::NP; ++p) {
      const int r = r0 + p * S::RPP, m = m0 + r;
      if (m >= M) continue;
      const floatx4 a0 = *reinterpret_cast<const floatx4*>(tile + r * LDT + cg * VEC);
      const floatx4 a1 = *reinterpret_cast<const floatx4*>(tile + r * LDT + cg * VEC + 4);
      float xv[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      if (x != nullptr) unpack8(cp.v[p], xv);
      const float o[8] = {a0.x + xv[0], a0.y + xv[1], a0.z + xv[2], a0.w + xv[3],
                          a1.x + xv[4], a1.y + xv[5], a1.z + xv[6], a1.w + xv[7]};
      st8<T>(y + map(m) * N + n0 + cg * VEC, o);
    }
  }
};

// fp32 output of a block tile staged in LDS in chunks of up to 64 rows (split-K
// slice z at C + z * zstride): each wave store instruction writes 64 consecutive
// 16-byte pieces of a row (whole rows of up to 256 columns).
struct EpiStoreTileF32 {
  static constexpr int TILE_ROWS = 64;
  int M, N;
  float* __restrict__ C;
  long zstride;
  RowMap map = RowMap{};   // output row of GEMM row m
  struct TilePre {};
  DM_DEV TilePre tile_prefetch(int, int) const { return TilePre{}; }
  template <int TR, int BN, int LDT>
  DM_DEV void tile_apply(const float* tile, int m0, int n0, const float*, const TilePre&, int z) const {
    constexpr int C4 = BN / 4, NV = TR * C4;   // 16-byte pieces per row, per chunk
    static_assert(NV % 256 == 0, "whole passes of the block");
    float* __restrict__ C = this->C + (long)z * zstride;
#pragma unroll
    for (int it = 0; it < NV / 256; ++it) {
      const int idx = it * 256 + threadIdx.x, r = idx / C4, c = 4 * (idx % C4);
      const floatx4 v = *reinterpret_cast<const floatx4*>(tile + r * LDT + c);
      if (m0 + r < M) *reinterpret_cast<floatx4*>(C + map(m0 + r) * N + n0 + c) = v;
    }
  }
};
// C (fp32) = acc, or C += acc when accumulate != 0
// C [M, N] fp32 (+)= acc; split-K slice z stores into C + z * zstride.
struct EpiStoreF32 {
  int M, N, accumulate;
  float* __restrict__ C;
  long zstride = 0;
  // With accumulate, each 16-row group's old values are loaded before its stores
  // (one group at a time: a whole 128 x 128 wave tile of old values would not fit
  // in registers next to the accumulators).
  template <int FM, int FN>
  DM_DEV void operator()(const floatx4 (&acc)[FM][FN], int row0, int col0, const float*, int z) const {
    const int lane = threadIdx.x & 63, lc = lane & 15;
    float* __restrict__ C = this->C + (long)z * zstride;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      float old[4][FN];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int m = min(row0 + 16 * i + 4 * (lane >> 4) + q, M - 1);
#pragma unroll
        for (int j = 0; j < FN; ++j) old[q][j] = accumulate ? C[(long)m * N + col0 + 16 * j + lc] : 0.f;
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int m = row0 + 16 * i + 4 * (lane >> 4) + q;
        if (m >= M) continue;
#pragma unroll
        for (int j = 0; j < FN; ++j) C[(long)m * N + col0 + 16 * j + lc] = old[q][j] + acc[i][j][q];
      }
    }
  }
};

}  // namespace dm
