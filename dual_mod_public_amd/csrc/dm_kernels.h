// Kernels of the DM forward cell, layer projection and decode step.
#pragma once

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

__global__ __launch_bounds__(256) void k_pack(PackArgs a) {
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

// ---------------------------------------------------------------------------
// row RMSNorm (attn_norm, models/dualmod/attention.py:74-83): one wave per row
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void k_rmsnorm_rows(const T* __restrict__ x, const T* __restrict__ w,
                                                      T* __restrict__ y, int M, int d, float eps) {
  const int lane = threadIdx.x & 63;
  const int m = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (m >= M) return;
  const T* xr = x + (long)m * d;
  float ss = 0.f;
  for (int j = lane; j < d; j += 64) {
    float v = to_f(xr[j]);
    ss += v * v;
  }
  ss = wave_sum(ss);
  const float rs = rsqrtf(ss / (float)d + eps);
  T* yr = y + (long)m * d;
  for (int j = lane; j < d; j += 64) yr[j] = from_f<T>(to_f(xr[j]) * rs * to_f(w[j]));
}

// ---------------------------------------------------------------------------
// projection epilogue: xhat . [wq | wk | wv | w_gk_x | w_gv_x | v_gate]^T
// ---------------------------------------------------------------------------
template <typename T> struct EpiProj {
  int M, bm, d, h, dh;
  int Tl;        // rows per batch element in this call
  int Tbuf;      // T of the destination head buffers
  int buf_t0;    // buffer row of local row 0
  int rope_t0;   // RoPE position of local row 0
  const float* cos;
  const float* sin;
  const float* bias;   // [3d] fp32
  T* qr; T* kraw; T* kself; T* vraw;
  float* glogx; float* sig;
  DM_DEV void operator()(const float* Cs, int ldc, int m0, int n0) const {
    const int bn = ldc - 4;
    const int seg = n0 / d, j0 = n0 - seg * d;
    const int half = dh / 2;
    if (seg <= 1) {
      const int nh = bn / dh;
      for (int it = threadIdx.x; it < bm * nh * half; it += 256) {
        const int r = it / (nh * half), rem = it - r * nh * half;
        const int hi = rem / half, jj = rem - hi * half;
        const int m = m0 + r;
        if (m >= M) continue;
        const int b = m / Tl, tl = m - b * Tl;
        const int hh = j0 / dh + hi;
        const float a = Cs[r * ldc + hi * dh + jj], bb = Cs[r * ldc + hi * dh + jj + half];
        const float c = cos[(long)(rope_t0 + tl) * half + jj], s = sin[(long)(rope_t0 + tl) * half + jj];
        const long off = (((long)b * h + hh) * Tbuf + buf_t0 + tl) * dh;
        if (seg == 0) {
          qr[off + jj] = from_f<T>(a * c - bb * s);
          qr[off + jj + half] = from_f<T>(bb * c + a * s);
        } else {
          kraw[off + jj] = from_f<T>(a);
          kraw[off + jj + half] = from_f<T>(bb);
          kself[off + jj] = from_f<T>(a * c - bb * s);
          kself[off + jj + half] = from_f<T>(bb * c + a * s);
        }
      }
    } else if (seg == 2) {
      for (int it = threadIdx.x; it < bm * bn; it += 256) {
        const int r = it / bn, jj = it - r * bn;
        const int m = m0 + r;
        if (m >= M) continue;
        const int b = m / Tl, tl = m - b * Tl;
        const int j = j0 + jj, hh = j / dh, e = j - hh * dh;
        vraw[(((long)b * h + hh) * Tbuf + buf_t0 + tl) * dh + e] = from_f<T>(Cs[r * ldc + jj]);
      }
    } else if (seg <= 4) {
      const int gs = seg - 3;
      for (int it = threadIdx.x; it < bm * bn; it += 256) {
        const int r = it / bn, jj = it - r * bn;
        const int m = m0 + r;
        if (m >= M) continue;
        const int b = m / Tl, tl = m - b * Tl;
        const int j = j0 + jj;
        glogx[((long)b * Tbuf + buf_t0 + tl) * 2 * d + gs * d + j] = Cs[r * ldc + jj] + bias[gs * d + j];
      }
    } else {
      for (int it = threadIdx.x; it < bm * bn; it += 256) {
        const int r = it / bn, jj = it - r * bn;
        const int m = m0 + r;
        if (m >= M) continue;
        const int b = m / Tl, tl = m - b * Tl;
        const int j = j0 + jj;
        sig[((long)b * Tbuf + buf_t0 + tl) * d + j] = sigmoidf_(Cs[r * ldc + jj] + bias[2 * d + j]);
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
};

// rows [pos0, pos0+c) of the cache := raw rows (sweep 0 reads raw intra rows)
template <typename T>
__global__ void k_init_rows(CellGeom g, const T* __restrict__ kself, const T* __restrict__ vraw,
                            T* __restrict__ Kc, T* __restrict__ Vc) {
  const long n = (long)g.B * g.h * g.c * g.dh;
  for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) {
    const int e = i % g.dh;
    const long r = i / g.dh;
    const int p = r % g.c;
    const long bh = r / g.c;
    const long src = (bh * g.Tbuf + g.buf_t0 + p) * g.dh + e;
    const long dst = (bh * g.cache_T + g.pos0 + p) * g.dh + e;
    Kc[dst] = kself[src];
    Vc[dst] = vraw[src];
  }
}

// ---------------------------------------------------------------------------
// committed-prefix accumulator (scan_cell_fwd.py:119-129): per (split, b, h),
// keys [s*L, min((s+1)*L, pos0)) -> unnormalised A [c, dh], Z [c], m [c]
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
};

struct KeyBound {
  int n;
  DM_DEV bool operator()(int, int key) const { return key < n; }
};
struct KeyStrictLower {
  DM_DEV bool operator()(int q, int key) const { return key < q; }
};

template <typename T, int DH>
__global__ __launch_bounds__(256) void k_comm_partial(CommArgs<T> a) {
  using C = AttnCfg<T, DH>;
  __shared__ __attribute__((aligned(16))) T lds[C::LDS_ELEMS];
  T* Ks = lds;
  T* Vt = Ks + C::KT * C::LDK;
  T* Ps = Vt + DH * C::LDV;
  const CellGeom& g = a.g;
  const int s = blockIdx.x, bh = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int BH = g.B * g.h;
  const int k_begin = s * a.split_len;
  const int k_end = min(k_begin + a.split_len, g.pos0);
  const int qrow = 16 * wave + (lane & 15);

  typename Mfma<T>::frag qf[C::NKS];
  load_q_frags<T, DH>(a.qr + ((long)bh * g.Tbuf + g.buf_t0 + qrow) * DH, qrow < g.c, qf);
  FlashState<T, DH> st;
  flash_init(st);
  const T* Kb = a.Kc + (long)bh * g.cache_T * DH;
  const T* Vb = a.Vc + (long)bh * g.cache_T * DH;
  for (int k0 = k_begin; k0 < k_end; k0 += C::KT) {
    const int nv = min(C::KT, k_end - k0);
    __syncthreads();
    stage_kv<T, DH>(Kb + (long)k0 * DH, Vb + (long)k0 * DH, DH, nv, Ks, Vt);
    __syncthreads();
    flash_tile<T, DH>(qf, Ks, Vt, Ps + wave * 16 * C::LDP, a.scale, KeyBound{nv}, st);
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

// merge the split partials into split 0's slots' twin buffers (A, Z, m)
__global__ __launch_bounds__(256) void k_comm_merge(int nsplit, int BH, int c, int dh,
                                                    const float* __restrict__ Ap,
                                                    const float* __restrict__ Zp,
                                                    const float* __restrict__ Mp, float* __restrict__ A,
                                                    float* __restrict__ Z, float* __restrict__ Mx) {
  const int bh = blockIdx.x;
  for (int i = threadIdx.x; i < c * dh; i += 256) {
    const int q = i / dh, e = i - q * dh;
    float M = NEG_INF;
    for (int s = 0; s < nsplit; ++s) M = fmaxf(M, Mp[((long)s * BH + bh) * c + q]);
    float acc = 0.f, z = 0.f;
    for (int s = 0; s < nsplit; ++s) {
      const long b = ((long)s * BH + bh) * c + q;
      const float w = (Mp[b] == NEG_INF) ? 0.f : __expf(Mp[b] - M);
      acc += w * Ap[b * dh + e];
      z += w * Zp[b];
    }
    const long o = (long)bh * c + q;
    A[o * dh + e] = acc;
    if (e == 0) {
      Z[o] = z;
      Mx[o] = M;
    }
  }
}

// ---------------------------------------------------------------------------
// one sweep's read (scan_cell_fwd.py:63-85 / :132-149): intra rows (strict
// lower) + raw self column, merged with the committed accumulator.
// writes o [B*c, d] fp32, per-head sums of squares ssq [B*c, h]
// ---------------------------------------------------------------------------
template <typename T> struct AttendArgs {
  CellGeom g;
  const T* qr; const T* kself; const T* vraw;   // layer buffers
  const T* Kc; const T* Vc;                     // cache (intra rows at pos0)
  const float* A; const float* Z; const float* Mx;   // committed (nullptr if pos0 == 0)
  float scale;
  float* o;     // [B*c, d]
  float* ssq;   // [B*c, h]
  T* ocat;      // [B, Tbuf, d] or nullptr (buffer rows buf_t0 + p)
  float* o_last;   // [B*c, d] or nullptr
};

template <typename T, int DH>
__global__ __launch_bounds__(256) void k_attend(AttendArgs<T> a) {
  using C = AttnCfg<T, DH>;
  __shared__ __attribute__((aligned(16))) T lds[C::LDS_ELEMS];
  T* Ks = lds;
  T* Vt = Ks + C::KT * C::LDK;
  T* Ps = Vt + DH * C::LDV;
  const CellGeom& g = a.g;
  const int bh = blockIdx.x;
  const int b = bh / g.h, hh = bh - b * g.h;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g4 = lane >> 4, col = lane & 15;
  const int qrow = 16 * wave + col;
  const long lrow0 = (long)bh * g.Tbuf + g.buf_t0;   // layer-buffer row of chunk row 0

  typename Mfma<T>::frag qf[C::NKS];
  load_q_frags<T, DH>(a.qr + (lrow0 + qrow) * DH, qrow < g.c, qf);
  FlashState<T, DH> st;
  flash_init(st);
  if (a.A != nullptr) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int q = 16 * wave + 4 * g4 + r;
      if (q < g.c) {
        const long o = (long)bh * g.c + q;
        st.m[r] = a.Mx[o];
        st.z[r] = (col == 0) ? a.Z[o] : 0.f;
#pragma unroll
        for (int dt = 0; dt < C::NDT; ++dt) st.O[dt][r] = a.A[o * DH + col + 16 * dt];
      }
    }
  }
  stage_kv<T, DH>(a.Kc + ((long)bh * g.cache_T + g.pos0) * DH, a.Vc + ((long)bh * g.cache_T + g.pos0) * DH,
                  DH, g.c, Ks, Vt);
  __syncthreads();
  flash_tile<T, DH>(qf, Ks, Vt, Ps + wave * 16 * C::LDP, a.scale, KeyStrictLower{}, st);

  // raw self column: s_self = scale * <q_r, k_self_r> (fp32), value v_raw
  constexpr int PER = DH / 16;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int q = 16 * wave + 4 * g4 + r;
    const int qc = min(q, g.c - 1);
    const T* qp = a.qr + (lrow0 + qc) * DH + col * PER;
    const T* kp = a.kself + (lrow0 + qc) * DH + col * PER;
    float dot = 0.f;
#pragma unroll
    for (int e = 0; e < PER; ++e) dot += to_f(qp[e]) * to_f(kp[e]);
    const float ss = group16_sum(dot) * a.scale;
    const float mnew = fmaxf(st.m[r], ss);
    const float alpha = (st.m[r] == NEG_INF) ? 0.f : __expf(st.m[r] - mnew);
    const float es = __expf(ss - mnew);
    const T* vp = a.vraw + (lrow0 + qc) * DH;
#pragma unroll
    for (int dt = 0; dt < C::NDT; ++dt) st.O[dt][r] = st.O[dt][r] * alpha + es * to_f(vp[col + 16 * dt]);
    st.z[r] = st.z[r] * alpha + (col == 0 ? es : 0.f);
    st.m[r] = mnew;
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int q = 16 * wave + 4 * g4 + r;
    const float inv = 1.0f / group16_sum(st.z[r]);
    float sq = 0.f;
    float ov[C::NDT];
#pragma unroll
    for (int dt = 0; dt < C::NDT; ++dt) {
      ov[dt] = st.O[dt][r] * inv;
      sq += ov[dt] * ov[dt];
    }
    sq = group16_sum(sq);
    if (q < g.c) {
      const long n = (long)b * g.c + q;
      float* orow = a.o + n * g.d + hh * DH;
#pragma unroll
      for (int dt = 0; dt < C::NDT; ++dt) orow[col + 16 * dt] = ov[dt];
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
      if (col == 0) a.ssq[n * g.h + hh] = sq;
    }
  }
}

// ---------------------------------------------------------------------------
// sweep GEMM 1 epilogue: u . W_sweep^T, one (2*dh)-wide column group per tile
//   groups [0, h)        : k_ctx | g_k(u) of head g -> blend, RoPE, write K rows
//   linear   [h, 2h)     : v_ctx | g_v(u) of head g -> blend, write V rows
//   mult fam [h, h+G)    : v_map(u) -> v_in = lam*u + sig * tanh(.)   (G = d/(2dh))
//            [h+G, h+2G) : g_v(u) -> fp32 scratch for GEMM 2
// (attention.py:314-387; fused_sweep.py:514-611, :1064-1089)
// ---------------------------------------------------------------------------
template <typename T> struct EpiSweep1 {
  CellGeom g;
  int M, bm, ctx_mod;
  float lam;
  const T* kraw; const T* vraw;
  const float* glogx; const float* sig;
  const float* cos; const float* sin;
  const float* o; const T* normw;   // for u = o * rs * w (v_in's lam*u term)
  T* Kc; T* Vc;
  T* vin; float* gvu;
  DM_DEV void operator()(const float* Cs, int ldc, int m0, int n0, const float* rs) const {
    const int dh = g.dh, half = dh / 2, d = g.d;
    const int grp = n0 / (2 * dh);
    if (grp < g.h || ctx_mod == 0) {
      const bool is_k = grp < g.h;
      const int hd = is_k ? grp : grp - g.h;
      for (int it = threadIdx.x; it < bm * half; it += 256) {
        const int r = it / half, jj = it - r * half;
        const int m = m0 + r;
        if (m >= M) continue;
        const int b = m / g.c, p = m - b * g.c;
        const long lrow = ((long)b * g.h + hd) * g.Tbuf + g.buf_t0 + p;
        const long crow = ((long)b * g.h + hd) * g.cache_T + g.pos0 + p;
        const float* gx = glogx + ((long)b * g.Tbuf + g.buf_t0 + p) * 2 * d + (is_k ? 0 : d) + hd * dh;
        const float ca = Cs[r * ldc + jj], cb = Cs[r * ldc + jj + half];
        const float ga = sigmoidf_(gx[jj] + Cs[r * ldc + dh + jj]);
        const float gb = sigmoidf_(gx[jj + half] + Cs[r * ldc + dh + jj + half]);
        if (is_k) {
          const float ka = ga * to_f(kraw[lrow * dh + jj]) + (1.f - ga) * ca;
          const float kb = gb * to_f(kraw[lrow * dh + jj + half]) + (1.f - gb) * cb;
          const long t = g.pos0 + p;
          const float cs = cos[t * half + jj], sn = sin[t * half + jj];
          Kc[crow * dh + jj] = from_f<T>(ka * cs - kb * sn);
          Kc[crow * dh + jj + half] = from_f<T>(kb * cs + ka * sn);
        } else {
          Vc[crow * dh + jj] = from_f<T>(ga * to_f(vraw[lrow * dh + jj]) + (1.f - ga) * ca);
          Vc[crow * dh + jj + half] =
              from_f<T>(gb * to_f(vraw[lrow * dh + jj + half]) + (1.f - gb) * cb);
        }
      }
      return;
    }
    const int bn = 2 * dh;
    const int j0 = (grp - g.h) * bn;   // column in [0, 2d)
    if (j0 < d) {
      for (int it = threadIdx.x; it < bm * bn; it += 256) {
        const int r = it / bn, jj = it - r * bn;
        const int m = m0 + r;
        if (m >= M) continue;
        const int b = m / g.c, p = m - b * g.c;
        const int col = j0 + jj;
        const float sg = sig[((long)b * g.Tbuf + g.buf_t0 + p) * d + col];
        float v = sg * tanhf_(Cs[r * ldc + jj]);
        if (ctx_mod == 1) v += lam * (o[(long)m * d + col] * rs[r] * to_f(normw[col]));
        vin[(long)m * d + col] = from_f<T>(v);
      }
    } else {
      for (int it = threadIdx.x; it < bm * bn; it += 256) {
        const int r = it / bn, jj = it - r * bn;
        const int m = m0 + r;
        if (m >= M) continue;
        gvu[(long)m * d + j0 - d + jj] = Cs[r * ldc + jj];
      }
    }
  }
};

// sweep GEMM 2 epilogue (mult family): v_ctx = v_in . w_vctx^T, one head per
// tile -> v'' = g_v v_raw + (1 - g_v) v_ctx -> V rows
template <typename T> struct EpiSweep2 {
  CellGeom g;
  int M, bm;
  const T* vraw;
  const float* glogx;
  const float* gvu;
  T* Vc;
  DM_DEV void operator()(const float* Cs, int ldc, int m0, int n0, const float*) const {
    const int dh = g.dh, d = g.d;
    const int hd = n0 / dh;
    for (int it = threadIdx.x; it < bm * dh; it += 256) {
      const int r = it / dh, jj = it - r * dh;
      const int m = m0 + r;
      if (m >= M) continue;
      const int b = m / g.c, p = m - b * g.c;
      const long lrow = ((long)b * g.h + hd) * g.Tbuf + g.buf_t0 + p;
      const long crow = ((long)b * g.h + hd) * g.cache_T + g.pos0 + p;
      const int col = hd * dh + jj;
      const float gv = sigmoidf_(glogx[((long)b * g.Tbuf + g.buf_t0 + p) * 2 * d + d + col] +
                                 gvu[(long)m * d + col]);
      Vc[crow * dh + jj] = from_f<T>(gv * to_f(vraw[lrow * dh + jj]) + (1.f - gv) * Cs[r * ldc + jj]);
    }
  }
};

// y = x + C (W_O projection with the block residual), or y = C when x == nullptr
template <typename T> struct EpiResidual {
  int M, N, bm;
  const T* x;
  T* y;
  DM_DEV void operator()(const float* Cs, int ldc, int m0, int n0) const {
    const int bn = ldc - 4;
    for (int it = threadIdx.x; it < bm * bn; it += 256) {
      const int r = it / bn, jj = it - r * bn;
      const int m = m0 + r;
      if (m >= M) continue;
      const long idx = (long)m * N + n0 + jj;
      float v = Cs[r * ldc + jj];
      if (x != nullptr) v += to_f(x[idx]);
      y[idx] = from_f<T>(v);
    }
  }
};

struct EpiStoreF32 {
  int M, N, bm;
  float* C;
  DM_DEV void operator()(const float* Cs, int ldc, int m0, int n0) const {
    const int bn = ldc - 4;
    for (int it = threadIdx.x; it < bm * bn; it += 256) {
      const int r = it / bn, jj = it - r * bn;
      const int m = m0 + r;
      if (m < M) C[(long)m * N + n0 + jj] = Cs[r * ldc + jj];
    }
  }
};

// GEMM kernel whose epilogue also sees the per-row scale scratch of the A loader
template <typename T, int BM, int BN, int WM, int WN, class AL, class EPI>
__global__ __launch_bounds__(256) void k_gemm_rs(AL al, const T* __restrict__ Bw, long ldb, int K,
                                                 EPI epi) {
  __shared__ __attribute__((aligned(16))) char smem[gemm_lds_bytes<T, BM, BN>()];
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  float* Cs;
  gemm_tile<T, BM, BN, WM, WN, AL>(al, Bw, ldb, K, m0, n0, smem, Cs);
  const float* rs = reinterpret_cast<const float*>(smem + (gemm_lds_bytes<T, BM, BN>() - BM * 4));
  epi(Cs, BN + 4, m0, n0, rs);
}

template <typename T, int BM, int BN, int WM, int WN, class AL, class EPI>
__global__ __launch_bounds__(256) void k_gemm_plain(AL al, const T* __restrict__ Bw, long ldb, int K,
                                                    EPI epi) {
  __shared__ __attribute__((aligned(16))) char smem[gemm_lds_bytes<T, BM, BN>()];
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  float* Cs;
  gemm_tile<T, BM, BN, WM, WN, AL>(al, Bw, ldb, K, m0, n0, smem, Cs);
  epi(Cs, BN + 4, m0, n0);
}

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
};

template <typename T, int DH, int L>
__global__ __launch_bounds__(256) void k_decode_partial(DecodeArgs<T> a) {
  constexpr int VEC = 16 / (int)sizeof(T);
  constexpr int LPK = DH / VEC;          // lanes per key row
  constexpr int KPP = 256 / LPK;         // keys per pass
  constexpr int NP = L / KPP;            // passes
  static_assert(L % KPP == 0, "split length");
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
    raw[i] = (key < k_end) ? ld_nt(Kb + (long)key * DH) : uint4{0u, 0u, 0u, 0u};
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
    raw[i] = (key < k_end) ? ld_nt(Vb + (long)key * DH) : uint4{0u, 0u, 0u, 0u};
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
