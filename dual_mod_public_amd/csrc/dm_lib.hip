// libdm_hip.so — host side of the C ABI declared in include/dm_abi.h.
//
// Argument validation, workspace carving, kernel selection by (dtype, head_dim)
// and launch sequencing. Never allocates device memory, never synchronizes.
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>

#include "../../include/dm_abi.h"
#include "dm_kernels.h"
#include "dm_prof.h"

using namespace dm;

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

#define DM_REQUIRE(cond, code, ...) \
  do {                              \
    if (!(cond)) return fail(code, __VA_ARGS__); \
  } while (0)

#define DM_HIP(call)                                                                  \
  do {                                                                                \
    hipError_t e_ = (call);                                                           \
    if (e_ != hipSuccess) return fail(DM_ERR_HIP, "%s: %s", #call, hipGetErrorString(e_)); \
  } while (0)

inline hipStream_t S(void* s) { return reinterpret_cast<hipStream_t>(s); }
inline size_t esz(int dtype) { return dtype == DM_BF16 ? 2 : 4; }
inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }
inline int cdiv(long a, long b) { return (int)((a + b - 1) / b); }

constexpr int CMAX = 64;              // max chunk length of one cell
constexpr int COMM_SPLIT_MIN = 256;   // committed keys per split (lower bound)
constexpr int COMM_MAX_SPLITS = 16;
constexpr int DEC_SPLIT = 512;        // tape keys per decode split

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

int check_cfg(const dm_config* c) {
  DM_REQUIRE(c != nullptr, DM_ERR_INVALID, "null config");
  DM_REQUIRE(c->dtype == DM_F32 || c->dtype == DM_BF16, DM_ERR_INVALID, "dtype %d", c->dtype);
  DM_REQUIRE(c->B > 0 && c->d > 0 && c->h > 0 && c->dh > 0, DM_ERR_INVALID, "non-positive dims");
  DM_REQUIRE(c->d == c->h * c->dh, DM_ERR_INVALID, "d=%d != h*dh=%d", c->d, c->h * c->dh);
  DM_REQUIRE(c->dh == 64 || c->dh == 128, DM_ERR_UNSUPPORTED, "head_dim %d (64 or 128)", c->dh);
  DM_REQUIRE(c->d % 128 == 0, DM_ERR_UNSUPPORTED, "d_model %d not a multiple of 128", c->d);
  DM_REQUIRE(c->ctx_mod >= 0 && c->ctx_mod <= 2, DM_ERR_UNSUPPORTED, "ctx_mod %d", c->ctx_mod);
  DM_REQUIRE(c->local_window >= 0, DM_ERR_INVALID, "local_window %d", c->local_window);
  return DM_OK;
}

// ---- cell workspace --------------------------------------------------------
struct CellWs {
  float* o; float* ssq;
  float* Ap; float* Zp; float* Mp;
  float* A; float* Z; float* M;
  void* vin; float* gvu;
  size_t bytes;
};

int comm_splits_max(int cache_T) {
  int n = cdiv(cache_T, COMM_SPLIT_MIN);
  return n < 1 ? 1 : (n > COMM_MAX_SPLITS ? COMM_MAX_SPLITS : n);
}

CellWs carve_cell(const dm_config* c, int cache_T, void* base) {
  CellWs w{};
  const size_t N = (size_t)c->B * CMAX, BH = (size_t)c->B * c->h;
  const size_t ns = comm_splits_max(cache_T);
  char* p = reinterpret_cast<char*>(base);
  size_t off = 0;
  auto take = [&](size_t bytes) { char* r = p ? p + off : nullptr; off += align256(bytes); return r; };
  w.o = (float*)take(N * c->d * 4);
  w.ssq = (float*)take(N * c->h * 4);
  w.Ap = (float*)take(ns * BH * CMAX * c->dh * 4);
  w.Zp = (float*)take(ns * BH * CMAX * 4);
  w.Mp = (float*)take(ns * BH * CMAX * 4);
  w.A = (float*)take(BH * CMAX * c->dh * 4);
  w.Z = (float*)take(BH * CMAX * 4);
  w.M = (float*)take(BH * CMAX * 4);
  w.vin = take(N * c->d * esz(c->dtype));
  w.gvu = (float*)take(N * c->d * 4);
  w.bytes = off;
  return w;
}

// ---- GEMM launch helpers ---------------------------------------------------
template <typename T, int BM, int BN, int WM, int WN, class AL, class EPI>
void launch_gemm(const AL& al, const T* Bw, long ldb, int M, int N, int K, const EPI& epi, hipStream_t s) {
  dim3 grid(N / BN, cdiv(M, BM));
  hipLaunchKernelGGL((k_gemm_plain<T, BM, BN, WM, WN, AL, EPI>), grid, dim3(256), 0, s, al, Bw, ldb, K, epi);
}
template <typename T, int BM, int BN, int WM, int WN, class AL, class EPI>
void launch_gemm_rs(const AL& al, const T* Bw, long ldb, int M, int N, int K, const EPI& epi, hipStream_t s) {
  dim3 grid(N / BN, cdiv(M, BM));
  hipLaunchKernelGGL((k_gemm_rs<T, BM, BN, WM, WN, AL, EPI>), grid, dim3(256), 0, s, al, Bw, ldb, K, epi);
}

// ---- projection --------------------------------------------------------------
template <typename T>
int run_proj(const dm_config* c, const dm_packed* w, const T* xhat, int M, int Tl, int Tbuf, int buf_t0,
             int rope_t0, const float* cos, const float* sin, T* qr, T* kraw, T* kself, T* vraw,
             float* glogx, float* sig, hipStream_t s) {
  const int nseg = (c->ctx_mod == DM_CTX_LINEAR) ? 5 : 6;
  EpiProj<T> epi{M, 64, c->d, c->h, c->dh, Tl, Tbuf, buf_t0, rope_t0, cos, sin, w->b_proj,
                 qr, kraw, kself, vraw, glogx, sig};
  ALoadPlain<T> al{xhat, c->d, M};
  ProfScope ps(PROF_PROJ, s);
  launch_gemm<T, 64, 128, 2, 2>(al, (const T*)w->w_proj, c->d, M, nseg * c->d, c->d, epi, s);
  return DM_OK;
}

// ---- one cell ------------------------------------------------------------------
template <typename T, int DH>
int run_cell(const dm_config* c, const dm_packed* w, const dm_layer_bufs* L, const float* cos,
             const float* sin, int pos0, int cc, int n_sweeps, int buf_t0, int Tbuf, T* Kc, T* Vc,
             int cache_T, T* ocat, float* o_last, const CellWs& ws, hipStream_t s) {
  CellGeom g{c->B, cc, c->d, c->h, DH, pos0, buf_t0, Tbuf, cache_T};
  const int BH = c->B * c->h;
  const float scale = 1.0f / sqrtf((float)DH);
  const T* qr = (const T*)L->qr;
  const T* kself = (const T*)L->kself;
  const T* vraw = (const T*)L->vraw;
  const T* kraw = (const T*)L->kraw;

  hipLaunchKernelGGL(k_init_rows<T>, dim3(cdiv((long)BH * cc * DH, 256 * 4)), dim3(256), 0, s, g, kself,
                     vraw, Kc, Vc);
  const float *A = nullptr, *Z = nullptr, *Mx = nullptr;
  if (pos0 > 0) {
    int nsplit = cdiv(pos0, COMM_SPLIT_MIN);
    if (nsplit > COMM_MAX_SPLITS) nsplit = COMM_MAX_SPLITS;
    int split_len = cdiv(cdiv(pos0, nsplit), 64) * 64;
    nsplit = cdiv(pos0, split_len);
    CommArgs<T> ca{g, qr, Kc, Vc, split_len, scale, ws.Ap, ws.Zp, ws.Mp};
    ProfScope ps(PROF_COMM, s);
    if (nsplit == 1) { ca.A = ws.A; ca.Z = ws.Z; ca.Mx = ws.M; }
    hipLaunchKernelGGL((k_comm_partial<T, DH>), dim3(nsplit, BH), dim3(256), 0, s, ca);
    if (nsplit > 1)
      hipLaunchKernelGGL(k_comm_merge, dim3(BH), dim3(256), 0, s, nsplit, BH, cc, DH, ws.Ap, ws.Zp, ws.Mp,
                         ws.A, ws.Z, ws.M);
    A = ws.A; Z = ws.Z; Mx = ws.M;
  }
  const int N = c->B * cc;
  const int lin = c->ctx_mod == DM_CTX_LINEAR;
  for (int sw = 0; sw < n_sweeps; ++sw) {
    const bool last = sw == n_sweeps - 1;
    AttendArgs<T> aa{g, qr, kself, vraw, Kc, Vc, A, Z, Mx, scale, ws.o, ws.ssq,
                     last ? ocat : nullptr, last ? o_last : nullptr};
    {
      ProfScope ps(PROF_ATTEND, s);
      hipLaunchKernelGGL((k_attend<T, DH>), dim3(BH), dim3(256), 0, s, aa);
    }

    ALoadRms<T, 64> al{ws.o, c->d, ws.ssq, c->h, (const T*)w->norm_ctx_w, N, c->d, c->rms_eps};
    EpiSweep1<T> e1{g, N, 64, c->ctx_mod, c->mult_res_lambda, kraw, vraw, L->glogx, L->sig, cos, sin,
                    ws.o, (const T*)w->norm_ctx_w, Kc, Vc, (T*)ws.vin, ws.gvu};
    {
      ProfScope ps(PROF_SWEEP1, s);
      launch_gemm_rs<T, 64, 2 * DH, 2, 2>(al, (const T*)w->w_sweep, c->d, N, 4 * c->d, c->d, e1, s);
    }
    if (!lin) {
      ALoadPlain<T> av{(const T*)ws.vin, c->d, N};
      EpiSweep2<T> e2{g, N, 64, vraw, L->glogx, ws.gvu, Vc};
      ProfScope ps(PROF_SWEEP2, s);
      launch_gemm_rs<T, 64, DH, 2, 2>(av, (const T*)w->w_vctx, c->d, N, c->d, c->d, e2, s);
    }
  }
  return DM_OK;
}

template <typename T>
int dispatch_cell(const dm_config* c, const dm_packed* w, const dm_layer_bufs* L, const float* cos,
                  const float* sin, int pos0, int cc, int n_sweeps, int buf_t0, int Tbuf, void* Kc, void* Vc,
                  int cache_T, void* ocat, float* o_last, const CellWs& ws, hipStream_t s) {
  if (c->dh == 64)
    return run_cell<T, 64>(c, w, L, cos, sin, pos0, cc, n_sweeps, buf_t0, Tbuf, (T*)Kc, (T*)Vc, cache_T,
                           (T*)ocat, o_last, ws, s);
  return run_cell<T, 128>(c, w, L, cos, sin, pos0, cc, n_sweeps, buf_t0, Tbuf, (T*)Kc, (T*)Vc, cache_T,
                          (T*)ocat, o_last, ws, s);
}

int check_bufs(const dm_config* c, const dm_layer_bufs* L) {
  DM_REQUIRE(L != nullptr, DM_ERR_INVALID, "null layer buffers");
  DM_REQUIRE(L->T > 0, DM_ERR_INVALID, "layer buffer T=%d", L->T);
  DM_REQUIRE(L->qr && L->kraw && L->kself && L->vraw && L->glogx, DM_ERR_INVALID, "null layer buffer");
  DM_REQUIRE(aligned16(L->qr) && aligned16(L->kraw) && aligned16(L->kself) && aligned16(L->vraw),
             DM_ERR_INVALID, "layer buffers must be 16-byte aligned");
  DM_REQUIRE(c->ctx_mod == DM_CTX_LINEAR || L->sig != nullptr, DM_ERR_INVALID,
             "ctx_mod mult/mult_res needs the sig buffer");
  return DM_OK;
}

int check_packed(const dm_config* c, const dm_packed* w) {
  DM_REQUIRE(w != nullptr, DM_ERR_INVALID, "null packed weights");
  DM_REQUIRE(w->w_proj && w->b_proj && w->w_sweep && w->norm_ctx_w, DM_ERR_INVALID, "null packed weight");
  DM_REQUIRE(c->ctx_mod == DM_CTX_LINEAR || w->w_vctx, DM_ERR_INVALID, "mult family needs w_vctx");
  DM_REQUIRE(aligned16(w->w_proj) && aligned16(w->w_sweep) && aligned16(w->norm_ctx_w) &&
                 (w->w_vctx == nullptr || aligned16(w->w_vctx)),
             DM_ERR_INVALID, "packed weights must be 16-byte aligned");
  return DM_OK;
}

}  // namespace

extern "C" {

int dm_abi_version(void) { return DM_ABI_VERSION; }

const char* dm_last_error(void) { return g_err.c_str(); }

int dm_pack_weights(const dm_config* c, const dm_params* p, const dm_packed* out, void* stream) {
  int rc = check_cfg(c);
  if (rc) return rc;
  DM_REQUIRE(p && out, DM_ERR_INVALID, "null params/packed");
  const int d = c->d, dh = c->dh, h = c->h;
  const bool mult = c->ctx_mod != DM_CTX_LINEAR;
  DM_REQUIRE(p->wq && p->wk && p->wv && p->wo && p->w_kctx && p->w_vctx && p->w_gk && p->w_gv && p->b_gk &&
                 p->b_gv && p->norm_ctx_w,
             DM_ERR_INVALID, "null parameter pointer");
  DM_REQUIRE(!mult || (p->v_gate && p->b_vgate && p->v_map), DM_ERR_INVALID, "mult family needs v_gate/v_map");
  DM_REQUIRE(out->w_proj && out->b_proj && out->w_sweep && out->norm_ctx_w && out->wo, DM_ERR_INVALID,
             "null packed output");
  DM_REQUIRE(!mult || out->w_vctx, DM_ERR_INVALID, "mult family needs packed w_vctx");
  hipStream_t s = S(stream);
  const int e = (int)esz(c->dtype);

  // each call copies <= PACK_MAX_SEG segments
  auto run = [&](PackSeg* segs, int n, void* dst) -> int {
    for (int i0 = 0; i0 < n; i0 += PACK_MAX_SEG) {
      PackArgs a{};
      a.nseg = n - i0 < PACK_MAX_SEG ? n - i0 : PACK_MAX_SEG;
      int rows = 0;
      for (int i = 0; i < a.nseg; ++i) { a.seg[i] = segs[i0 + i]; rows += segs[i0 + i].nrows; }
      a.ncols = d;
      a.esz = e;
      a.dst = dst;
      hipLaunchKernelGGL(k_pack, dim3(rows), dim3(256), 0, s, a);
    }
    return DM_OK;
  };
  PackSeg segs[4 * 64 + 8];
  int n = 0;
  // w_proj: wq | wk | wv | w_gk[:, :d] | w_gv[:, :d] | v_gate
  segs[n++] = PackSeg{p->wq, d, 0, d, 0, 0};
  segs[n++] = PackSeg{p->wk, d, 0, d, d, 0};
  segs[n++] = PackSeg{p->wv, d, 0, d, 2 * d, 0};
  segs[n++] = PackSeg{p->w_gk, 2 * d, 0, d, 3 * d, 0};
  segs[n++] = PackSeg{p->w_gv, 2 * d, 0, d, 4 * d, 0};
  if (mult) segs[n++] = PackSeg{p->v_gate, d, 0, d, 5 * d, 0};
  run(segs, n, out->w_proj);
  // w_sweep
  n = 0;
  for (int g = 0; g < h; ++g) {
    segs[n++] = PackSeg{(const char*)p->w_kctx + (size_t)g * dh * d * e, d, 0, dh, 2 * dh * g, 0};
    segs[n++] = PackSeg{(const char*)p->w_gk + (size_t)g * dh * 2 * d * e, 2 * d, d, dh, 2 * dh * g + dh, 0};
  }
  if (mult) {
    segs[n++] = PackSeg{p->v_map, d, 0, d, 2 * d, 0};
    segs[n++] = PackSeg{p->w_gv, 2 * d, d, d, 3 * d, 0};
  } else {
    for (int g = 0; g < h; ++g) {
      segs[n++] = PackSeg{(const char*)p->w_vctx + (size_t)g * dh * d * e, d, 0, dh, 2 * d + 2 * dh * g, 0};
      segs[n++] = PackSeg{(const char*)p->w_gv + (size_t)g * dh * 2 * d * e, 2 * d, d, dh,
                          2 * d + 2 * dh * g + dh, 0};
    }
  }
  DM_REQUIRE(n <= (int)(sizeof(segs) / sizeof(segs[0])), DM_ERR_UNSUPPORTED, "too many heads (%d)", h);
  run(segs, n, out->w_sweep);
  // plain copies
  DM_HIP(hipMemcpyAsync(out->wo, p->wo, (size_t)d * d * e, hipMemcpyDeviceToDevice, s));
  DM_HIP(hipMemcpyAsync(out->norm_ctx_w, p->norm_ctx_w, (size_t)d * e, hipMemcpyDeviceToDevice, s));
  if (out->attn_norm_w && p->attn_norm_w)
    DM_HIP(hipMemcpyAsync(out->attn_norm_w, p->attn_norm_w, (size_t)d * e, hipMemcpyDeviceToDevice, s));
  if (mult) DM_HIP(hipMemcpyAsync(out->w_vctx, p->w_vctx, (size_t)d * d * e, hipMemcpyDeviceToDevice, s));
  // biases -> fp32
  const void* bsrc[3] = {p->b_gk, p->b_gv, mult ? p->b_vgate : nullptr};
  for (int i = 0; i < 3; ++i) {
    if (!bsrc[i]) continue;
    if (c->dtype == DM_BF16)
      hipLaunchKernelGGL(k_to_f32<bf16>, dim3(cdiv(d, 256)), dim3(256), 0, s, (const bf16*)bsrc[i],
                         out->b_proj + (size_t)i * d, d);
    else
      DM_HIP(hipMemcpyAsync(out->b_proj + (size_t)i * d, bsrc[i], (size_t)d * 4, hipMemcpyDeviceToDevice, s));
  }
  DM_HIP(hipGetLastError());
  return DM_OK;
}

int dm_layer_proj(const dm_config* c, const dm_packed* w, const void* x, const float* cos, const float* sin,
                  const dm_layer_bufs* L, void* stream) {
  int rc = check_cfg(c);
  if (rc) return rc;
  if ((rc = check_packed(c, w)) || (rc = check_bufs(c, L))) return rc;
  DM_REQUIRE(x && cos && sin && aligned16(x), DM_ERR_INVALID, "null/misaligned x or null rope tables");
  const bool norm = w->attn_norm_w != nullptr;
  DM_REQUIRE(!norm || L->xhat, DM_ERR_INVALID, "attn_norm needs the xhat buffer");
  const int M = c->B * L->T;
  hipStream_t s = S(stream);
  if (c->dtype == DM_BF16) {
    const bf16* xin = (const bf16*)x;
    if (norm) {
      hipLaunchKernelGGL(k_rmsnorm_rows<bf16>, dim3(cdiv(M, 4)), dim3(256), 0, s, (const bf16*)x,
                         (const bf16*)w->attn_norm_w, (bf16*)L->xhat, M, c->d, c->rms_eps);
      xin = (const bf16*)L->xhat;
    }
    run_proj<bf16>(c, w, xin, M, L->T, L->T, 0, 0, cos, sin, (bf16*)L->qr, (bf16*)L->kraw, (bf16*)L->kself,
                   (bf16*)L->vraw, L->glogx, L->sig, s);
  } else {
    const float* xin = (const float*)x;
    if (norm) {
      hipLaunchKernelGGL(k_rmsnorm_rows<float>, dim3(cdiv(M, 4)), dim3(256), 0, s, (const float*)x,
                         (const float*)w->attn_norm_w, (float*)L->xhat, M, c->d, c->rms_eps);
      xin = (const float*)L->xhat;
    }
    run_proj<float>(c, w, xin, M, L->T, L->T, 0, 0, cos, sin, (float*)L->qr, (float*)L->kraw,
                    (float*)L->kself, (float*)L->vraw, L->glogx, L->sig, s);
  }
  DM_HIP(hipGetLastError());
  return DM_OK;
}

size_t dm_cell_workspace_bytes(const dm_config* c, int32_t cache_T) {
  if (check_cfg(c) != DM_OK || cache_T <= 0) return 0;
  return carve_cell(c, cache_T, nullptr).bytes;
}

int dm_cell_fwd(const dm_config* c, const dm_packed* w, const dm_layer_bufs* L, const float* cos,
                const float* sin, const dm_cell_args* a, void* stream) {
  int rc = check_cfg(c);
  if (rc) return rc;
  if ((rc = check_packed(c, w)) || (rc = check_bufs(c, L))) return rc;
  DM_REQUIRE(a != nullptr && cos && sin, DM_ERR_INVALID, "null cell args / rope tables");
  DM_REQUIRE(a->c >= 1 && a->c <= CMAX, DM_ERR_UNSUPPORTED, "chunk length c=%d (1..%d)", a->c, CMAX);
  DM_REQUIRE(a->n_sweeps >= 1, DM_ERR_INVALID, "n_sweeps=%d", a->n_sweeps);
  DM_REQUIRE(a->pos0 >= 0 && a->pos0 + a->c <= L->T && L->T <= a->cache_T, DM_ERR_INVALID,
             "pos0=%d c=%d T=%d cache_T=%d", a->pos0, a->c, L->T, a->cache_T);
  DM_REQUIRE(a->K_cache && a->V_cache && aligned16(a->K_cache) && aligned16(a->V_cache), DM_ERR_INVALID,
             "K/V cache must be non-null and 16-byte aligned");
  DM_REQUIRE(c->local_window == 0, DM_ERR_UNSUPPORTED, "local_window is decode-only");
  const CellWs need = carve_cell(c, a->cache_T, nullptr);
  DM_REQUIRE(a->workspace && a->workspace_bytes >= need.bytes, DM_ERR_WORKSPACE,
             "workspace %zu < %zu bytes", a->workspace_bytes, need.bytes);
  const CellWs ws = carve_cell(c, a->cache_T, a->workspace);
  hipStream_t s = S(stream);
  if (c->dtype == DM_BF16)
    rc = dispatch_cell<bf16>(c, w, L, cos, sin, a->pos0, a->c, a->n_sweeps, a->pos0, L->T, a->K_cache,
                             a->V_cache, a->cache_T, a->ocat, a->o_last, ws, s);
  else
    rc = dispatch_cell<float>(c, w, L, cos, sin, a->pos0, a->c, a->n_sweeps, a->pos0, L->T, a->K_cache,
                              a->V_cache, a->cache_T, a->ocat, a->o_last, ws, s);
  if (rc) return rc;
  DM_HIP(hipGetLastError());
  return DM_OK;
}

int dm_layer_fwd(const dm_config* c, const dm_packed* w, const void* x, void* y, const float* cos,
                 const float* sin, const dm_layer_bufs* L, const int32_t* sched, int32_t n_cells,
                 void* K_cache, void* V_cache, int32_t cache_T, void* ocat, void* workspace,
                 size_t workspace_bytes, void* stream) {
  int rc = check_cfg(c);
  if (rc) return rc;
  if ((rc = check_packed(c, w)) || (rc = check_bufs(c, L))) return rc;
  DM_REQUIRE(x && y && ocat && sched && n_cells > 0, DM_ERR_INVALID, "null x/y/ocat/schedule");
  int expect = 0;
  for (int i = 0; i < n_cells; ++i) {
    DM_REQUIRE(sched[3 * i] == expect, DM_ERR_INVALID, "schedule cell %d starts at %d, expected %d", i,
               sched[3 * i], expect);
    DM_REQUIRE(sched[3 * i + 1] >= 1 && sched[3 * i + 1] <= CMAX, DM_ERR_UNSUPPORTED, "cell %d: c=%d", i,
               sched[3 * i + 1]);
    DM_REQUIRE(sched[3 * i + 2] >= 1, DM_ERR_INVALID, "cell %d: n_sweeps=%d", i, sched[3 * i + 2]);
    expect += sched[3 * i + 1];
  }
  DM_REQUIRE(expect == L->T, DM_ERR_INVALID, "schedule covers %d positions, T=%d", expect, L->T);
  DM_REQUIRE(L->T <= cache_T, DM_ERR_INVALID, "T=%d > cache_T=%d", L->T, cache_T);
  ProfScope whole(PROF_LAYER, S(stream));
  if ((rc = dm_layer_proj(c, w, x, cos, sin, L, stream))) return rc;
  for (int i = 0; i < n_cells; ++i) {
    dm_cell_args a{sched[3 * i], sched[3 * i + 1], sched[3 * i + 2], cache_T, K_cache, V_cache, ocat,
                   nullptr, workspace, workspace_bytes};
    if ((rc = dm_cell_fwd(c, w, L, cos, sin, &a, stream))) return rc;
  }
  const int M = c->B * L->T;
  hipStream_t s = S(stream);
  ProfScope ps(PROF_WO, s);
  if (c->dtype == DM_BF16) {
    ALoadPlain<bf16> al{(const bf16*)ocat, c->d, M};
    EpiResidual<bf16> ep{M, c->d, 64, (const bf16*)x, (bf16*)y};
    launch_gemm<bf16, 64, 128, 2, 2>(al, (const bf16*)w->wo, c->d, M, c->d, c->d, ep, s);
  } else {
    ALoadPlain<float> al{(const float*)ocat, c->d, M};
    EpiResidual<float> ep{M, c->d, 64, (const float*)x, (float*)y};
    launch_gemm<float, 64, 128, 2, 2>(al, (const float*)w->wo, c->d, M, c->d, c->d, ep, s);
  }
  DM_HIP(hipGetLastError());
  return DM_OK;
}

}  // extern "C"

// ---- decode ----------------------------------------------------------------------
namespace {

struct DecWs {
  void* q; void* kraw; void* kself; void* vraw;
  float* glogx; float* sig; float* o; float* ssq; float* part;
  void* vin; float* gvu;
  size_t bytes;
};

DecWs carve_dec(const dm_config* c, int tape_T, void* base) {
  DecWs w{};
  const size_t B = c->B, d = c->d, e = esz(c->dtype);
  const size_t ns = cdiv(tape_T, DEC_SPLIT);
  char* p = reinterpret_cast<char*>(base);
  size_t off = 0;
  auto take = [&](size_t bytes) { char* r = p ? p + off : nullptr; off += align256(bytes); return r; };
  w.q = take(B * d * e);
  w.kraw = take(B * d * e);
  w.kself = take(B * d * e);
  w.vraw = take(B * d * e);
  w.glogx = (float*)take(B * 2 * d * 4);
  w.sig = (float*)take(B * d * 4);
  w.o = (float*)take(B * d * 4);
  w.ssq = (float*)take(B * c->h * 4);
  w.part = (float*)take((ns ? ns : 1) * B * c->h * (c->dh + 2) * 4);
  w.vin = take(B * d * e);
  w.gvu = (float*)take(B * d * 4);
  w.bytes = off;
  return w;
}

template <typename T, int DH>
int run_decode(const dm_config* c, const dm_packed* w, const float* cos, const float* sin,
               const dm_decode_args* a, const DecWs& ws, hipStream_t s) {
  const int B = c->B, d = c->d, h = c->h;
  const int pos = a->pos;
  const int lo = (c->local_window > 0 && pos > c->local_window - 1) ? pos - (c->local_window - 1) : 0;
  run_proj<T>(c, w, (const T*)a->xhat, B, 1, 1, 0, pos, cos, sin, (T*)ws.q, (T*)ws.kraw, (T*)ws.kself,
              (T*)ws.vraw, ws.glogx, ws.sig, s);
  const int nsplit = pos > lo ? cdiv(pos - lo, DEC_SPLIT) : 0;
  DecodeArgs<T> da{B, h, d, a->tape_T, pos, lo, DEC_SPLIT, nsplit, 1.0f / sqrtf((float)DH),
                   (const T*)ws.q, (const T*)ws.kself, (const T*)ws.vraw, (const T*)a->K_tape,
                   (const T*)a->V_tape, ws.part, ws.o, ws.ssq, (T*)a->o_cat};
  if (nsplit > 0) {
    ProfScope ps(PROF_DEC_READ, s);
    hipLaunchKernelGGL((k_decode_partial<T, DH, DEC_SPLIT>), dim3(nsplit, B * h), dim3(256), 0, s, da);
  }
  {
    ProfScope ps(PROF_DEC_MERGE, s);
    hipLaunchKernelGGL((k_decode_merge<T, DH>), dim3(B * h), dim3(64), 0, s, da);
  }
  ProfScope ps(PROF_DEC_REFINE, s);

  // refine_kv for the B rows (c = 1, position pos), write slot pos of the tape
  CellGeom g{B, 1, d, h, DH, pos, 0, 1, a->tape_T};
  ALoadRms<T, 64> al{ws.o, d, ws.ssq, h, (const T*)w->norm_ctx_w, B, d, c->rms_eps};
  EpiSweep1<T> e1{g, B, 64, c->ctx_mod, c->mult_res_lambda, (const T*)ws.kraw, (const T*)ws.vraw, ws.glogx,
                  ws.sig, cos, sin, ws.o, (const T*)w->norm_ctx_w, (T*)a->K_tape, (T*)a->V_tape, (T*)ws.vin,
                  ws.gvu};
  launch_gemm_rs<T, 64, 2 * DH, 2, 2>(al, (const T*)w->w_sweep, d, B, 4 * d, d, e1, s);
  if (c->ctx_mod != DM_CTX_LINEAR) {
    ALoadPlain<T> av{(const T*)ws.vin, d, B};
    EpiSweep2<T> e2{g, B, 64, (const T*)ws.vraw, ws.glogx, ws.gvu, (T*)a->V_tape};
    launch_gemm_rs<T, 64, DH, 2, 2>(av, (const T*)w->w_vctx, d, B, d, d, e2, s);
  }
  if (a->y != nullptr) {
    ALoadPlain<T> ao{(const T*)a->o_cat, d, B};
    EpiResidual<T> ep{B, d, 64, nullptr, (T*)a->y};
    launch_gemm<T, 64, 128, 2, 2>(ao, (const T*)w->wo, d, B, d, d, ep, s);
  }
  return DM_OK;
}

}  // namespace

extern "C" {

size_t dm_decode_workspace_bytes(const dm_config* c, int32_t tape_T) {
  if (check_cfg(c) != DM_OK || tape_T <= 0) return 0;
  return carve_dec(c, tape_T, nullptr).bytes;
}

int dm_decode_step(const dm_config* c, const dm_packed* w, const float* cos, const float* sin,
                   const dm_decode_args* a, void* stream) {
  int rc = check_cfg(c);
  if (rc) return rc;
  if ((rc = check_packed(c, w))) return rc;
  DM_REQUIRE(a && cos && sin && a->xhat && a->K_tape && a->V_tape && a->o_cat, DM_ERR_INVALID,
             "null decode argument");
  DM_REQUIRE(a->pos >= 0 && a->pos < a->tape_T, DM_ERR_INVALID, "pos=%d outside tape of %d", a->pos,
             a->tape_T);
  DM_REQUIRE(aligned16(a->K_tape) && aligned16(a->V_tape) && aligned16(a->xhat), DM_ERR_INVALID,
             "tape/xhat must be 16-byte aligned");
  const DecWs need = carve_dec(c, a->tape_T, nullptr);
  DM_REQUIRE(a->workspace && a->workspace_bytes >= need.bytes, DM_ERR_WORKSPACE, "workspace %zu < %zu bytes",
             a->workspace_bytes, need.bytes);
  const DecWs ws = carve_dec(c, a->tape_T, a->workspace);
  hipStream_t s = S(stream);
  ProfScope whole(PROF_LAYER, s);
  if (c->dtype == DM_BF16)
    rc = c->dh == 64 ? run_decode<bf16, 64>(c, w, cos, sin, a, ws, s) : run_decode<bf16, 128>(c, w, cos, sin, a, ws, s);
  else
    rc = c->dh == 64 ? run_decode<float, 64>(c, w, cos, sin, a, ws, s) : run_decode<float, 128>(c, w, cos, sin, a, ws, s);
  if (rc) return rc;
  DM_HIP(hipGetLastError());
  return DM_OK;
}

int dm_linear(int32_t dtype, const void* x, const void* W, const void* r, void* y, int32_t M, int32_t N,
              int32_t K, void* stream) {
  DM_REQUIRE(x && W && y, DM_ERR_INVALID, "null operand");
  DM_REQUIRE(M > 0 && N > 0 && K > 0 && N % 128 == 0 && K % 64 == 0, DM_ERR_INVALID,
             "M=%d N=%d K=%d (N multiple of 128, K of 64)", M, N, K);
  DM_REQUIRE(aligned16(x) && aligned16(W), DM_ERR_INVALID, "operands must be 16-byte aligned");
  hipStream_t s = S(stream);
  if (dtype == DM_BF16) {
    ALoadPlain<bf16> al{(const bf16*)x, K, M};
    EpiResidual<bf16> ep{M, N, 64, (const bf16*)r, (bf16*)y};
    launch_gemm<bf16, 64, 128, 2, 2>(al, (const bf16*)W, K, M, N, K, ep, s);
  } else if (dtype == DM_F32) {
    ALoadPlain<float> al{(const float*)x, K, M};
    EpiResidual<float> ep{M, N, 64, (const float*)r, (float*)y};
    launch_gemm<float, 64, 128, 2, 2>(al, (const float*)W, K, M, N, K, ep, s);
  } else {
    return fail(DM_ERR_INVALID, "dtype %d", dtype);
  }
  DM_HIP(hipGetLastError());
  return DM_OK;
}

int dm_gemm_nt(int32_t dtype, const void* A, const void* Bm, float* C, int32_t M, int32_t N, int32_t K,
               void* stream) {
  DM_REQUIRE(A && Bm && C, DM_ERR_INVALID, "null operand");
  DM_REQUIRE(M > 0 && N > 0 && K > 0 && M % 64 == 0 && N % 64 == 0 && K % 64 == 0, DM_ERR_INVALID,
             "M=%d N=%d K=%d must be positive multiples of 64", M, N, K);
  hipStream_t s = S(stream);
  EpiStoreF32 ep{M, N, 64, C};
  if (dtype == DM_BF16) {
    ALoadPlain<bf16> al{(const bf16*)A, K, M};
    launch_gemm<bf16, 64, 64, 2, 2>(al, (const bf16*)Bm, K, M, N, K, ep, s);
  } else if (dtype == DM_F32) {
    ALoadPlain<float> al{(const float*)A, K, M};
    launch_gemm<float, 64, 64, 2, 2>(al, (const float*)Bm, K, M, N, K, ep, s);
  } else {
    return fail(DM_ERR_INVALID, "dtype %d", dtype);
  }
  DM_HIP(hipGetLastError());
  return DM_OK;
}

}  // extern "C"

// ---- optional per-kernel-class timing --------------------------------------------
extern "C" {

int dm_prof_start(int32_t kernel_class, int32_t max_launches) {
  ProfState& p = prof();
  DM_REQUIRE(p.armed == PROF_NONE, DM_ERR_INVALID, "timing already armed for class %d", p.armed);
  DM_REQUIRE(kernel_class > PROF_NONE && kernel_class < PROF_NCLASS, DM_ERR_INVALID, "kernel class %d",
             kernel_class);
  DM_REQUIRE(max_launches > 0 && max_launches <= (1 << 16), DM_ERR_INVALID, "max_launches %d", max_launches);
  if ((int)p.ev.size() < 2 * max_launches) {
    const size_t have = p.ev.size();
    p.ev.resize(2 * (size_t)max_launches);
    for (size_t i = have; i < p.ev.size(); ++i) DM_HIP(hipEventCreate(&p.ev[i]));
  }
  p.cap = max_launches;
  p.n = 0;
  p.armed = kernel_class;
  return DM_OK;
}

int dm_prof_stop(float* total_ms, int32_t* n_launches) {
  ProfState& p = prof();
  DM_REQUIRE(p.armed != PROF_NONE, DM_ERR_INVALID, "timing not armed");
  p.armed = PROF_NONE;
  float tot = 0.f;
  for (int i = 0; i < p.n; ++i) {
    DM_HIP(hipEventSynchronize(p.ev[2 * i + 1]));
    float ms = 0.f;
    DM_HIP(hipEventElapsedTime(&ms, p.ev[2 * i], p.ev[2 * i + 1]));
    tot += ms;
  }
  if (total_ms) *total_ms = tot;
  if (n_launches) *n_launches = p.n;
  return DM_OK;
}

}  // extern "C"
