// libdm_hip.so — forward, decode and utility entry points of the C ABI declared
// in include/dm_abi.h (the backward lives in dm_bwd.hip).
//
// Argument validation, workspace carving, kernel selection by (dtype, head_dim)
// and launch sequencing. Never allocates device memory, never synchronizes.
#include "dm_decode.h"
#include "dm_fwd_host.h"
#include "dm_mlp.h"

#include <mutex>
#include <vector>

using namespace dm;

extern "C" {

int dm_abi_version(void) { return DM_ABI_VERSION; }

const char* dm_last_error(void) { return last_error().c_str(); }

int dm_pack_weights(const dm_config* c, const dm_params* p, const dm_packed* out, void* stream) {
  int rc = check_cfg(c);
  if (rc) return rc;
  DM_REQUIRE(p && out, DM_ERR_INVALID, "null params/packed");
  const int d = c->d, dh = c->dh, h = c->h;
  const bool mult = c->ctx_mod != DM_CTX_LINEAR;
  DM_REQUIRE(p->wq && p->wk && p->wv && p->wo && p->w_kctx && p->w_vctx && p->w_gk && p->w_gv && p->b_gk &&
                 p->b_gv && p->norm_ctx_w,
             DM_ERR_INVALID, "null parameter pointer");
  const bool fusion = c->ctx_mod == DM_CTX_FUSION;
  DM_REQUIRE(!mult || fusion || (p->v_gate && p->b_vgate && p->v_map), DM_ERR_INVALID,
             "mult family needs v_gate/v_map");
  DM_REQUIRE(!fusion || p->v_pre, DM_ERR_INVALID, "ctx_mod fusion needs v_pre");
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
  std::vector<PackSeg> segs;
  // w_proj: wq | wk | wv | w_gk[:, :d] | w_gv[:, :d] | v_gate
  segs.push_back(PackSeg{p->wq, d, 0, d, 0, 0});
  segs.push_back(PackSeg{p->wk, d, 0, d, d, 0});
  segs.push_back(PackSeg{p->wv, d, 0, d, 2 * d, 0});
  segs.push_back(PackSeg{p->w_gk, 2 * d, 0, d, 3 * d, 0});
  segs.push_back(PackSeg{p->w_gv, 2 * d, 0, d, 4 * d, 0});
  if (fusion) segs.push_back(PackSeg{p->v_pre, 2 * d, 0, d, 5 * d, 0});   // x-half of v_pre
  else if (mult) segs.push_back(PackSeg{p->v_gate, d, 0, d, 5 * d, 0});
  run(segs.data(), (int)segs.size(), out->w_proj);
  // w_sweep, in the 64-row groups of the sweep GEMM 1 epilogue
  segs.clear();
  auto rows_of = [&](const void* W, long ld, int row) { return (const char*)W + (size_t)row * ld * e; };
  for (int g = 0; g < h; ++g)
    for (int q = 0; q < dh / 32; ++q) {
      const int base = 2 * dh * g + 64 * q, r0 = g * dh + 16 * q, r1 = r0 + dh / 2;
      segs.push_back(PackSeg{rows_of(p->w_kctx, d, r0), d, 0, 16, base, 0});
      segs.push_back(PackSeg{rows_of(p->w_kctx, d, r1), d, 0, 16, base + 16, 0});
      segs.push_back(PackSeg{rows_of(p->w_gk, 2 * d, r0), 2 * d, d, 16, base + 32, 0});
      segs.push_back(PackSeg{rows_of(p->w_gk, 2 * d, r1), 2 * d, d, 16, base + 48, 0});
    }
  if (mult) {
    if (fusion) segs.push_back(PackSeg{p->v_pre, 2 * d, d, d, 2 * d, 0});   // u-half of v_pre
    else segs.push_back(PackSeg{p->v_map, d, 0, d, 2 * d, 0});
    segs.push_back(PackSeg{p->w_gv, 2 * d, d, d, 3 * d, 0});
  } else {
    for (int g = 0; g < h; ++g)
      for (int q = 0; q < dh / 32; ++q) {
        const int base = 2 * d + 2 * dh * g + 64 * q, r0 = g * dh + 32 * q;
        segs.push_back(PackSeg{rows_of(p->w_vctx, d, r0), d, 0, 32, base, 0});
        segs.push_back(PackSeg{rows_of(p->w_gv, 2 * d, r0), 2 * d, d, 32, base + 32, 0});
      }
  }
  run(segs.data(), (int)segs.size(), out->w_sweep);
  // plain copies
  DM_HIP(hipMemcpyAsync(out->wo, p->wo, (size_t)d * d * e, hipMemcpyDeviceToDevice, s));
  DM_HIP(hipMemcpyAsync(out->norm_ctx_w, p->norm_ctx_w, (size_t)d * e, hipMemcpyDeviceToDevice, s));
  if (out->attn_norm_w && p->attn_norm_w)
    DM_HIP(hipMemcpyAsync(out->attn_norm_w, p->attn_norm_w, (size_t)d * e, hipMemcpyDeviceToDevice, s));
  if (mult) DM_HIP(hipMemcpyAsync(out->w_vctx, p->w_vctx, (size_t)d * d * e, hipMemcpyDeviceToDevice, s));
  // biases -> fp32
  const void* bsrc[3] = {p->b_gk, p->b_gv, (mult && !fusion) ? p->b_vgate : nullptr};
  for (int i = 0; i < 3; ++i) {
    if (!bsrc[i]) continue;
    if (c->dtype == DM_BF16)
      hipLaunchKernelGGL(k_to_f32<bf16>, dim3(cdiv(d, 256)), dim3(256), 0, s, (const bf16*)bsrc[i],
                         out->b_proj + (size_t)i * d, d);
    else
      DM_HIP(hipMemcpyAsync(out->b_proj + (size_t)i * d, bsrc[i], (size_t)d * 4, hipMemcpyDeviceToDevice, s));
  }
  // per-head norm gains -> fp32 gains[k_gain | ctx_gain | v_gain]
  const void* gsrc[3] = {p->k_gain, p->ctx_gain, p->v_gain};
  const int gbit[3] = {DM_NORM_K_CTX, DM_NORM_V_CTX, DM_NORM_V};
  for (int i = 0; i < 3; ++i) {
    if (!(c->norms & gbit[i])) continue;
    DM_REQUIRE(gsrc[i] != nullptr && out->gains != nullptr, DM_ERR_INVALID, "norm gain %d: null pointer", i);
    if (c->dtype == DM_BF16)
      hipLaunchKernelGGL(k_to_f32<bf16>, dim3(cdiv(h, 256)), dim3(256), 0, s, (const bf16*)gsrc[i],
                         out->gains + (size_t)i * h, h);
    else
      DM_HIP(hipMemcpyAsync(out->gains + (size_t)i * h, gsrc[i], (size_t)h * 4, hipMemcpyDeviceToDevice, s));
  }
  // transposed copies for the backward's NT GEMMs
  auto tr = [&](const void* src, void* dst, int rows, int cols) {
    if (dst == nullptr) return;
    dim3 grid(cdiv(cols, 64), cdiv(rows, 64));
    if (c->dtype == DM_BF16)
      hipLaunchKernelGGL(k_transpose<bf16>, grid, dim3(256), 0, s, (const bf16*)src, (bf16*)dst, rows, cols);
    else
      hipLaunchKernelGGL(k_transpose<float>, grid, dim3(256), 0, s, (const float*)src, (float*)dst, rows, cols);
  };
  const int nproj = mult ? 6 : 5;
  tr(out->w_proj, out->w_proj_t, nproj * d, d);
  tr(out->w_sweep, out->w_sweep_t, 4 * d, d);   // unscaled rows: the backward's du = dctx . W
  // fold norm_ctx.weight into the forward's packed rows: W[:, k] *= w[k]
  if (c->dtype == DM_BF16)
    hipLaunchKernelGGL(k_scale_cols<bf16>, dim3(cdiv((long)4 * d * d, 256)), dim3(256), 0, s, (bf16*)out->w_sweep,
                       (const bf16*)p->norm_ctx_w, 4 * d, d);
  else
    hipLaunchKernelGGL(k_scale_cols<float>, dim3(cdiv((long)4 * d * d, 256)), dim3(256), 0, s, (float*)out->w_sweep,
                       (const float*)p->norm_ctx_w, 4 * d, d);
  if (mult) tr(p->w_vctx, out->w_vctx_t, d, d);
  tr(p->wo, out->wo_t, d, d);
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
    run_proj_dispatch<bf16>(c, w, xin, M, L->T, L->T, 0, 0, cos, sin, (bf16*)L->qr, (bf16*)L->kraw,
                            (bf16*)L->kself, (bf16*)L->vraw, (bf16*)L->vpre, (bf16*)L->glogx, (bf16*)L->sig, s);
  } else {
    const float* xin = (const float*)x;
    if (norm) {
      hipLaunchKernelGGL(k_rmsnorm_rows<float>, dim3(cdiv(M, 4)), dim3(256), 0, s, (const float*)x,
                         (const float*)w->attn_norm_w, (float*)L->xhat, M, c->d, c->rms_eps);
      xin = (const float*)L->xhat;
    }
    run_proj_dispatch<float>(c, w, xin, M, L->T, L->T, 0, 0, cos, sin, (float*)L->qr, (float*)L->kraw,
                             (float*)L->kself, (float*)L->vraw, (float*)L->vpre, (float*)L->glogx, (float*)L->sig,
                             s);
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
  const bool local = a->K_rows != nullptr;
  if (local) {
    // chunk-local form: layer buffer row p, RoPE table row p and ocat row p belong to chunk row p;
    // the committed prefix is K_cache / V_cache rows [0, pos0); the rows go to K_rows / V_rows
    DM_REQUIRE(a->pos0 >= 0 && a->c <= L->T && a->pos0 <= a->cache_T && a->c <= a->rows_T, DM_ERR_INVALID,
               "pos0=%d c=%d T=%d cache_T=%d rows_T=%d", a->pos0, a->c, L->T, a->cache_T, a->rows_T);
    DM_REQUIRE(a->pos0 == 0 || (a->K_cache && a->V_cache && aligned16(a->K_cache) && aligned16(a->V_cache)),
               DM_ERR_INVALID, "committed K/V must be non-null and 16-byte aligned");
    DM_REQUIRE(a->V_rows && aligned16(a->K_rows) && aligned16(a->V_rows), DM_ERR_INVALID,
               "K/V rows must be non-null and 16-byte aligned");
  } else {
    DM_REQUIRE(a->pos0 >= 0 && a->pos0 + a->c <= L->T && L->T <= a->cache_T, DM_ERR_INVALID,
               "pos0=%d c=%d T=%d cache_T=%d", a->pos0, a->c, L->T, a->cache_T);
    DM_REQUIRE(a->K_cache && a->V_cache && aligned16(a->K_cache) && aligned16(a->V_cache), DM_ERR_INVALID,
               "K/V cache must be non-null and 16-byte aligned");
  }
  const int cache_T = a->cache_T > 0 ? a->cache_T : 1;
  // the committed-prefix splits scale with the committed rows (the chunk-local form's cache_T is
  // only the stride of the caller's view); dm_cell_workspace_bytes(cfg, n) covers n >= pos0
  const int carve_T = local ? std::max(a->pos0, 1) : cache_T;
  const CellWs need = carve_cell(c, carve_T, nullptr);
  DM_REQUIRE(a->workspace && a->workspace_bytes >= need.bytes, DM_ERR_WORKSPACE,
             "workspace %zu < %zu bytes", a->workspace_bytes, need.bytes);
  const CellWs ws = carve_cell(c, carve_T, a->workspace);
  hipStream_t s = S(stream);
  const int buf_t0 = local ? 0 : a->pos0;
  auto run = [&](auto tag) {
    using T = decltype(tag);
    CellRows<T> rows;
    if (local) {
      rows.K = (T*)a->K_rows;
      rows.V = (T*)a->V_rows;
      rows.stride = (long)a->rows_T * c->dh;
      rows.row0 = 0;
      rows.rope_t0 = 0;
    }
    run_cell_dispatch<T>(c, w, L, cos, sin, a->pos0, a->c, a->n_sweeps, buf_t0, L->T, a->K_cache, a->V_cache,
                         cache_T, a->ocat, a->o_last, ws, nullptr, s, rows);
  };
  if (c->dtype == DM_BF16) run(bf16{});
  else run(float{});
  DM_HIP(hipGetLastError());
  return DM_OK;
}

int dm_check_schedule(const int32_t* sched, int32_t n_cells, int32_t T) {
  DM_REQUIRE(sched && n_cells > 0, DM_ERR_INVALID, "null/empty schedule");
  int expect = 0;
  for (int i = 0; i < n_cells; ++i) {
    DM_REQUIRE(sched[3 * i] == expect, DM_ERR_INVALID, "schedule cell %d starts at %d, expected %d", i,
               sched[3 * i], expect);
    DM_REQUIRE(sched[3 * i + 1] >= 1 && sched[3 * i + 1] <= CMAX, DM_ERR_UNSUPPORTED, "cell %d: c=%d", i,
               sched[3 * i + 1]);
    DM_REQUIRE(sched[3 * i + 2] >= 1, DM_ERR_INVALID, "cell %d: n_sweeps=%d", i, sched[3 * i + 2]);
    expect += sched[3 * i + 1];
  }
  DM_REQUIRE(expect == T, DM_ERR_INVALID, "schedule covers %d positions, T=%d", expect, T);
  return DM_OK;
}

size_t dm_layer_tape_bytes(const dm_config* c, const int32_t* sched, int32_t n_cells) {
  if (check_cfg(c) != DM_OK || sched == nullptr || n_cells <= 0) return 0;
  return c->dtype == DM_BF16 ? tape_offsets<bf16>(c, sched, n_cells)[n_cells + 1]
                             : tape_offsets<float>(c, sched, n_cells)[n_cells + 1];
}

int dm_layer_fwd(const dm_config* c, const dm_packed* w, const void* x, void* y, const float* cos,
                 const float* sin, const dm_layer_bufs* L, const int32_t* sched, int32_t n_cells,
                 void* K_cache, void* V_cache, int32_t cache_T, void* ocat, void* tape, size_t tape_bytes,
                 void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_cfg(c);
  if (rc) return rc;
  if ((rc = check_packed(c, w)) || (rc = check_bufs(c, L))) return rc;
  DM_REQUIRE(x && y && ocat, DM_ERR_INVALID, "null x/y/ocat");
  if ((rc = dm_check_schedule(sched, n_cells, L->T))) return rc;
  DM_REQUIRE(L->T <= cache_T, DM_ERR_INVALID, "T=%d > cache_T=%d", L->T, cache_T);
  if (tape != nullptr) {
    DM_REQUIRE(tape_bytes >= dm_layer_tape_bytes(c, sched, n_cells), DM_ERR_WORKSPACE, "tape %zu < %zu bytes",
               tape_bytes, dm_layer_tape_bytes(c, sched, n_cells));
    DM_REQUIRE(aligned16(tape), DM_ERR_INVALID, "tape must be 16-byte aligned");
  }
  ProfScope whole(PROF_LAYER, S(stream));
  if ((rc = dm_layer_proj(c, w, x, cos, sin, L, stream))) return rc;
  DM_REQUIRE(K_cache && V_cache && aligned16(K_cache) && aligned16(V_cache), DM_ERR_INVALID,
             "K/V cache must be non-null and 16-byte aligned");
  const CellWs need = carve_cell(c, cache_T, nullptr);
  DM_REQUIRE(workspace && workspace_bytes >= need.bytes, DM_ERR_WORKSPACE, "workspace %zu < %zu bytes",
             workspace_bytes, need.bytes);
  const CellWs ws = carve_cell(c, cache_T, workspace);
  auto run = [&](auto tag) {
    using T = decltype(tag);
    std::vector<size_t> off;
    if (tape != nullptr) off = tape_offsets<T>(c, sched, n_cells);
    // each cell computes the next one's committed-prefix split partials where it can (run_cell)
    int handed = -1;
    for (int i = 0; i < n_cells; ++i) {
      const int pos0 = sched[3 * i], cc = sched[3 * i + 1], K = sched[3 * i + 2];
      CellSave<T> sv{};
      CellWs cws = ws;
      if (tape != nullptr) {
        Carver cv(static_cast<char*>(tape) + off[i]);
        sv = carve_save<T>(c, (size_t)c->B * cc, K, true, pos0 > 0, cv);
        if (c->ctx_mod != DM_CTX_LINEAR)
          sv.vin = reinterpret_cast<T*>(static_cast<char*>(tape) + off[n_cells]) +
                   vin_row(c, sched, n_cells, i) * c->d;
        if (sv.Mx) cws.M = sv.Mx;   // the committed row max is part of the saved state
      }
      const bool more = i + 1 < n_cells;
      handed = run_cell_dispatch<T>(c, w, L, cos, sin, pos0, cc, K, pos0, L->T, K_cache, V_cache, cache_T, ocat,
                                    nullptr, cws, tape != nullptr ? &sv : nullptr, S(stream), CellRows<T>{}, handed,
                                    more ? sched[3 * (i + 1)] : -1, more ? sched[3 * (i + 1) + 1] : 0);
    }
  };
  if (c->dtype == DM_BF16) run(bf16{});
  else run(float{});
  DM_HIP(hipGetLastError());
  return dm_linear(c->dtype, ocat, w->wo, (c->flags & DM_FLAG_NO_RESIDUAL) ? nullptr : x, y, c->B * L->T,
                   c->d, c->d, stream);
}

}  // extern "C"

// ---- decode ----------------------------------------------------------------------
namespace dm {

struct DecWs {
  void* q; void* kraw; void* kself; void* vraw;
  void* glogx; void* sig; float* o; float* ssq; float* part;   // glogx, sig: storage dtype
  void* vin; void* gvu;
  float* rope; void* kst; void* vst;   // device position: RoPE rows, refined rows before the tape write
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
  w.glogx = take(B * 2 * d * e);
  w.sig = take(B * d * e);
  w.o = (float*)take(B * d * 4);
  w.ssq = (float*)take(B * c->h * 4);
  w.part = (float*)take((ns ? ns : 1) * B * c->h * (c->dh + 2) * 4);
  w.vin = take(B * d * e);
  w.gvu = take(B * d * e);
  w.rope = (float*)take(c->dh * 4);
  w.kst = take(B * d * e);
  w.vst = take(B * d * e);
  w.bytes = off;
  return w;
}

template <typename T, int DH>
int run_decode(const dm_config* c, const dm_packed* w, const float* cos, const float* sin,
               const dm_decode_args* a, const DecWs& ws, hipStream_t s) {
  const int B = c->B, d = c->d, h = c->h;
  // device position (a->pos_dev): one launch shape for every position — the RoPE rows are
  // gathered first, the split grid covers the whole tape, the refined pair is staged and
  // written into the tape slot last; host position: the launches are sized to a->pos
  const bool dev_pos = a->pos_dev != nullptr;
  const int pos = dev_pos ? 0 : a->pos;
  const int W = window_of(c);
  const int lo = (W > 0 && pos > W - 1) ? pos - (W - 1) : 0;
  // device position without per-head context norms or the v'' clamp: the projection and refine
  // epilogues read the position themselves (RoPE rows of the full tables, the refined pair written
  // straight into tape slot pos); otherwise the RoPE rows are gathered and the pair staged first
  const bool dev_direct = dev_pos && kctx_gain(c, w) == nullptr && vctx_gain(c, w) == nullptr &&
                          c->v_clamp_tau <= 0.f;
  const float* rc = cos;
  const float* rs = sin;
  if (dev_pos && !dev_direct) {
    hipLaunchKernelGGL(k_decode_pos_rope, dim3(1), dim3(64), 0, s, a->pos_dev, a->tape_T, cos, sin, DH / 2,
                       ws.rope);
    rc = ws.rope;
    rs = ws.rope + DH / 2;
  }
  run_proj<T, DH>(c, w, (const T*)a->xhat, B, 1, 1, 0, dev_pos ? 0 : pos, rc, rs, (T*)ws.q, (T*)ws.kraw,
                  (T*)ws.kself, (T*)ws.vraw, nullptr, (T*)ws.glogx, (T*)ws.sig, s,
                  dev_direct ? (const int*)a->pos_dev : nullptr, a->tape_T);
  const int nsplit = dev_pos ? cdiv(a->tape_T, DEC_SPLIT) : (pos > lo ? cdiv(pos - lo, DEC_SPLIT) : 0);
  DecodeArgs<T> da{B, h, d, a->tape_T, pos, lo, DEC_SPLIT, nsplit, 1.0f / sqrtf((float)DH),
                   (const T*)ws.q, (const T*)ws.kself, (const T*)ws.vraw, (const T*)a->K_tape,
                   (const T*)a->V_tape, ws.part, ws.o, ws.ssq, (T*)a->o_cat, nullptr,
                   (const int*)a->pos_dev, window_of(c)};
  if (nsplit > 0) {
    const int idx = prof_launch_begin(PROF_DEC_READ, true, da.prof_ts);
    launch_timed(idx, k_decode_partial<T, DH, DEC_SPLIT>, dim3(nsplit, B * h), dim3(256), 0, s, da);
    da.prof_ts = nullptr;
  }
  launch_k(PROF_DEC_MERGE, k_decode_merge<T, DH>, dim3(B * h), dim3(64), 0, s, da);

  // refine_kv for the B rows (c = 1, position pos), write slot pos of the tape (device
  // position: a staging row, copied into the slot by k_decode_commit)
  CellGeom g{B, 1, d, h, DH, pos, 0, 1, dev_pos ? 1 : a->tape_T};
  g.kmod_cols = c->kmod_vraw_heads * DH;
  g.kmod_mode = c->kmod_mode;
  g.v_clamp_tau = c->v_clamp_tau;
  ProfScope pr(PROF_DEC_REFINE, s);
  if (dev_direct) {
    g.pos_dev = (const int*)a->pos_dev;
    g.pos_cap = a->tape_T;
    g.cache_T = a->tape_T;
    run_refine<T, DH>(c, w, g, B, (const T*)a->o_cat, ws.ssq, (const T*)ws.kraw, (const T*)ws.vraw,
                      (const T*)ws.glogx, (const T*)ws.sig, cos, sin, (T*)a->K_tape, (T*)a->V_tape,
                      (long)a->tape_T * DH, 0, (T*)ws.vin, (T*)ws.gvu, nullptr, nullptr, s);
  } else if (dev_pos) {
    run_refine<T, DH>(c, w, g, B, (const T*)a->o_cat, ws.ssq, (const T*)ws.kraw, (const T*)ws.vraw,
                      (const T*)ws.glogx, (const T*)ws.sig, rc, rs, (T*)ws.kst, (T*)ws.vst, (long)DH, 0, (T*)ws.vin,
                      (T*)ws.gvu, nullptr, nullptr, s);
    hipLaunchKernelGGL((k_decode_commit<T, DH>), dim3(B * h), dim3(DH), 0, s, (const int*)a->pos_dev, a->tape_T,
                       (const T*)ws.kst, (const T*)ws.vst, (T*)a->K_tape, (T*)a->V_tape);
  } else {
    run_refine<T, DH>(c, w, g, B, (const T*)a->o_cat, ws.ssq, (const T*)ws.kraw, (const T*)ws.vraw,
                      (const T*)ws.glogx, (const T*)ws.sig, cos, sin, (T*)a->K_tape, (T*)a->V_tape,
                      (long)a->tape_T * DH, pos, (T*)ws.vin, (T*)ws.gvu, nullptr, nullptr, s);
  }
  if (a->y != nullptr) {
    SrcRows<T> ao{(const T*)a->o_cat, d, B};
    SrcRows<T> bo{(const T*)w->wo, d, d};
    EpiResidual<T> ep{B, d, nullptr, (T*)a->y};
    bool done = false;
    if constexpr (sizeof(T) == 2) {
      if (B <= MLP_ROWS && d % 32 == 0 && aligned16(a->o_cat) && aligned16(w->wo)) {
        // bf16, one token per row: the weight-streaming product
        launch_rows_wt<T>((const T*)a->o_cat, (const T*)w->wo, (T*)a->y, B, d, d, s);
        done = true;
      }
    }
    if (!done) {
      // one row block: 64 x 32 tiles give d / 32 blocks
      if (B <= 64) launch_gemm_auto<T, 64, 32, 4, 1, 3, 4>(ao, bo, B, d, d, ep, s);
      else launch_gemm_auto<T, 64, 128, 2, 2, 3, 4>(ao, bo, B, d, d, ep, s);
    }
  }
  return DM_OK;
}

}  // namespace dm

using namespace dm;

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
  DM_REQUIRE(a->pos_dev != nullptr || (a->pos >= 0 && a->pos < a->tape_T), DM_ERR_INVALID,
             "pos=%d outside tape of %d", a->pos, a->tape_T);
  DM_REQUIRE(a->pos_dev == nullptr || (reinterpret_cast<uintptr_t>(a->pos_dev) & 3) == 0, DM_ERR_INVALID,
             "pos_dev must be 4-byte aligned");
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

}  // extern "C"

// ---- attend_one / refine_kv as separate calls --------------------------------------
namespace dm {

// per-(row, head) sums of squares of stored rows o [N, h * DH] -> ssq [N, h]
template <typename T, int DH>
static __global__ __launch_bounds__(256) void k_head_ssq(const T* __restrict__ o, long nrh, float* __restrict__ ssq) {
  constexpr int V = 16 / (int)sizeof(T);
  const long i = blockIdx.x * 256L + threadIdx.x;
  if (i >= nrh) return;
  const T* p = o + i * DH;   // row i / h, head i % h: d = h * DH
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < DH; e += V) {
    float f[V];
    unpack16<T>(*reinterpret_cast<const uint4*>(p + e), f);
#pragma unroll
    for (int j = 0; j < V; ++j) s += f[j] * f[j];
  }
  ssq[i] = s;
}

struct RefineWs {
  float* ssq; void* vin; void* gvu;
  size_t bytes;
};
inline RefineWs carve_refine(const dm_config* c, int t, void* base) {
  RefineWs w{};
  const size_t N = (size_t)c->B * t;
  Carver cv(base);
  w.ssq = cv.take<float>(N * c->h * 4);
  w.vin = cv.take<void>(N * c->d * esz(c->dtype));
  w.gvu = cv.take<void>(N * c->d * esz(c->dtype));
  w.bytes = cv.off;
  return w;
}

template <typename T, int DH>
void run_attend_one(const dm_config* c, const void* q, const void* ks, const void* vs, const void* Kp, const void* Vp,
                    int P, int past_T, void* o, const DecWs& ws, hipStream_t s) {
  const int B = c->B, h = c->h, d = c->d;
  const int W = window_of(c);
  const int lo = (W > 0 && P > W - 1) ? P - (W - 1) : 0;
  const int nsplit = P > lo ? cdiv(P - lo, DEC_SPLIT) : 0;
  DecodeArgs<T> da{B, h, d, past_T, P, lo, DEC_SPLIT, nsplit, 1.0f / sqrtf((float)DH), (const T*)q, (const T*)ks,
                   (const T*)vs, (const T*)Kp, (const T*)Vp, ws.part, ws.o, ws.ssq, (T*)o, nullptr};
  if (nsplit > 0)
    hipLaunchKernelGGL((k_decode_partial<T, DH, DEC_SPLIT>), dim3(nsplit, B * h), dim3(256), 0, s, da);
  hipLaunchKernelGGL((k_decode_merge<T, DH>), dim3(B * h), dim3(64), 0, s, da);
}

template <typename T, int DH>
void run_refine_kv(const dm_config* c, const dm_packed* w, const dm_layer_bufs* L, const void* o_cat,
                   const float* cos, const float* sin, void* K_out, void* V_out, const RefineWs& ws, hipStream_t s) {
  const int t = L->T, N = c->B * t;
  const long nrh = (long)N * c->h;
  hipLaunchKernelGGL((k_head_ssq<T, DH>), dim3(cdiv(nrh, 256)), dim3(256), 0, s, (const T*)o_cat, nrh, ws.ssq);
  CellGeom g{c->B, t, c->d, c->h, DH, 0, 0, t, t};
  g.kmod_cols = c->kmod_vraw_heads * DH;
  g.kmod_mode = c->kmod_mode;
  g.v_clamp_tau = c->v_clamp_tau;
  g.rope_t0 = 0;
  run_refine<T, DH>(c, w, g, N, (const T*)o_cat, ws.ssq, (const T*)L->kraw, (const T*)L->vraw, (const T*)L->glogx,
                    (const T*)L->sig, cos, sin, (T*)K_out, (T*)V_out, (long)t * DH, 0, (T*)ws.vin, (T*)ws.gvu, nullptr,
                    nullptr, s);
}

}  // namespace dm

extern "C" {

int dm_attend_one(const dm_config* c, const void* q_r, const void* k_self_r, const void* v_self, const void* K_past,
                  const void* V_past, int32_t P, int32_t past_T, void* o, void* workspace, size_t workspace_bytes,
                  void* stream) {
  int rc = check_cfg(c);
  if (rc) return rc;
  DM_REQUIRE(q_r && k_self_r && v_self && o, DM_ERR_INVALID, "null attend_one argument");
  DM_REQUIRE(P >= 0 && past_T >= P, DM_ERR_INVALID, "P=%d past_T=%d", P, past_T);
  DM_REQUIRE(P == 0 || (K_past && V_past && aligned16(K_past) && aligned16(V_past)), DM_ERR_INVALID,
             "K_past / V_past must be non-null and 16-byte aligned");
  DM_REQUIRE(aligned16(q_r) && aligned16(k_self_r) && aligned16(v_self), DM_ERR_INVALID,
             "q_r / k_self_r / v_self must be 16-byte aligned");
  const DecWs need = carve_dec(c, P > 0 ? P : 1, nullptr);
  DM_REQUIRE(workspace && workspace_bytes >= need.bytes, DM_ERR_WORKSPACE, "workspace %zu < %zu bytes",
             workspace_bytes, need.bytes);
  const DecWs ws = carve_dec(c, P > 0 ? P : 1, workspace);
  hipStream_t s = S(stream);
  if (c->dtype == DM_BF16)
    c->dh == 64 ? run_attend_one<bf16, 64>(c, q_r, k_self_r, v_self, K_past, V_past, P, past_T, o, ws, s)
                : run_attend_one<bf16, 128>(c, q_r, k_self_r, v_self, K_past, V_past, P, past_T, o, ws, s);
  else
    c->dh == 64 ? run_attend_one<float, 64>(c, q_r, k_self_r, v_self, K_past, V_past, P, past_T, o, ws, s)
                : run_attend_one<float, 128>(c, q_r, k_self_r, v_self, K_past, V_past, P, past_T, o, ws, s);
  DM_HIP(hipGetLastError());
  return DM_OK;
}

size_t dm_refine_kv_workspace_bytes(const dm_config* c, int32_t t) {
  if (check_cfg(c) != DM_OK || t <= 0) return 0;
  return carve_refine(c, t, nullptr).bytes;
}

int dm_refine_kv(const dm_config* c, const dm_packed* w, const dm_layer_bufs* L, const void* o_cat, const float* cos,
                 const float* sin, void* K_out, void* V_out, void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_cfg(c);
  if (rc) return rc;
  if ((rc = check_packed(c, w)) || (rc = check_bufs(c, L))) return rc;
  DM_REQUIRE(o_cat && cos && sin && K_out && V_out, DM_ERR_INVALID, "null refine_kv argument");
  DM_REQUIRE(aligned16(o_cat) && aligned16(K_out) && aligned16(V_out), DM_ERR_INVALID,
             "o_cat / K_out / V_out must be 16-byte aligned");
  const RefineWs need = carve_refine(c, L->T, nullptr);
  DM_REQUIRE(workspace && workspace_bytes >= need.bytes, DM_ERR_WORKSPACE, "workspace %zu < %zu bytes",
             workspace_bytes, need.bytes);
  const RefineWs ws = carve_refine(c, L->T, workspace);
  hipStream_t s = S(stream);
  if (c->dtype == DM_BF16)
    c->dh == 64 ? run_refine_kv<bf16, 64>(c, w, L, o_cat, cos, sin, K_out, V_out, ws, s)
                : run_refine_kv<bf16, 128>(c, w, L, o_cat, cos, sin, K_out, V_out, ws, s);
  else
    c->dh == 64 ? run_refine_kv<float, 64>(c, w, L, o_cat, cos, sin, K_out, V_out, ws, s)
                : run_refine_kv<float, 128>(c, w, L, o_cat, cos, sin, K_out, V_out, ws, s);
  DM_HIP(hipGetLastError());
  return DM_OK;
}

}  // extern "C"

// ---- decode without a workspace argument -------------------------------------------
// The decode workspace (this step's projections, the split-P partials, the refine's
// v_in and gate logits) lives in one file-scope device array instead. Host code never
// passes `scratch` itself to a kernel (in host code the name is a host-side stand-in):
// each device's address of it is looked up once, with that device current, and kept.
namespace {
constexpr size_t SCRATCH_BYTES = DM_DECODE_SCRATCH_MAX;
__device__ __align__(256) char scratch[SCRATCH_BYTES];
constexpr int SCRATCH_MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[SCRATCH_MAX_DEVICES] = {};

int scratch_for_current_device(void** out) {
  int dev = 0;
  DM_HIP(hipGetDevice(&dev));
  DM_REQUIRE(dev >= 0 && dev < SCRATCH_MAX_DEVICES, DM_ERR_UNSUPPORTED, "device %d (at most %d devices)", dev,
             SCRATCH_MAX_DEVICES);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    DM_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    DM_REQUIRE(p != nullptr, DM_ERR_HIP, "no device address for the decode scratch array on device %d", dev);
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return DM_OK;
}
}  // namespace

extern "C" {

int dm_decode_step_noalloc(const dm_config* c, const dm_packed* w, const float* cos, const float* sin,
                           const dm_decode_args* a, void* stream) {
  int rc = check_cfg(c);
  if (rc) return rc;
  DM_REQUIRE(a != nullptr, DM_ERR_INVALID, "null decode argument");
  DM_REQUIRE(a->tape_T > 0, DM_ERR_INVALID, "tape_T=%d", a->tape_T);
  const size_t need = carve_dec(c, a->tape_T, nullptr).bytes;
  DM_REQUIRE(need <= SCRATCH_BYTES, DM_ERR_WORKSPACE,
             "decode step needs %zu bytes of scratch (B=%d, d=%d, tape_T=%d); the static scratch holds %zu",
             need, c->B, c->d, a->tape_T, SCRATCH_BYTES);
  void* base = nullptr;
  if ((rc = scratch_for_current_device(&base))) return rc;
  dm_decode_args b = *a;
  b.workspace = base;
  b.workspace_bytes = SCRATCH_BYTES;
  return dm_decode_step(c, w, cos, sin, &b, stream);
}

int dm_linear(int32_t dtype, const void* x, const void* W, const void* r, void* y, int32_t M, int32_t N,
              int32_t K, void* stream) {
  DM_REQUIRE(x && W && y, DM_ERR_INVALID, "null operand");
  DM_REQUIRE(M > 0 && N > 0 && K > 0 && N % 128 == 0 && K % 64 == 0, DM_ERR_INVALID,
             "M=%d N=%d K=%d (N multiple of 128, K of 64)", M, N, K);
  DM_REQUIRE(aligned16(x) && aligned16(W), DM_ERR_INVALID, "operands must be 16-byte aligned");
  hipStream_t s = S(stream);
  ProfScope ps(PROF_WO, s);
  if (dtype == DM_BF16) {
    SrcRows<bf16> sa{(const bf16*)x, K, M};
    SrcRows<bf16> sb{(const bf16*)W, K, N};
    EpiResidual<bf16> ep{M, N, (const bf16*)r, (bf16*)y};
    launch_gemm_big<bf16>(sa, sb, M, N, K, ep, s);
  } else if (dtype == DM_F32) {
    SrcRows<float> sa{(const float*)x, K, M};
    SrcRows<float> sb{(const float*)W, K, N};
    EpiResidual<float> ep{M, N, (const float*)r, (float*)y};
    launch_gemm<float, 128, 128, 2, 2, 4>(sa, sb, M, N, K, ep, s);
  } else {
    return fail(DM_ERR_INVALID, "dtype %d", dtype);
  }
  DM_HIP(hipGetLastError());
  return DM_OK;
}

int dm_swiglu_rows(int32_t dtype, const void* x, const void* w1, const void* w3, const void* w2, void* act,
                   void* out, int32_t M, int32_t d, int32_t H, void* stream) {
  DM_REQUIRE(x && w1 && w3 && w2 && act && out, DM_ERR_INVALID, "null operand");
  DM_REQUIRE(dtype == DM_BF16, DM_ERR_UNSUPPORTED, "dm_swiglu_rows: bf16 only (dtype %d)", dtype);
  DM_REQUIRE(M >= 1 && M <= MLP_ROWS, DM_ERR_INVALID, "M=%d (1..%d rows)", M, MLP_ROWS);
  DM_REQUIRE(d > 0 && H > 0 && d % 128 == 0 && H % 32 == 0, DM_ERR_INVALID,
             "d=%d H=%d (d a multiple of 128, H of 32)", d, H);
  DM_REQUIRE(aligned16(x) && aligned16(w1) && aligned16(w3) && aligned16(w2) && aligned16(act), DM_ERR_INVALID,
             "operands must be 16-byte aligned");
  hipStream_t s = S(stream);
  auto up = [&](auto rt) {
    constexpr int RT = decltype(rt)::value;
    hipLaunchKernelGGL((k_swiglu_up<bf16, RT>), dim3(H / 16), dim3(256), 0, s, (const bf16*)x, (const bf16*)w1,
                       (const bf16*)w3, (bf16*)act, M, d, H);
  };
  const int rts = (M + 15) / 16;
  if (rts == 1) up(std::integral_constant<int, 1>{});
  else if (rts == 2) up(std::integral_constant<int, 2>{});
  else if (rts == 3) up(std::integral_constant<int, 3>{});
  else up(std::integral_constant<int, 4>{});
  launch_rows_wt<bf16>((const bf16*)act, (const bf16*)w2, (bf16*)out, M, d, H, s);
  DM_HIP(hipGetLastError());
  return DM_OK;
}

int dm_residual_rmsnorm(int32_t dtype, float* x, const void* delta, const float* w, void* y, int32_t M,
                        int32_t d, float eps, void* stream) {
  DM_REQUIRE(x != nullptr && (w == nullptr || y != nullptr), DM_ERR_INVALID, "null operand");
  DM_REQUIRE(M > 0 && d > 0, DM_ERR_INVALID, "M=%d d=%d", M, d);
  hipStream_t s = S(stream);
  DM_REQUIRE(dtype == DM_BF16 || dtype == DM_F32, DM_ERR_INVALID, "dtype %d", dtype);
  // rows of up to 4096 held in registers; longer rows by the streaming kernel
  auto run = [&](auto tag) {
    using T = decltype(tag);
    const T* dl = (const T*)delta;
    T* yy = (T*)y;
    if (d <= 1024) hipLaunchKernelGGL((k_residual_rmsnorm_reg<T, 4>), dim3(M), dim3(256), 0, s, x, dl, w, yy, d, eps);
    else if (d <= 2048) hipLaunchKernelGGL((k_residual_rmsnorm_reg<T, 8>), dim3(M), dim3(256), 0, s, x, dl, w, yy, d, eps);
    else if (d <= 4096) hipLaunchKernelGGL((k_residual_rmsnorm_reg<T, 16>), dim3(M), dim3(256), 0, s, x, dl, w, yy, d, eps);
    else hipLaunchKernelGGL(k_residual_rmsnorm<T>, dim3(M), dim3(256), 0, s, x, dl, w, yy, d, eps);
  };
  if (dtype == DM_BF16) run(bf16{});
  else run(float{});
  DM_HIP(hipGetLastError());
  return DM_OK;
}

int dm_argmax_rows(int32_t dtype, const void* x, int32_t rows, int32_t cols, int64_t ld, int64_t* out,
                   void* stream) {
  DM_REQUIRE(x && out, DM_ERR_INVALID, "null operand");
  DM_REQUIRE(rows > 0 && cols > 0 && ld >= cols, DM_ERR_INVALID, "rows=%d cols=%d ld=%lld", rows, cols,
             (long long)ld);
  hipStream_t s = S(stream);
  // 16-byte aligned rows: the vector-load kernel; otherwise the scalar scan
  const bool vec = aligned16(x) && ld % (dtype == DM_BF16 ? 8 : 4) == 0;
  if (dtype == DM_BF16) {
    if (vec) hipLaunchKernelGGL(k_argmax_rows_vec<bf16>, dim3(rows), dim3(1024), 0, s, (const bf16*)x, (long)ld, cols, out);
    else hipLaunchKernelGGL(k_argmax_rows<bf16>, dim3(rows), dim3(256), 0, s, (const bf16*)x, (long)ld, cols, out);
  } else if (dtype == DM_F32) {
    if (vec) hipLaunchKernelGGL(k_argmax_rows_vec<float>, dim3(rows), dim3(1024), 0, s, (const float*)x, (long)ld, cols, out);
    else hipLaunchKernelGGL(k_argmax_rows<float>, dim3(rows), dim3(256), 0, s, (const float*)x, (long)ld, cols, out);
  } else {
    return fail(DM_ERR_INVALID, "dtype %d", dtype);
  }
  DM_HIP(hipGetLastError());
  return DM_OK;
}

}  // extern "C"

namespace {
template <typename T>
void gemm_any(int ta, int tb, const void* A, const void* Bm, float* C, int M, int N, int K, int accumulate,
              hipStream_t s) {
  EpiStoreF32 ep{M, N, accumulate, C};
  const T* a = (const T*)A;
  const T* b = (const T*)Bm;
  if (!ta && !tb)
    launch_gemm_big<T>(SrcRows<T>{a, K, M}, SrcRows<T>{b, K, N}, M, N, K, ep, s);
  else if (!ta && tb)
    launch_gemm<T, 128, 128, 2, 2, 4>(SrcRows<T>{a, K, M}, SrcKMajor<T>{b, N, N}, M, N, K, ep, s);
  else if (ta && !tb)
    launch_gemm<T, 128, 128, 2, 2, 4>(SrcKMajor<T>{a, M, M}, SrcRows<T>{b, K, N}, M, N, K, ep, s);
  else
    launch_gemm_kk<T>(SrcKMajor<T>{a, M, M}, SrcKMajor<T>{b, N, N}, M, N, K, ep, s);
}
}  // namespace

extern "C" {

int dm_gemm(int32_t dtype, int32_t trans_a, int32_t trans_b, const void* A, const void* Bm, float* C, int32_t M,
            int32_t N, int32_t K, int32_t accumulate, void* stream) {
  DM_REQUIRE(A && Bm && C, DM_ERR_INVALID, "null operand");
  DM_REQUIRE(M > 0 && N > 0 && K > 0 && M % 128 == 0 && N % 128 == 0 && K % 64 == 0, DM_ERR_INVALID,
             "M=%d N=%d K=%d (M, N multiples of 128, K of 64)", M, N, K);
  DM_REQUIRE(aligned16(A) && aligned16(Bm), DM_ERR_INVALID, "operands must be 16-byte aligned");
  hipStream_t s = S(stream);
  if (dtype == DM_BF16)
    gemm_any<bf16>(trans_a, trans_b, A, Bm, C, M, N, K, accumulate, s);
  else if (dtype == DM_F32)
    gemm_any<float>(trans_a, trans_b, A, Bm, C, M, N, K, accumulate, s);
  else
    return fail(DM_ERR_INVALID, "dtype %d", dtype);
  DM_HIP(hipGetLastError());
  return DM_OK;
}

}  // extern "C"

// ---- optional per-kernel-class timing --------------------------------------------
static __global__ void k_prof_init(uint64_t* ts, long n) {
  const long i = blockIdx.x * 256L + threadIdx.x;
  if (i < n) ts[i] = ((i / dm::PROF_SLOTS) % 2 == 0) ? ~0ull : 0ull;
}

extern "C" {

int dm_prof_start(int32_t kernel_class, int32_t max_launches) {
  ProfState& p = prof();
  DM_REQUIRE(p.armed == PROF_NONE, DM_ERR_INVALID, "timing already armed for class %d", p.armed);
  p.dev_clock = !(kernel_class & DM_PROF_EVENTS_ONLY);
  kernel_class &= ~DM_PROF_EVENTS_ONLY;
  DM_REQUIRE(kernel_class > PROF_NONE && kernel_class < PROF_NCLASS, DM_ERR_INVALID, "kernel class %d",
             kernel_class);
  DM_REQUIRE(max_launches > 0 && max_launches <= (1 << 16), DM_ERR_INVALID, "max_launches %d", max_launches);
  if ((int)p.ev.size() < 2 * max_launches) {
    const size_t have = p.ev.size();
    p.ev.resize(2 * (size_t)max_launches);
    for (size_t i = have; i < p.ev.size(); ++i) DM_HIP(hipEventCreate(&p.ev[i]));
  }
  if (p.dts_cap < max_launches) {
    if (p.dts) DM_HIP(hipFree(p.dts));
    p.dts = nullptr;
    p.dts_cap = 0;
    DM_HIP(hipMalloc(&p.dts, (size_t)max_launches * 2 * PROF_SLOTS * sizeof(uint64_t)));
    p.dts_cap = max_launches;
  }
  {   // starts: all ones (min-reduced), ends: zero (max-reduced)
    const long n = (long)max_launches * 2 * PROF_SLOTS;
    hipLaunchKernelGGL(k_prof_init, dim3(cdiv(n, 256)), dim3(256), 0, nullptr, p.dts, n);
    DM_HIP(hipGetLastError());
    DM_HIP(hipDeviceSynchronize());
  }
  p.dev_timed.assign(max_launches, 0);
  p.cap = max_launches;
  p.n = 0;
  p.armed = kernel_class;
  return DM_OK;
}

int dm_prof_stop(float* total_ms, int32_t* n_launches) {
  return dm_prof_stop2(total_ms, nullptr, n_launches);
}

int dm_prof_stop2(float* event_ms, float* device_ms, int32_t* n_launches) {
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
  double dev_tot = -1.0;
  int ndev = 0;
  for (int i = 0; i < p.n; ++i) ndev += p.dev_timed[i];
  if (ndev == p.n && p.n > 0) {
    int dev = 0, khz = 0;
    DM_HIP(hipGetDevice(&dev));
    DM_HIP(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev));
    DM_REQUIRE(khz > 0, DM_ERR_HIP, "device wall clock rate unavailable");
    std::vector<uint64_t> h((size_t)p.n * 2 * PROF_SLOTS);
    DM_HIP(hipMemcpy(h.data(), p.dts, h.size() * sizeof(uint64_t), hipMemcpyDeviceToHost));
    dev_tot = 0.0;
    for (int i = 0; i < p.n; ++i) {
      const uint64_t* st = h.data() + (size_t)i * 2 * PROF_SLOTS;
      uint64_t lo = ~0ull, hi = 0;
      for (int k = 0; k < PROF_SLOTS; ++k) {
        lo = std::min(lo, st[k]);
        hi = std::max(hi, st[PROF_SLOTS + k]);
      }
      DM_REQUIRE(hi >= lo && lo != ~0ull, DM_ERR_HIP, "launch %d left no device timestamps", i);
      dev_tot += (double)(hi - lo) / (double)khz;   // ticks / (ticks per ms)
    }
  }
  if (event_ms) *event_ms = tot;
  if (device_ms) *device_ms = (float)dev_tot;
  if (n_launches) *n_launches = p.n;
  return DM_OK;
}

}  // extern "C"
