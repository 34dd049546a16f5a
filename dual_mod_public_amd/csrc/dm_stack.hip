// libdm_hip.so — the layer-batched (wavefront) forward of a stack of DM attention sublayers
// (dm_stack_fwd in include/dm_abi.h; the schedule of engines/wave3d/wave3d.py:1-47 applied
// to the chained chunk cells).
//
// Layer l runs cell t - l at global step t. What one layer launches for one cell — the
// chunk's attn_norm rows and projection, the committed-prefix partials, the K sweeps, W_O
// with the residual — is recorded (launch_log) instead of launched, for every active layer;
// the records of a step line up position by position (uniform schedule), and each position
// becomes one grouped launch (k_grouped<Body>, grid z = active layer) whose argument table
// lives in the caller's plan buffer.
#include <algorithm>
#include <map>
#include <mutex>
#include <vector>

#include "dm_block.h"
#include "dm_fwd_host.h"

namespace dm {
namespace {

// One layer's cell i, recorded: the same kernels and arguments as dm_layer_fwd's projection,
// cell and W_O, restricted to the chunk's rows.
template <typename T, int DH>
void record_chunk(const dm_config* c, const dm_stack_layer& ly, const float* cos, const float* sin,
                  const int32_t* sched, int n_cells, int i, int cache_T, const std::vector<size_t>& toff) {
  const dm_packed* w = ly.w;
  const dm_layer_bufs* L = ly.bufs;
  const int pos0 = sched[3 * i], cc = sched[3 * i + 1], K = sched[3 * i + 2];
  const int M = c->B * cc, d = c->d;
  const RowMap map{log2_exact(cc), L->T, pos0};
  const T* x = (const T*)ly.x;
  // attn_norm of the chunk's rows into the layer's x-hat rows, then the projections
  SrcChunkRows<T> sx{x, d, M, map.lc, L->T, pos0};
  if (w->attn_norm_w != nullptr) {
    record_launch<RmsRowsBody<T>>(dim3(cdiv(M, 4)), dim3(256),
                                  typename RmsRowsBody<T>::Args{x, (const T*)w->attn_norm_w, (T*)L->xhat, M, d,
                                                                c->rms_eps, map});
    sx.p = (const T*)L->xhat;
  }
  // (a chunk's M = B * c rows: 128 x 128 blocks, several per layer and CU)
  run_proj_src<T, DH>(c, w, sx, M, cc, L->T, pos0, pos0, cos, sin, (T*)L->qr, (T*)L->kraw, (T*)L->kself,
                      (T*)L->vraw, (T*)L->vpre, (T*)L->glogx, (T*)L->sig, nullptr, true);
  // the cell (as dm_layer_fwd: with the tape its sweep states go there)
  const CellWs ws = carve_cell(c, cache_T, ly.workspace);
  const T* o_last;
  if (ly.tape == nullptr) {
    run_cell<T, DH>(c, w, L, cos, sin, pos0, cc, K, pos0, L->T, (T*)ly.K_cache, (T*)ly.V_cache, cache_T,
                    (T*)ly.ocat, nullptr, ws, nullptr, nullptr, CellRows<T>{}, true);
    o_last = (const T*)ws.o;
  } else {
    Carver cv(static_cast<char*>(ly.tape) + toff[i]);
    CellSave<T> sv = carve_save<T>(c, (size_t)M, K, true, pos0 > 0, cv);
    if (c->ctx_mod != DM_CTX_LINEAR)
      sv.vin = reinterpret_cast<T*>(static_cast<char*>(ly.tape) + toff[n_cells]) + vin_row(c, sched, n_cells, i) * d;
    CellWs cws = ws;
    if (sv.Mx) cws.M = sv.Mx;
    run_cell<T, DH>(c, w, L, cos, sin, pos0, cc, K, pos0, L->T, (T*)ly.K_cache, (T*)ly.V_cache, cache_T,
                    (T*)ly.ocat, nullptr, cws, &sv, nullptr, CellRows<T>{}, true);
    o_last = sv.o + (size_t)(K - 1) * M * d;
  }
  // W_O (+ the residual) of the chunk's rows: the last sweep's o holds the chunk's o_cat rows
  EpiResidual<T> ep{M, d, (c->flags & DM_FLAG_NO_RESIDUAL) ? nullptr : x, (T*)ly.y, map};
  SrcRows<T> ao{o_last, d, M};
  SrcRows<T> bo{(const T*)w->wo, d, d};
  // 64 x 64 blocks (the per-layer product's k-order, so its result)
  if constexpr (sizeof(T) == 2)
    launch_gemm_auto<T, 64, 64, 2, 2, 3, 4>(ao, bo, M, d, d, ep, nullptr);
  else
    launch_gemm<T, 64, 64, 2, 2, 4>(ao, bo, M, d, d, ep, nullptr);
  // the block tail (wave3d.py:26-28): the MLP sublayer of the chunk's rows, y -> z
  if (ly.mlp_w != nullptr)
    mlp_fwd_rows<T>(ly.mlp_w, (const T*)ly.y, (T*)ly.z, ly.mlp_bufs, M, d, ly.mlp_H, c->rms_eps, map.lc, L->T, pos0,
                    nullptr);
}

// Records every step and lines the layers' launches up; fills `tab` (when non-null) with the
// argument tables and returns the plan size in *bytes.
int plan_stack(const dm_config* c, int nl, const dm_stack_layer* layers, const float* cos, const float* sin,
               const int32_t* sched, int n_cells, int cache_T, std::vector<GroupedLaunch>& out,
               std::vector<unsigned char>* tab, size_t* bytes) {
  const std::vector<size_t> toff =
      c->dtype == DM_BF16 ? tape_offsets<bf16>(c, sched, n_cells) : tape_offsets<float>(c, sched, n_cells);
  size_t off = 0;
  std::vector<LaunchLog> logs;
  for (int t = 0; t < n_cells + nl - 1; ++t) {
    const int la = std::max(0, t - n_cells + 1), lb = std::min(nl - 1, t);
    logs.assign(lb - la + 1, LaunchLog{});
    for (int l = la; l <= lb; ++l) {
      launch_log() = &logs[l - la];
      if (c->dtype == DM_BF16) {
        if (c->dh == 64) record_chunk<bf16, 64>(c, layers[l], cos, sin, sched, n_cells, t - l, cache_T, toff);
        else record_chunk<bf16, 128>(c, layers[l], cos, sin, sched, n_cells, t - l, cache_T, toff);
      } else {
        if (c->dh == 64) record_chunk<float, 64>(c, layers[l], cos, sin, sched, n_cells, t - l, cache_T, toff);
        else record_chunk<float, 128>(c, layers[l], cos, sin, sched, n_cells, t - l, cache_T, toff);
      }
      launch_log() = nullptr;
    }
    const int rc = merge_step(t, logs, out, tab, off);
    if (rc) return rc;
  }
  *bytes = off;
  return DM_OK;
}

int check_stack(const dm_config* c, int nl, const dm_stack_layer* layers, const int32_t* sched, int n_cells,
                int cache_T) {
  int rc = check_cfg(c);
  if (rc) return rc;
  DM_REQUIRE(nl >= 1 && layers != nullptr, DM_ERR_INVALID, "n_layers=%d", nl);
  DM_REQUIRE(layers[0].bufs != nullptr, DM_ERR_INVALID, "null layer buffers");
  const int T = layers[0].bufs->T;
  if ((rc = dm_check_schedule(sched, n_cells, T))) return rc;
  for (int i = 0; i < n_cells; ++i)
    DM_REQUIRE(sched[3 * i + 1] == sched[1] && sched[3 * i + 2] == sched[2], DM_ERR_UNSUPPORTED,
               "the layer-batched forward needs equal cells (cell %d: c=%d K=%d, cell 0: c=%d K=%d)", i,
               sched[3 * i + 1], sched[3 * i + 2], sched[1], sched[2]);
  DM_REQUIRE(log2_exact(sched[1]) >= 0, DM_ERR_UNSUPPORTED, "cell length %d is not a power of two", sched[1]);
  DM_REQUIRE(T <= cache_T, DM_ERR_INVALID, "T=%d > cache_T=%d", T, cache_T);
  const bool tape = layers[0].tape != nullptr;
  const size_t need_ws = carve_cell(c, cache_T, nullptr).bytes;
  for (int l = 0; l < nl; ++l) {
    const dm_stack_layer& ly = layers[l];
    if ((rc = check_packed(c, ly.w)) || (rc = check_bufs(c, ly.bufs))) return rc;
    DM_REQUIRE(ly.bufs->T == T, DM_ERR_INVALID, "layer %d: T=%d, layer 0: T=%d", l, ly.bufs->T, T);
    DM_REQUIRE(ly.w->attn_norm_w == nullptr || ly.bufs->xhat != nullptr, DM_ERR_INVALID,
               "layer %d: attn_norm needs the xhat buffer", l);
    DM_REQUIRE(ly.x && ly.y && ly.ocat && aligned16(ly.x) && aligned16(ly.y), DM_ERR_INVALID,
               "layer %d: null/misaligned x, y or ocat", l);
    DM_REQUIRE(ly.K_cache && ly.V_cache && aligned16(ly.K_cache) && aligned16(ly.V_cache), DM_ERR_INVALID,
               "layer %d: K/V cache must be non-null and 16-byte aligned", l);
    DM_REQUIRE(ly.workspace && ly.workspace_bytes >= need_ws && aligned16(ly.workspace), DM_ERR_WORKSPACE,
               "layer %d: workspace %zu < %zu bytes", l, ly.workspace_bytes, need_ws);
    DM_REQUIRE((ly.tape != nullptr) == tape, DM_ERR_INVALID, "layer %d: all layers with a tape or none", l);
    if (ly.mlp_w != nullptr) {
      if ((rc = check_mlp(c->dtype, ly.mlp_w, ly.mlp_bufs, c->B * T, c->d, ly.mlp_H))) return rc;
      DM_REQUIRE(ly.z && aligned16(ly.z) && ly.z != ly.y, DM_ERR_INVALID, "layer %d: the block tail needs its own "
                 "16-byte aligned z", l);
    }
    if (tape) {
      const size_t need = dm_layer_tape_bytes(c, sched, n_cells);
      DM_REQUIRE(ly.tape_bytes >= need && aligned16(ly.tape), DM_ERR_WORKSPACE, "layer %d: tape %zu < %zu bytes",
                 l, ly.tape_bytes, need);
    }
  }
  return DM_OK;
}

// The launch list of every plan written by this process (keyed by the plan's device
// address): a call with build == 0 replays it without recording the steps again.
struct PlanCache {
  std::mutex mu;
  std::map<const void*, std::vector<GroupedLaunch>> lists;
};
PlanCache& plan_cache() {
  static PlanCache c;
  return c;
}

}  // namespace
}  // namespace dm

using namespace dm;

extern "C" {

size_t dm_stack_fwd_plan_bytes(const dm_config* c, int32_t n_layers, const dm_stack_layer* layers,
                               const int32_t* sched, int32_t n_cells, int32_t cache_T) {
  if (check_stack(c, n_layers, layers, sched, n_cells, cache_T) != DM_OK) return 0;
  std::vector<GroupedLaunch> launches;
  size_t bytes = 0;
  if (plan_stack(c, n_layers, layers, nullptr, nullptr, sched, n_cells, cache_T, launches, nullptr, &bytes) != DM_OK)
    return 0;
  return bytes;
}

int dm_stack_fwd(const dm_config* c, int32_t n_layers, const dm_stack_layer* layers, const float* cos,
                 const float* sin, const int32_t* sched, int32_t n_cells, int32_t cache_T, void* plan,
                 size_t plan_bytes, int32_t build, void* stream) {
  int rc = check_stack(c, n_layers, layers, sched, n_cells, cache_T);
  if (rc) return rc;
  DM_REQUIRE(cos && sin, DM_ERR_INVALID, "null rope tables");
  DM_REQUIRE(plan != nullptr && (reinterpret_cast<uintptr_t>(plan) & 255) == 0, DM_ERR_INVALID,
             "plan must be non-null and 256-byte aligned");
  ArgSig sig;
  sig.val(*c); sig.val(n_layers); sig.val(cos); sig.val(sin); sig.val(n_cells); sig.val(cache_T);
  sig.val(plan_bytes); sig.add(sched, sizeof(int32_t) * 3 * (size_t)n_cells);
  for (int l = 0; l < n_layers; ++l) {
    const dm_stack_layer& ly = layers[l];
    sig.val(*ly.w); sig.bufs(ly.bufs);
    sig.val(ly.x); sig.val(ly.y); sig.val(ly.K_cache); sig.val(ly.V_cache); sig.val(ly.ocat);
    sig.val(ly.tape); sig.val(ly.tape_bytes); sig.val(ly.workspace); sig.val(ly.workspace_bytes);
    sig.val(ly.mlp_w); sig.val(ly.z); sig.val(ly.mlp_H);
    if (ly.mlp_w != nullptr) { sig.val(*ly.mlp_w); sig.val(*ly.mlp_bufs); }
  }
  std::vector<GroupedLaunch> launches;
  if (!build) {
    DM_REQUIRE(plan_sig_matches(plan, sig.h), DM_ERR_INVALID,
               "plan %p was not written for these arguments (call once with build != 0)", plan);
    PlanCache& pc = plan_cache();
    std::lock_guard<std::mutex> lk(pc.mu);
    auto it = pc.lists.find(plan);
    DM_REQUIRE(it != pc.lists.end(), DM_ERR_INVALID, "plan %p has no launch list", plan);
    launches = it->second;
  } else {
    plan_sig_forget(plan);
    std::vector<unsigned char> tab;
    size_t bytes = 0;
    if ((rc = plan_stack(c, n_layers, layers, cos, sin, sched, n_cells, cache_T, launches, &tab, &bytes)))
      return rc;
    DM_REQUIRE(plan_bytes >= bytes, DM_ERR_WORKSPACE, "plan %zu < %zu bytes", plan_bytes, bytes);
    if ((rc = write_plan(plan, tab.data(), bytes, S(stream)))) return rc;
    {
      PlanCache& pc = plan_cache();
      std::lock_guard<std::mutex> lk(pc.mu);
      pc.lists[plan] = launches;
    }
    plan_sig_store(plan, sig.h);
  }
  hipStream_t s = S(stream);
  for (const GroupedLaunch& g : launches)
    if ((rc = issue_grouped(g, plan, s))) return rc;
  DM_HIP(hipGetLastError());
  return DM_OK;
}

}  // extern "C"
