// Host-side helpers shared by the translation units of libdm_hip.so:
// error reporting, argument checks, launch helpers, workspace carving.
#pragma once

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdint>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/dm_abi.h"
#include "dm_kernels.h"
#include "dm_prof.h"

namespace dm {

// Launch shapes of the per-sweep GEMMs (M = B*c rows). Their k-loops are bound by LDS
// traffic; two 64 x 64 blocks per CU let one block's epilogue overlap the other's k-loop
// (64 x 128 blocks, one per CU, measured slower). The defaults are the measured best on
// MI355X; -D overrides exist for tuning builds.
#ifndef DM_SW1_STAGES
#define DM_SW1_STAGES 3   // sweep GEMM 1: direct-to-LDS stages of the 64 x 64 blocks
#endif
#ifndef DM_SW2_STAGES
#define DM_SW2_STAGES 3   // GEMM 2 / dv_in GEMM (64 x 32 blocks): direct-to-LDS stages (0 = register ring of depth 8)
#endif
#ifndef DM_DU_STAGES
#define DM_DU_STAGES 3    // du split-K GEMM: direct-to-LDS stages of the 64 x 64 blocks
#endif
#ifndef DM_DU_SPLIT
#define DM_DU_SPLIT 4     // du split-K slices (K = 4d is long, M = B*c short)
#endif
// Layer-level GEMMs (M = B*T rows, outside the sweep chain): block tile and
// direct-to-LDS stages of the K-contiguous products, stages of the K-major (weight-grad)
// 256 x 256 products.
#ifndef DM_BIG_BM
#define DM_BIG_BM 256
#endif
#ifndef DM_BIG_BN
#define DM_BIG_BN 256
#endif
#ifndef DM_BIG_STAGES
#define DM_BIG_STAGES 2
#endif
#ifndef DM_GROUPED_WIDE_SW1
#define DM_GROUPED_WIDE_SW1 1  // layer-batched sweep GEMM 1 in 64 x 128 tiles
#endif
#ifndef DM_SW1_EIGHT_WAVES
#define DM_SW1_EIGHT_WAVES 1   // sweep GEMM 1 in 64 x 128 blocks of eight waves (one column group per half)
#endif
#ifndef DM_KK_STAGES
#define DM_KK_STAGES 2
#endif
constexpr int SW1_STAGES = DM_SW1_STAGES, SW2_STAGES = DM_SW2_STAGES, DU_STAGES = DM_DU_STAGES;
constexpr int BIG_BM = DM_BIG_BM, BIG_BN = DM_BIG_BN, BIG_STAGES = DM_BIG_STAGES, KK_STAGES = DM_KK_STAGES;

inline std::string& last_error() {
  static thread_local std::string e;
  return e;
}

inline int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
inline int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  last_error() = buf;
  return code;
}

#define DM_REQUIRE(cond, code, ...)                  \
  do {                                               \
    if (!(cond)) return ::dm::fail(code, __VA_ARGS__); \
  } while (0)

#define DM_HIP(call)                                                                             \
  do {                                                                                           \
    hipError_t e_ = (call);                                                                      \
    if (e_ != hipSuccess) return ::dm::fail(DM_ERR_HIP, "%s: %s", #call, hipGetErrorString(e_)); \
  } while (0)

inline hipStream_t S(void* s) { return reinterpret_cast<hipStream_t>(s); }
inline size_t esz(int dtype) { return dtype == DM_BF16 ? 2 : 4; }
inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }
inline int cdiv(long a, long b) { return (int)((a + b - 1) / b); }
inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

constexpr int COMM_SPLIT_MIN = 256;   // committed keys per split (lower bound)
constexpr int DEC_SPLIT = 512;        // tape keys per decode split

inline int check_cfg(const dm_config* c) {
  DM_REQUIRE(c != nullptr, DM_ERR_INVALID, "null config");
  DM_REQUIRE(c->dtype == DM_F32 || c->dtype == DM_BF16, DM_ERR_INVALID, "dtype %d", c->dtype);
  DM_REQUIRE(c->B > 0 && c->d > 0 && c->h > 0 && c->dh > 0, DM_ERR_INVALID, "non-positive dims");
  DM_REQUIRE(c->d == c->h * c->dh, DM_ERR_INVALID, "d=%d != h*dh=%d", c->d, c->h * c->dh);
  DM_REQUIRE(c->dh == 64 || c->dh == 128, DM_ERR_UNSUPPORTED, "head_dim %d (64 or 128)", c->dh);
  DM_REQUIRE(c->d % (2 * c->dh) == 0 && c->d % 128 == 0, DM_ERR_UNSUPPORTED,
             "d_model %d must be a multiple of 128 and of 2*head_dim", c->d);
  DM_REQUIRE(c->d <= RMS_MAXK, DM_ERR_UNSUPPORTED, "d_model %d > %d", c->d, RMS_MAXK);
  DM_REQUIRE(c->h <= MAX_HEADS && c->d / 32 <= MAX_ROWDOT, DM_ERR_UNSUPPORTED, "%d heads (at most %d)", c->h,
             MAX_HEADS);
  DM_REQUIRE(c->ctx_mod >= 0 && c->ctx_mod <= DM_CTX_FUSION, DM_ERR_UNSUPPORTED, "ctx_mod %d", c->ctx_mod);
  DM_REQUIRE(c->kmod_vraw_heads >= 0 && c->kmod_vraw_heads <= c->h && c->kmod_mode >= DM_KMOD_RAW &&
                 c->kmod_mode <= DM_KMOD_GATED_NORM,
             DM_ERR_UNSUPPORTED, "kmod_vraw_heads %d / kmod_mode %d", c->kmod_vraw_heads, c->kmod_mode);
  DM_REQUIRE(c->v_clamp_tau >= 0.f, DM_ERR_INVALID, "v_clamp_tau %g", (double)c->v_clamp_tau);
  DM_REQUIRE(c->local_window >= 0, DM_ERR_INVALID, "local_window %d", c->local_window);
  DM_REQUIRE((c->norms & ~(DM_NORM_K_CTX | DM_NORM_V_CTX | DM_NORM_V)) == 0, DM_ERR_UNSUPPORTED, "norms bits 0x%x",
             c->norms);
  return DM_OK;
}

// committed-prefix split plan for a cell at pos0
struct CommPlan {
  int nsplit, split_len;
};
// forward: enough splits for ~512 blocks over the B*h heads (the first sweep's
// attention merges them, so no more than that)
// (n: the committed keys the cell reads, pos0 or, with a window, fewer)
inline CommPlan comm_plan(int n, int BH) {
  if (n <= 0) return CommPlan{0, 0};
  int nsplit = cdiv(n, COMM_SPLIT_MIN);
  nsplit = std::min(nsplit, std::max(1, std::min(COMM_MAX_SPLITS, cdiv(512, BH))));
  const int split_len = cdiv(cdiv(n, nsplit), 64) * 64;
  return CommPlan{cdiv(n, split_len), split_len};
}
// The window the kernels apply for local_window W (attention.py:291-293): a row at position i
// reads keys >= i - W + 1, committed and intra (0 = none). W = 1 reads like no window, as the
// reference's attend_one does: it keeps K_past[:, :, -(W - 1):], and for W = 1 that is
// K_past[:, :, -0:], the whole past.
inline int window_of(const dm_config* c) { return c->local_window > 1 ? c->local_window : 0; }

// first committed key a cell at pos0 reads (chunk row 0's window start)
inline int comm_kstart(int pos0, int window) { return window > 0 ? std::max(0, pos0 - window + 1) : 0; }
// the cell's last committed keys [comm_prev_lo, pos0), at most one 64-key tile: its first sweep's
// attention reads them itself; the split partials cover [kstart, comm_prev_lo)
inline int comm_prev_lo(int pos0, int kstart) { return std::max(kstart, pos0 - 64); }
inline int comm_splits_max(int cache_T) {
  int n = cdiv(cache_T, COMM_SPLIT_MIN);
  return n < 1 ? 1 : (n > COMM_MAX_SPLITS ? COMM_MAX_SPLITS : n);
}

// bump allocator over a caller-provided workspace (base == nullptr: size query)
struct Carver {
  char* base;
  size_t off = 0;
  explicit Carver(void* b) : base(reinterpret_cast<char*>(b)) {}
  template <typename P> P* take(size_t bytes) {
    char* r = base ? base + off : nullptr;
    off += align256(bytes);
    return reinterpret_cast<P*>(r);
  }
};

// ---- grouped launches of the layer-batched stack passes ------------------------------
// One grouped launch (argument table at plan + off), or the per-layer closing work of
// layer `layer_end` (issued directly, not grouped).
struct GroupedLaunch {
  const void* f;
  dim3 grid, block;
  unsigned shmem;
  size_t off;
  int layer_end;
};

// Lines one step's per-layer records up position by position into grouped launches (their
// argument tables appended to tab when non-null, at 256-byte aligned offsets from off).
inline int merge_step(int t, const std::vector<LaunchLog>& logs, std::vector<GroupedLaunch>& out,
                      std::vector<unsigned char>* tab, size_t& off) {
  for (const LaunchLog& lg : logs)
    DM_REQUIRE(!lg.unsupported, DM_ERR_UNSUPPORTED, "step %d: a launch has no grouped form", t);
  const size_t n = logs[0].recs.size();
  for (const LaunchLog& lg : logs)
    DM_REQUIRE(lg.recs.size() == n, DM_ERR_UNSUPPORTED, "step %d: layers record %zu and %zu launches", t,
               lg.recs.size(), n);
  const int G = (int)logs.size();
  for (size_t r = 0; r < n; ++r) {
    const LaunchRec& r0 = logs[0].recs[r];
    unsigned gx = 0;
    for (const LaunchLog& lg : logs) {
      const LaunchRec& x = lg.recs[r];
      DM_REQUIRE(x.gfunc == r0.gfunc && x.grid.y == r0.grid.y && x.block.x == r0.block.x &&
                     x.shmem == r0.shmem && x.args_bytes == r0.args_bytes,
                 DM_ERR_UNSUPPORTED, "step %d, launch %zu differs between layers", t, r);
      gx = std::max(gx, x.grid.x);
    }
    if (gx == 0) continue;   // nothing to do for any layer
    off = (off + 255) / 256 * 256;
    out.push_back(GroupedLaunch{r0.gfunc, dim3(gx, r0.grid.y, G), r0.block, r0.shmem, off, -1});
    if (tab != nullptr) {
      tab->resize(off + (size_t)G * r0.args_bytes);
      for (int g = 0; g < G; ++g)
        std::memcpy(tab->data() + off + (size_t)g * r0.args_bytes, logs[g].recs[r].args.data(), r0.args_bytes);
    }
    off += (size_t)G * r0.args_bytes;
  }
  return DM_OK;
}

inline int issue_grouped(const GroupedLaunch& g, void* plan, hipStream_t s) {
  void* p = static_cast<char*>(plan) + g.off;
  void* args[] = {&p};
  DM_HIP(hipLaunchKernel(g.f, g.grid, g.block, args, g.shmem, s));
  return DM_OK;
}

// ---- plans of the layer-batched passes -----------------------------------------------------
// A plan's device table holds the argument structs of a pass's grouped launches. The library
// remembers, per plan address, a signature (FNV-1a) of every argument the table was written
// for; a call that launches from a written plan (build == 0) must present the same arguments,
// so a plan never written, overwritten by another pass, or written for other buffers is refused
// instead of being launched.
struct ArgSig {
  uint64_t h = 1469598103934665603ull;
  void add(const void* p, size_t n) {
    const unsigned char* b = static_cast<const unsigned char*>(p);
    for (size_t i = 0; i < n; ++i) {
      h ^= b[i];
      h *= 1099511628211ull;
    }
  }
  template <class X> void val(const X& x) { add(&x, sizeof(x)); }
  void bufs(const dm_layer_bufs* L) {   // field by field: the struct has padding after T
    val(L->T); val(L->xhat); val(L->qr); val(L->kraw); val(L->kself); val(L->vraw); val(L->glogx);
    val(L->sig); val(L->vpre);
  }
};
inline std::mutex& plan_sig_mu() {
  static std::mutex m;
  return m;
}
inline std::map<const void*, uint64_t>& plan_sigs() {
  static std::map<const void*, uint64_t> m;
  return m;
}
// a build forgets the plan's signature first (a failed build leaves no usable plan) and stores it
// once the pass has gone through
inline void plan_sig_forget(const void* plan) {
  std::lock_guard<std::mutex> lk(plan_sig_mu());
  plan_sigs().erase(plan);
}
inline void plan_sig_store(const void* plan, uint64_t sig) {
  std::lock_guard<std::mutex> lk(plan_sig_mu());
  plan_sigs()[plan] = sig;
}
inline bool plan_sig_matches(const void* plan, uint64_t sig) {
  std::lock_guard<std::mutex> lk(plan_sig_mu());
  auto it = plan_sigs().find(plan);
  return it != plan_sigs().end() && it->second == sig;
}
// Write a plan's argument table (host staging -> device) for the grouped launches that read it on
// stream s. A build is a one-time set-up step and is refused while s is being captured; otherwise
// s is drained first, so that no launch still in flight on s reads an earlier table at the same
// address, and the blocking copy has landed before the new launches are issued.
inline int write_plan(void* plan, const void* tab, size_t bytes, hipStream_t s) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  DM_HIP(hipStreamIsCapturing(s, &cs));
  DM_REQUIRE(cs == hipStreamCaptureStatusNone, DM_ERR_INVALID,
             "a plan cannot be built (build != 0) on a stream under capture: build it once before capturing");
  DM_HIP(hipStreamSynchronize(s));
  DM_HIP(hipMemcpy(plan, tab, bytes, hipMemcpyHostToDevice));
  return DM_OK;
}

inline int log2_exact(int v) {
  int l = 0;
  while ((1 << l) < v) ++l;
  return (1 << l) == v ? l : -1;
}

// GEMM launch: grid (N/BN, ceil(M/BM)), 64 WM WN threads (grouped-launch bodies: 4 waves only)
template <typename T, int BM, int BN, int WM, int WN, int D, class SA, class SB, class EPI>
void launch_gemm(const SA& sa, const SB& sb, int M, int N, int K, const EPI& epi, hipStream_t s,
                 int prof_cls = PROF_NONE) {
  dim3 grid(N / BN, cdiv(M, BM));
  if constexpr (WM * WN == 4) {
    if (launch_log() != nullptr) {
      using Body = GemmBody<T, BM, BN, WM, WN, D, SA, SB, EPI>;
      record_launch<Body>(grid, dim3(256), typename Body::Args{sa, sb, K, epi});
      return;
    }
  }
  uint64_t* ts;
  const int idx = prof_launch_begin(prof_cls, true, ts);
  launch_timed(idx, k_gemm<T, BM, BN, WM, WN, D, SA, SB, EPI>, grid, dim3(64 * WM * WN), 0, s, sa, sb, K, epi,
               ts);
}

// bf16 with K-contiguous operands and K a multiple of 64: the direct-to-LDS k-loop
// with S stages; otherwise the register-ring k-loop of depth D.
template <typename T, int BM, int BN, int WM, int WN, int S, int D, class SA, class SB, class EPI>
void launch_gemm_auto(const SA& sa, const SB& sb, int M, int N, int K, const EPI& epi, hipStream_t s,
                      int prof_cls = PROF_NONE) {
  if constexpr (sizeof(T) == 2 && !SA::KMAJOR && !SB::KMAJOR) {
    if (K % 64 == 0) {
      launch_gemm<T, BM, BN, WM, WN, -S>(sa, sb, M, N, K, epi, s, prof_cls);
      return;
    }
  }
  launch_gemm<T, BM, BN, WM, WN, D>(sa, sb, M, N, K, epi, s, prof_cls);
}

// Large GEMMs (M, N multiples of 256, bf16, K-contiguous, K a multiple of 64): 256 x 256
// blocks of four 128 x 128 wave tiles with two 64 KB direct-to-LDS stages (a quarter of
// the LDS traffic per MFMA of 64 x 64 wave tiles); otherwise 128 x 128.
template <typename T, class SA, class SB, class EPI>
void launch_gemm_big(const SA& sa, const SB& sb, int M, int N, int K, const EPI& epi, hipStream_t s,
                     int prof_cls = PROF_NONE) {
  if constexpr (sizeof(T) == 2 && !SA::KMAJOR && !SB::KMAJOR) {
    if (M % BIG_BM == 0 && N % BIG_BN == 0 && K % 64 == 0) {
      launch_gemm<T, BIG_BM, BIG_BN, 2, 2, -BIG_STAGES>(sa, sb, M, N, K, epi, s, prof_cls);
      return;
    }
  }
  launch_gemm_auto<T, 128, 128, 2, 2, 3, 4>(sa, sb, M, N, K, epi, s, prof_cls);
}

// K-major operands (C = A^T B summed over rows; element (r, k) at p[k * ld + r]):
// bf16 whole tiles with K a multiple of 64 take the direct-to-LDS path (256 x 256
// blocks where M and N allow), otherwise the register ring.
template <typename T, class EPI>
void launch_gemm_kk(const SrcKMajor<T>& sa, const SrcKMajor<T>& sb, int M, int N, int K, const EPI& epi,
                    hipStream_t s, int prof_cls = PROF_NONE) {
  if constexpr (sizeof(T) == 2) {
    if (K % 64 == 0 && sa.kmax >= K && sb.kmax >= K) {
      if (M % 256 == 0 && N % 256 == 0) {
        launch_gemm<T, 256, 256, 2, 2, -KK_STAGES>(sa, sb, M, N, K, epi, s, prof_cls);
        return;
      }
      if (M % 128 == 0 && N % 128 == 0) {
        launch_gemm<T, 128, 128, 2, 2, -3>(sa, sb, M, N, K, epi, s, prof_cls);
        return;
      }
    }
  }
  launch_gemm<T, 128, 128, 2, 2, 4>(sa, sb, M, N, K, epi, s, prof_cls);
}

// Two independent GEMMs (GemmPart) in one launch: the first's blocks, then the second's.
template <class P1, class P2>
void launch_gemm_pair(const P1& p1, const P2& p2, hipStream_t s) {
  using Body = GemmPairBody<P1, P2>;
  const int n = p1.gx * p1.gy * p1.nz + p2.gx * p2.gy * p2.nz;
  const typename Body::Args a{p1, p2};
  if (launch_log() != nullptr) {
    record_launch<Body>(dim3(n), dim3(256), a);
    return;
  }
  hipLaunchKernelGGL((k_gemm_pair<P1, P2>), dim3(n), dim3(256), 0, s, a);
}

// Split-K: S slices of K/S each (K/S a multiple of the k-tile), slice z in grid.z.
template <typename T, int BM, int BN, int WM, int WN, int D, class SA, class SB, class EPI>
void launch_gemm_splitk(const SA& sa, const SB& sb, int M, int N, int K, int S, const EPI& epi, hipStream_t s,
                        int prof_cls = PROF_NONE) {
  dim3 grid(N / BN, cdiv(M, BM), S);
  if (launch_log() != nullptr) {   // grouped: the slices stacked along grid y
    using Body = SplitGemmBody<T, BM, BN, WM, WN, D, SA, SB, EPI>;
    record_launch<Body>(dim3(N / BN, cdiv(M, BM) * S), dim3(256), typename Body::Args{sa, sb, K / S, epi, cdiv(M, BM)});
    return;
  }
  uint64_t* ts;
  const int idx = prof_launch_begin(prof_cls, true, ts);
  launch_timed(idx, k_gemm<T, BM, BN, WM, WN, D, SA, SB, EPI>, grid, dim3(256), 0, s, sa, sb, K / S, epi, ts);
}

}  // namespace dm
