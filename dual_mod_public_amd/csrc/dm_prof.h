// Optional per-kernel-class timing (host side).
//
// When a class is armed (dm_prof_start), every launch of that class is timed:
//  * a HIP start/stop event pair that the launch itself stamps (hipExtLaunchKernel: the
//    kernel dispatch's own begin and end, the interval a kernel-trace profiler reports);
//    launch groups (ProfScope) record ordinary events around the group instead;
//  * the GEMM kernels and the decode tape read also take their span from the device
//    clock (first block start to last block end, folded into PROF_SLOTS slots per
//    launch; see prof_begin / prof_end): the execution without dispatch and drain.
// dm_prof_stop waits for the last event and returns the summed times and the
// launch count. Unarmed, a launch costs one integer compare. Used by bench.py to
// time the dominant kernel inside its timed region; never armed on the product path.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <vector>

namespace dm {

enum ProfClass {
  PROF_NONE = 0,
  PROF_PROJ = 1,         // layer projection GEMM (+ its RMSNorm)
  PROF_COMM = 2,         // committed-prefix accumulator (partials + merge)
  PROF_ATTEND = 3,       // per-sweep intra attention + merge
  PROF_SWEEP1 = 4,       // per-sweep packed GEMM (k_ctx | g_k | v_map | g_v) + epilogue
  PROF_SWEEP2 = 5,       // per-sweep w_vctx GEMM + blend epilogue
  PROF_WO = 6,           // W_O projection + residual
  PROF_DEC_READ = 7,     // decode tape read (split partials)
  PROF_DEC_MERGE = 8,    // decode LSE merge + self column
  PROF_DEC_REFINE = 9,   // decode refine GEMMs
  PROF_BWD = 10,         // backward kernels (all classes of the reverse sweep)
  PROF_LAYER = 11,       // one whole entry-point call (dm_layer_fwd / dm_layer_bwd / dm_decode_step)
  PROF_NCLASS = 12
};

struct ProfState {
  int armed = PROF_NONE;
  int cap = 0;
  int n = 0;
  std::vector<hipEvent_t> ev;   // 2 * cap events: start, stop
  uint64_t* dts = nullptr;      // [cap][2 * PROF_SLOTS] device-clock slots
  int dts_cap = 0;
  std::vector<char> dev_timed;  // per launch: took device-clock slots
  bool dev_clock = true;        // false: events only (the kernels write no device-clock slots)
};

inline ProfState& prof() {
  static ProfState s;
  return s;
}

// RAII bracket around one launch (or one group of launches) of class `cls`.
struct ProfScope {
  hipEvent_t stop_ = nullptr;
  hipStream_t s_;
  ProfScope(int cls, hipStream_t s) : s_(s) {
    ProfState& p = prof();
    if (p.armed != cls || p.n >= p.cap) return;
    (void)hipEventRecord(p.ev[2 * p.n], s);
    stop_ = p.ev[2 * p.n + 1];
    ++p.n;
  }
  ~ProfScope() {
    if (stop_ != nullptr) (void)hipEventRecord(stop_, s_);
  }
};

// Timing of one launch of class `cls`: when armed, reserves the launch's event pair and
// returns its index (else -1). `ts` receives the launch's device-clock slots when the
// kernel supports them (dev_ts) — nullptr otherwise.
inline int prof_launch_begin(int cls, bool dev_ts, uint64_t*& ts) {
  ProfState& p = prof();
  ts = nullptr;
  if (p.armed != cls || cls == PROF_NONE || p.n >= p.cap) return -1;
  if (dev_ts && p.dev_clock && p.dts != nullptr) {
    ts = p.dts + (size_t)p.n * 2 * PROF_SLOTS;
    p.dev_timed[p.n] = 1;
  }
  return p.n++;
}

// The launch: with a reserved event pair (idx >= 0) the dispatch stamps both events.
template <typename F, typename... Args>
inline void launch_timed(int idx, F kernel, dim3 grid, dim3 block, uint32_t shmem, hipStream_t s, Args... args) {
  if (idx >= 0)
    hipExtLaunchKernelGGL(kernel, grid, block, shmem, s, prof().ev[2 * idx], prof().ev[2 * idx + 1], 0, args...);
  else
    hipLaunchKernelGGL(kernel, grid, block, shmem, s, args...);
}

// a launch of class `cls` with event timing
template <typename F, typename... Args>
inline void launch_k(int cls, F kernel, dim3 grid, dim3 block, uint32_t shmem, hipStream_t s, Args... args) {
  uint64_t* ts;
  const int idx = prof_launch_begin(cls, false, ts);
  launch_timed(idx, kernel, grid, block, shmem, s, args...);
}

}  // namespace dm
