// Optional per-kernel-class timing with HIP events (host side).
//
// When a class is armed (dm_prof_start), every launch of that class records a
// start and a stop event on the launch's own stream; dm_prof_stop waits for the
// last event and returns the summed elapsed time and the launch count. Unarmed,
// a ProfScope costs one integer compare. Used by bench.py to time the dominant
// kernel inside its timed region; never armed on the product path.
#pragma once

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

}  // namespace dm
