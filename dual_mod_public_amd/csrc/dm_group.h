// Grouped launches for the layer-batched (wavefront) forward of a layer stack.
//
// A kernel written as a Body (static constexpr int THREADS; struct Args; static
// run(const Args&, int bx, int by)) can run as its ordinary kernel or as k_grouped<Body>: one
// launch over several independent argument sets, set g in grid z, read from a table in device
// memory. The wavefront driver records what one layer's chunk would launch (launch_log() set:
// the launch helpers append a LaunchRec instead of launching), for every active layer, and
// then issues each recorded position once for all of them.
#pragma once

#include <hip/hip_runtime.h>

#include <cstring>
#include <vector>

namespace dm {

// Body::MIN_WAVES (optional): the waves per SIMD the kernel is built for (register budget)
template <class Body, class = void> struct min_waves_of {
  static constexpr int value = 1;
};
template <class Body> struct min_waves_of<Body, decltype(void(Body::MIN_WAVES))> {
  static constexpr int value = Body::MIN_WAVES;
};

template <class Body>
__global__ __launch_bounds__(Body::THREADS, min_waves_of<Body>::value) void k_grouped(
    const typename Body::Args* __restrict__ tab) {
  Body::run(tab[blockIdx.z], (int)blockIdx.x, (int)blockIdx.y);
}

struct LaunchRec {
  const void* gfunc;   // k_grouped<Body>
  dim3 grid, block;    // grid.x of this argument set (0: nothing to do for it), grid.y, block
  unsigned shmem;      // dynamic LDS bytes
  size_t args_bytes;
  std::vector<unsigned char> args;
};
struct LaunchLog {
  std::vector<LaunchRec> recs;
  bool unsupported = false;   // a launch with no grouped form was reached
};
// non-null while launches are recorded instead of issued (per host thread)
inline LaunchLog*& launch_log() {
  static thread_local LaunchLog* log = nullptr;
  return log;
}

template <class Body>
inline void record_launch(dim3 grid, dim3 block, const typename Body::Args& a, unsigned shmem = 0) {
  LaunchRec r;
  r.gfunc = reinterpret_cast<const void*>(&k_grouped<Body>);
  r.grid = grid;
  r.block = block;
  r.shmem = shmem;
  r.args_bytes = sizeof(a);
  r.args.resize(sizeof(a));
  std::memcpy(r.args.data(), &a, sizeof(a));
  launch_log()->recs.push_back(std::move(r));
}

}  // namespace dm
