// Kernels as functors: a body `void operator()(int64_t block, int64_t nblocks) const` that takes its block index
// from the caller instead of blockIdx, launched on its own (k_run) or beside an independent body in one launch
// (k_run2: blocks [0, n1) run the first, the others the second).  The step's executor pairs the directory's small
// launches, which wait on one another, with the large row kernels that do not depend on them, so that the small
// ones cost no launch of their own.  Every body here uses 256-thread blocks.
#pragma once

#include "elr_common.h"

namespace elr {

constexpr int kFunctorBlock = 256;

template <class F>
__global__ __launch_bounds__(kFunctorBlock) void k_run(F f) {
  f((int64_t)blockIdx.x, (int64_t)gridDim.x);
}

template <class F1, class F2>
__global__ __launch_bounds__(kFunctorBlock) void k_run2(F1 f1, int64_t n1, F2 f2) {
  const int64_t b = blockIdx.x;
  if (b < n1) f1(b, n1);
  else f2(b - n1, (int64_t)gridDim.x - n1);
}

template <class F>
inline void launch1(const F& f, int64_t blocks, hipStream_t st) {
  if (blocks > 0) k_run<F><<<(unsigned)blocks, kFunctorBlock, 0, st>>>(f);
}

// f1 on n1 blocks and f2 on n2 blocks in one launch (a body without blocks is left out).
template <class F1, class F2>
inline void launch2(const F1& f1, int64_t n1, const F2& f2, int64_t n2, hipStream_t st) {
  if (n1 <= 0) launch1(f2, n2, st);
  else if (n2 <= 0) launch1(f1, n1, st);
  else k_run2<F1, F2><<<(unsigned)(n1 + n2), kFunctorBlock, 0, st>>>(f1, n1, f2);
}

// Global wave index and wave count of a body's block, wave-uniform (SGPR) values: indices derived from them address
// kernel arguments and row bases with scalar instructions.
__device__ __forceinline__ int64_t body_wave(int64_t block) {
  return (int64_t)__builtin_amdgcn_readfirstlane((int)(block * (kFunctorBlock / 64) + (threadIdx.x >> 6)));
}
__device__ __forceinline__ int64_t body_waves(int64_t nblocks) { return nblocks * (kFunctorBlock / 64); }

}  // namespace elr
