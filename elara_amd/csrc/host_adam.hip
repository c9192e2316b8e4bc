// Row-sparse Adam on the host (elr_cpu_adam): the host workers' op of the reference's capacity tier, for a C caller
// of this library that updates rows held in host memory (srm2/csrc/srm2_cpu.cpp:37-56 cpu_adam, which the
// reference's update worker runs on its host arenas, srm2/elara.py:567).  Host code only: no GPU is touched.
//
// Each element is one IEEE binary32 operation per statement, in the reference's order, with no contraction (this
// file is compiled with -ffp-contract=off like every source of the library), so the results are bitwise those of
// the GPU kernels and of the reference's CPU extension.  Work split: nthreads contiguous ranges of the row list,
// one thread each; a single thread below 256 rows.  A row outside [0, R) is skipped, as the GPU kernels skip it.
#include <thread>
#include <vector>

#include "elr_common.h"

namespace {

void adam_host_rows(float* state, int64_t R, const int64_t* rows, const float* grad, int64_t lo, int64_t hi,
                    int64_t D, const float* sc) {
  const float lr = sc[0], b1 = sc[1], omb1 = sc[2], b2 = sc[3], omb2 = sc[4], bc1 = sc[5], bc2 = sc[6], eps = sc[7];
  for (int64_t i = lo; i < hi; ++i) {
    const int64_t r = rows[i];
    if (r < 0 || r >= R) continue;
    float* w = state + r * 3 * D;
    float* m = w + D;
    float* v = w + 2 * D;
    const float* g = grad + i * D;
    for (int64_t j = 0; j < D; ++j) {
      const float gj = g[j];
      const float mj = b1 * m[j] + omb1 * gj;
      const float t2 = omb2 * gj;
      const float vj = b2 * v[j] + t2 * gj;
      const float den = __builtin_sqrtf(vj / bc2) + eps;
      w[j] = w[j] - (lr * (mj / bc1)) / den;
      m[j] = mj;
      v[j] = vj;
    }
  }
}

}  // namespace

extern "C" int elr_cpu_adam(float* state, int64_t R, const int64_t* rows, const float* grad, int64_t n, int64_t D,
                            const float sc[8], int nthreads) {
  if (n < 0 || D < 1 || R < 0 || !sc) return ELR_EINVAL;
  if (n == 0) return ELR_OK;
  if (!state || !rows || !grad) return ELR_EINVAL;
  if (nthreads <= 1 || n < 256) {
    adam_host_rows(state, R, rows, grad, 0, n, D, sc);
    return ELR_OK;
  }
  const int64_t chunk = (n + nthreads - 1) / nthreads;
  std::vector<std::thread> pool;
  for (int64_t lo = 0; lo < n; lo += chunk) {
    const int64_t hi = lo + chunk < n ? lo + chunk : n;
    pool.emplace_back(adam_host_rows, state, R, rows, grad, lo, hi, D, sc);
  }
  for (std::thread& t : pool) t.join();
  return ELR_OK;
}
