// Row copies between HBM arrays of fixed-width fp32 rows: gradient-log appends and the executor's gathers and
// scatters (HBM-bound, no arithmetic).
//
// dst[dst_idx[i]] = src[src_idx[i]] for i < n (a NULL index array means the identity).  Replaces, with the HBM-resident
// log arena of this build:
//   - the gradient-log append logs[A_ids] = g (srm2/elara.py:569-570 cpu_scatter(logs, A_ids); srm2/csrc/srm2_cpu.cpp
//     cs_append semantics, :167-180);
//   - the resident-history record glog.index_put_((dyn, j), g) (srm2/elara.py:501, 524) on glog viewed as
//     [(Cdyn+1)*K, D];
//   - index_select / index_copy_ of rows between the pool, the staging buffers and W (srm2/elara.py:480-488,
//     506-531; srm2/executor.py:190-199).
// One wave per row, 16-byte accesses when the width and both bases allow it; a row whose source or destination
// index is out of range is skipped.  Duplicate destinations race (the reference's index_put_ leaves their
// value unspecified too).
#include "elr_rowio.h"

namespace elr {

template <bool V4>
__global__ __launch_bounds__(256) void k_copy_rows(float* __restrict__ dst, int64_t dst_rows,
                                                   const int64_t* __restrict__ dst_idx, const float* __restrict__ src,
                                                   int64_t src_rows, const int64_t* __restrict__ src_idx, int64_t n,
                                                   int64_t W) {
  const int lane = threadIdx.x & 63;
  for (int64_t i = wave_id(); i < n; i += wave_count()) {
    const int64_t d = dst_idx ? dst_idx[i] : i;
    const int64_t s = src_idx ? src_idx[i] : i;
    if (d < 0 || d >= dst_rows || s < 0 || s >= src_rows) continue;
    if (V4) {
      const f32x4* sp = reinterpret_cast<const f32x4*>(src + s * W);
      f32x4* dp = reinterpret_cast<f32x4*>(dst + d * W);
      for (int64_t c = lane; c < W / 4; c += 64) dp[c] = sp[c];
    } else {
      const float* sp = src + s * W;
      float* dp = dst + d * W;
      for (int64_t c = lane; c < W; c += 64) dp[c] = sp[c];
    }
  }
}

}  // namespace elr

extern "C" int elr_copy_rows(float* dst, int64_t dst_rows, const int64_t* dst_idx, const float* src, int64_t src_rows,
                             const int64_t* src_idx, int64_t n, int64_t W, void* stream) {
  using namespace elr;
  if (n < 0 || W <= 0 || dst_rows < 0 || src_rows < 0) return ELR_EINVAL;
  if (n == 0) return ELR_OK;
  if (!dst || !src) return ELR_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  int64_t blocks = (n + 3) / 4;
  if (blocks > 256 * 32) blocks = 256 * 32;
  if (W % 4 == 0 && aligned16(dst) && aligned16(src))
    k_copy_rows<true><<<(unsigned)blocks, 256, 0, st>>>(dst, dst_rows, dst_idx, src, src_rows, src_idx, n, W);
  else
    k_copy_rows<false><<<(unsigned)blocks, 256, 0, st>>>(dst, dst_rows, dst_idx, src, src_rows, src_idx, n, W);
  return launch_status();
}

// out[rows[i]] = value for i < *n_dev (a device-side count, e.g. the unique rows of a batch whose count the host has
// not read yet): the TTL lookahead's record of when rows appear next (srm2/elara.py:160-161), without a
// synchronisation.  Rows out of range are skipped.
__global__ __launch_bounds__(256) void k_mark_rows(const int64_t* __restrict__ rows, const int64_t* __restrict__ n_dev,
                                                   int64_t n_max, int32_t value, int32_t* __restrict__ out,
                                                   int64_t out_rows) {
  const int64_t n = *n_dev < n_max ? *n_dev : n_max;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const int64_t r = rows[i];
  if (r >= 0 && r < out_rows) out[r] = value;
}

extern "C" int elr_mark_rows(const int64_t* rows, const int64_t* n_dev, int64_t n_max, int32_t value, int32_t* out,
                             int64_t out_rows, void* stream) {
  if (n_max < 0 || out_rows < 0) return ELR_EINVAL;
  if (n_max == 0) return ELR_OK;
  if (!rows || !n_dev || !out) return ELR_EINVAL;
  const int64_t blocks = (n_max + 255) / 256;
  if (blocks >= (int64_t(1) << 31)) return ELR_EINVAL;
  k_mark_rows<<<(unsigned)blocks, 256, 0, (hipStream_t)stream>>>(rows, n_dev, n_max, value, out, out_rows);
  return elr::launch_status();
}
