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
#include "elr_copy_dev.h"

namespace elr {

template <bool V4, class DI, class SI>
__global__ __launch_bounds__(256) void k_copy_rows(CopyPart<DI, SI> c) {
  copy_part<V4>(c, wave_id(), wave_count());
}

template <class DI, class SI>
static int copy_rows_launch(float* dst, int64_t dst_rows, DI dix, const float* src, int64_t src_rows, SI six,
                            int64_t n, int64_t W, void* stream, int64_t max_blocks = kCopyMaxBlocks) {
  hipStream_t st = (hipStream_t)stream;
  const CopyPart<DI, SI> c{dst, dst_rows, dix, src, src_rows, six, n, W};
  const unsigned blocks = (unsigned)copy_blocks(n, max_blocks);
  if (copy_v4(c)) k_copy_rows<true><<<blocks, 256, 0, st>>>(c);
  else k_copy_rows<false><<<blocks, 256, 0, st>>>(c);
  return launch_status();
}

}  // namespace elr

extern "C" int elr_copy_rows(float* dst, int64_t dst_rows, const int64_t* dst_idx, const float* src, int64_t src_rows,
                             const int64_t* src_idx, int64_t n, int64_t W, void* stream) {
  using namespace elr;
  if (n < 0 || W <= 0 || dst_rows < 0 || src_rows < 0) return ELR_EINVAL;
  if (n == 0) return ELR_OK;
  if (!dst || !src) return ELR_EINVAL;
  return copy_rows_launch(dst, dst_rows, IxList{dst_idx}, src, src_rows, IxList{src_idx}, n, W, stream);
}

// Resident-history record glog.index_put_((dyn - dyn_off, j), g) (srm2/elara.py:501, 524): glog [nd, K, W],
// g [n, W]; j NULL means entry 0 (the admission record); items whose slot or entry is out of range are skipped.
extern "C" int elr_glog_put(float* glog, int64_t nd, int64_t K, const int64_t* dyn, int64_t dyn_off,
                            const int64_t* j, const float* g, int64_t n, int64_t W, void* stream) {
  using namespace elr;
  if (n < 0 || W <= 0 || nd < 0 || K < 1) return ELR_EINVAL;
  if (n == 0) return ELR_OK;
  if (!glog || !dyn || !g) return ELR_EINVAL;
  return copy_rows_launch(glog, nd * K, IxPair{dyn, dyn_off, j, K, nd}, g, n, IxList{nullptr}, n, W, stream);
}

// History of rows going back to L (srm2/elara.py:396, 507): logs[ids[r*K + k]] = glog[clamp(dyn[r], 0, nd-1), k]
// for r < n, k < K; entries whose id is out of range (-1: none) are skipped.
extern "C" int elr_glog_take(float* logs, int64_t nlogs, const int64_t* ids, const float* glog, int64_t nd,
                             int64_t K, const int64_t* dyn, int64_t n, int64_t W, void* stream) {
  using namespace elr;
  if (n < 0 || W <= 0 || nd < 1 || K < 1 || nlogs < 0) return ELR_EINVAL;
  if (n == 0) return ELR_OK;
  if (!logs || !ids || !glog || !dyn) return ELR_EINVAL;
  return copy_rows_launch(logs, nlogs, IxList{ids}, glog, nd * K, IxExpand{dyn, K, nd}, n * K, W, stream);
}

extern "C" int elr_mark_rows(const int64_t* rows, const int64_t* n_dev, int64_t n_max, int32_t value, int32_t* out,
                             int64_t out_rows, uint32_t* bits, uint32_t bit, void* stream) {
  if (n_max < 0 || out_rows < 0) return ELR_EINVAL;
  if (n_max == 0) return ELR_OK;
  if (!rows || !n_dev || !out) return ELR_EINVAL;
  elr::launch1(elr::MarkRows{rows, n_dev, n_max, value, out, out_rows, bits, bit}, elr::mark_rows_blocks(n_max),
               (hipStream_t)stream);
  return elr::launch_status();
}
