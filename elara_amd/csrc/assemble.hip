// Fused weight assembly of one ELARA step (srm2/elara.py:471-489, ELARAExecutor.assemble): the full states of the
// non-resident rows the step touches, written into one work array in the planner's class-rank order, in a single
// launch.  Each work row belongs to a segment of one kind:
//   INIT    counter-hash initial state of an implicit (N) row                         (srm2/gpu_ops.py:26-48)
//   REPLAY  init plus exact replay of a logged (L) row's entries, read from the log arena by entry id
//                                                                                     (srm2/gpu_ops.py:51-79)
//   GATHER  the state of a materialised (M) row, read from the MAT arena at loc[row]
// The segments are ranges of work positions given by the caller; a replay segment names where its rows' entry ids,
// steps and counts start in the directory's replay inputs (elr_dir_a's steps / ids, in the caller's L-row order).
// Rows whose inputs are out of range are skipped (left unwritten), as elsewhere in this library.
// D = 64, 128, 256, 512 with 16-byte aligned arrays: a wave per row, each lane holding D/64 consecutive floats
// (elr_rowio.h).  Any other D or alignment: the generic kernel, a wave per row whose lanes step through the row one
// float at a time.  K <= 8.
#include "elr_rowio.h"

namespace elr {

// Work row k's segment: its index g, and the first work position of that segment.
__device__ __forceinline__ int seg_of(const elr_assemble_args& a, int64_t k, int64_t& s0) {
  int g = 0;
  while (g + 1 < a.nseg && k >= a.seg_end[g]) ++g;
  s0 = g == 0 ? 0 : a.seg_end[g - 1];
  return g;
}

// Replay inputs of work row k in segment g: count c (clamped to [0, K]), entry ids and steps; false when a used
// entry id or step is out of range (the row is then skipped).
template <int K>
__device__ __forceinline__ bool replay_inputs(const elr_assemble_args& a, int g, int64_t k, int64_t s0, int& c,
                                              int32_t (&id)[K], int32_t (&st)[K]) {
  const int64_t j = a.seg_aux[g] + (k - s0);
  if (j < 0 || j >= a.nL) return false;
  const int ci = a.L_cnt[j];
  c = ci < 0 ? 0 : (ci > K ? K : ci);
  int bad = 0;
#pragma unroll
  for (int q = 0; q < K; ++q) {
    id[q] = a.L_ids[j * K + q];
    st[q] = a.L_steps[j * K + q];
    bad |= (q < c) & ((id[q] < 0) | (id[q] >= a.nlogs) | (st[q] < 0) | (st[q] >= a.table_rows));
  }
  return !bad;
}

// Any D and alignment: one wave per work row, lane l handling elements l, l + 64, ...
template <int K>
__global__ __launch_bounds__(256) void k_assemble_gen(elr_assemble_args a, const float* __restrict__ table,
                                                      const double* __restrict__ recip) {
  const int lane = threadIdx.x & 63;
  const int64_t k = wave_id();
  if (k >= a.n) return;
  int64_t s0;
  const int g = seg_of(a, k, s0);
  const int kind = a.seg_kind[g];
  const int64_t r = a.rows[k], D = a.D;
  float* dst = a.work + k * 3 * D;
  if (kind == ELR_ASM_GATHER) {
    if (r < 0 || r >= a.R) return;
    const int64_t slot = a.loc[r];
    if (slot < 0 || slot >= a.mat_rows) return;
    const float* src = a.mat + slot * 3 * D;
    for (int64_t j = lane; j < 3 * D; j += 64) dst[j] = src[j];
    return;
  }
  int c = 0;
  int32_t id[K], st[K];
  if (kind == ELR_ASM_REPLAY && !replay_inputs<K>(a, g, k, s0, c, id, st)) return;
  const uint32_t rk = init_row_key(r, a.seed);
  for (int64_t j = lane; j < D; j += 64) {
    float w = init_elem((uint32_t)((uint64_t)r * (uint64_t)D + (uint64_t)j), rk, a.seed, a.bound), m = 0.f, v = 0.f;
#pragma unroll
    for (int q = 0; q < K; ++q)
      if (q < c) adam_elem(w, m, v, a.logs[(int64_t)id[q] * D + j], table_scalars(table, recip, st[q]));
    dst[j] = w;
    dst[D + j] = m;
    dst[2 * D + j] = v;
  }
}

template <int VPL, int K>
__global__ __launch_bounds__(256) void k_assemble_wpr(elr_assemble_args a, const float* __restrict__ table,
                                                      const double* __restrict__ recip) {
  constexpr int64_t D = 64 * VPL;
  const int lane = threadIdx.x & 63;
  const int64_t k = wave_id();
  if (k >= a.n) return;
  int64_t s0;
  const int g = seg_of(a, k, s0);
  const int kind = a.seg_kind[g];
  const int64_t r = a.rows[k];
  float* dst = a.work + k * 3 * D + lane * VPL;
  if (kind == ELR_ASM_GATHER) {
    if (r < 0 || r >= a.R) return;
    const int64_t slot = a.loc[r];
    if (slot < 0 || slot >= a.mat_rows) return;
    const float* src = a.mat + slot * 3 * D + lane * VPL;
    const RowFrag<VPL> w = frag_load<VPL, true>(src), m = frag_load<VPL, true>(src + D),
                       v = frag_load<VPL, true>(src + 2 * D);
    frag_store<VPL>(dst, w);
    frag_store<VPL>(dst + D, m);
    frag_store<VPL>(dst + 2 * D, v);
    return;
  }
  RowFrag<VPL> w = frag_init<VPL>(r, lane, a.seed, a.bound), m = frag_zero<VPL>(), v = frag_zero<VPL>();
  if (kind == ELR_ASM_REPLAY) {
    int c = 0;
    int32_t id[K], st[K];
    if (!replay_inputs<K>(a, g, k, s0, c, id, st)) return;
    RowFrag<VPL> gr[K];
#pragma unroll
    for (int q = 0; q < K; ++q)
      if (q < c) gr[q] = frag_load<VPL, true>(a.logs + (int64_t)id[q] * D + lane * VPL);
#pragma unroll
    for (int q = 0; q < K; ++q)
      if (q < c) frag_adam<VPL>(w, m, v, gr[q], table_scalars(table, recip, st[q]));
  }
  frag_store<VPL>(dst, w);
  frag_store<VPL>(dst + D, m);
  frag_store<VPL>(dst + 2 * D, v);
}

// VPL = 0: the generic kernel.
template <int VPL, int K>
static void launch_k(const elr_assemble_args& a, const float* table, const double* recip, hipStream_t st) {
  const unsigned blocks = (unsigned)((a.n + 3) / 4);
  if constexpr (VPL == 0) k_assemble_gen<K><<<blocks, 256, 0, st>>>(a, table, recip);
  else k_assemble_wpr<VPL, K><<<blocks, 256, 0, st>>>(a, table, recip);
}

template <int VPL>
static void launch_assemble(const elr_assemble_args& a, const float* table, const double* recip, hipStream_t st) {
  switch (a.K) {
    case 1: launch_k<VPL, 1>(a, table, recip, st); break;
    case 2: launch_k<VPL, 2>(a, table, recip, st); break;
    case 3: launch_k<VPL, 3>(a, table, recip, st); break;
    case 4: launch_k<VPL, 4>(a, table, recip, st); break;
    case 5: launch_k<VPL, 5>(a, table, recip, st); break;
    case 6: launch_k<VPL, 6>(a, table, recip, st); break;
    case 7: launch_k<VPL, 7>(a, table, recip, st); break;
    default: launch_k<VPL, 8>(a, table, recip, st); break;
  }
}

}  // namespace elr

extern "C" int elr_assemble(const elr_assemble_args* args, void* stream) {
  using namespace elr;
  if (!args) return ELR_EINVAL;
  const elr_assemble_args& a = *args;
  if (a.n < 0 || a.nseg < 1 || a.nseg > ELR_ASM_MAX_SEG || a.K < 1 || a.D < 1) return ELR_EINVAL;
  if (a.K > 8) return ELR_EUNSUPPORTED;
  if (a.n == 0) return ELR_OK;
  if (a.n > (int64_t(1) << 31) - 4 || !a.work || !a.rows) return ELR_EINVAL;
  int64_t prev = 0;
  bool need_replay = false, need_gather = false;
  for (int g = 0; g < a.nseg; ++g) {
    if (a.seg_end[g] < prev || a.seg_kind[g] < ELR_ASM_INIT || a.seg_kind[g] > ELR_ASM_GATHER) return ELR_EINVAL;
    if (a.seg_end[g] > prev) {
      need_replay |= a.seg_kind[g] == ELR_ASM_REPLAY;
      need_gather |= a.seg_kind[g] == ELR_ASM_GATHER;
    }
    prev = a.seg_end[g];
  }
  if (prev != a.n) return ELR_EINVAL;
  if (need_replay && (!a.L_ids || !a.L_steps || !a.L_cnt || !a.logs || !a.table || !a.recip || a.nL < 0))
    return ELR_EINVAL;
  if (need_gather && (!a.mat || !a.loc)) return ELR_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  const bool al = aligned16(a.work) && (!a.logs || aligned16(a.logs)) && (!a.mat || aligned16(a.mat));
  switch (al ? a.D : 0) {
    case 64: launch_assemble<1>(a, a.table, a.recip, st); break;
    case 128: launch_assemble<2>(a, a.table, a.recip, st); break;
    case 256: launch_assemble<4>(a, a.table, a.recip, st); break;
    case 512: launch_assemble<8>(a, a.table, a.recip, st); break;
    default: launch_assemble<0>(a, a.table, a.recip, st); break;
  }
  return launch_status();
}
