// Device side of the fused assembly (assemble.hip): the work-row kernels as functors (elr_launch.h), so that the
// step's executor can launch them beside the directory's eviction count.
#pragma once

#include "elr_desc.h"
#include "elr_launch.h"
#include "elr_rowio.h"

namespace elr {

// Work row k's segment: its index g, and the first work position of that segment.
__device__ __forceinline__ int seg_of(const elr_assemble_args& a, int64_t k, int64_t& s0) {
  int g = 0;
  while (g + 1 < a.nseg && k >= a.seg_end[g]) ++g;
  s0 = g == 0 ? 0 : a.seg_end[g - 1];
  return g;
}

// The work row k's kind and, for a replayed row, its index j among the L rows (segments of the argument).
__device__ __forceinline__ int row_kind(const elr_assemble_args& a, int64_t k, int64_t& j) {
  int64_t s0;
  const int g = seg_of(a, k, s0);
  j = a.seg_aux[g] + (k - s0);
  return a.seg_kind[g];
}

// The same in a device-driven step: the work rows are the positions from b[NADM] to b[S] of the class order, whose
// ranks fix the kind (admitted N, L, F; appended N, L; compacted N, L; transient F) and the L rows' order (admitted,
// appended, compacted).
__device__ __forceinline__ int row_kind_dev(const int64_t* __restrict__ desc, int64_t k, int64_t& j) {
  const int64_t pos = desc[kDW0] + k;
  int r = ELR_RANK_NADM;
  while (r < ELR_RANK_FN && pos >= desc[kDB + r + 1]) ++r;
  const int64_t within = pos - desc[kDB + r];
  j = within + (r == ELR_RANK_LAPP ? desc[kDNLa] : r == ELR_RANK_LCMP ? desc[kDNLa] + desc[kDNLp] : 0);
  return (r == ELR_RANK_LADM || r == ELR_RANK_LAPP || r == ELR_RANK_LCMP) ? ELR_ASM_REPLAY
         : (r == ELR_RANK_FADM || r == ELR_RANK_FN)                      ? ELR_ASM_GATHER
                                                                         : ELR_ASM_INIT;
}

// Replay inputs of the L row j (of nL): count c (clamped to [0, K]), entry ids and steps; false when a used entry id
// or step is out of range (the row is then skipped).
template <int K>
__device__ __forceinline__ bool replay_inputs(const elr_assemble_args& a, int64_t j, int64_t nL, int& c,
                                              int32_t (&id)[K], int32_t (&st)[K]) {
  if (j < 0 || j >= nL) return false;
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

// Any D and alignment: one wave per work row, lane l handling elements l, l + 64, ...  desc (a device-driven step):
// the work rows' count and segments come from the descriptor, a.rows is the class-ordered rows (offset by b[NADM]
// on the device), and each wave loops over the rows (the grid is capped, not sized to the upper bound).
template <int K>
struct AsmGen {
  elr_assemble_args a;
  const int64_t* desc;
  __device__ void operator()(int64_t blk, int64_t nblk) const;
  __device__ __forceinline__ void row(int64_t k, const int64_t* rows, int64_t nL) const;
};

template <int K>
__device__ void AsmGen<K>::operator()(int64_t blk, int64_t nblk) const {
  if (desc) {   // within the bounds the arrays were sized for (a.n rows, a.nL L rows)
    const int64_t n = clampi(desc[kDNw], 0, a.n), nL = clampi(desc[kDNL], 0, a.nL);
    const int64_t* rows = a.rows + clampi(desc[kDW0], 0, a.n - n);
    for (int64_t k = body_wave(blk); k < n; k += body_waves(nblk)) row(k, rows, nL);
    return;
  }
  const int64_t k = body_wave(blk);
  if (k < a.n) row(k, a.rows, a.nL);
}

template <int K>
__device__ __forceinline__ void AsmGen<K>::row(int64_t k, const int64_t* rows, int64_t nL) const {
  const float* __restrict__ table = a.table;
  const double* __restrict__ recip = a.recip;
  const int lane = threadIdx.x & 63;
  int64_t j;
  const int kind = desc ? row_kind_dev(desc, k, j) : row_kind(a, k, j);
  const int64_t r = rows[k], D = a.D;
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
  if (kind == ELR_ASM_REPLAY && !replay_inputs<K>(a, j, nL, c, id, st)) return;
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

// D = 64 * VPL: one wave per work row, each lane holding VPL consecutive floats.  desc: as AsmGen.
template <int VPL, int K>
struct AsmWpr {
  elr_assemble_args a;
  const int64_t* desc;
  __device__ void operator()(int64_t blk, int64_t nblk) const;
  __device__ __forceinline__ void row(int64_t k, const int64_t* rows, int64_t nL) const;
};

template <int VPL, int K>
__device__ void AsmWpr<VPL, K>::operator()(int64_t blk, int64_t nblk) const {
  if (desc) {   // within the bounds the arrays were sized for (a.n rows, a.nL L rows)
    const int64_t n = clampi(desc[kDNw], 0, a.n), nL = clampi(desc[kDNL], 0, a.nL);
    const int64_t* rows = a.rows + clampi(desc[kDW0], 0, a.n - n);
    for (int64_t k = body_wave(blk); k < n; k += body_waves(nblk)) row(k, rows, nL);
    return;
  }
  const int64_t k = body_wave(blk);
  if (k < a.n) row(k, a.rows, a.nL);
}

template <int VPL, int K>
__device__ __forceinline__ void AsmWpr<VPL, K>::row(int64_t k, const int64_t* rows, int64_t nL) const {
  const float* __restrict__ table = a.table;
  const double* __restrict__ recip = a.recip;
  constexpr int64_t D = 64 * VPL;
  const int lane = threadIdx.x & 63;
  int64_t j;
  const int kind = desc ? row_kind_dev(desc, k, j) : row_kind(a, k, j);
  const int64_t r = rows[k];
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
    if (!replay_inputs<K>(a, j, nL, c, id, st)) return;
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

// The functor and grid for a's D, K and alignment (checked by assemble_check), passed to visit(functor, blocks).
// desc: a device-driven step, a.n its upper bound; the grid is capped at max_blocks (the waves loop over the rows).
template <int VPL, int K, class Visit>
inline void asm_visit_k(const elr_assemble_args& a, const int64_t* desc, int64_t max_blocks, Visit&& visit) {
  int64_t blocks = (a.n + 3) / 4;
  if (desc && blocks > max_blocks) blocks = max_blocks;
  if constexpr (VPL == 0) visit(AsmGen<K>{a, desc}, blocks);
  else visit(AsmWpr<VPL, K>{a, desc}, blocks);
}

template <int VPL, class Visit>
inline void asm_visit_vpl(const elr_assemble_args& a, const int64_t* desc, int64_t max_blocks, Visit&& visit) {
  switch (a.K) {
    case 1: asm_visit_k<VPL, 1>(a, desc, max_blocks, visit); break;
    case 2: asm_visit_k<VPL, 2>(a, desc, max_blocks, visit); break;
    case 3: asm_visit_k<VPL, 3>(a, desc, max_blocks, visit); break;
    case 4: asm_visit_k<VPL, 4>(a, desc, max_blocks, visit); break;
    case 5: asm_visit_k<VPL, 5>(a, desc, max_blocks, visit); break;
    case 6: asm_visit_k<VPL, 6>(a, desc, max_blocks, visit); break;
    case 7: asm_visit_k<VPL, 7>(a, desc, max_blocks, visit); break;
    default: asm_visit_k<VPL, 8>(a, desc, max_blocks, visit); break;
  }
}

template <class Visit>
inline void assemble_visit(const elr_assemble_args& a, Visit&& visit, const int64_t* desc = nullptr,
                           int64_t max_blocks = 0) {
  const bool al = aligned16(a.work) && (!a.logs || aligned16(a.logs)) && (!a.mat || aligned16(a.mat));
  switch (al ? a.D : 0) {
    case 64: asm_visit_vpl<1>(a, desc, max_blocks, visit); break;
    case 128: asm_visit_vpl<2>(a, desc, max_blocks, visit); break;
    case 256: asm_visit_vpl<4>(a, desc, max_blocks, visit); break;
    case 512: asm_visit_vpl<8>(a, desc, max_blocks, visit); break;
    default: asm_visit_vpl<0>(a, desc, max_blocks, visit); break;
  }
}

// The checks of elr_assemble's arguments (assemble.hip).
int assemble_check(const elr_assemble_args& a);

}  // namespace elr
