// Device side of the row copies (rows.hip): row index maps, one copy's rows per wave, and the executor's two
// eviction copies as one functor (elr_launch.h).
#pragma once

#include "elr_desc.h"
#include "elr_launch.h"
#include "elr_rowio.h"

namespace elr {

// out[rows[i]] = value for i < min(*n_dev, n_max) (a device-side count, e.g. the unique rows of a batch whose count
// the host has not read): the TTL lookahead's record of when rows appear next (srm2/elara.py:160-161).  With bits,
// also bits[r] |= bit (the planner's ring of loaded batches): the rows of one batch are distinct, so no two threads
// write the same word.  Rows out of range are skipped.  Grid-stride over the blocks it is given.
struct MarkRows {
  const int64_t* rows;
  const int64_t* n_dev;
  int64_t n_max;
  int32_t value;
  int32_t* out;
  int64_t out_rows;
  uint32_t* bits;
  uint32_t bit;
  __device__ __forceinline__ void operator()(int64_t block, int64_t nblocks) const {
    const int64_t v = *n_dev, n = v < 0 ? 0 : (v < n_max ? v : n_max);
    for (int64_t i = block * kFunctorBlock + threadIdx.x; i < n; i += nblocks * kFunctorBlock) {
      const int64_t r = rows[i];
      if (r >= 0 && r < out_rows) {
        out[r] = value;
        if (bits) bits[r] |= bit;
      }
    }
  }
};
// Blocks of a MarkRows launch of at most n_max rows: one row per thread, at most 512 blocks.
inline int64_t mark_rows_blocks(int64_t n_max) {
  const int64_t b = (n_max + kFunctorBlock - 1) / kFunctorBlock;
  return b < 512 ? b : 512;
}

// Row index maps: the row of item i, or -1 to skip the item.
struct IxList {   // idx[i] (NULL: i)
  const int64_t* idx;
  __device__ __forceinline__ int64_t operator()(int64_t i) const { return idx ? idx[i] : i; }
};
struct IxPair {   // row (dyn[i] - off) * K + j[i] of a [nd, K] grid of rows (j NULL: entry 0)
  const int64_t* dyn;
  int64_t off;
  const int64_t* j;
  int64_t K, nd;
  __device__ __forceinline__ int64_t operator()(int64_t i) const {
    const int64_t d = dyn[i] - off, q = j ? j[i] : 0;
    return d >= 0 && d < nd && q >= 0 && q < K ? d * K + q : -1;
  }
};
struct IxExpand {   // item i = r * K + k: row clamp(dyn[r], 0, nd - 1) * K + k
  const int64_t* dyn;
  int64_t K, nd;
  __device__ __forceinline__ int64_t operator()(int64_t i) const {
    const int64_t r = i / K, k = i - r * K;
    int64_t d = dyn[r];
    d = d < 0 ? 0 : (d >= nd ? nd - 1 : d);
    return d * K + k;
  }
};

// One row copy: n rows of W floats, dst row dix(i) = src row six(i).  n_dev (a device-driven step): the row count
// is n_dev[0] * n_mul, n its upper bound (the grid).
template <class DI, class SI>
struct CopyPart {
  float* dst;
  int64_t dst_rows;
  DI dix;
  const float* src;
  int64_t src_rows;
  SI six;
  int64_t n, W;
  const int64_t* n_dev;
  int64_t n_mul;
};

// Rows wid, wid + wcount, ... of copy c by one wave.
template <bool V4, class DI, class SI>
__device__ __forceinline__ void copy_part(const CopyPart<DI, SI>& c, int64_t wid, int64_t wcount) {
  const int lane = threadIdx.x & 63;
  const int64_t W = c.W;
  const int64_t n = c.n_dev ? clampi(*c.n_dev * c.n_mul, 0, c.n) : c.n;
  for (int64_t i = wid; i < n; i += wcount) {
    const int64_t d = c.dix(i);
    const int64_t s = c.six(i);
    if (d < 0 || d >= c.dst_rows || s < 0 || s >= c.src_rows) continue;
    if (V4) {
      const f32x4* sp = reinterpret_cast<const f32x4*>(c.src + s * W);
      f32x4* dp = reinterpret_cast<f32x4*>(c.dst + d * W);
      for (int64_t k = lane; k < W / 4; k += 64) dp[k] = sp[k];
    } else {
      const float* sp = c.src + s * W;
      float* dp = c.dst + d * W;
      for (int64_t k = lane; k < W; k += 64) dp[k] = sp[k];
    }
  }
}

// Two independent copies in one body: blocks [0, nb1) take the first, the others the second.
template <bool V4, class DI1, class SI1, class DI2, class SI2>
struct CopyRows2 {
  CopyPart<DI1, SI1> c1;
  CopyPart<DI2, SI2> c2;
  int64_t nb1;
  __device__ void operator()(int64_t b, int64_t nblocks) const {
    if (b < nb1) copy_part<V4>(c1, body_wave(b), body_waves(nb1));
    else copy_part<V4>(c2, body_wave(b - nb1), body_waves(nblocks - nb1));
  }
};

template <class DI, class SI>
inline bool copy_v4(const CopyPart<DI, SI>& c) {
  return c.W % 4 == 0 && aligned16(c.dst) && aligned16(c.src);
}

inline int64_t copy_blocks(int64_t n, int64_t max_blocks) {
  const int64_t b = (n + 3) / 4;
  return b > max_blocks ? max_blocks : b;
}

constexpr int64_t kCopyMaxBlocks = 256 * 32;

// The executor's eviction moves: mat[evf_slots[i]] = pool[ev_slot[i]] (rows of 3D floats, i < nev) and the
// resident histories logs[evl_ids[r*K + k]] = glog[clamp(ev_dyn[r], 0, nd-1), k] (elr_glog_take), with their grids.
struct EvictMove {
  CopyPart<IxList, IxList> c1;
  CopyPart<IxList, IxExpand> c2;
  int64_t nb1, nb2;
  bool v4;
};

// desc (a device-driven step): nev is an upper bound, the count comes from the descriptor.
inline EvictMove evict_move_prep(float* mat, int64_t mat_rows, const int64_t* evf_slots, const float* pool,
                                 int64_t pool_rows, const int64_t* ev_slot, float* logs, int64_t log_rows,
                                 const int64_t* evl_ids, const float* glog, int64_t nd, int64_t K,
                                 const int64_t* ev_dyn, int64_t nev, int64_t D, const int64_t* desc = nullptr) {
  const int64_t* nv = desc ? desc + kDNev : nullptr;
  EvictMove m{{mat, mat_rows, IxList{evf_slots}, pool, pool_rows, IxList{ev_slot}, nev, 3 * D, nv, 1},
              {logs, log_rows, IxList{evl_ids}, glog, nd * K, IxExpand{ev_dyn, K, nd}, nev * K, D, nv, K}, 0, 0,
              false};
  m.nb1 = copy_blocks(m.c1.n, kCopyMaxBlocks);
  m.nb2 = copy_blocks(m.c2.n, kCopyMaxBlocks);
  m.v4 = copy_v4(m.c1) && copy_v4(m.c2);
  return m;
}

// visit(functor, blocks) with the move's functor (16-byte or 4-byte accesses).
template <class Visit>
inline void evict_move_visit(const EvictMove& m, Visit&& visit) {
  if (m.v4) visit(CopyRows2<true, IxList, IxList, IxList, IxExpand>{m.c1, m.c2, m.nb1}, m.nb1 + m.nb2);
  else visit(CopyRows2<false, IxList, IxList, IxList, IxExpand>{m.c1, m.c2, m.nb1}, m.nb1 + m.nb2);
}

}  // namespace elr
