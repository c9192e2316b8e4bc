// Device side of the segment sum's partial chunks (dedup.hip), as a functor (elr_launch.h): the planner's count
// kernel of a step can share a launch with them (elr_plan_classify_seg), since they read only the batch's dedup plan
// and its occurrence gradients.
#pragma once

#include "elr_launch.h"
#include "elr_rowio.h"

namespace elr {

constexpr int kAtenGroup = 10;                          // NROWS_PER_THREAD of ATen's sort path
constexpr int kGroupsPerChunk = 6;
constexpr int kSegChunk = kAtenGroup * kGroupsPerChunk;   // occurrences per parallel chunk (sort path)
constexpr int64_t kHotLen = 240;                          // sort-path segments longer than this are hot

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Sort path.  A segment of more than kHotLen occurrences is hot: the partial-chunk kernel sums all of its runs (its
// first chunk included) and one block of the final kernel folds the run sums, its four waves loading together.  Any
// other segment folds its first chunk in the final kernel's wave, and only its later chunks are partial chunks.
__device__ __forceinline__ bool seg_hot(int64_t L) { return L > kHotLen; }

// Group sums of the extra chunks (sort path), one wave per chunk (grid-stride over the E work items): chunk wi's
// group gi goes to parts row wi * kGroupsPerChunk + gi.  The rows of GB groups load together; the sums are stored
// after the last load (a store in flight would hold up the wait for the next loads).  NQ: floats per lane
// (ceil(D / 64), rounded up to 1, 2, 4 or 8).
template <int NQ>
struct SegPartials {
  const float* grad;
  int64_t D;
  const int32_t* sv;
  const int64_t* seg_start;
  const int32_t* chunk_off;
  const int32_t* chunk_seg;
  const int64_t* d_E;
  float* parts;
  __device__ void operator()(int64_t blk, int64_t nblk) const;
};

template <int NQ>
__device__ void SegPartials<NQ>::operator()(int64_t blk, int64_t nblk) const {
  constexpr int GB = NQ == 1 ? 6 : (NQ == 2 ? 3 : 1);
  constexpr int RB = GB * kAtenGroup;
  static_assert(kGroupsPerChunk % GB == 0, "whole batches of groups per chunk");
  const float* __restrict__ g_ = grad;
  const int lane = threadIdx.x & 63;
  const int64_t E = *d_E;
  for (int64_t wi = body_wave(blk); wi < E; wi += body_waves(nblk)) {
    const int64_t u = chunk_seg[wi];
    const int64_t c = wi - chunk_off[u] + (seg_hot(seg_start[u + 1] - seg_start[u]) ? 0 : 1);
    const int64_t p0 = seg_start[u] + c * kSegChunk;
    int64_t p1 = p0 + kSegChunk;
    const int64_t e = seg_start[u + 1];
    if (p1 > e) p1 = e;
    const int len = (int)(p1 - p0);
    const int32_t my = lane < len ? sv[p0 + lane] : 0;
    float acc[kGroupsPerChunk][NQ];
#pragma unroll
    for (int b = 0; b < kGroupsPerChunk / GB; ++b) {
      const int k0 = b * RB;
      if (k0 >= len) break;
      float g[RB][NQ];
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        if (k0 + r < len) {
          const int64_t o = (int64_t)__builtin_amdgcn_readlane(my, k0 + r);
          const float* row = g_ + o * D;
#pragma unroll
          for (int q = 0; q < NQ; ++q) {
            const int64_t j = lane + 64 * q;
            g[r][q] = j < D ? __builtin_nontemporal_load(row + j) : 0.0f;
          }
        }
      }
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        if (k0 + r < len) {
          const int gi = b * GB + r / kAtenGroup;
#pragma unroll
          for (int q = 0; q < NQ; ++q) acc[gi][q] = r % kAtenGroup == 0 ? g[r][q] : acc[gi][q] + g[r][q];
        }
      }
    }
#pragma unroll
    for (int gi = 0; gi < kGroupsPerChunk; ++gi) {
      if (gi * kAtenGroup >= len) break;
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        const int64_t j = lane + 64 * q;
        if (j < D) parts[(wi * kGroupsPerChunk + gi) * D + j] = acc[gi][q];
      }
    }
  }
}

// Grid of a grid-stride wave loop: enough blocks to fill the chip several times over, at most one wave per item.
inline unsigned wave_grid(int64_t items) {
  int64_t b = cdiv(items, 4);
  const int64_t cap = 256 * 16;
  if (b > cap) b = cap;
  if (b < 1) b = 1;
  return (unsigned)b;
}

// Blocks of the partial-chunk launch of n occurrences (an upper bound of the chunks; waves beyond E exit at once).
inline int64_t seg_partials_blocks(int64_t n) { return wave_grid(n / kSegChunk + n / kHotLen + 2); }

// NQ of the partial chunks for row width D.
inline int seg_nq(int64_t D) {
  const int64_t q = cdiv(D, 64);
  return q <= 2 ? (int)q : (q <= 4 ? 4 : 8);
}

// The partial chunks of one batch's dedup plan (dedup.hip: seg_partials_prep), and visit(functor, blocks) with the
// functor for its width.  blocks == 0: the batch needs none (ATen's windowed path sums every segment in one wave).
struct SegPartialsLaunch {
  SegPartials<1> a;   // the arguments (the same for every NQ)
  int64_t blocks;
};
int seg_partials_prep(const float* grad, int64_t n, int64_t D, int key_bits, const void* plan, int64_t plan_bytes,
                      SegPartialsLaunch& out);

struct DirLstepsHits;   // elr_dir_dev.h

// elr_segment_sum_plan_final's launch with `first` (nb1 blocks; the directory's replay inputs and hit records of the
// device-driven step, which touch none of the sum's arrays) in the same launch, its blocks first.  ELR_EUNSUPPORTED,
// with nothing launched, when the plan's final kernel is not the single wave-per-row launch (the caller then
// launches the two on their own).
int segment_sum_plan_final_with(const float* grad, int64_t n, int64_t D, int key_bits, const void* plan,
                                int64_t plan_bytes, const int64_t* perm, float* out, int64_t out_rows,
                                const DirLstepsHits& first, int64_t nb1, void* stream);

template <class Visit>
inline void seg_partials_visit(const SegPartialsLaunch& L, Visit&& visit) {
  const SegPartials<1>& a = L.a;
  switch (seg_nq(a.D)) {
    case 1: visit(a, L.blocks); break;
    case 2: visit(SegPartials<2>{a.grad, a.D, a.sv, a.seg_start, a.chunk_off, a.chunk_seg, a.d_E, a.parts}, L.blocks);
      break;
    case 4: visit(SegPartials<4>{a.grad, a.D, a.sv, a.seg_start, a.chunk_off, a.chunk_seg, a.d_E, a.parts}, L.blocks);
      break;
    default:
      visit(SegPartials<8>{a.grad, a.D, a.sv, a.seg_start, a.chunk_off, a.chunk_seg, a.d_E, a.parts}, L.blocks);
      break;
  }
}

}  // namespace elr
