// Wave, block and device-wide prefix sums (wave64), shared by the directory and dedup kernels.
//
// Device-wide exclusive scans use three launches: a per-block count kernel writes one total per block and
// channel, one block scans those totals in place (scan_channels_block) and stores the channel totals, and an
// apply kernel adds its block's offset to an in-block exclusive scan.  Nothing spins on other blocks.
#pragma once

#include "elr_common.h"

namespace elr {

constexpr int kScanBlock = 1024;

template <typename T>
__device__ __forceinline__ T wave_incl_scan(T v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const T t = __shfl_up(v, d, 64);
    if (lane >= d) v += t;
  }
  return v;
}

// Exclusive prefix of v[c] over the BLOCK threads of the block, and the block totals.  Every thread of the block
// must call it (it synchronises once); its LDS is private to the call site.
template <int BLOCK, int NCH>
__device__ __forceinline__ void block_excl_scan(const int (&v)[NCH], int (&ex)[NCH], int (&tot)[NCH]) {
  __shared__ int wsum[NCH][BLOCK / 64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int inc[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    inc[c] = wave_incl_scan(v[c]);
    if (lane == 63) wsum[c][w] = inc[c];
  }
  __syncthreads();
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    int base = 0, t = 0;
#pragma unroll
    for (int q = 0; q < BLOCK / 64; ++q) {
      const int x = wsum[c][q];
      base += q < w ? x : 0;
      t += x;
    }
    ex[c] = base + inc[c] - v[c];
    tot[c] = t;
  }
}

// In-place exclusive scan of `nch` channels of `n` int64 values each (channel c at bsum[c*n .. c*n+n)), by one
// block of NT threads; channel totals to tot[c] (device memory) when tot is not null.
template <int NT = kScanBlock>
__device__ __forceinline__ void scan_channels_block(int64_t* __restrict__ bsum, int64_t n, int nch,
                                                    int64_t* __restrict__ tot) {
  __shared__ int64_t wtot[NT / 64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  for (int c = 0; c < nch; ++c) {
    int64_t carry = 0;
    for (int64_t b0 = 0; b0 < n; b0 += NT) {
      const int64_t b = b0 + threadIdx.x;
      const int64_t x = b < n ? bsum[c * n + b] : 0;
      const int64_t inc = wave_incl_scan<int64_t>(x);
      if (lane == 63) wtot[w] = inc;
      __syncthreads();
      int64_t base = 0, all = 0;
      for (int q = 0; q < NT / 64; ++q) {
        base += q < w ? wtot[q] : 0;
        all += wtot[q];
      }
      if (b < n) bsum[c * n + b] = carry + base + inc - x;
      carry += all;
      __syncthreads();
    }
    if (tot && threadIdx.x == 0) tot[c] = carry;
  }
}

// Lanes below this one in the wave (for ranks from ballots).
__device__ __forceinline__ uint64_t lanemask_lt() {
  const int lane = threadIdx.x & 63;
  return lane == 0 ? 0ull : (~0ull >> (64 - lane));
}

}  // namespace elr
