// Batch dedup and duplicate-id gradient reduction in a fixed order, optionally fused with row-sparse Adam
// (HBM-bound; no MFMA).
//
// Replaces the step before Adam on every batch: torch.unique(ids, return_inverse=True) (srm2/train.py:352) and
// aten.embedding_dense_backward (srm2/train.py:429), and gives config C3 its fused form (dedup, fixed-order
// segment sum, Adam on each unique row).
//
// Sort.  Stable LSD radix sort of (id, occurrence index) pairs, 8-bit digits, ceil(key_bits / 8) passes (or one
// pass fewer with 9- or 10-bit digits), keys held as uint32 when key_bits <= 32.  Tiles of 4096 keys, or 1024 below
// 2^18 keys.  A pass is three launches: per-tile digit histograms, a wave per digit scanning that digit's per-tile
// counts, and a scatter in which each key's rank among equal digits of its tile comes from wave ballots (peer mask
// of the digit bits), a per-wave running count in LDS and a scan over the tile's waves, so equal keys keep their
// occurrence order.
//
// Segments.  Sorted position i starts a segment when its key differs from position i-1; per-block head counts, then
// a launch in which each block adds up the counts of the blocks before it (or, above kFoldMaxBlocks blocks, a
// one-block scan launch in between), gives every position its unique index (the inverse) and every unique id its
// first position.  The extra-chunk plan is laid out the same way.
//
// Summation order: ATen's, as torch.ops.aten.embedding_dense_backward computes it on this GPU
// (aten/src/ATen/native/cuda/Embedding.cu embedding_dense_backward_cuda and EmbeddingBackwardKernel.cu, PyTorch
// 2.10 / 2.11; third-party code the reference calls, restated here).  Every id's sum is ((0 + G1) + G2) + ..., G
// the left-to-right sum of one group of that id's occurrences, taken in ascending occurrence index:
//   n <= 3072 indices (embedding_backward_feature_kernel): a group is the id's occurrences inside one window of
//       16 consecutive indices (the kernel's blockDim.y in ATen's ROCm build; 32 in its CUDA build);
//   n >  3072 (embedding_backward_cuda_kernel on a stable sort): groups are the id's occurrences cut into runs of
//       NROWS_PER_THREAD = 10 from its first.
// ATen starts every group sum from zero as well; the total never is -0 (it starts at +0 and a rounded sum is -0
// only when both terms are), so starting a group from its first gradient gives the same bits.  Long (Zipf-hot)
// segments are cut into chunks of 6 groups summed in parallel by different waves (partial sums per group, added in
// order by the segment's own wave).
#include "elr_dir_dev.h"
#include "elr_scan.h"
#include "elr_seg_dev.h"

namespace elr {

constexpr int kSortThreads = 256;
// Keys per thread of a sort tile and positions per thread of a segment tile: 16 (tiles of 4,096) from kBigBatch
// keys, 4 below it, so that a small batch still spreads over a few hundred blocks.  The threshold is set for a batch
// sorted beside other kernels, as the ELARA step sorts the batches it loads ahead: at config C5 (425,984 keys)
// tiles of 4,096 make a sort alone 124 us against 81 us with tiles of 1,024, but its launches of a quarter as many
// blocks take fewer CUs from the step's kernels beside them, and the step is faster (0.342 against 0.357 ms
// device-driven, 0.279 against 0.297 ms host-planned; three alternations on one box; tiles of 2,048 in between,
// 8,192 slower than both).
constexpr int kItemsBig = 16;
constexpr int kItemsSmall = 4;
constexpr int64_t kBigBatch = int64_t(1) << 18;
inline int items_for(int64_t n) { return n >= kBigBatch ? kItemsBig : kItemsSmall; }
constexpr int kRadixBins = 256;      // bins of an 8-bit digit; passes take 8, 9 or 10 bits (sort_plan)
constexpr int kRadixMaxBits = 10;
constexpr int kRadixMaxBins = 1 << kRadixMaxBits;
constexpr int64_t kAtenSmall = 3072;                      // ATen's windowed path up to this many indices
constexpr int kAtenWinShift = 4;                          // its window: 16 indices
constexpr int kSegParts = 8;                              // run sums a final-kernel wave loads together
constexpr int kSegBlock = 256;

static_assert(kSortThreads == kRadixBins, "at least one histogram bin per sort thread");

template <int RB, typename Key>
__device__ __forceinline__ uint32_t digit_of(Key k, int shift) {
  return (uint32_t)((k >> shift) & (Key)((1u << RB) - 1));
}

// Passes and digit width of a sort of key_bits-bit keys: one pass fewer than 8-bit digits need when digits of at
// most max_bits bits then suffice (27-bit keys: 3 passes of 9 bits instead of 4 of 8), else 8-bit digits.
inline void sort_plan(int key_bits, int max_bits, int& passes, int& rb) {
  const int p8 = (key_bits + 7) / 8;
  if (p8 > 1) {
    const int w = (key_bits + p8 - 2) / (p8 - 1);
    if (w <= max_bits) {
      passes = p8 - 1;
      rb = w < 8 ? 8 : w;
      return;
    }
  }
  passes = p8;
  rb = 8;
}

// Per-tile histogram of RB-bit digits, digit-major: hist[d * nblk + tile].
template <typename Src, typename Key, int ITEMS, int RB>
__global__ __launch_bounds__(kSortThreads) void k_radix_hist(const Src* __restrict__ src, int64_t n, int shift,
                                                             int64_t* __restrict__ hist, int64_t nblk) {
  constexpr int BINS = 1 << RB;
  __shared__ int h[BINS];
  for (int b = threadIdx.x; b < BINS; b += kSortThreads) h[b] = 0;
  __syncthreads();
  const int64_t base = (int64_t)blockIdx.x * kSortThreads * ITEMS;
  for (int r = 0; r < ITEMS; ++r) {
    const int64_t pos = base + (int64_t)r * kSortThreads + threadIdx.x;
    if (pos < n) atomicAdd(&h[digit_of<RB>((Key)src[pos], shift)], 1);
  }
  __syncthreads();
  for (int b = threadIdx.x; b < BINS; b += kSortThreads) hist[(int64_t)b * nblk + blockIdx.x] = h[b];
}

// Exclusive prefix over BINS values held BPT per thread (thread t holds bins t*BPT .. t*BPT + BPT - 1, in x[]):
// the prefixes to ex[], the total of all bins to *total.
template <int BPT>
__device__ __forceinline__ void bins_excl_scan(const int (&x)[BPT], int (&ex)[BPT], int& total) {
  int loc = 0;
#pragma unroll
  for (int j = 0; j < BPT; ++j) {
    ex[j] = loc;
    loc += x[j];
  }
  int v[1] = {loc}, e[1], tot[1];
  block_excl_scan<kSortThreads, 1>(v, e, tot);
#pragma unroll
  for (int j = 0; j < BPT; ++j) ex[j] += e[0];
  total = tot[0];
}

// One wave per digit: exclusive scan of that digit's per-tile counts (in place) and the digit's total.  The wave
// loads up to 512 counts (8 per lane) before it scans them, so a few hundred tiles cost one round of loads; no
// block barrier.
__global__ __launch_bounds__(kSortThreads) void k_radix_hist_scan(int64_t* __restrict__ hist, int64_t ntile,
                                                                  int nbins, int64_t* __restrict__ dtot) {
  constexpr int kWaves = kSortThreads / 64, kPer = 8;
  const int lane = threadIdx.x & 63;
  const int d = blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (d >= nbins) return;
  int64_t* h = hist + (int64_t)d * ntile;
  int64_t carry = 0;
  for (int64_t g0 = 0; g0 < ntile; g0 += 64 * kPer) {
    int64_t x[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int64_t b = g0 + k * 64 + lane;
      x[k] = b < ntile ? h[b] : 0;
    }
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int64_t b = g0 + k * 64 + lane;
      const int64_t inc = wave_incl_scan<int64_t>(x[k]);
      if (b < ntile) h[b] = carry + inc - x[k];
      carry += __shfl(inc, 63, 64);
    }
  }
  if (lane == 0) dtot[d] = carry;
}

// One block: exclusive scan of per-block counts in place (grids above kFoldMaxBlocks; see k_seg_apply).
__global__ __launch_bounds__(kScanBlock) void k_scan_blocks(int64_t* __restrict__ bsum, int64_t n) {
  scan_channels_block(bsum, n, 1, nullptr);
}

// Stable scatter of one pass.  FIRST: the source keys are the caller's int64 ids and the values are their
// positions.  Wave w of the block takes the tile's w-th quarter, 64 consecutive positions per round, so an item's
// rank among the tile's items of its digit is: items of that digit in earlier waves' quarters, plus those of its
// own wave's earlier rounds (a per-wave running count in LDS, which only that wave touches, in program order), plus
// its peers in the same round below its lane (ballots).  The waves run their rounds without block barriers; one
// scan over the waves' counts per digit at the end gives the first term.  The tile is then sorted by digit in LDS
// and written out run by run, so consecutive threads write consecutive addresses of one digit's bucket instead of
// 64 scattered ones.
template <typename Src, typename Key, bool FIRST, int ITEMS, int RB>
__global__ __launch_bounds__(kSortThreads) void k_radix_scatter(const Src* __restrict__ src_keys,
                                                                const int32_t* __restrict__ src_vals, int64_t n,
                                                                int shift, const int64_t* __restrict__ offs,
                                                                const int64_t* __restrict__ dtot, int64_t nblk,
                                                                Key* __restrict__ dst_keys,
                                                                int32_t* __restrict__ dst_vals) {
  constexpr int NW = kSortThreads / 64;
  constexpr int TILE = kSortThreads * ITEMS;
  constexpr int BINS = 1 << RB, BPT = BINS / kSortThreads;   // digits per thread in the per-digit steps
  static_assert(BPT * kSortThreads == BINS, "RB >= 8");
  __shared__ int bo[BINS];       // global position of this tile's first item of digit d (n < 2^31)
  __shared__ int run[BINS];      // items of digit d in the tile
  __shared__ int lbase[BINS];    // position of digit d's first item in the tile sorted by digit
  __shared__ int wc[NW][BINS];   // per wave: running count of digit d, then the count in earlier waves
  __shared__ Key lk[TILE];
  __shared__ int32_t lv[TILE];
  const int t = threadIdx.x, w = t >> 6, lane = t & 63;
  const int64_t tile0 = (int64_t)blockIdx.x * TILE, base = tile0 + (int64_t)w * (ITEMS * 64);
  // the tile's items first, so that their loads overlap the digit bases' loads and scan
  Key kk[ITEMS];
  int32_t vv[ITEMS];
#pragma unroll
  for (int r = 0; r < ITEMS; ++r) {
    const int64_t pos = base + (int64_t)r * 64 + lane;
    const bool valid = pos < n;
    kk[r] = valid ? (Key)src_keys[pos] : (Key)0;
    vv[r] = valid ? (FIRST ? (int32_t)pos : src_vals[pos]) : 0;
  }
  {
    // digit bases: exclusive scan of the digit totals (n < 2^31, so they fit in int)
    int x[BPT], ex[BPT], total;
#pragma unroll
    for (int j = 0; j < BPT; ++j) x[j] = (int)dtot[t * BPT + j];
    bins_excl_scan<BPT>(x, ex, total);
#pragma unroll
    for (int j = 0; j < BPT; ++j) bo[t * BPT + j] = ex[j] + (int)offs[(int64_t)(t * BPT + j) * nblk + blockIdx.x];
  }
#pragma unroll
  for (int q = 0; q < NW; ++q)
#pragma unroll
    for (int j = 0; j < BPT; ++j) wc[q][t * BPT + j] = 0;
  __syncthreads();
  int rk[ITEMS];
#pragma unroll
  for (int r = 0; r < ITEMS; ++r) {
    const int64_t pos = base + (int64_t)r * 64 + lane;
    const bool valid = pos < n;
    const uint32_t d = digit_of<RB>(kk[r], shift);
    uint64_t m = __ballot(valid);
#pragma unroll
    for (int b = 0; b < RB; ++b) {
      const bool bit = (d >> b) & 1u;
      const uint64_t bal = __ballot(bit);
      m &= bit ? bal : ~bal;
    }
    const int lr = __popcll(m & lanemask_lt());
    // every lane reads its digit's running count before the group's lowest lane adds the group's size: one wave's
    // LDS accesses take effect in program order
    const int before = valid ? wc[w][d] : 0;
    rk[r] = valid ? before + lr : -1;
    if (valid && lr == 0) wc[w][d] = before + __popcll(m);
  }
  __syncthreads();
  int runs[BPT];
#pragma unroll
  for (int j = 0; j < BPT; ++j) {
    // per digit: exclusive scan over the waves, and the tile's total
    const int dd = t * BPT + j;
    int acc = 0;
#pragma unroll
    for (int q = 0; q < NW; ++q) {
      const int c = wc[q][dd];
      wc[q][dd] = acc;
      acc += c;
    }
    runs[j] = acc;
    run[dd] = acc;
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < ITEMS; ++r)
    if (rk[r] >= 0) rk[r] += wc[w][digit_of<RB>(kk[r], shift)];
  {
    // the tile sorted by digit: digit d's items start at the exclusive scan of the tile's digit counts
    int ex[BPT], total;
    bins_excl_scan<BPT>(runs, ex, total);
#pragma unroll
    for (int j = 0; j < BPT; ++j) lbase[t * BPT + j] = ex[j];
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < ITEMS; ++r) {
    if (rk[r] >= 0) {
      const int lp = lbase[digit_of<RB>(kk[r], shift)] + rk[r];
      lk[lp] = kk[r];
      lv[lp] = vv[r];
    }
  }
  __syncthreads();
  const int64_t rem = n - tile0;
  const int nvalid = rem < TILE ? (int)rem : TILE;
  for (int j = t; j < nvalid; j += kSortThreads) {
    const Key k = lk[j];
    const uint32_t d = digit_of<RB>(k, shift);
    const int64_t dst = (int64_t)bo[d] + (j - lbase[d]);
    if (dst >= 0 && dst < n) {
      dst_keys[dst] = k;
      dst_vals[dst] = lv[j];
    }
  }
}

// Segment kernels take a tile of kSegBlock * ITEMS positions per block, in ITEMS rounds of kSegBlock consecutive
// positions (thread t takes position base + r * kSegBlock + t in round r: every load is coalesced).  Positions are
// ranked in that order, round by round, with one block scan per round.

template <typename Key>
__device__ __forceinline__ int is_head(const Key* __restrict__ sk, int64_t i, int64_t n) {
  return i < n && (i == 0 || sk[i] != sk[i - 1]) ? 1 : 0;
}

// Segment heads: per-block head counts.
template <typename Key, int ITEMS>
__global__ __launch_bounds__(kSegBlock) void k_seg_count(const Key* __restrict__ sk, int64_t n,
                                                         int64_t* __restrict__ bsum) {
  const int64_t base = (int64_t)blockIdx.x * kSegBlock * ITEMS + threadIdx.x;
  int v[1] = {0}, ex[1], tot[1];
  for (int r = 0; r < ITEMS; ++r) v[0] += is_head(sk, base + (int64_t)r * kSegBlock, n);
  block_excl_scan<kSegBlock, 1>(v, ex, tot);
  if (threadIdx.x == 0) bsum[blockIdx.x] = tot[0];
}

// Grids of at most this many blocks take their block offsets by block_offset; larger ones from a one-block scan
// launch (k_scan_blocks) between the count and apply launches.  At config C3 (830 blocks) the summing blocks made the
// step 55 us slower where the sort runs beside the final segment kernel; at C5 (104 blocks) they save the launch.
constexpr int64_t kFoldMaxBlocks = 256;

// Sum of cnt[0 .. b) over the whole block, returned to every thread: the offset of block b from the per-block
// counts of the launch before, without a scan launch in between.
__device__ __forceinline__ int64_t block_offset(const int64_t* __restrict__ cnt, int64_t b) {
  __shared__ int64_t wpart[kSegBlock / 64];
  int64_t x = 0;
  for (int64_t i = threadIdx.x; i < b; i += kSegBlock) x += cnt[i];
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) x += __shfl_xor(x, d, 64);
  if ((threadIdx.x & 63) == 0) wpart[threadIdx.x >> 6] = x;
  __syncthreads();
  int64_t t = 0;
#pragma unroll
  for (int q = 0; q < kSegBlock / 64; ++q) t += wpart[q];
  __syncthreads();   // wpart is reused by the caller's next call
  return t;
}

// Segment heads: unique ids, segment starts, each segment's first occurrence index and the inverse.  The block's
// first segment index: the sum of the earlier blocks' head counts (k_seg_count), or, with `scanned`, bcnt[block]
// after k_scan_blocks.  The last block stores U to d_U (and n_unique) and seg_start[U] = n.
template <typename Key, int ITEMS>
__global__ __launch_bounds__(kSegBlock) void k_seg_apply(const Key* __restrict__ sk, const int32_t* __restrict__ sv,
                                                         int64_t n, const int64_t* __restrict__ bcnt, int scanned,
                                                         int64_t* __restrict__ d_U, int64_t* __restrict__ n_unique,
                                                         int64_t* __restrict__ uniq, int64_t* __restrict__ seg_start,
                                                         int32_t* __restrict__ seg_occ0,
                                                         int64_t* __restrict__ inverse) {
  const int64_t base = (int64_t)blockIdx.x * kSegBlock * ITEMS + threadIdx.x;
  // heads in earlier positions of the tile's earlier rounds
  int64_t before = scanned ? bcnt[blockIdx.x] : block_offset(bcnt, blockIdx.x);
  for (int r = 0; r < ITEMS; ++r) {
    const int64_t i = base + (int64_t)r * kSegBlock;
    const int f = is_head(sk, i, n);
    int v[1] = {f}, ex[1], tot[1];
    block_excl_scan<kSegBlock, 1>(v, ex, tot);
    const int64_t u = before + ex[0] + f - 1;   // segment of position i
    if (i < n) {
      const int32_t o = sv[i];
      if (f) {
        uniq[u] = (int64_t)sk[i];
        seg_start[u] = i;
        seg_occ0[u] = o;
      }
      if (inverse && o >= 0 && o < n) inverse[o] = u;
    }
    before += tot[0];
    __syncthreads();   // block_excl_scan's LDS is reused by the next round
  }
  if (blockIdx.x == gridDim.x - 1 && threadIdx.x == 0) {
    *d_U = before;
    if (n_unique) *n_unique = before;
    seg_start[before] = n;
  }
}

// Sort path.  A segment of more than kHotLen occurrences is hot: the partial-chunk kernel sums all of its runs (its
// first chunk included) and one block of the final kernel folds the run sums, its four waves loading together.  Any
// other segment folds its first chunk in the final kernel's wave, and only its later chunks are partial chunks.
__device__ __forceinline__ int part_chunks(int64_t L) {
  return (int)(seg_hot(L) ? (L + kSegChunk - 1) / kSegChunk : (L - 1) / kSegChunk);
}
__device__ __forceinline__ int extra_chunks(const int64_t* __restrict__ seg_start, int64_t u, int64_t U) {
  return u < U ? part_chunks(seg_start[u + 1] - seg_start[u]) : 0;
}

// Partial chunks of each segment: per-block counts.  Also clears the hot-segment count.
template <int ITEMS>
__global__ __launch_bounds__(kSegBlock) void k_chunk_count(const int64_t* __restrict__ seg_start,
                                                           const int64_t* __restrict__ d_U,
                                                           int64_t* __restrict__ bsum, int64_t* __restrict__ d_hot) {
  const int64_t base = (int64_t)blockIdx.x * kSegBlock * ITEMS + threadIdx.x;
  const int64_t U = *d_U;
  if (blockIdx.x == 0 && threadIdx.x == 0) *d_hot = 0;
  int v[1] = {0}, ex[1], tot[1];
  for (int r = 0; r < ITEMS; ++r) v[0] += extra_chunks(seg_start, base + (int64_t)r * kSegBlock, U);
  block_excl_scan<kSegBlock, 1>(v, ex, tot);
  if (threadIdx.x == 0) bsum[blockIdx.x] = tot[0];
}

// chunk_off[u] = first work item of segment u's partial chunks; chunk_seg[item] = u; hot segments are listed in
// hot_list[0 .. *d_hot) (in no particular order: each is summed on its own).  The block's first work item is the sum
// of the earlier blocks' counts (k_chunk_count), or bcnt[block] with `scanned`; the last block stores the number of
// work items to *d_E.
template <int ITEMS>
__global__ __launch_bounds__(kSegBlock) void k_chunk_apply(const int64_t* __restrict__ seg_start,
                                                           const int64_t* __restrict__ d_U,
                                                           const int64_t* __restrict__ bcnt, int scanned,
                                                           int32_t* __restrict__ chunk_off,
                                                           int32_t* __restrict__ chunk_seg,
                                                           int32_t* __restrict__ hot_list,
                                                           int64_t* __restrict__ d_hot, int64_t* __restrict__ d_E) {
  const int64_t base = (int64_t)blockIdx.x * kSegBlock * ITEMS + threadIdx.x;
  const int64_t U = *d_U;
  int64_t before = scanned ? bcnt[blockIdx.x] : block_offset(bcnt, blockIdx.x);
  for (int r = 0; r < ITEMS; ++r) {
    const int64_t u = base + (int64_t)r * kSegBlock;
    const int e = extra_chunks(seg_start, u, U);
    int v[1] = {e}, ex[1], tot[1];
    block_excl_scan<kSegBlock, 1>(v, ex, tot);
    if (u < U) {
      const int64_t off = before + ex[0];
      chunk_off[u] = (int32_t)off;
      for (int c = 0; c < e; ++c) chunk_seg[off + c] = (int32_t)u;
      if (seg_hot(seg_start[u + 1] - seg_start[u]))
        hot_list[atomicAdd(reinterpret_cast<unsigned long long*>(d_hot), 1ull)] = (int32_t)u;
    }
    before += tot[0];
    __syncthreads();
  }
  if (blockIdx.x == gridDim.x - 1 && threadIdx.x == 0) *d_E = before;
}

// ---- dedup plan of a batch laid out by field -------------------------------------------------------------------
// A batch of nrows samples x nf fields in (sample, field) order, field c holding rows [lo[c], lo[c + 1]) of the
// table with the bounds ascending: every id of field c is below every id of field c + 1, so the stable sort of the
// whole batch is field 0's column sorted stably, then field 1's, and so on (within a column, sample order is
// occurrence order).  One block per field sorts its column of at most kFieldRows ids in LDS: LSD passes of at most
// kFieldDigit bits over the id's offset in its field, each key ranked as in k_radix_scatter (ballots, a running
// count per wave, a scan over the waves), the column re-read from LDS after each pass.  The plan is then the
// general path's, bit for bit, in three launches (k_field_keys, the columns' keys; k_field_sort; k_field_apply, which
// adds the earlier fields' segment and chunk counts) instead of three per radix pass and four for the segments and
// chunks.  An id outside
// its field's rows takes the key R_c (the field's row count), sorts after the field's ids and comes out as -1 in
// uniq: a row out of range for the caller.
constexpr int kFieldThreads = 1024;
constexpr int kFieldItems = 16;
constexpr int64_t kFieldRows = (int64_t)kFieldThreads * kFieldItems;   // samples per batch: the row index is 16-bit
constexpr int kFieldDigit = 9;
constexpr int kFieldMax = 128;                      // fields per batch (the bounds travel as a kernel argument)
constexpr int64_t kFieldSpanMax = (int64_t(1) << 31) - 2;   // rows per field: keys 0 .. R_c fit in 31 bits

struct FieldBounds {
  int64_t lo[kFieldMax + 1];
};

// Passes and digit width for keys in [0, span]: ceil(bits / kFieldDigit) passes of equal width.
__device__ __forceinline__ void field_digits(int64_t span, int& passes, int& rb) {
  int bits = 1;
  while (bits < 31 && (int64_t(1) << bits) <= span) ++bits;
  passes = (bits + kFieldDigit - 1) / kFieldDigit;
  rb = (bits + passes - 1) / passes;
}

// Head flags of the sorted column in lk (bit r: this thread's item r, position w * kFieldItems * 64 + r * 64 +
// lane) and this wave's head count.
__device__ __forceinline__ uint32_t field_heads(const uint32_t* lk, int n, int& wcount) {
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  uint32_t hm = 0;
  wcount = 0;
#pragma unroll
  for (int r = 0; r < kFieldItems; ++r) {
    const int j = w * kFieldItems * 64 + r * 64 + lane;
    const bool h = j < n && (j == 0 || lk[j - 1] != lk[j]);
    hm |= h ? 1u << r : 0u;
    wcount += __popcll(__ballot(h));
  }
  return hm;
}

// Positions of the column's segment heads, hpos[u] for u < U, and hpos[U] = n, from the head flags; returns U.
// Synchronises the block before writing (hpos may share LDS with what the head test read) and after.
__device__ __forceinline__ int field_head_positions(uint32_t hm, int wcount, int n, int* wtot, int* hpos) {
  constexpr int NW = kFieldThreads / 64;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) wtot[w] = wcount;
  __syncthreads();
  int U = 0, run = 0;
#pragma unroll
  for (int q = 0; q < NW; ++q) {
    U += wtot[q];
    run += q < w ? wtot[q] : 0;
  }
#pragma unroll
  for (int r = 0; r < kFieldItems; ++r) {
    const bool h = (hm >> r) & 1u;
    const uint64_t bal = __ballot(h);
    if (h) hpos[run + __popcll(bal & lanemask_lt())] = w * kFieldItems * 64 + r * 64 + lane;
    run += __popcll(bal);
  }
  if (threadIdx.x == 0) hpos[U] = n;
  __syncthreads();
  return U;
}

// Each field's ids as offsets in its field (the key R_c for an id outside it), field after field: keys[c * nrows + j].
// One block per field and kFieldKeyRows samples, so that the gather of a column (each wave's 64 loads touch 64
// different cache lines) is spread over the whole GPU instead of being done by the field's sorting block alone.
constexpr int kFieldKeyRows = 1024;
__global__ __launch_bounds__(256) void k_field_keys(const int64_t* __restrict__ ids, int64_t nrows, int nf,
                                                    FieldBounds fb, uint32_t* __restrict__ keys) {
  const int c = blockIdx.y;
  const int64_t lo = fb.lo[c], hi = fb.lo[c + 1];
  const int64_t j0 = (int64_t)blockIdx.x * kFieldKeyRows;
#pragma unroll
  for (int r = 0; r < kFieldKeyRows / 256; ++r) {
    const int64_t j = j0 + r * 256 + threadIdx.x;
    if (j < nrows) {
      const int64_t id = ids[j * nf + c];
      keys[(int64_t)c * nrows + j] = id >= lo && id < hi ? (uint32_t)(id - lo) : (uint32_t)(hi - lo);
    }
  }
}

__global__ __launch_bounds__(kFieldThreads) void k_field_sort(const uint32_t* __restrict__ keys, int64_t nrows,
                                                              int nf, FieldBounds fb, uint32_t* __restrict__ skeys,
                                                              int32_t* __restrict__ svals, int64_t* __restrict__ cnt,
                                                              int64_t* __restrict__ d_hot) {
  constexpr int NW = kFieldThreads / 64, WSPAN = kFieldItems * 64, BINS = 1 << kFieldDigit;
  __shared__ uint32_t lk[kFieldRows + 1];   // the column by digit; at the end the head positions (U + 1 of them)
  __shared__ uint16_t lv[2][kFieldRows];    // sample index of each key: pass p writes lv[p & 1]
  __shared__ uint16_t wc[NW][BINS];         // per wave: running count of digit d, then the count in earlier waves
  __shared__ int lbase[BINS];
  __shared__ int wtot[NW];
  const int c = blockIdx.x, t = threadIdx.x, w = t >> 6, lane = t & 63;
  const int n = (int)nrows;
  const int64_t R = fb.lo[c + 1] - fb.lo[c];
  int passes, rb;
  field_digits(R, passes, rb);
  const int nbins = 1 << rb;
  const uint32_t mask = (uint32_t)nbins - 1u;
  if (c == 0 && t == 0) *d_hot = 0;
  uint32_t kk[kFieldItems];
#pragma unroll
  for (int r = 0; r < kFieldItems; ++r) {
    const int j = w * WSPAN + r * 64 + lane;
    kk[r] = j < n ? keys[(int64_t)c * nrows + j] : 0u;
  }
  for (int p = 0; p < passes; ++p) {
    const int shift = p * rb;
    const uint16_t* vsrc = lv[(p + 1) & 1];
    uint16_t* vdst = lv[p & 1];
    if (t < nbins)
#pragma unroll
      for (int q = 0; q < NW; ++q) wc[q][t] = 0;
    __syncthreads();
    int rk[kFieldItems];
#pragma unroll
    for (int r = 0; r < kFieldItems; ++r) {
      const bool valid = w * WSPAN + r * 64 + lane < n;
      const uint32_t d = (kk[r] >> shift) & mask;
      uint64_t m = __ballot(valid);
      for (int b = 0; b < rb; ++b) {
        const bool bit = (d >> b) & 1u;
        const uint64_t bal = __ballot(bit);
        m &= bit ? bal : ~bal;
      }
      const int lr = __popcll(m & lanemask_lt());
      // one wave's LDS accesses take effect in program order: every lane reads the count before the lowest lane of
      // its digit group adds the group's size
      const int before = valid ? (int)wc[w][d] : 0;
      rk[r] = valid ? before + lr : -1;
      if (valid && lr == 0) wc[w][d] = (uint16_t)(before + __popcll(m));
    }
    __syncthreads();
    int run = 0;
    if (t < nbins)
#pragma unroll
      for (int q = 0; q < NW; ++q) {
        const int x = wc[q][t];
        wc[q][t] = (uint16_t)run;
        run += x;
      }
    {
      int v[1] = {run}, ex[1], tot[1];
      block_excl_scan<kFieldThreads, 1>(v, ex, tot);
      if (t < nbins) lbase[t] = ex[0];
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < kFieldItems; ++r)
      if (rk[r] >= 0) {
        const int j = w * WSPAN + r * 64 + lane;
        const uint32_t d = (kk[r] >> shift) & mask;
        const int lp = lbase[d] + wc[w][d] + rk[r];
        lk[lp] = kk[r];
        vdst[lp] = p == 0 ? (uint16_t)j : vsrc[j];
      }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < kFieldItems; ++r) {
      const int j = w * WSPAN + r * 64 + lane;
      if (j < n) kk[r] = lk[j];
    }
  }
  const uint16_t* vfin = lv[(passes - 1) & 1];
  const int64_t out0 = (int64_t)c * nrows;
#pragma unroll
  for (int r = 0; r < kFieldItems; ++r) {
    const int j = w * WSPAN + r * 64 + lane;
    if (j < n) {
      skeys[out0 + j] = kk[r];
      svals[out0 + j] = (int32_t)vfin[j] * nf + c;
    }
  }
  int wcount;
  const uint32_t hm = field_heads(lk, n, wcount);
  int* hpos = reinterpret_cast<int*>(lk);
  const int U = field_head_positions(hm, wcount, n, wtot, hpos);
  int e = 0;
  for (int u = t; u < U; u += kFieldThreads) e += part_chunks(hpos[u + 1] - hpos[u]);
  int v[1] = {e}, ex[1], tot[1];
  block_excl_scan<kFieldThreads, 1>(v, ex, tot);
  if (t == 0) {
    cnt[2 * c] = U;
    cnt[2 * c + 1] = tot[0];
  }
}

// Field c's unique ids, segment starts, first occurrences, inverse and chunk plan, offset by the earlier fields'
// segment and chunk counts (cnt, from k_field_sort).  The last field's block stores U, E and seg_start[U] = n.
__global__ __launch_bounds__(kFieldThreads) void k_field_apply(const uint32_t* __restrict__ skeys,
                                                               const int32_t* __restrict__ svals, int64_t nrows,
                                                               int nf, FieldBounds fb, const int64_t* __restrict__ cnt,
                                                               int64_t* __restrict__ d_tot,
                                                               int64_t* __restrict__ n_unique,
                                                               int64_t* __restrict__ uniq,
                                                               int64_t* __restrict__ seg_start,
                                                               int32_t* __restrict__ seg_occ0,
                                                               int64_t* __restrict__ inverse,
                                                               int32_t* __restrict__ chunk_off,
                                                               int32_t* __restrict__ chunk_seg,
                                                               int32_t* __restrict__ hot_list) {
  constexpr int NW = kFieldThreads / 64, WSPAN = kFieldItems * 64;
  __shared__ uint32_t lk[kFieldRows];
  __shared__ int hpos[kFieldRows + 1];
  __shared__ int wtot[NW];
  __shared__ int64_t pre[2][NW];
  const int c = blockIdx.x, t = threadIdx.x, w = t >> 6, lane = t & 63;
  const int n = (int)nrows;
  const int64_t lo = fb.lo[c], R = fb.lo[c + 1] - lo, out0 = (int64_t)c * nrows;
  {
    // segments and chunks of the earlier fields (nf <= kFieldMax <= kFieldThreads)
    int64_t a = t < c ? cnt[2 * t] : 0, b = t < c ? cnt[2 * t + 1] : 0;
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
      a += __shfl_xor(a, d, 64);
      b += __shfl_xor(b, d, 64);
    }
    if (lane == 0) {
      pre[0][w] = a;
      pre[1][w] = b;
    }
  }
#pragma unroll
  for (int r = 0; r < kFieldItems; ++r) {
    const int j = w * WSPAN + r * 64 + lane;
    if (j < n) lk[j] = skeys[out0 + j];
  }
  __syncthreads();
  int64_t su = 0, se = 0;
#pragma unroll
  for (int q = 0; q < NW; ++q) {
    su += pre[0][q];
    se += pre[1][q];
  }
  int wcount;
  const uint32_t hm = field_heads(lk, n, wcount);
  const int U = field_head_positions(hm, wcount, n, wtot, hpos);
  // every position's segment: heads at or before it, less one (this wave's earlier heads from the head flags)
  int run = 0;
#pragma unroll
  for (int q = 0; q < NW; ++q) run += q < w ? wtot[q] : 0;
#pragma unroll
  for (int r = 0; r < kFieldItems; ++r) {
    const int j = w * WSPAN + r * 64 + lane;
    const bool h = (hm >> r) & 1u;
    const uint64_t bal = __ballot(h);
    if (j < n) {
      const int64_t gu = su + run + __popcll(bal & lanemask_lt()) + (h ? 0 : -1);
      const int32_t o = svals[out0 + j];
      if (h) {
        const uint32_t k = lk[j];
        uniq[gu] = (int64_t)k == R ? -1 : lo + (int64_t)k;
        seg_start[gu] = out0 + j;
        seg_occ0[gu] = o;
      }
      if (inverse) inverse[o] = gu;
    }
    run += __popcll(bal);
  }
  int64_t before = se;
  for (int u0 = 0; u0 < U; u0 += kFieldThreads) {
    const int u = u0 + t;
    const int L = u < U ? hpos[u + 1] - hpos[u] : 0;
    const int e = u < U ? part_chunks(L) : 0;
    int v[1] = {e}, ex[1], tot[1];
    block_excl_scan<kFieldThreads, 1>(v, ex, tot);
    if (u < U) {
      const int64_t off = before + ex[0];
      const int32_t gu = (int32_t)(su + u);
      chunk_off[gu] = (int32_t)off;
      for (int k = 0; k < e; ++k) chunk_seg[off + k] = gu;
      if (seg_hot(L)) hot_list[atomicAdd(reinterpret_cast<unsigned long long*>(d_tot + 2), 1ull)] = gu;
    }
    before += tot[0];
    __syncthreads();   // block_excl_scan's LDS is reused by the next round
  }
  if (c == nf - 1 && t == 0) {
    const int64_t Ut = su + U;
    d_tot[0] = Ut;
    if (n_unique) *n_unique = Ut;
    seg_start[Ut] = out0 + n;
    d_tot[1] = before;
  }
}

// Does occurrence k of a segment (occurrence index o, previous one prev) start a new group?  Sort path
// (win_shift == 0): every kAtenGroup occurrences; windowed path: when its index window differs from the previous
// occurrence's.  Wave-uniform (all arguments are).
__device__ __forceinline__ bool group_head(int64_t k, int32_t o, int32_t prev, int win_shift) {
  return k == 0 || (win_shift ? (o >> win_shift) != (prev >> win_shift) : k % kAtenGroup == 0);
}

// Folds the gradients at sorted positions [p0, p1) (p1 - p0 <= 64), occurrences k0.. of their segment, into the
// open group acc and the segment total tot (this lane's NQ elements j = lane + 64 q < D).  Occurrence indices are
// loaded once per wave and broadcast with readlane; prev carries the previous occurrence index across calls.
template <int NQ>
__device__ __forceinline__ void fold_range(const float* __restrict__ grad, int64_t D, const int32_t* __restrict__ sv,
                                           int64_t p0, int64_t p1, int64_t k0, int win_shift, int32_t& prev,
                                           float (&acc)[NQ], float (&tot)[NQ]) {
  const int lane = threadIdx.x & 63;
  const int len = (int)(p1 - p0);
  const int32_t my = lane < len ? sv[p0 + lane] : 0;
  constexpr int UN = 8;
  for (int b0 = 0; b0 < len; b0 += UN) {
    float g[UN][NQ];
#pragma unroll
    for (int u = 0; u < UN; ++u) {
      if (b0 + u < len) {
        const int64_t o = (int64_t)__builtin_amdgcn_readlane(my, b0 + u);
        const float* row = grad + o * D;
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
          const int64_t j = lane + 64 * q;
          g[u][q] = j < D ? __builtin_nontemporal_load(row + j) : 0.0f;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < UN; ++u) {
      if (b0 + u < len) {
        const int32_t o = __builtin_amdgcn_readlane(my, b0 + u);
        const int64_t k = k0 + b0 + u;
        if (group_head(k, o, prev, win_shift)) {
#pragma unroll
          for (int q = 0; q < NQ; ++q) {
            if (k) tot[q] = tot[q] + acc[q];
            acc[q] = g[u][q];
          }
        } else {
#pragma unroll
          for (int q = 0; q < NQ; ++q) acc[q] = acc[q] + g[u][q];
        }
        prev = o;
      }
    }
  }
}

// The group sums of a segment's partial chunks are consecutive parts rows from chunk_off[u] * kGroupsPerChunk (every
// partial chunk but the last is full): ceil(L / kAtenGroup) of them for a hot segment, else
// ceil((L - kSegChunk) / kAtenGroup).  inline_len: the occurrences the segment's own wave folds.
__device__ __forceinline__ int64_t seg_parts(int64_t L, int win_shift) {
  if (win_shift) return 0;
  if (seg_hot(L)) return (L + kAtenGroup - 1) / kAtenGroup;
  return L <= kSegChunk ? 0 : (L - kSegChunk + kAtenGroup - 1) / kAtenGroup;
}
__device__ __forceinline__ int64_t inline_len(int64_t L, int win_shift) {
  if (win_shift) return L;
  return seg_hot(L) ? 0 : (L < kSegChunk ? L : kSegChunk);
}

// Final per-segment sum (the inline part -- the first chunk, or the whole segment on the windowed path -- then the
// extra chunks' group sums in order), then either written to out[uniq[u]] (MODE 0) or applied as an Adam step to
// state[uniq[u]] (MODE 1).  One wave per segment.
template <int NQ, int MODE>
__global__ __launch_bounds__(256) void k_seg_final(const float* __restrict__ grad, int64_t D,
                                                   const int32_t* __restrict__ sv,
                                                   const int64_t* __restrict__ seg_start,
                                                   const int64_t* __restrict__ uniq,
                                                   const int32_t* __restrict__ chunk_off,
                                                   const float* __restrict__ parts, const int64_t* __restrict__ d_U,
                                                   int win_shift, float* __restrict__ out, int64_t nrows,
                                                   AdamScalars s) {
  const int lane = threadIdx.x & 63;
  const int64_t U = *d_U;
  for (int64_t u = wave_id(); u < U; u += wave_count()) {
    const int64_t s0 = seg_start[u], s1 = seg_start[u + 1];
    const int64_t L = s1 - s0;
    const int64_t row = uniq ? uniq[u] : u;   // NULL: segment u goes to row u
    const int64_t inl = inline_len(L, win_shift);
    float acc[NQ], tot[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) acc[q] = tot[q] = 0.0f;
    int32_t prev = 0;
    for (int64_t b0 = 0; b0 < inl; b0 += 64)
      fold_range<NQ>(grad, D, sv, s0 + b0, s0 + (inl - b0 < 64 ? inl : b0 + 64), b0, win_shift, prev, acc, tot);
#pragma unroll
    for (int q = 0; q < NQ; ++q) tot[q] = tot[q] + acc[q];
    const int64_t np = seg_parts(L, win_shift);
    const float* pr = np ? parts + (int64_t)chunk_off[u] * kGroupsPerChunk * D : parts;
    constexpr int PB = 8;
    for (int64_t c0 = 0; c0 < np; c0 += PB) {
      float pc[PB][NQ];
#pragma unroll
      for (int e = 0; e < PB; ++e)
        if (c0 + e < np) {
#pragma unroll
          for (int q = 0; q < NQ; ++q) {
            const int64_t j = lane + 64 * q;
            pc[e][q] = j < D ? pr[(c0 + e) * D + j] : 0.0f;
          }
        }
#pragma unroll
      for (int e = 0; e < PB; ++e)
        if (c0 + e < np) {
#pragma unroll
          for (int q = 0; q < NQ; ++q) tot[q] = tot[q] + pc[e][q];
        }
    }
    if (row < 0 || row >= nrows) continue;
    if (MODE == 0) {
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        const int64_t j = lane + 64 * q;
        if (j < D) out[row * D + j] = tot[q];
      }
    } else {
      float* rec = out + row * 3 * D;
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        const int64_t j = lane + 64 * q;
        if (j < D) {
          float w = rec[j], m = rec[D + j], v = rec[2 * D + j];
          adam_elem(w, m, v, tot[q], s);
          rec[j] = w;
          rec[D + j] = m;
          rec[2 * D + j] = v;
        }
      }
    }
  }
}

// Wave-per-row form of k_seg_final for D = 64*VPL (lane l holds floats [l*VPL, l*VPL + VPL)): no grid-stride
// loop, each wave owns kSegPerWave consecutive segments starting at u_base + wave * kSegPerWave; waves past U exit.
// All per-segment metadata (bounds, row id, first occurrence) are scalar loads issued together, then the first
// gradient row, the row's w, m, v (MODE 1) and the next 63 occurrence indices load in parallel: a one-occurrence
// segment -- the common case -- costs two dependent memory round trips.
constexpr int kSegPerWave = 2;

// The result of one segment: written to out[row] (MODE 0) or applied as an Adam step to state row `row` (MODE 1).
template <int VPL, int MODE>
__device__ __forceinline__ void seg_emit(float* __restrict__ out, int64_t row, const RowFrag<VPL>& sum,
                                         const AdamScalars& s) {
  constexpr int64_t D = 64 * VPL;
  const int lane = threadIdx.x & 63;
  if (MODE == 0) {
    frag_store<VPL>(out + row * D + lane * VPL, sum);
  } else {
    float* rec = out + row * 3 * D + lane * VPL;
    RowFrag<VPL> w = frag_load<VPL, false>(rec), m = frag_load<VPL, false>(rec + D),
                 v = frag_load<VPL, false>(rec + 2 * D);
    frag_adam<VPL>(w, m, v, sum, s);
    frag_store<VPL>(rec, w);
    frag_store<VPL>(rec + D, m);
    frag_store<VPL>(rec + 2 * D, v);
  }
}

// Hot segments, one block each (grid-stride over hot_list by hot_blocks blocks): the total is
// ((0 + G1) + G2) + ... over the segment's ceil(L / 10) run sums, consecutive parts rows.  The four waves load
// 4 * PB run sums together; then wave 0, 1, 2, 3 in turn adds its PB of them to the running total, which passes
// from wave to wave through LDS, so the additions keep their order.  Every loop bound is block-uniform.
template <int VPL, int MODE>
__device__ __forceinline__ void seg_hot_block(const int64_t* __restrict__ seg_start,
                                              const int64_t* __restrict__ uniq,
                                              const int32_t* __restrict__ chunk_off,
                                              const float* __restrict__ parts,
                                              const int32_t* __restrict__ hot_list, const int64_t* __restrict__ d_hot,
                                              int64_t hot_blocks, float* __restrict__ out, int64_t nrows,
                                              const AdamScalars& s, float* __restrict__ relay, int64_t block) {
  constexpr int64_t D = 64 * VPL;
  constexpr int PB = VPL <= 2 ? kSegParts : kSegParts / 2;
  constexpr int NWV = 4;
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int64_t nh = *d_hot;
  for (int64_t h = block; h < nh; h += hot_blocks) {
    const int64_t u = hot_list[h];
    const int64_t L = seg_start[u + 1] - seg_start[u];
    const int64_t nr = (L + kAtenGroup - 1) / kAtenGroup;
    const float* pr = parts + (int64_t)chunk_off[u] * kGroupsPerChunk * D + lane * VPL;
    for (int64_t i0 = 0; i0 < nr; i0 += NWV * PB) {
      const int64_t mine = i0 + wv * PB;
      RowFrag<VPL> pc[PB];
#pragma unroll
      for (int e = 0; e < PB; ++e)
        if (mine + e < nr) pc[e] = frag_load<VPL, false>(pr + (mine + e) * D);
      for (int w = 0; w < NWV; ++w) {
        if (wv == w && mine < nr) {
          RowFrag<VPL> tot;
          if (mine == 0) {
            tot = frag_zero<VPL>();
          } else {
#pragma unroll
            for (int j = 0; j < VPL; ++j) tot.v[j] = relay[lane * VPL + j];
          }
#pragma unroll
          for (int e = 0; e < PB; ++e)
            if (mine + e < nr) {
#pragma unroll
              for (int j = 0; j < VPL; ++j) tot.v[j] = tot.v[j] + pc[e].v[j];
            }
#pragma unroll
          for (int j = 0; j < VPL; ++j) relay[lane * VPL + j] = tot.v[j];
        }
        __syncthreads();
      }
    }
    if (wv == 0) {
      const int64_t row = uniq ? uniq[u] : u;
      if (row >= 0 && row < nrows) {
        RowFrag<VPL> tot;
#pragma unroll
        for (int j = 0; j < VPL; ++j) tot.v[j] = relay[lane * VPL + j];
        seg_emit<VPL, MODE>(out, row, tot, s);
      }
    }
    __syncthreads();   // the relay is reused by the block's next hot segment
  }
}

// The final kernel as a functor (elr_launch.h): block `block` of the launch, the first hot_blocks of them on the hot
// segments.  k_seg_final_wpr launches it on its own; the device-driven step also runs it beside the directory's
// first launch of the executor (k_run2).
template <int VPL, int MODE>
struct SegFinalWpr {
  const float* grad;
  const int32_t* sv;
  const int64_t* seg_start;
  const int32_t* seg_occ0;
  const int64_t* uniq;
  const int32_t* chunk_off;
  const float* parts;
  const int64_t* d_U;
  int64_t u_base;
  const int32_t* hot_list;
  const int64_t* d_hot;
  int64_t hot_blocks;
  float* out;
  int64_t nrows;
  AdamScalars s;
  __device__ void operator()(int64_t block, int64_t nblocks) const;
};

template <int VPL, int MODE>
__device__ void SegFinalWpr<VPL, MODE>::operator()(int64_t block, int64_t) const {
  constexpr int64_t D = 64 * VPL;
  constexpr int SW = kSegPerWave;
  __shared__ float relay[D];
  if (block < hot_blocks) {
    seg_hot_block<VPL, MODE>(seg_start, uniq, chunk_off, parts, hot_list, d_hot, hot_blocks, out, nrows, s, relay,
                             block);
    return;
  }
  const int lane = threadIdx.x & 63;
  const int64_t U = *d_U;
  const int64_t u0 = u_base + ((block - hot_blocks) * 4 + (threadIdx.x >> 6)) * SW;
  if (u0 >= U) return;
  int64_t s0[SW], len[SW], row[SW], o0[SW];
  bool ok[SW];
#pragma unroll
  for (int q = 0; q < SW; ++q) {
    const int64_t u = u0 + q;
    ok[q] = u < U;
    s0[q] = ok[q] ? seg_start[u] : 0;
    len[q] = ok[q] ? seg_start[u + 1] - s0[q] : 0;
    row[q] = ok[q] ? (uniq ? uniq[u] : u) : -1;   // NULL: segment u goes to row u
    o0[q] = ok[q] ? (int64_t)seg_occ0[u] : 0;
    ok[q] = ok[q] && row[q] >= 0 && row[q] < nrows && !seg_hot(len[q]);   // hot segments: a block's
  }
  RowFrag<VPL> w[SW], m[SW], v[SW], acc[SW];
  int32_t my[SW];
  // short: every segment of the wave fits one run of at most FB occurrences (wave-uniform: the lengths are scalar
  // loads).  Their remaining rows then load together, all segments' at once, before any addition.
  constexpr int FB = VPL <= 2 ? kAtenGroup : 4;
  bool short_segs = true;
#pragma unroll
  for (int q = 0; q < SW; ++q) {
    short_segs = short_segs && (!ok[q] || len[q] <= FB);
    if (!ok[q]) continue;
    acc[q] = frag_load<VPL, true>(grad + o0[q] * D + lane * VPL);
    if (MODE == 1) {
      const float* rec = out + row[q] * 3 * D + lane * VPL;
      w[q] = frag_load<VPL, false>(rec);
      m[q] = frag_load<VPL, false>(rec + D);
      v[q] = frag_load<VPL, false>(rec + 2 * D);
    }
    my[q] = (lane >= 1 && lane < len[q]) ? sv[s0[q] + lane] : 0;
  }
  if (short_segs) {
    // the same additions as the general loop below for one run: ((first + g1) + g2) + ..., then +0 + run
    RowFrag<VPL> g[SW][FB - 1];
#pragma unroll
    for (int q = 0; q < SW; ++q)
#pragma unroll
      for (int e = 1; e < FB; ++e)
        if (ok[q] && e < len[q]) {
          const int64_t o = (int64_t)__builtin_amdgcn_readlane(my[q], e);
          g[q][e - 1] = frag_load<VPL, true>(grad + o * D + lane * VPL);
        }
#pragma unroll
    for (int q = 0; q < SW; ++q) {
      if (!ok[q]) continue;
      RowFrag<VPL> run = acc[q];
#pragma unroll
      for (int e = 1; e < FB; ++e)
        if (e < len[q]) {
#pragma unroll
          for (int j = 0; j < VPL; ++j) run.v[j] = run.v[j] + g[q][e - 1].v[j];
        }
#pragma unroll
      for (int j = 0; j < VPL; ++j) acc[q].v[j] = 0.0f + run.v[j];
    }
  }
#pragma unroll
  for (int q = 0; q < SW; ++q) {
    if (!ok[q] || short_segs) continue;
    // the first chunk folds here, run by run (runs of kAtenGroup from the segment's first occurrence, which is
    // already in acc); then the later chunks' run sums, kSegParts at a time
    const int inl = (int)(len[q] < kSegChunk ? len[q] : kSegChunk);
    RowFrag<VPL> tot = frag_zero<VPL>();
    constexpr int RB = VPL <= 2 ? kAtenGroup : kAtenGroup / 2;   // rows of a run loaded together
    constexpr int PB = VPL <= 2 ? kSegParts : kSegParts / 2;     // run sums loaded together
    for (int r0 = 0; r0 < inl; r0 += kAtenGroup) {
      const int rl = inl - r0 < kAtenGroup ? inl - r0 : kAtenGroup;
      RowFrag<VPL> run = acc[q];
      for (int h = 0; h < rl; h += RB) {
        RowFrag<VPL> g[RB];
#pragma unroll
        for (int e = 0; e < RB; ++e)
          if (h + e < rl && r0 + h + e > 0) {
            const int64_t o = (int64_t)__builtin_amdgcn_readlane(my[q], r0 + h + e);
            g[e] = frag_load<VPL, true>(grad + o * D + lane * VPL);
          }
#pragma unroll
        for (int e = 0; e < RB; ++e) {
          if (h + e >= rl) continue;
          if (h + e == 0) {
            if (r0 > 0) run = g[e];   // run 0 starts from the preloaded first gradient
          } else {
#pragma unroll
            for (int j = 0; j < VPL; ++j) run.v[j] = run.v[j] + g[e].v[j];
          }
        }
      }
#pragma unroll
      for (int j = 0; j < VPL; ++j) tot.v[j] = tot.v[j] + run.v[j];
    }
    const int64_t np = seg_parts(len[q], 0);
    if (np) {
      const float* pr = parts + (int64_t)chunk_off[u0 + q] * kGroupsPerChunk * D + lane * VPL;
      for (int64_t c0 = 0; c0 < np; c0 += PB) {
        RowFrag<VPL> pc[PB];
#pragma unroll
        for (int e = 0; e < PB; ++e)
          if (c0 + e < np) pc[e] = frag_load<VPL, false>(pr + (c0 + e) * D);
#pragma unroll
        for (int e = 0; e < PB; ++e)
          if (c0 + e < np) {
#pragma unroll
            for (int j = 0; j < VPL; ++j) tot.v[j] = tot.v[j] + pc[e].v[j];
          }
      }
    }
    acc[q] = tot;
  }
#pragma unroll
  for (int q = 0; q < SW; ++q) {
    if (!ok[q]) continue;
    if (MODE == 0) {
      frag_store<VPL>(out + row[q] * D + lane * VPL, acc[q]);
    } else {
      frag_adam<VPL>(w[q], m[q], v[q], acc[q], s);
      float* rec = out + row[q] * 3 * D + lane * VPL;
      frag_store<VPL>(rec, w[q]);
      frag_store<VPL>(rec + D, m[q]);
      frag_store<VPL>(rec + 2 * D, v[q]);
    }
  }
}

template <int VPL, int MODE>
__global__ __launch_bounds__(256) void k_seg_final_wpr(SegFinalWpr<VPL, MODE> f) {
  f((int64_t)blockIdx.x, (int64_t)gridDim.x);
}

// ---- host side -------------------------------------------------------------------------------------------------
inline int64_t al256(int64_t b) { return (b + 255) & ~int64_t(255); }

// Scratch carve-up for n occurrences of width D.
struct DedupScratch {
  void* keys[2];
  int32_t* vals[2];
  int64_t* hist;      // [kRadixMaxBins * ntile], ntile = n / (kSortThreads * items_for(n)) rounded up
  int64_t* dtot;      // [256] digit totals
  int64_t* bsum;      // [n / (kSegBlock * items_for(n)) + 1]
  int64_t* d_tot;     // [3]: U, E (partial chunks), hot segments
  int64_t* uniq;      // [n]
  int64_t* seg_start; // [n + 1]
  int32_t* seg_occ0;  // [n] first occurrence index of each segment
  int32_t* chunk_off; // [n]
  int32_t* chunk_seg; // [nch]: n / kSegChunk + n / kHotLen + 2 bounds the partial chunks
  float* parts;       // [nch * kGroupsPerChunk * D] group sums of the partial chunks
  int32_t* hot_list;  // [n / kHotLen + 1] hot segments
};

inline int64_t dedup_scratch_bytes(int64_t n, int64_t D, DedupScratch* out, void* base) {
  const int64_t ntile = cdiv(n, kSortThreads * items_for(n)), nblk = cdiv(n, kSegBlock * items_for(n));
  const int64_t nch = n / kSegChunk + n / kHotLen + 2;
  int64_t o = 0;
  char* b = (char*)base;
  auto take = [&](int64_t bytes) {
    void* p = b ? (void*)(b + o) : nullptr;
    o += al256(bytes);
    return p;
  };
  DedupScratch s;
  s.keys[0] = take(n * 8);
  s.keys[1] = take(n * 8);
  s.vals[0] = (int32_t*)take(n * 4);
  s.vals[1] = (int32_t*)take(n * 4);
  s.hist = (int64_t*)take(kRadixMaxBins * ntile * 8);
  s.dtot = (int64_t*)take(kRadixMaxBins * 8);
  s.bsum = (int64_t*)take(nblk * 8);
  s.d_tot = (int64_t*)take(3 * 8);
  s.uniq = (int64_t*)take(n * 8);
  s.seg_start = (int64_t*)take((n + 1) * 8);
  s.seg_occ0 = (int32_t*)take(n * 4);
  s.chunk_off = (int32_t*)take(n * 4);
  s.chunk_seg = (int32_t*)take(nch * 4);
  s.parts = (float*)take(nch * kGroupsPerChunk * D * 4);
  s.hot_list = (int32_t*)take((n / kHotLen + 1) * 4);
  if (out) *out = s;
  return o;
}

// Widest digit of a sort with Key keys: 64-bit keys stop at 9 bits to keep the scatter's LDS tile within 64 KiB.
template <typename Key>
constexpr int max_digit_bits() { return sizeof(Key) == 8 ? 9 : kRadixMaxBits; }

// Passes of a sort of key_bits-bit Key keys (sort_plan); the result sits in buffer (passes - 1) % 2.
template <typename Key>
inline int sort_passes(int key_bits) {
  int passes, rb;
  sort_plan(key_bits, max_digit_bits<Key>(), passes, rb);
  return passes;
}

// One pass over RB-bit digit p of the keys: histogram, scan, stable scatter from buffer cur (the caller's ids on
// the first pass) to buffer nxt.
template <typename Key, int ITEMS, int RB>
static void radix_pass(const int64_t* ids, int64_t n, int p, int cur, int nxt, DedupScratch& S, hipStream_t st) {
  const int64_t ntile = cdiv(n, kSortThreads * ITEMS);
  const int shift = RB * p;
  constexpr int BINS = 1 << RB;
  constexpr unsigned kScanGrid = (unsigned)(BINS / (kSortThreads / 64));   // a wave per digit
  Key* kb[2] = {(Key*)S.keys[0], (Key*)S.keys[1]};
  if (p == 0) {
    k_radix_hist<int64_t, Key, ITEMS, RB><<<(unsigned)ntile, kSortThreads, 0, st>>>(ids, n, shift, S.hist, ntile);
    k_radix_hist_scan<<<kScanGrid, kSortThreads, 0, st>>>(S.hist, ntile, BINS, S.dtot);
    k_radix_scatter<int64_t, Key, true, ITEMS, RB><<<(unsigned)ntile, kSortThreads, 0, st>>>(
        ids, nullptr, n, shift, S.hist, S.dtot, ntile, kb[nxt], S.vals[nxt]);
  } else {
    k_radix_hist<Key, Key, ITEMS, RB><<<(unsigned)ntile, kSortThreads, 0, st>>>(kb[cur], n, shift, S.hist, ntile);
    k_radix_hist_scan<<<kScanGrid, kSortThreads, 0, st>>>(S.hist, ntile, BINS, S.dtot);
    k_radix_scatter<Key, Key, false, ITEMS, RB><<<(unsigned)ntile, kSortThreads, 0, st>>>(
        kb[cur], S.vals[cur], n, shift, S.hist, S.dtot, ntile, kb[nxt], S.vals[nxt]);
  }
}

// Sort (ids, positions) by id; returns which buffer holds the result.
template <typename Key, int ITEMS>
static int radix_sort(const int64_t* ids, int64_t n, int key_bits, DedupScratch& S, hipStream_t st) {
  int passes, rb;
  sort_plan(key_bits, max_digit_bits<Key>(), passes, rb);
  int cur = 0;
  for (int p = 0; p < passes; ++p) {
    const int nxt = p == 0 ? 0 : cur ^ 1;
    if constexpr (max_digit_bits<Key>() >= 10) {
      if (rb == 10) {
        radix_pass<Key, ITEMS, 10>(ids, n, p, cur, nxt, S, st);
        cur = nxt;
        continue;
      }
    }
    if (rb == 9) radix_pass<Key, ITEMS, 9>(ids, n, p, cur, nxt, S, st);
    else radix_pass<Key, ITEMS, 8>(ids, n, p, cur, nxt, S, st);
    cur = nxt;
  }
  return cur;
}

// Sort, segment heads (uniq / seg_start / inverse, U in d_tot[0]) and the extra-chunk plan (E in d_tot[1]).
template <typename Key, int ITEMS>
static int dedup_core_items(const int64_t* ids, int64_t n, int key_bits, DedupScratch& S, int64_t* uniq_out,
                            int64_t* inverse, int64_t* n_unique, hipStream_t st) {
  const int cur = radix_sort<Key, ITEMS>(ids, n, key_bits, S, st);
  const Key* sk = (const Key*)S.keys[cur];
  const int32_t* sv = S.vals[cur];
  const int64_t nblk = cdiv(n, kSegBlock * ITEMS);
  int64_t* uniq = uniq_out ? uniq_out : S.uniq;
  const int scanned = nblk > kFoldMaxBlocks;
  k_seg_count<Key, ITEMS><<<(unsigned)nblk, kSegBlock, 0, st>>>(sk, n, S.bsum);
  if (scanned) k_scan_blocks<<<1, kScanBlock, 0, st>>>(S.bsum, nblk);
  k_seg_apply<Key, ITEMS><<<(unsigned)nblk, kSegBlock, 0, st>>>(sk, sv, n, S.bsum, scanned, S.d_tot, n_unique, uniq,
                                                                S.seg_start, S.seg_occ0, inverse);
  return cur;
}

template <typename Key>
static int dedup_core(const int64_t* ids, int64_t n, int key_bits, DedupScratch& S, int64_t* uniq_out,
                      int64_t* inverse, int64_t* n_unique, hipStream_t st) {
  return items_for(n) == kItemsBig
             ? dedup_core_items<Key, kItemsBig>(ids, n, key_bits, S, uniq_out, inverse, n_unique, st)
             : dedup_core_items<Key, kItemsSmall>(ids, n, key_bits, S, uniq_out, inverse, n_unique, st);
}

// ATen's windowed order applies up to kAtenSmall indices: returns the window's shift there, 0 on the sort path.
inline int win_shift_for(int64_t n) { return n <= kAtenSmall ? kAtenWinShift : 0; }

template <int ITEMS>
static void chunk_plan_items(int64_t n, DedupScratch& S, hipStream_t st) {
  const int64_t nblk = cdiv(n, kSegBlock * ITEMS);
  const int scanned = nblk > kFoldMaxBlocks;
  k_chunk_count<ITEMS><<<(unsigned)nblk, kSegBlock, 0, st>>>(S.seg_start, S.d_tot, S.bsum, S.d_tot + 2);
  if (scanned) k_scan_blocks<<<1, kScanBlock, 0, st>>>(S.bsum, nblk);
  k_chunk_apply<ITEMS><<<(unsigned)nblk, kSegBlock, 0, st>>>(S.seg_start, S.d_tot, S.bsum, scanned, S.chunk_off,
                                                             S.chunk_seg, S.hot_list, S.d_tot + 2, S.d_tot + 1);
}

static void chunk_plan(int64_t n, DedupScratch& S, hipStream_t st) {
  if (win_shift_for(n)) return;   // the windowed path sums every segment in one wave: no extra chunks
  if (items_for(n) == kItemsBig) chunk_plan_items<kItemsBig>(n, S, st);
  else chunk_plan_items<kItemsSmall>(n, S, st);
}


template <int NQ>
inline SegPartials<NQ> seg_partials_of(const float* grad, int64_t D, const int32_t* sv, const DedupScratch& S) {
  return SegPartials<NQ>{grad, D, sv, S.seg_start, S.chunk_off, S.chunk_seg, S.d_tot + 1, S.parts};
}

template <int NQ, int MODE>
static void seg_reduce(const float* grad, int64_t D, const int32_t* sv, DedupScratch& S, const int64_t* uniq,
                       int64_t n, float* out, int64_t nrows, const AdamScalars& s, hipStream_t st, bool partials) {
  const int ws = win_shift_for(n);
  if (!ws && partials) launch1(seg_partials_of<NQ>(grad, D, sv, S), seg_partials_blocks(n), st);
  k_seg_final<NQ, MODE><<<wave_grid(n), 256, 0, st>>>(grad, D, sv, S.seg_start, uniq, S.chunk_off, S.parts, S.d_tot,
                                                       ws, out, nrows, s);
}

template <int VPL, int MODE>
static void seg_reduce_wpr(const float* grad, const int32_t* sv, DedupScratch& S, const int64_t* uniq, int64_t n,
                           float* out, int64_t nrows, const AdamScalars& s, hipStream_t st, bool partials) {
  constexpr int64_t D = 64 * VPL;   // sort path only (n > kAtenSmall)
  if (partials) launch1(seg_partials_of<VPL>(grad, D, sv, S), seg_partials_blocks(n), st);
  // one launch per range of at most 2^22 blocks (4 waves of kSegPerWave segments each); U <= n.  The first launch
  // starts with one block per possible hot segment (fewer than n / kHotLen; blocks beyond the count exit at once).
  const int64_t per = kOneShotBlocks * 4 * kSegPerWave;
  for (int64_t a = 0; a < n; a += per) {
    const int64_t m = n - a < per ? n - a : per;
    const int64_t hb = a == 0 ? n / kHotLen + 1 : 0;
    const SegFinalWpr<VPL, MODE> f{grad, sv, S.seg_start, S.seg_occ0, uniq, S.chunk_off, S.parts, S.d_tot, a,
                                   S.hot_list, S.d_tot + 2, hb, out, nrows, s};
    k_seg_final_wpr<VPL, MODE><<<(unsigned)(hb + cdiv(m, 4 * kSegPerWave)), 256, 0, st>>>(f);
  }
}

template <int MODE>
static int seg_reduce_d(const float* grad, int64_t D, const int32_t* sv, DedupScratch& S, const int64_t* uniq,
                        int64_t n, float* out, int64_t nrows, const AdamScalars& s, hipStream_t st,
                        bool partials = true) {
  if (aligned16(grad) && aligned16(out) && !win_shift_for(n)) {   // ATen's windowed order: the generic kernels
    switch (D) {
      case 64: seg_reduce_wpr<1, MODE>(grad, sv, S, uniq, n, out, nrows, s, st, partials); return ELR_OK;
      case 128: seg_reduce_wpr<2, MODE>(grad, sv, S, uniq, n, out, nrows, s, st, partials); return ELR_OK;
      case 256: seg_reduce_wpr<4, MODE>(grad, sv, S, uniq, n, out, nrows, s, st, partials); return ELR_OK;
      case 512: seg_reduce_wpr<8, MODE>(grad, sv, S, uniq, n, out, nrows, s, st, partials); return ELR_OK;
      default: break;
    }
  }
  const int64_t nq = cdiv(D, 64);
  switch (nq) {
    case 1: seg_reduce<1, MODE>(grad, D, sv, S, uniq, n, out, nrows, s, st, partials); break;
    case 2: seg_reduce<2, MODE>(grad, D, sv, S, uniq, n, out, nrows, s, st, partials); break;
    case 3:
    case 4: seg_reduce<4, MODE>(grad, D, sv, S, uniq, n, out, nrows, s, st, partials); break;
    case 5: case 6: case 7:
    case 8: seg_reduce<8, MODE>(grad, D, sv, S, uniq, n, out, nrows, s, st, partials); break;
    default: return ELR_EUNSUPPORTED;
  }
  return ELR_OK;
}

inline int bits_for(int64_t bound) {  // smallest b with bound <= 2^b (keys in [0, bound))
  int b = 1;
  while (b < 63 && (int64_t(1) << b) < bound) ++b;
  return b;
}

inline bool dedup_sizes_ok(int64_t n) { return n >= 0 && n < (int64_t(1) << 31); }

}  // namespace elr

extern "C" int64_t elr_dedup_scratch_bytes(int64_t n, int64_t D) {
  if (!elr::dedup_sizes_ok(n) || D < 0) return ELR_EINVAL;
  return elr::dedup_scratch_bytes(n, D < 1 ? 1 : D, nullptr, nullptr);
}

extern "C" int elr_unique(const int64_t* ids, int64_t n, int key_bits, int64_t* uniq, int64_t* inverse,
                          int64_t* n_unique, void* scratch, int64_t scratch_bytes, void* stream) {
  using namespace elr;
  if (!dedup_sizes_ok(n) || key_bits < 1 || key_bits > 64) return ELR_EINVAL;
  if (n == 0) return ELR_OK;
  if (!ids || !uniq || !n_unique || !scratch) return ELR_EINVAL;
  DedupScratch S;
  if (scratch_bytes < dedup_scratch_bytes(n, 1, &S, scratch)) return ELR_ECAPACITY;
  hipStream_t st = (hipStream_t)stream;
  if (key_bits <= 32) dedup_core<uint32_t>(ids, n, key_bits, S, uniq, inverse, n_unique, st);
  else dedup_core<uint64_t>(ids, n, key_bits, S, uniq, inverse, n_unique, st);
  return launch_status();
}

extern "C" int elr_segment_sum(const float* grad, const int64_t* idx, int64_t n, int64_t D, int64_t num_rows,
                               float* out, void* scratch, int64_t scratch_bytes, void* stream) {
  using namespace elr;
  if (!dedup_sizes_ok(n) || D < 1 || num_rows < 0) return ELR_EINVAL;
  if (n == 0) return ELR_OK;
  if (!grad || !idx || !out || !scratch) return ELR_EINVAL;
  if (D > 512) return ELR_EUNSUPPORTED;
  DedupScratch S;
  if (scratch_bytes < dedup_scratch_bytes(n, D, &S, scratch)) return ELR_ECAPACITY;
  hipStream_t st = (hipStream_t)stream;
  const int kb = bits_for(num_rows);
  const int cur = kb <= 32 ? dedup_core<uint32_t>(idx, n, kb, S, nullptr, nullptr, nullptr, st)
                           : dedup_core<uint64_t>(idx, n, kb, S, nullptr, nullptr, nullptr, st);
  chunk_plan(n, S, st);
  const AdamScalars none{};
  const int rc = seg_reduce_d<0>(grad, D, S.vals[cur], S, S.uniq, n, out, num_rows, none, st);
  return rc != ELR_OK ? rc : launch_status();
}

extern "C" int elr_adam_dedup(float* state, int64_t C, const int64_t* ids, const float* grad, int64_t n, int64_t D,
                              const float sc[8], void* scratch, int64_t scratch_bytes, void* stream) {
  using namespace elr;
  if (!dedup_sizes_ok(n) || D < 1 || C < 0 || !sc) return ELR_EINVAL;
  if (n == 0) return ELR_OK;
  if (!state || !ids || !grad || !scratch) return ELR_EINVAL;
  if (D > 512) return ELR_EUNSUPPORTED;
  DedupScratch S;
  if (scratch_bytes < dedup_scratch_bytes(n, D, &S, scratch)) return ELR_ECAPACITY;
  hipStream_t st = (hipStream_t)stream;
  const AdamScalars s = make_scalars(sc);
  const int kb = bits_for(C);
  const int cur = kb <= 32 ? dedup_core<uint32_t>(ids, n, kb, S, nullptr, nullptr, nullptr, st)
                           : dedup_core<uint64_t>(ids, n, kb, S, nullptr, nullptr, nullptr, st);
  chunk_plan(n, S, st);
  const int rc = seg_reduce_d<1>(grad, D, S.vals[cur], S, S.uniq, n, state, C, s, st);
  return rc != ELR_OK ? rc : launch_status();
}

// ---- dedup plan: one sort per batch, reused by the segment sum -------------------------------------------------
// elr_dedup_plan sorts the batch and finds its segments exactly as elr_unique does, and also lays out the extra
// chunks; the scratch then holds the plan (sorted positions, segment starts, first occurrences, chunk plan, U).
// elr_segment_sum_plan sums a gradient batch over that plan without sorting again.  The sorted result lives in the
// scratch buffer that the last radix pass wrote: with p passes, buffer (p - 1) % 2.
static int plan_result_buffer(int key_bits) {
  return ((key_bits <= 32 ? elr::sort_passes<uint32_t>(key_bits) : elr::sort_passes<uint64_t>(key_bits)) - 1) % 2;
}

extern "C" int64_t elr_dedup_plan_bytes(int64_t n, int64_t D) {
  using namespace elr;
  if (!dedup_sizes_ok(n) || D < 1) return ELR_EINVAL;
  return dedup_scratch_bytes(n, D, nullptr, nullptr);
}

extern "C" int elr_dedup_plan(const int64_t* ids, int64_t n, int key_bits, int64_t* uniq, int64_t* inverse,
                              int64_t* n_unique, void* plan, int64_t plan_bytes, int64_t D, void* stream) {
  using namespace elr;
  if (!dedup_sizes_ok(n) || key_bits < 1 || key_bits > 64 || D < 1) return ELR_EINVAL;
  if (n == 0) return ELR_OK;
  if (!ids || !uniq || !n_unique || !plan) return ELR_EINVAL;
  DedupScratch S;
  if (plan_bytes < dedup_scratch_bytes(n, D, &S, plan)) return ELR_ECAPACITY;
  hipStream_t st = (hipStream_t)stream;
  const int cur = key_bits <= 32 ? dedup_core<uint32_t>(ids, n, key_bits, S, uniq, inverse, n_unique, st)
                                 : dedup_core<uint64_t>(ids, n, key_bits, S, uniq, inverse, n_unique, st);
  if (cur != plan_result_buffer(key_bits)) return ELR_EINVAL;
  chunk_plan(n, S, st);
  return launch_status();
}

extern "C" int elr_dedup_plan_fields(const int64_t* ids, int64_t nrows, int64_t nfields, const int64_t* field_lo,
                                     int key_bits, int64_t* uniq, int64_t* inverse, int64_t* n_unique, void* plan,
                                     int64_t plan_bytes, int64_t D, void* stream) {
  using namespace elr;
  if (nrows < 0 || nfields < 1 || !field_lo || key_bits < 1 || key_bits > 64 || D < 1) return ELR_EINVAL;
  if (nrows > 0 && nfields > ((int64_t(1) << 31) - 1) / nrows) return ELR_EINVAL;
  const int64_t n = nrows * nfields;
  if (n == 0) return ELR_OK;
  if (field_lo[0] < 0) return ELR_EINVAL;
  for (int64_t c = 0; c < nfields; ++c)
    if (field_lo[c + 1] < field_lo[c]) return ELR_EINVAL;
  if (nrows > kFieldRows || nfields > kFieldMax || n <= kAtenSmall)
    return elr_dedup_plan(ids, n, key_bits, uniq, inverse, n_unique, plan, plan_bytes, D, stream);
  for (int64_t c = 0; c < nfields; ++c)
    if (field_lo[c + 1] - field_lo[c] > kFieldSpanMax)
      return elr_dedup_plan(ids, n, key_bits, uniq, inverse, n_unique, plan, plan_bytes, D, stream);
  if (!ids || !uniq || !n_unique || !plan) return ELR_EINVAL;
  DedupScratch S;
  if (plan_bytes < dedup_scratch_bytes(n, D, &S, plan)) return ELR_ECAPACITY;
  static_assert(2 * kFieldMax <= kRadixMaxBins, "the per-field counts fit in the first histogram's space");
  FieldBounds fb;
  for (int64_t c = 0; c <= nfields; ++c) fb.lo[c] = field_lo[c];
  hipStream_t st = (hipStream_t)stream;
  int32_t* sv = S.vals[plan_result_buffer(key_bits)];
  k_field_keys<<<dim3((unsigned)cdiv(nrows, kFieldKeyRows), (unsigned)nfields), 256, 0, st>>>(
      ids, nrows, (int)nfields, fb, (uint32_t*)S.keys[1]);
  k_field_sort<<<(unsigned)nfields, kFieldThreads, 0, st>>>((const uint32_t*)S.keys[1], nrows, (int)nfields, fb,
                                                            (uint32_t*)S.keys[0], sv, S.hist, S.d_tot + 2);
  k_field_apply<<<(unsigned)nfields, kFieldThreads, 0, st>>>((const uint32_t*)S.keys[0], sv, nrows, (int)nfields, fb,
                                                             S.hist, S.d_tot, n_unique, uniq, S.seg_start,
                                                             S.seg_occ0, inverse, S.chunk_off, S.chunk_seg,
                                                             S.hot_list);
  return launch_status();
}

namespace elr {

int seg_partials_prep(const float* grad, int64_t n, int64_t D, int key_bits, const void* plan, int64_t plan_bytes,
                      SegPartialsLaunch& out) {
  out.blocks = 0;
  if (!dedup_sizes_ok(n) || D < 1 || key_bits < 1 || key_bits > 64) return ELR_EINVAL;
  if (n == 0) return ELR_OK;
  if (!grad || !plan) return ELR_EINVAL;
  if (D > 512) return ELR_EUNSUPPORTED;
  DedupScratch S;
  if (plan_bytes < dedup_scratch_bytes(n, D, &S, const_cast<void*>(plan))) return ELR_ECAPACITY;
  if (win_shift_for(n)) return ELR_OK;
  out.a = seg_partials_of<1>(grad, D, S.vals[plan_result_buffer(key_bits)], S);
  out.blocks = seg_partials_blocks(n);
  return ELR_OK;
}

// elr_segment_sum_plan, with or without the partial chunks (computed earlier by elr_plan_classify_seg).
static int segment_sum_plan(const float* grad, int64_t n, int64_t D, int key_bits, const void* plan,
                            int64_t plan_bytes, const int64_t* perm, float* out, int64_t out_rows, void* stream,
                            bool partials) {
  if (!dedup_sizes_ok(n) || D < 1 || key_bits < 1 || key_bits > 64 || out_rows < 0) return ELR_EINVAL;
  if (n == 0) return ELR_OK;
  if (!grad || !plan || !out) return ELR_EINVAL;
  if (D > 512) return ELR_EUNSUPPORTED;
  DedupScratch S;
  if (plan_bytes < dedup_scratch_bytes(n, D, &S, const_cast<void*>(plan))) return ELR_ECAPACITY;
  hipStream_t st = (hipStream_t)stream;
  const AdamScalars none{};
  const int rc = seg_reduce_d<0>(grad, D, S.vals[plan_result_buffer(key_bits)], S, perm, n, out, out_rows, none, st,
                                 partials);
  return rc != ELR_OK ? rc : launch_status();
}

template <int VPL>
static void seg_final_with(const float* grad, const int32_t* sv, DedupScratch& S, const int64_t* perm, int64_t n,
                           float* out, int64_t nrows, const DirLstepsHits& first, int64_t nb1, hipStream_t st) {
  const int64_t hb = n / kHotLen + 1;
  const SegFinalWpr<VPL, 0> f{grad, sv, S.seg_start, S.seg_occ0, perm, S.chunk_off, S.parts, S.d_tot, 0,
                              S.hot_list, S.d_tot + 2, hb, out, nrows, AdamScalars{}};
  launch2(first, nb1, f, hb + cdiv(n, 4 * kSegPerWave), st);
}

int segment_sum_plan_final_with(const float* grad, int64_t n, int64_t D, int key_bits, const void* plan,
                                int64_t plan_bytes, const int64_t* perm, float* out, int64_t out_rows,
                                const DirLstepsHits& first, int64_t nb1, void* stream) {
  if (!dedup_sizes_ok(n) || D < 1 || key_bits < 1 || key_bits > 64 || out_rows < 0 || nb1 < 0) return ELR_EINVAL;
  if (n == 0 || !grad || !plan || !out) return ELR_EUNSUPPORTED;
  // the wave-per-row final kernel in one launch: aligned rows of 64, 128, 256 or 512, the sort path, at most one
  // launch's worth of segments (seg_reduce_wpr)
  if (!aligned16(grad) || !aligned16(out) || win_shift_for(n) || n > kOneShotBlocks * 4 * kSegPerWave)
    return ELR_EUNSUPPORTED;
  DedupScratch S;
  if (plan_bytes < dedup_scratch_bytes(n, D, &S, const_cast<void*>(plan))) return ELR_ECAPACITY;
  const int32_t* sv = S.vals[plan_result_buffer(key_bits)];
  hipStream_t st = (hipStream_t)stream;
  switch (D) {
    case 64: seg_final_with<1>(grad, sv, S, perm, n, out, out_rows, first, nb1, st); break;
    case 128: seg_final_with<2>(grad, sv, S, perm, n, out, out_rows, first, nb1, st); break;
    case 256: seg_final_with<4>(grad, sv, S, perm, n, out, out_rows, first, nb1, st); break;
    case 512: seg_final_with<8>(grad, sv, S, perm, n, out, out_rows, first, nb1, st); break;
    default: return ELR_EUNSUPPORTED;
  }
  return launch_status();
}

}  // namespace elr

extern "C" int elr_segment_sum_plan(const float* grad, int64_t n, int64_t D, int key_bits, const void* plan,
                                    int64_t plan_bytes, const int64_t* perm, float* out, int64_t out_rows,
                                    void* stream) {
  return elr::segment_sum_plan(grad, n, D, key_bits, plan, plan_bytes, perm, out, out_rows, stream, true);
}

extern "C" int elr_segment_sum_plan_final(const float* grad, int64_t n, int64_t D, int key_bits, const void* plan,
                                          int64_t plan_bytes, const int64_t* perm, float* out, int64_t out_rows,
                                          void* stream) {
  return elr::segment_sum_plan(grad, n, D, key_bits, plan, plan_bytes, perm, out, out_rows, stream, false);
}

extern "C" int elr_adam_dedup_plan(float* state, int64_t C, const int64_t* uniq, const float* grad, int64_t n,
                                   int64_t D, int key_bits, const void* plan, int64_t plan_bytes, const float sc[8],
                                   void* stream) {
  using namespace elr;
  if (!dedup_sizes_ok(n) || D < 1 || C < 0 || key_bits < 1 || key_bits > 64 || !sc) return ELR_EINVAL;
  if (n == 0) return ELR_OK;
  if (!state || !uniq || !grad || !plan) return ELR_EINVAL;
  if (D > 512) return ELR_EUNSUPPORTED;
  DedupScratch S;
  if (plan_bytes < dedup_scratch_bytes(n, D, &S, const_cast<void*>(plan))) return ELR_ECAPACITY;
  hipStream_t st = (hipStream_t)stream;
  const int rc = seg_reduce_d<1>(grad, D, S.vals[plan_result_buffer(key_bits)], S, uniq, n, state, C,
                                 make_scalars(sc), st);
  return rc != ELR_OK ? rc : launch_status();
}

// ---- duplicate-id Adam that allocates nothing ------------------------------------------------------------------
// elr_adam_dedup with its scratch in a file-scope device array instead of a caller buffer, for callers that cannot
// allocate device memory (code under graph capture, tight serving loops).  The array (ELR_NOALLOC_SCRATCH_BYTES)
// exists once per GPU the library runs on, for the life of the process.  In host code `scratch` names only a
// host-side stand-in; the device address is obtained once per device with hipGetSymbolAddress, with that device
// current, and only that address is handed to kernels.  Every kernel writes the parts of the scratch it later
// reads (the hot-segment counter is zeroed by the segment kernel itself), so nothing needs clearing between calls.
// All calls on one GPU share its array: calls that overlap in time on one GPU (two streams, two host threads) race.
#include <atomic>
#include <mutex>

namespace elr {
constexpr int kNoAllocMaxDevices = 64;
std::atomic<void*> g_noalloc_ptr[kNoAllocMaxDevices];
std::mutex g_noalloc_mu;
}  // namespace elr

static __device__ __align__(256) unsigned char scratch[ELR_NOALLOC_SCRATCH_BYTES];

// Device address of `scratch` on the current device (resolved on the first call per device).  A stream of another
// device is refused (ELR_EINVAL): its kernels would be handed this device's address.
static int noalloc_scratch(void** out, hipStream_t stream) {
  using namespace elr;
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kNoAllocMaxDevices) return ELR_EUNSUPPORTED;
  if (stream) {
    hipDevice_t sdev = -1;
    e = hipStreamGetDevice(stream, &sdev);
    if (e != hipSuccess) return (int)e;
    if ((int)sdev != dev) return ELR_EINVAL;
  }
  void* p = g_noalloc_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> g(g_noalloc_mu);
    p = g_noalloc_ptr[dev].load(std::memory_order_relaxed);
    if (!p) {
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess) return (int)e;
      if (!p) return ELR_EINVAL;
      g_noalloc_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return ELR_OK;
}

extern "C" int elr_adam_dedup_noalloc(float* state, int64_t C, const int64_t* ids, const float* grad, int64_t n,
                                      int64_t D, const float sc[8], void* stream) {
  using namespace elr;
  if (!dedup_sizes_ok(n) || D < 1 || C < 0 || !sc) return ELR_EINVAL;
  if (n == 0) return ELR_OK;
  if (!state || !ids || !grad) return ELR_EINVAL;
  if (D > 512) return ELR_EUNSUPPORTED;
  if (dedup_scratch_bytes(n, D, nullptr, nullptr) > (int64_t)ELR_NOALLOC_SCRATCH_BYTES) return ELR_ECAPACITY;
  void* base = nullptr;
  const int rc = noalloc_scratch(&base, static_cast<hipStream_t>(stream));
  if (rc != ELR_OK) return rc;
  return elr_adam_dedup(state, C, ids, grad, n, D, sc, base, (int64_t)ELR_NOALLOC_SCRATCH_BYTES, stream);
}
