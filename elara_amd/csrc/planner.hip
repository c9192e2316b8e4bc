// Planner classification of one ELARA step (srm2/elara.py:214-267, the part before the class counts go to the host):
// three launches in place of the reference planner's chain of elementwise torch ops, bincount and stable argsorts.
//
//   unique rows u[i] of the batch: slot sl = slot_of[u], hit = sl >= 0, in_next = u appears in one of the next
//     batches, admit = !hit && (ttl: last_seen[u] > s; carry: in_next), c = code[u], app = c < kthr[table_of(u)],
//     and the class
//       hit -> HIT;  c == 0 (N) -> admit ? NADM : app ? NAPP : NCMP;  1 <= c <= K (L) -> LADM / LAPP / LCMP;
//       otherwise (M) -> admit ? FADM : want_T ? FNADM : S                              (elara.py:244-258)
//   dynamic pool slots d = dyn[j] (row r = slot_row[d]): protected when r appears in one of the next batches
//     (the slot holds a row the pipeline needs, elara.py:227-229), expired when last_seen[r] <= s (ttl: the row's
//     TTL is over) or always (carry) (elara.py:231-233); class 0 = expired and unprotected, 1 = unprotected
//     (preemptible), 2 = protected.
//
// Outputs: the positions of u sorted stably by class rank (`order`, and its inverse `rank`), the dynamic slots
// partitioned stably by class ([class 0 | class 1 | class 2] and [class 0 | classes 1, 2 in dyn order], so that the
// evicted and kept slots of both the plain and the preempting plan are contiguous slices), per-position flags, slots
// and codes, and a small block of counts for the host: 10 class counts, the 3 dynamic-slot counts, mat_top and
// log_top.
//
// A dynamic slot is protected in the reference when slot_of[un] == d for a row un of the next batches; every
// occupied dynamic slot satisfies slot_of[slot_row[d]] == d, so the test here is the membership of slot_row[d] in
// the (ascending, unique) next batches: by binary search, or with one load from the ring of loaded batches
// (next_bits) when the caller keeps one.
#include "elr_admit_dev.h"
#include "elr_desc.h"
#include "elr_seg_dev.h"
#include "elr_scan.h"

namespace elr {

constexpr int kPlanBlock = 256;
constexpr int kNumCls = 10;     // HIT, NADM, NAPP, NCMP, LADM, LAPP, LCMP, FADM, FNADM, S
constexpr int kDynCh = 4;       // expired, preemptible, protected, not expired (= preemptible + protected)

enum : int { kHit = 0, kNAdm, kNApp, kNCmp, kLAdm, kLApp, kLCmp, kFAdm, kFNAdm, kS };

// Position of each class in `order` (the class rank): hits, then the admitted N, L and F rows, the N and L appends,
// the N and L compactions, the transient F rows and the S rows.  Each group the executor treats alike -- the
// admissions (ascending N, L, F as the reference concatenates them, srm2/elara.py:345-350), the appends and the
// compactions (srm2/elara.py:379-386) -- is then one contiguous range.
__constant__ int kRankOf[kNumCls] = {0, 1, 4, 6, 2, 5, 7, 3, 8, 9};
__constant__ int kClsOfRank[kNumCls] = {kHit, kNAdm, kLAdm, kFAdm, kNApp, kLApp, kNCmp, kLCmp, kFNAdm, kS};

__device__ __forceinline__ bool sorted_has(const int64_t* __restrict__ a, int64_t n, int64_t x) {
  int64_t lo = 0, hi = n;   // first index with a[idx] >= x
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (a[mid] < x) lo = mid + 1;
    else hi = mid;
  }
  return lo < n && a[lo] == x;
}

__device__ __forceinline__ bool in_next(const elr_plan_in& p, int64_t r) {
  if (p.next_bits) return (p.next_bits[r] & p.next_mask) != 0;
  bool f = false;
#pragma unroll
  for (int k = 0; k < 4; ++k)   // constant indices keep the lists' pointers in registers (nnext <= 4)
    if (k < p.nnext) f = f || sorted_has(p.next[k], p.n_next[k], r);
  return f;
}

// Table of row r: the last t with toff[t] <= r (searchsorted(toff, r, right=True) - 1, srm2/elara_dir.cpp:46-48).
__device__ __forceinline__ int64_t table_of(const int64_t* __restrict__ toff, int64_t T, int64_t r) {
  int64_t lo = 0, hi = T;   // first index with toff[idx] > r
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (toff[mid] <= r) lo = mid + 1;
    else hi = mid;
  }
  return lo - 1;
}

struct RowClass {
  int cls, flags, sl, c;
};

__device__ __forceinline__ bool row_ok(const elr_plan_in& p, int64_t r) { return p.R <= 0 || (r >= 0 && r < p.R); }

// The batch's row count and the dynamic slot count: the arguments, or the device counts they bound.
__device__ __forceinline__ int64_t rows_n(const elr_plan_in& p) {
  if (!p.n_dev) return p.n;
  const int64_t v = *p.n_dev;
  return v < 0 ? 0 : (v < p.n ? v : p.n);
}
__device__ __forceinline__ int64_t dyn_n(const elr_plan_in& p) {
  if (!p.nd_dev) return p.nd;
  const int64_t v = *p.nd_dev;
  return v < 0 ? 0 : (v < p.nd ? v : p.nd);
}

__device__ __forceinline__ RowClass classify_row(const elr_plan_in& p, int64_t r) {
  RowClass o;
  if (!row_ok(p, r)) {   // out of range: class S with no slot, which the executor's copies and updates skip
    o.cls = kS;
    o.flags = 0;
    o.sl = -1;
    o.c = p.K + 1;
    return o;
  }
  o.sl = p.slot_of[r];
  const bool hit = o.sl >= 0;
  const bool nxt = in_next(p, r);
  const bool admit = !hit && (p.carry ? nxt : (int64_t)p.last_seen[r] > p.s);
  o.c = p.code[r];
  const int64_t t = table_of(p.toff, p.T, r);
  const int thr = (t >= 0 && t < p.T) ? (int)p.kthr[t] : 0;
  const bool isN = o.c == 0, isL = o.c >= 1 && o.c <= p.K, app = o.c < thr;
  int k;
  if (hit) k = kHit;
  else if (isN) k = admit ? kNAdm : (app ? kNApp : kNCmp);
  else if (isL) k = admit ? kLAdm : (app ? kLApp : kLCmp);
  else if (admit || p.want_t) k = admit ? kFAdm : kFNAdm;
  else k = kS;
  o.cls = k;
  o.flags = (hit ? ELR_PLAN_HIT : 0) | (isN ? ELR_PLAN_N : 0) | (isL ? ELR_PLAN_L : 0) | (app ? ELR_PLAN_APP : 0) |
            (admit ? ELR_PLAN_ADMIT : 0) | (nxt ? ELR_PLAN_NEXT : 0);
  return o;
}

__device__ __forceinline__ int dyn_class(const elr_plan_in& p, int64_t d) {
  const int64_t r = p.slot_row[d];
  if (r >= 0 && !row_ok(p, r)) return 1;   // a slot holding an out-of-range row: unprotected, not expired
  const bool prot = r >= 0 && in_next(p, r);
  if (prot) return 2;
  const bool expired = p.carry || r < 0 || (int64_t)p.last_seen[r] <= p.s;
  return expired ? 0 : 1;
}

// Wave ranks and block counts of NCH classes: for element class k (or -1 for none) the rank among the block's
// earlier elements of the same class (stable: thread order), and every class's block total in tot.
template <int NCH>
__device__ __forceinline__ int block_class_rank(int k, int (&tot)[NCH]) {
  constexpr int NW = kPlanBlock / 64;
  __shared__ int wc[NW][NCH];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int rank_w = 0;
#pragma unroll
  for (int q = 0; q < NCH; ++q) {
    const uint64_t m = __builtin_amdgcn_ballot_w64(k == q);
    if (k == q) rank_w = __builtin_popcountll(m & lanemask_lt());
    if (lane == 0) wc[w][q] = __builtin_popcountll(m);
  }
  __syncthreads();
  int before = 0;
#pragma unroll
  for (int q = 0; q < NCH; ++q) {
    int t = 0;
#pragma unroll
    for (int v = 0; v < NW; ++v) {
      const int x = wc[v][q];
      if (q == k && v < w) before += x;
      t += x;
    }
    tot[q] = t;
  }
  return before + rank_w;
}

// Pass 1: classify and count per block.  Blocks [0, nbu) take the unique rows, blocks [nbu, nbu + nbd) the dynamic
// slots.  Block counts go channel-major: bu[c * nbu + b], bd[c * nbd + b]; bbad[b]: the block's rows outside [0, R).
struct PlanCount {
  elr_plan_in p;
  elr_plan_out o;
  int64_t nbu, nbd;
  int64_t* bu;
  int64_t* bd;
  int64_t* bbad;
  __device__ void operator()(int64_t b, int64_t) const;
};

__device__ void PlanCount::operator()(int64_t b, int64_t) const {
  if (b < nbu) {
    __shared__ int nbad;
    if (threadIdx.x == 0) nbad = 0;
    const int64_t i = b * kPlanBlock + threadIdx.x;
    int k = -1;
    bool bad = false;
    if (i < rows_n(p)) {
      const int64_t r = p.u[i];
      const RowClass rc = classify_row(p, r);
      bad = !row_ok(p, r);
      k = kRankOf[rc.cls];
      o.cls[i] = (int8_t)rc.cls;
      o.flags[i] = (uint8_t)rc.flags;
      o.sl[i] = rc.sl;
      o.c[i] = (int8_t)rc.c;
    }
    int tot[kNumCls];
    block_class_rank<kNumCls>(k, tot);   // synchronises the block: nbad is zeroed before the adds below
    const uint64_t mb = __builtin_amdgcn_ballot_w64(bad);
    if ((threadIdx.x & 63) == 0 && mb) atomicAdd(&nbad, (int)__builtin_popcountll(mb));
    if (threadIdx.x < kNumCls) bu[threadIdx.x * nbu + b] = tot[threadIdx.x];
    __syncthreads();
    if (threadIdx.x == 0) bbad[b] = nbad;
  } else {
    const int64_t bb = b - nbu;
    const int64_t j = bb * kPlanBlock + threadIdx.x;
    const int k = j < dyn_n(p) ? dyn_class(p, p.dyn[j]) : -1;
    int tot[3];
    block_class_rank<3>(k, tot);
    if (threadIdx.x == 0) {
      bd[0 * nbd + bb] = tot[0];
      bd[1 * nbd + bb] = tot[1];
      bd[2 * nbd + bb] = tot[2];
      bd[3 * nbd + bb] = tot[1] + tot[2];
    }
  }
}

// ---- the device-driven step's resolution (elr_plan_step) ------------------------------------------------------
constexpr int kRW = kScanBlock / 64;   // waves of the resolving block

// The overflow path (srm2/elara.py:246-256) by the resolving block: the admitted rows are ordered as the reference's
// stable sort of pri = (admitted and in the next batches: 0, admitted otherwise: 2) orders them, the last `need` of
// them are not admitted after all and take the class they get without admission (their cls is rewritten), and the
// class-rank block offsets and totals are recomputed into bu2 and tot2 (exclusive offsets per block of kPlanBlock
// rows, as the scan launch makes them).  Returns, to thread 0, how many dropped rows appear in the next batches.
__device__ int64_t plan_overflow(const elr_plan_in& p, const elr_plan_out& o, int64_t n, int64_t nbu, int64_t n_adm,
                                 int64_t need, int64_t* __restrict__ bu2, int64_t* __restrict__ tot2) {
  __shared__ int64_t a0_w[kRW];
  __shared__ int wsum[kRW][3];
  __shared__ int wcls[kRW][kNumCls];
  __shared__ int64_t run[kNumCls + 3];   // class runs, then admitted rows in / not in the next batches, carry drops
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  // admitted rows that appear in the next batches: they come first in the reference's priority order
  int64_t a0 = 0;
  for (int64_t i = threadIdx.x; i < n; i += kScanBlock) {
    const int f = o.flags[i];
    a0 += ((f & ELR_PLAN_ADMIT) && (f & ELR_PLAN_NEXT)) ? 1 : 0;
  }
  a0 = wave_incl_scan<int64_t>(a0);
  if (lane == 63) a0_w[w] = a0;
  if (threadIdx.x < kNumCls + 3) run[threadIdx.x] = 0;
  __syncthreads();
  int64_t A0 = 0;
  for (int v = 0; v < kRW; ++v) A0 += a0_w[v];
  const int64_t T = n_adm - need;   // admitted rows at priority rank T and beyond are dropped
  for (int64_t c0 = 0; c0 < n; c0 += kScanBlock) {
    const int64_t i = c0 + threadIdx.x;
    const bool valid = i < n;
    const int f = valid ? o.flags[i] : 0;
    const bool adm = (f & ELR_PLAN_ADMIT) != 0, nx = (f & ELR_PLAN_NEXT) != 0;
    const uint64_t m_nx = __builtin_amdgcn_ballot_w64(adm && nx), m_x = __builtin_amdgcn_ballot_w64(adm && !nx);
    if (lane == 0) {
      wsum[w][0] = __builtin_popcountll(m_nx);
      wsum[w][1] = __builtin_popcountll(m_x);
    }
    __syncthreads();
    int64_t bnx = run[kNumCls], bx = run[kNumCls + 1];
    for (int v = 0; v < w; ++v) {
      bnx += wsum[v][0];
      bx += wsum[v][1];
    }
    const int64_t q_nx = bnx + __builtin_popcountll(m_nx & lanemask_lt());
    const int64_t q_x = bx + __builtin_popcountll(m_x & lanemask_lt());
    const bool drop = adm && (nx ? q_nx >= T : A0 + q_x >= T);
    int k = valid ? (int)o.cls[i] : -1;
    if (drop) {
      k = (f & ELR_PLAN_N) ? ((f & ELR_PLAN_APP) ? kNApp : kNCmp)
          : (f & ELR_PLAN_L) ? ((f & ELR_PLAN_APP) ? kLApp : kLCmp)
          : (p.want_t ? kFNAdm : kS);
      o.cls[i] = (int8_t)k;
    }
    const uint64_t m_cd = __builtin_amdgcn_ballot_w64(drop && nx);
    const int rk = k >= 0 ? kRankOf[k] : -1;
#pragma unroll
    for (int q = 0; q < kNumCls; ++q) {
      const uint64_t mq = __builtin_amdgcn_ballot_w64(rk == q);
      if (lane == 0) wcls[w][q] = __builtin_popcountll(mq);
    }
    if (lane == 0) wsum[w][2] = __builtin_popcountll(m_cd);
    __syncthreads();
    if (threadIdx.x < kNumCls) {
      const int q = threadIdx.x;
      for (int sb = 0; sb < kScanBlock / kPlanBlock; ++sb) {
        const int64_t blk = c0 / kPlanBlock + sb;
        if (blk < nbu) bu2[(int64_t)q * nbu + blk] = run[q];
        for (int v = sb * (kPlanBlock / 64); v < (sb + 1) * (kPlanBlock / 64); ++v) run[q] += wcls[v][q];
      }
    } else if (threadIdx.x < kNumCls + 3) {
      const int q = threadIdx.x - kNumCls;
      int64_t add = 0;
      for (int v = 0; v < kRW; ++v) add += wsum[v][q];
      run[threadIdx.x] += add;
    }
    __syncthreads();
  }
  if (threadIdx.x < kNumCls) tot2[threadIdx.x] = run[threadIdx.x];
  __syncthreads();
  return run[kNumCls + 2];
}

// The resolution of one step by the last block of the scan launch: everything the host planner decides from the
// class counts (srm2/elara.py:234-267, 345-347; the capacity bound and the rows out of range of this build), written
// into the step descriptor, with the dynamic pool's counters and the statistics advanced in the control state.
// One thread decides; it loads everything it reads at once (a single round trip) and the stores go out together.
__device__ void plan_resolve(const elr_plan_in& p, const elr_plan_out& o, const elr_plan_ctl& c, int64_t nbu,
                             const int64_t* __restrict__ tot, int64_t* __restrict__ bu2,
                             int64_t* __restrict__ tot2) {
  __shared__ int64_t sh[4];
  int64_t* S = c.state;
  int64_t* Dd = c.desc;
  const int64_t n = rows_n(p), nd = dyn_n(p);
  constexpr int NT = kNumCls + kDynCh + 1;
  int64_t t[NT], st[kNumStats], n_free = 0, err = 0, mat_top = 0, log_top = 0, live = 0;
  if (threadIdx.x == 0) {
#pragma unroll
    for (int q = 0; q < NT; ++q) t[q] = tot[q];   // by rank, then expired, preemptible, protected, not, bad
#pragma unroll
    for (int q = 0; q < kNumStats; ++q) st[q] = S[kSStats + q];
    n_free = S[kSNFree];
    err = S[kSErr];
    mat_top = p.mat_top ? *p.mat_top : 0;
    log_top = p.log_top ? *p.log_top : 0;
    live = p.live ? *p.live : 0;
    const int64_t n_exp = t[kNumCls], n_pre = t[kNumCls + 1];
    const int64_t n_adm = t[1] + t[2] + t[3];   // ranks NADM, LADM, FADM
    int64_t need = n_adm - (n_free + n_exp);
    const int64_t take = (need > 0 && nd > n_exp) ? (need < n_pre ? need : n_pre) : 0;
    need -= take;
    sh[0] = need > 0 ? need : 0;
    sh[1] = take;
    sh[2] = n_adm;
  }
  __syncthreads();
  const int64_t need = sh[0];
  const int64_t carry_drop = need > 0 ? plan_overflow(p, o, n, nbu, sh[2], need, bu2, tot2) : 0;
  if (threadIdx.x != 0) return;
  const int64_t take = sh[1];
  if (need > 0) {   // the reclassified totals (the dynamic-slot ones stay), for the scatter launch too
#pragma unroll
    for (int q = 0; q < kNumCls; ++q) t[q] = tot2[q];
#pragma unroll
    for (int q = kNumCls; q < NT; ++q) tot2[q] = t[q];
  }
  int64_t b[kNumCls + 1];
  b[0] = 0;
#pragma unroll
  for (int q = 0; q < kNumCls; ++q) b[q + 1] = b[q] + t[q];
  const int64_t nh = t[0], nNa = t[1], nLa = t[2], nFa = t[3], nNp = t[4], nLp = t[5], nNc = t[6], nLc = t[7],
                nFn = t[8], nS = t[9];
  const int64_t n_exp = t[kNumCls], bad = t[kNumCls + kDynCh];
  const int64_t nev = n_exp + take;
  const int64_t keep_off = take ? nev : nd + n_exp, nkeep = nd - (take ? nev : n_exp);
  const int64_t n_adm = nNa + nLa + nFa;
  const int64_t K = p.K;
  // the step's allocations at most: a MAT slot per eviction and compaction, a log entry per append and K per
  // eviction, the latter from the free stack first (n_lfree = log_top - live)
  const int64_t mt_hi = mat_top + nev + nNc + nLc;
  const int64_t lneed = nev * K + nNp + nLp - (log_top - live);
  const int64_t lt_hi = log_top + (lneed > 0 ? lneed : 0);
  const int64_t e = (bad > 0 ? ELR_STEP_ERR_ROWS : 0) | ((mt_hi > c.mat_cap || lt_hi > c.log_cap) ? ELR_STEP_ERR_CAPACITY : 0);
  if (!err && e) {
    S[kSErr] = e;
    S[kSErrStep] = p.s;
    S[kSErrA] = bad;
    S[kSErrB] = mt_hi;
    S[kSErrC] = lt_hi;
  }
  const bool skip = (err | e) != 0;
  // every descriptor word is written once (the words a skipped step leaves are zero)
  Dd[kDOverflow] = need;   // the scatter launch takes bu2 / tot2 whenever the overflow path ran
  Dd[kDNRows] = n;
  Dd[kDNd] = nd;
  Dd[kDMatHi] = mt_hi;
  Dd[kDLogHi] = lt_hi;
  Dd[kDSkip] = skip ? 1 : 0;
#pragma unroll
  for (int q = 0; q <= kNumCls; ++q) Dd[kDB + q] = skip ? 0 : b[q];
  const int64_t words[][2] = {{kDNev, nev},
                              {kDKeepOff, keep_off},
                              {kDNKeep, nkeep},
                              {kDNFree, n_free},
                              {kDNAdm, n_adm},
                              {kDLazy, nNa + nLa},
                              {kDNL, nLa + nLp + nLc},
                              {kDNLa, nLa},
                              {kDNLp, nLp},
                              {kDNa, nNp + nLp},
                              {kDNc, nNc + nLc},
                              {kDNr, c.triton ? nev : 0},
                              {kDNh, nh},
                              {kDW0, b[1]},
                              {kDNw, b[kNumCls - 1] - b[1]},
                              {kDNs, nS},
                              {kDNTail, b[kNumCls - 1] - b[6]},
                              {kDTake, take},
                              {kDBarrier, carry_drop > 0 ? 1 : 0}};
  constexpr int kNamed = sizeof(words) / sizeof(words[0]);
  static_assert(kDB + kNumCls + 1 + kNamed + 6 <= kDWords, "descriptor words");
#pragma unroll
  for (int q = 0; q < kNamed; ++q) Dd[words[q][0]] = skip ? 0 : words[q][1];
  if (skip) return;
  S[kSNFree] = n_free + nev - n_adm;
  S[kSNd] = nkeep + n_adm;
  const int64_t add[kNumStats] = {nh, nNa + nNp + nNc, nLa + nLp + nLc, nFa + nFn, nS, n_adm, nev, take, need,
                                  nNc + nLc, nNp + nLp, carry_drop > 0 ? 1 : 0, 1};
#pragma unroll
  for (int q = 0; q < kNumStats; ++q) S[kSStats + q] = st[q] + add[q];
}

// The host counts of pass 2 (class totals by class, the dynamic-slot totals, the rows outside [0, R) and the arena
// tops at plan time), by the thread that holds channel c's total.
__device__ __forceinline__ void plan_counts_out(const elr_plan_in& p, const elr_plan_out& o, int c, int64_t total) {
  if (c < kNumCls) o.counts[kClsOfRank[c]] = total;
  else if (c < kNumCls + 3) o.counts[c] = total;
  else if (c == kNumCls + kDynCh) o.counts[16] = total;
  if (c == 0) {
    o.counts[13] = p.mat_top ? *p.mat_top : 0;
    o.counts[14] = p.log_top ? *p.log_top : 0;
    o.counts[15] = p.live ? *p.live : 0;
  }
}

// Pass 2 (one block per channel): block offsets per class; class totals and the host counts.
__global__ __launch_bounds__(kScanBlock) void k_plan_scan(elr_plan_in p, elr_plan_out o, int64_t nbu, int64_t nbd,
                                                          int64_t* __restrict__ bu, int64_t* __restrict__ bd,
                                                          int64_t* __restrict__ bbad, int64_t* __restrict__ tot) {
  // one block per channel: the kNumCls class channels, the kDynCh dynamic-slot channels, then the rows outside
  // [0, R), which the caller raises on instead of letting the step skip them
  const int c = blockIdx.x;
  if (c < kNumCls) scan_channels_block(bu + (int64_t)c * nbu, nbu, 1, tot + c);
  else if (c < kNumCls + kDynCh) scan_channels_block(bd + (int64_t)(c - kNumCls) * nbd, nbd, 1, tot + c);
  else scan_channels_block(bbad, nbu, 1, tot + c);
  if (threadIdx.x == 0) plan_counts_out(p, o, c, tot[c]);   // the thread that stored tot[c]
}

// Pass 2 of the device-driven step, in one block: wave c scans channel c (its loads kScanQ * 64 entries at a time,
// all in flight together), then the same block resolves the step (plan_resolve) -- no block waits on another and
// no device-wide fence is needed.  Only the blocks that hold live rows or slots are scanned (the scatter reads no
// others).
constexpr int kPlanCh = kNumCls + kDynCh + 1;
constexpr int kScanQ = 8;
static_assert(kPlanCh <= kScanBlock / 64, "one wave per channel");

__global__ __launch_bounds__(kScanBlock) void k_plan_scan_dev(elr_plan_in p, elr_plan_out o, int64_t nbu,
                                                              int64_t nbd, int64_t* __restrict__ bu,
                                                              int64_t* __restrict__ bd, int64_t* __restrict__ bbad,
                                                              int64_t* __restrict__ tot, elr_plan_ctl ctl,
                                                              int64_t* __restrict__ bu2, int64_t* __restrict__ tot2) {
  __shared__ int64_t stot[kPlanCh];
  const int lane = threadIdx.x & 63, c = threadIdx.x >> 6;
  if (c < kPlanCh) {
    const bool rowch = c < kNumCls || c == kNumCls + kDynCh;
    const int64_t live = ((rowch ? rows_n(p) : dyn_n(p)) + kPlanBlock - 1) / kPlanBlock, cap = rowch ? nbu : nbd;
    const int64_t n = live < cap ? live : cap;
    int64_t* __restrict__ ch = c < kNumCls             ? bu + (int64_t)c * nbu
                               : c < kNumCls + kDynCh ? bd + (int64_t)(c - kNumCls) * nbd
                                                      : bbad;
    int64_t carry = 0;
    for (int64_t b0 = 0; b0 < n; b0 += 64 * kScanQ) {
      int x[kScanQ];   // a block's count is at most kPlanBlock
#pragma unroll
      for (int q = 0; q < kScanQ; ++q) {
        const int64_t b = b0 + q * 64 + lane;
        x[q] = b < n ? (int)ch[b] : 0;
      }
#pragma unroll
      for (int q = 0; q < kScanQ; ++q) {
        const int64_t b = b0 + q * 64 + lane;
        const int inc = wave_incl_scan<int>(x[q]);
        if (b < n) ch[b] = carry + inc - x[q];
        carry += __shfl(inc, 63, 64);
      }
    }
    if (lane == 0) {
      tot[c] = carry;
      stot[c] = carry;
      plan_counts_out(p, o, c, carry);
    }
  }
  __syncthreads();
  plan_resolve(p, o, ctl, nbu, stot, bu2, tot2);
}

// Pass 3: stable scatter by class.
__global__ __launch_bounds__(kPlanBlock) void k_plan_scatter(elr_plan_in p, elr_plan_out o, int64_t nbu, int64_t nbd,
                                                             const int64_t* __restrict__ bu_in,
                                                             const int64_t* __restrict__ bd,
                                                             const int64_t* __restrict__ tot_in,
                                                             const int64_t* __restrict__ desc,
                                                             const int64_t* __restrict__ bu2,
                                                             const int64_t* __restrict__ tot2) {
  const int64_t b = blockIdx.x;
  // after the device-driven overflow path: its reclassified offsets and totals
  const bool ovf = desc && desc[kDOverflow] > 0;
  const int64_t* __restrict__ bu = ovf ? bu2 : bu_in;
  const int64_t* __restrict__ tot = ovf ? tot2 : tot_in;
  if (b < nbu) {
    const int64_t i = b * kPlanBlock + threadIdx.x;
    const int k = i < rows_n(p) ? kRankOf[(int)o.cls[i]] : -1;
    int t[kNumCls];
    const int r = block_class_rank<kNumCls>(k, t);
    if (k >= 0) {
      int64_t base = 0;
      for (int q = 0; q < k; ++q) base += tot[q];
      const int64_t within = bu[(int64_t)k * nbu + b] + r;   // position among the rows of its class
      const int64_t pos = base + within;
      o.order[pos] = i;
      if (o.rank) o.rank[i] = pos;
      if (o.u_ord) o.u_ord[pos] = p.u[i];
      if (o.c_ord) o.c_ord[pos] = (int64_t)o.c[i];
      if (o.sl_ord) o.sl_ord[pos] = (int64_t)o.sl[i];
      if (o.loc_ord && p.loc) o.loc_ord[pos] = row_ok(p, p.u[i]) ? (int64_t)p.loc[p.u[i]] : -1;
      // L rows in the reference's list order: admitted (rank 2), append (rank 5), compact (rank 7)
      const int64_t loff = k == kRankOf[kLAdm] ? 0
                           : k == kRankOf[kLApp] ? tot[kRankOf[kLAdm]]
                           : k == kRankOf[kLCmp] ? tot[kRankOf[kLAdm]] + tot[kRankOf[kLApp]] : -1;
      if (loff >= 0) {
        if (o.L_row) o.L_row[loff + within] = p.u[i];
        if (o.L_cnt) o.L_cnt[loff + within] = (int32_t)o.c[i];
      }
      // this batch's bit in the ring: no later plan asks about step s (the rows of u are distinct, so no other
      // thread writes this word; the dynamic-slot threads read only the bits of next_mask)
      if (p.next_bits && row_ok(p, p.u[i]) && p.R > 0) p.next_bits[p.u[i]] &= ~(1u << (p.s & 31));
    }
  } else {
    const int64_t bb = b - nbu;
    const int64_t j = bb * kPlanBlock + threadIdx.x;
    // the step's slot count: in the device-driven step from the descriptor, since the resolution has already
    // advanced the control state's count to the one after this step
    const int64_t nd = desc ? clampi(desc[kDNd], 0, p.nd) : dyn_n(p);
    const int k = j < nd ? dyn_class(p, p.dyn[j]) : -1;
    int t3[3];
    const int r3 = block_class_rank<3>(k, t3);
    int t2[2];
    const int r2 = block_class_rank<2>(k < 0 ? -1 : (k == 0 ? 0 : 1), t2);
    if (k >= 0) {
      const int64_t* dt = tot + kNumCls;   // expired, preemptible, protected, not expired
      const int64_t base3 = k == 0 ? 0 : (k == 1 ? dt[0] : dt[0] + dt[1]);
      const int64_t d = p.dyn[j];
      o.dyn_out[base3 + bd[(int64_t)k * nbd + bb] + r3] = d;
      const int64_t pos2 = k == 0 ? bd[0 * nbd + bb] + r2 : dt[0] + bd[3 * nbd + bb] + r2;
      o.dyn_out[nd + pos2] = d;
    }
  }
}

inline int64_t plan_blocks(int64_t m) { return (m + kPlanBlock - 1) / kPlanBlock; }

__global__ __launch_bounds__(kPlanBlock) void k_plan_admit(const int64_t* __restrict__ adm_rows,
                                                           const int64_t* __restrict__ adm_slots, int64_t n_adm,
                                                           int64_t lazy_n, int evl, int64_t s, int64_t n0, int64_t C,
                                                           int64_t R, int K, const int8_t* __restrict__ code,
                                                           int32_t* __restrict__ slot_of,
                                                           int64_t* __restrict__ slot_row,
                                                           int8_t* __restrict__ adm_c0, int8_t* __restrict__ rj,
                                                           int8_t* __restrict__ rok, int32_t* __restrict__ pstep) {
  const int64_t i = (int64_t)blockIdx.x * kPlanBlock + threadIdx.x;
  if (i >= n_adm) return;
  admit_one(i, adm_rows[i], adm_slots[i], lazy_n, evl, s, n0, C, R, K, code, slot_of, slot_row, adm_c0, rj, rok,
            pstep);
}

}  // namespace elr

extern "C" int64_t elr_plan_scratch_bytes(int64_t n, int64_t nd) {
  using namespace elr;
  if (n < 0 || nd < 0) return -1;
  const int64_t nbu = plan_blocks(n), nbd = plan_blocks(nd);
  return ((kNumCls * nbu + kDynCh * nbd + nbu + kNumCls + kDynCh + 1) * 8 + 255) & ~int64_t(255);
}

namespace elr {

// elr_plan_classify's checks; 0 when the call may launch.
static int plan_classify_check(const elr_plan_in* in, const elr_plan_out* out, void* scratch, int64_t scratch_bytes) {
  if (!in || !out) return ELR_EINVAL;
  const elr_plan_in& p = *in;
  const elr_plan_out& o = *out;
  if (p.n < 0 || p.nd < 0 || p.n >= (int64_t(1) << 31) || p.nd >= (int64_t(1) << 31)) return ELR_EINVAL;
  if (p.nnext < 0 || p.nnext > 4 || p.T < 1 || p.K < 1 || !p.toff || !p.kthr || !o.counts) return ELR_EINVAL;
  for (int k = 0; k < p.nnext; ++k)
    if (p.n_next[k] < 0 || (p.n_next[k] > 0 && !p.next[k])) return ELR_EINVAL;
  if (p.n > 0 && (!p.u || !p.slot_of || !p.last_seen || !p.code || !o.cls || !o.flags || !o.sl || !o.c || !o.order))
    return ELR_EINVAL;
  if (p.nd > 0 && (!p.dyn || !p.slot_row || !p.last_seen || !o.dyn_out)) return ELR_EINVAL;
  if (p.next_bits && (p.R <= 0 || (p.next_mask & (1u << (p.s & 31))))) return ELR_EINVAL;
  if (!scratch || scratch_bytes < elr_plan_scratch_bytes(p.n, p.nd)) return ELR_ECAPACITY;
  return ELR_OK;
}

// The three launches of the classification; the count pass beside the segment sum's partial chunks when given
// (blocks of the count pass first).  ctl (the device-driven step): the scan launch also resolves the step, with
// the overflow path's offsets in the scratch after the plain layout.
static int plan_classify_launch(const elr_plan_in& p, const elr_plan_out& o, void* scratch, hipStream_t st,
                                const SegPartialsLaunch* seg, const elr_plan_ctl* ctl = nullptr) {
  const int64_t nbu = plan_blocks(p.n), nbd = plan_blocks(p.nd);
  int64_t* bu = (int64_t*)scratch;
  int64_t* bd = bu + kNumCls * nbu;
  int64_t* bbad = bd + kDynCh * nbd;
  int64_t* tot = bbad + nbu;
  elr_plan_ctl c{};
  int64_t* bu2 = nullptr;
  int64_t* tot2 = nullptr;
  if (ctl) {
    c = *ctl;
    bu2 = (int64_t*)((char*)scratch + elr_plan_scratch_bytes(p.n, p.nd));
    tot2 = bu2 + kNumCls * nbu;
  }
  const PlanCount count{p, o, nbu, nbd, bu, bd, bbad};
  if (seg && seg->blocks > 0)
    seg_partials_visit(*seg, [&](const auto& f, int64_t nb) { launch2(count, nbu + nbd, f, nb, st); });
  else
    launch1(count, nbu + nbd, st);
  if (ctl) k_plan_scan_dev<<<1, kScanBlock, 0, st>>>(p, o, nbu, nbd, bu, bd, bbad, tot, c, bu2, tot2);
  else k_plan_scan<<<kPlanCh, kScanBlock, 0, st>>>(p, o, nbu, nbd, bu, bd, bbad, tot);
  if (nbu + nbd > 0)
    k_plan_scatter<<<(unsigned)(nbu + nbd), kPlanBlock, 0, st>>>(p, o, nbu, nbd, bu, bd, tot, c.desc, bu2, tot2);
  return launch_status();
}

}  // namespace elr

extern "C" int elr_plan_classify(const elr_plan_in* in, const elr_plan_out* out, void* scratch, int64_t scratch_bytes,
                                 void* stream) {
  using namespace elr;
  const int rc = plan_classify_check(in, out, scratch, scratch_bytes);
  if (rc) return rc;
  return plan_classify_launch(*in, *out, scratch, (hipStream_t)stream, nullptr);
}

extern "C" int elr_plan_classify_seg(const elr_plan_in* in, const elr_plan_out* out, void* scratch,
                                     int64_t scratch_bytes, const float* grad, int64_t n_occ, int64_t D, int key_bits,
                                     const void* dplan, int64_t dplan_bytes, void* stream) {
  using namespace elr;
  int rc = plan_classify_check(in, out, scratch, scratch_bytes);
  if (rc) return rc;
  SegPartialsLaunch seg;
  if ((rc = seg_partials_prep(grad, n_occ, D, key_bits, dplan, dplan_bytes, seg))) return rc;
  return plan_classify_launch(*in, *out, scratch, (hipStream_t)stream, &seg);
}

extern "C" int64_t elr_plan_step_scratch_bytes(int64_t n, int64_t nd) {
  using namespace elr;
  const int64_t base = elr_plan_scratch_bytes(n, nd);
  if (base < 0) return base;
  return base + (((kNumCls * plan_blocks(n) + 16) * 8 + 255) & ~int64_t(255));
}

extern "C" int elr_plan_step(const elr_plan_in* in, const elr_plan_out* out, const elr_plan_ctl* ctl, void* scratch,
                             int64_t scratch_bytes, const float* grad, int64_t n_occ, int64_t D, int key_bits,
                             const void* dplan, int64_t dplan_bytes, void* stream) {
  using namespace elr;
  int rc = plan_classify_check(in, out, scratch, scratch_bytes);
  if (rc) return rc;
  if (!ctl || !ctl->state || !ctl->desc || ctl->mat_cap < 0 || ctl->log_cap < 0 || !in->nd_dev || !in->live ||
      !in->mat_top || !in->log_top || in->n < 1 || (in->nd > 0 && !in->dyn))
    return ELR_EINVAL;
  if (scratch_bytes < elr_plan_step_scratch_bytes(in->n, in->nd)) return ELR_ECAPACITY;
  SegPartialsLaunch seg{};
  if (grad && (rc = seg_partials_prep(grad, n_occ, D, key_bits, dplan, dplan_bytes, seg))) return rc;
  return plan_classify_launch(*in, *out, scratch, (hipStream_t)stream, grad ? &seg : nullptr, ctl);
}

extern "C" int elr_plan_admit(const int64_t* adm_rows, const int64_t* adm_slots, int64_t n_adm, int64_t lazy_n, int evl,
                              int64_t s, int64_t n0, int64_t C, int64_t R, int K, const int8_t* code, int32_t* slot_of,
                              int64_t* slot_row, int8_t* adm_c0, int8_t* rj, int8_t* rok, int32_t* pstep,
                              void* stream) {
  using namespace elr;
  if (n_adm < 0 || lazy_n < 0 || lazy_n > n_adm || n0 < 0 || n0 > C || K < 1 || R < 0) return ELR_EINVAL;
  if (n_adm == 0) return ELR_OK;
  if (!adm_rows || !adm_slots || !code || !slot_of || !slot_row || !adm_c0 || !rj || !rok || !pstep) return ELR_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  k_plan_admit<<<(unsigned)plan_blocks(n_adm), kPlanBlock, 0, st>>>(adm_rows, adm_slots, n_adm, lazy_n, evl, s, n0, C,
                                                                     R, K, code, slot_of, slot_row, adm_c0, rj, rok,
                                                                     pstep);
  return launch_status();
}

namespace elr {

int admit_slots_check(const elr_slots_args& sl, const int64_t* adm_rows, int64_t n_adm, int64_t lazy_n, int64_t n0,
                      int64_t C, int64_t R, int K, const int8_t* code, int32_t* slot_of, int64_t* slot_row,
                      int8_t* adm_c0, int8_t* rj, int8_t* rok, int32_t* pstep) {
  if (n_adm < 0 || lazy_n < 0 || lazy_n > n_adm || n0 < 0 || n0 > C || K < 1 || R < 0) return ELR_EINVAL;
  if (sl.n_free < 0 || sl.nev < 0 || sl.nkeep < 0 || n_adm > sl.n_free + sl.nev || sl.n_free + sl.nev > C)
    return ELR_EINVAL;
  if (admit_slots_blocks(sl, n_adm) == 0) return ELR_OK;
  if ((sl.n_free + sl.nev > 0 && !sl.free_stack) || (sl.nev > 0 && !sl.ev_slot) || (sl.nkeep > 0 && !sl.keep) ||
      (n_adm + sl.nkeep > 0 && !sl.dyn_out) || (n_adm > 0 && (!sl.adm_slots || !adm_rows || !code || !slot_of ||
                                                              !slot_row || !adm_c0 || !rj || !rok || !pstep)))
    return ELR_EINVAL;
  return ELR_OK;
}

}  // namespace elr

extern "C" int elr_plan_admit_slots(const elr_slots_args* slots, const int64_t* adm_rows, int64_t n_adm,
                                    int64_t lazy_n, int evl, int64_t s, int64_t n0, int64_t C, int64_t R, int K,
                                    const int8_t* code, int32_t* slot_of, int64_t* slot_row, int8_t* adm_c0, int8_t* rj,
                                    int8_t* rok, int32_t* pstep, void* stream) {
  using namespace elr;
  if (!slots) return ELR_EINVAL;
  const elr_slots_args& sl = *slots;
  const int rc = admit_slots_check(sl, adm_rows, n_adm, lazy_n, n0, C, R, K, code, slot_of, slot_row, adm_c0, rj, rok,
                                   pstep);
  const int64_t blocks = admit_slots_blocks(sl, n_adm);
  if (rc || blocks == 0) return rc;
  launch1(PlanAdmitSlots{sl, adm_rows, n_adm, lazy_n, evl, s, n0, C, R, K, code, slot_of, slot_row, adm_c0, rj, rok,
                         pstep},
          blocks, (hipStream_t)stream);
  return launch_status();
}
