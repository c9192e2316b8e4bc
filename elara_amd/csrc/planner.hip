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
  for (int k = 0; k < p.nnext; ++k) f = f || sorted_has(p.next[k], p.n_next[k], r);
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
    if (i < p.n) {
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
    const int k = j < p.nd ? dyn_class(p, p.dyn[j]) : -1;
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
  if (threadIdx.x == 0) {   // the thread that stored tot[c]
    if (c < kNumCls) o.counts[kClsOfRank[c]] = tot[c];
    else if (c < kNumCls + 3) o.counts[c] = tot[c];
    else if (c == kNumCls + kDynCh) o.counts[16] = tot[c];
    if (c == 0) {
      o.counts[13] = p.mat_top ? *p.mat_top : 0;
      o.counts[14] = p.log_top ? *p.log_top : 0;
      o.counts[15] = p.live ? *p.live : 0;
    }
  }
}

// Pass 3: stable scatter by class.
__global__ __launch_bounds__(kPlanBlock) void k_plan_scatter(elr_plan_in p, elr_plan_out o, int64_t nbu, int64_t nbd,
                                                             const int64_t* __restrict__ bu,
                                                             const int64_t* __restrict__ bd,
                                                             const int64_t* __restrict__ tot) {
  const int64_t b = blockIdx.x;
  if (b < nbu) {
    const int64_t i = b * kPlanBlock + threadIdx.x;
    const int k = i < p.n ? kRankOf[(int)o.cls[i]] : -1;
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
    const int k = j < p.nd ? dyn_class(p, p.dyn[j]) : -1;
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
      o.dyn_out[p.nd + pos2] = d;
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
// (blocks of the count pass first).
static int plan_classify_launch(const elr_plan_in& p, const elr_plan_out& o, void* scratch, hipStream_t st,
                                const SegPartialsLaunch* seg) {
  const int64_t nbu = plan_blocks(p.n), nbd = plan_blocks(p.nd);
  int64_t* bu = (int64_t*)scratch;
  int64_t* bd = bu + kNumCls * nbu;
  int64_t* bbad = bd + kDynCh * nbd;
  int64_t* tot = bbad + nbu;
  const PlanCount count{p, o, nbu, nbd, bu, bd, bbad};
  if (seg && seg->blocks > 0)
    seg_partials_visit(*seg, [&](const auto& f, int64_t nb) { launch2(count, nbu + nbd, f, nb, st); });
  else
    launch1(count, nbu + nbd, st);
  k_plan_scan<<<kNumCls + kDynCh + 1, kScanBlock, 0, st>>>(p, o, nbu, nbd, bu, bd, bbad, tot);
  if (nbu + nbd > 0) k_plan_scatter<<<(unsigned)(nbu + nbd), kPlanBlock, 0, st>>>(p, o, nbu, nbd, bu, bd, tot);
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
