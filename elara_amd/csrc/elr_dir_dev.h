// Device side of the state directory (directory.hip): the shared helpers and the eviction and call-B kernels as
// functors (elr_launch.h), so that the step's executor can launch them beside independent row kernels.
#pragma once

#include "elr_desc.h"
#include "elr_launch.h"
#include "elr_scan.h"

namespace elr {

constexpr int kDirBlock = 256;

// Old counter values kept for the apply steps: block 0 of the count kernel stores nf0, top0 and mt0 (every block of
// it reads the same counters, which nothing writes during that launch); nf1 comes with the counter update.
struct DirHdr {
  int64_t nf0;   // n_lfree before this call's log allocation
  int64_t top0;  // log_top before it
  int64_t mt0;   // mat_top before this call's MAT allocation
  int64_t nf1;   // n_lfree after the log allocation (push base of the releases)
};

// Grids of at most this many blocks skip the single-block scan launch: each block of the apply kernel sums the
// per-block counts of the blocks before it itself (one count per thread), and its block 0 advances the counters.
// Larger grids scan the counts in a launch of their own (k_dir_scan) rather than have every block read them all.
constexpr int64_t kFusedScanBlocks = kDirBlock;

template <int NCH>
__device__ __forceinline__ void dir_block_scan(const int (&v)[NCH], int (&ex)[NCH], int (&tot)[NCH]) {
  block_excl_scan<kDirBlock, NCH>(v, ex, tot);
}

__device__ __forceinline__ void dir_snapshot(int64_t blk, const elr_dir_state& st, DirHdr* hdr) {
  if (blk == 0 && threadIdx.x == 0) {
    hdr->nf0 = *st.n_lfree;
    hdr->top0 = *st.log_top;
    hdr->mt0 = *st.mat_top;
  }
}

// n_lfree after `nalloc` log allocations (elara_dir.cpp:18: the free stack is popped first).
__device__ __forceinline__ int64_t nf_after_alloc(int64_t nf0, int64_t nalloc) {
  return nf0 - (nalloc < nf0 ? nalloc : nf0);
}

// Counter update of one call from the counters' old values nf0, top0, mt0 (elara_dir.cpp:18-19 alloc, 31 release,
// 42 MAT, in the reference's order: log allocation, MAT allocation, release); returns n_lfree after the allocation.
__device__ __forceinline__ int64_t dir_advance(const elr_dir_state& st, int64_t nf0, int64_t top0, int64_t mt0,
                                               int64_t nalloc, int64_t nmat, int64_t nrel) {
  const int64_t nf1 = nf_after_alloc(nf0, nalloc);
  *st.log_top = top0 + nalloc - (nf0 - nf1);
  *st.mat_top = mt0 + nmat;
  *st.n_lfree = nf1 + nrel;
  *st.live = *st.live + nalloc - nrel;
  return nf1;
}

// Block offsets of a grid of nblk <= kFusedScanBlocks blocks from its raw per-block counts (channel c at
// bsum[c*nblk .. c*nblk+nblk)): off[c] = sum over the blocks before this one, tot[c] = sum over all.  Every thread
// of the block must call it; it synchronises before and after, so it may sit beside other block scans.
template <int NCH>
__device__ __forceinline__ void fused_offsets(int64_t blk, const int64_t* __restrict__ bsum, int64_t nblk,
                                              int64_t (&off)[NCH], int64_t (&tot)[NCH]) {
  __shared__ int sh[NCH];
  int v[NCH], ex[NCH], t[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) v[c] = (int64_t)threadIdx.x < nblk ? (int)bsum[c * nblk + threadIdx.x] : 0;
  __syncthreads();
  block_excl_scan<kDirBlock, NCH>(v, ex, t);
  if ((int64_t)threadIdx.x == blk)
#pragma unroll
    for (int c = 0; c < NCH; ++c) sh[c] = ex[c];
  __syncthreads();
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    off[c] = sh[c];
    tot[c] = t[c];
  }
  __syncthreads();
}

// fused_offsets for a device-driven step, whose grid is sized from an upper bound: only the first nlive blocks hold
// items (and wrote counts), any number of them; each thread sums the counts of every kDirBlock-th live block.
template <int NCH>
__device__ __forceinline__ void live_offsets(int64_t blk, const int64_t* __restrict__ bsum, int64_t nblk, int64_t nlive,
                                             int64_t (&off)[NCH], int64_t (&tot)[NCH]) {
  __shared__ int64_t sh[2][NCH][kDirBlock / 64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int64_t before[NCH], all[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) before[c] = all[c] = 0;
  for (int64_t b = threadIdx.x; b < nlive; b += kDirBlock)
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int64_t x = bsum[c * nblk + b];
      all[c] += x;
      before[c] += b < blk ? x : 0;
    }
  __syncthreads();
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int64_t sb = wave_incl_scan<int64_t>(before[c]), sa = wave_incl_scan<int64_t>(all[c]);
    if (lane == 63) {
      sh[0][c][w] = sb;
      sh[1][c][w] = sa;
    }
  }
  __syncthreads();
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    int64_t a = 0, t = 0;
    for (int v = 0; v < kDirBlock / 64; ++v) {
      a += sh[0][c][v];
      t += sh[1][c][v];
    }
    off[c] = a;
    tot[c] = t;
  }
  __syncthreads();
}

__device__ __forceinline__ bool in_range(int64_t x, int64_t hi) { return x >= 0 && x < hi; }

// searchsorted(toff, row, right=True) - 1, with ATen's wrap of index -1 to T-1 (elara_dir.cpp:46-48, 75).
__device__ __forceinline__ int64_t table_of(const int64_t* __restrict__ toff, int64_t T, int64_t row) {
  int64_t lo = 0, hi = T;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (toff[mid] <= row) lo = mid + 1; else hi = mid;
  }
  const int64_t t = lo - 1;
  return t < 0 ? t + T : t;
}

// Log id of allocation rank `rank` (elara_dir.cpp:15-17): free stack top-down first, then the bump pointer.
__device__ __forceinline__ int64_t log_id_of_rank(const int32_t* __restrict__ lfree, int64_t Lcap, int64_t nf0,
                                                  int64_t top0, int64_t rank) {
  if (rank < nf0) {
    const int64_t fi = nf0 - 1 - rank;
    return in_range(fi, Lcap + 1) ? (int64_t)lfree[fi] : -1;
  }
  return top0 + rank - nf0;
}

// ---------------------------------------------------------------------------------------------------------------
// A1: replay inputs of L rows (elara_dir.cpp:56-59) and resident-history recording of hits (elara_dir.cpp:60-71).
// Threads [0, nL*K) take one (row, k) entry each; threads [nL*K, nL*K + nh) take one hit slot each.  The two parts
// touch disjoint arrays (ent/lstep are read; pstep/rj/rok are written), and hit slots are unique.
struct DirLstepsHits {
  elr_dir_state st;
  elr_dir_params p;
  const int64_t* hs;
  DevCount nh_;
  const int64_t* L_row;
  const int32_t* L_cnt;
  DevCount nL_;
  int32_t s;
  int32_t* L_steps;
  int32_t* L_ids;
  int64_t* hrec_dyn;
  int64_t* hrec_j;
  __device__ void operator()(int64_t block, int64_t) const {
    const int64_t t = block * kDirBlock + threadIdx.x;
    const int64_t nh = nh_.get(), nL = nL_.get();
    const int64_t K = p.K, nLK = nL * K;
    if (t < nLK) {
      const int64_t i = t / K, k = t - i * K;
      const int64_t row = L_row[i];
      int32_t e = -1;
      if (in_range(row, p.R + 1)) e = st.ent[row * K + k];
      L_steps[t] = (e >= 0 && e <= p.Lcap) ? st.lstep[e] : 0;
      L_ids[t] = k < (int64_t)L_cnt[i] ? e : -1;
      return;
    }
    const int64_t i = t - nLK;
    if (i >= nh) return;
    const int64_t sl = hs[i];
    const int64_t C = p.n0 + p.Cdyn;
    if (!in_range(sl, C)) {
      hrec_dyn[i] = p.Cdyn;
      hrec_j[i] = 0;
      return;
    }
    const bool dyn = sl >= p.n0;
    const int64_t c0 = st.adm_c0[sl], j = st.rj[sl];
    const bool ok = st.rok[sl] != 0;
    const bool rec = p.evl && dyn && ok && (c0 + j < K);
    const int64_t hd = rec ? sl - p.n0 : p.Cdyn, hj = rec ? j : 0;
    hrec_dyn[i] = hd;
    hrec_j[i] = hj;
    if (in_range(hj, K)) st.pstep[hd * K + hj] = s;  // non-recorded hits write the trash row (Cdyn, 0), as the reference
    st.rj[sl] = (int8_t)(j + (rec ? 1 : 0));
    st.rok[sl] = (int8_t)(ok && !(dyn && !rec));
  }
};

// Per-item quantities of an eviction (elara_dir.cpp:73-77, 80, 89, 92).
struct EvCounts {
  int nalloc;  // log ids for the resident history (rows going back to L): k < j
  int nmat;    // 1 if the row goes to M and has no MAT slot yet
  int nrel;    // host-log entries released (rows going to M): k < max(c0, 0) with ent >= 0
};

__device__ __forceinline__ EvCounts ev_counts(const elr_dir_state& st, const elr_dir_params& p, int64_t row, bool rep,
                                              int64_t c0, int64_t j) {
  EvCounts c{0, 0, 0};
  if (!in_range(row, p.R)) return c;
  const int64_t K = p.K;
  if (rep) {
    c.nalloc = (int)(j < 0 ? 0 : (j > K ? K : j));
  } else {
    c.nmat = st.loc[row] < 0 ? 1 : 0;
    const int64_t cnt = c0 > 0 ? c0 : 0;
    for (int64_t k = 0; k < K && k < cnt; ++k) c.nrel += st.ent[row * K + k] >= 0 ? 1 : 0;
  }
  return c;
}

// A2: eviction representation and per-block allocation counts (elara_dir.cpp:73-78).  With ev_row_in (the
// Directory.evict form, srm2/elara_kernels.py:152-171) the caller supplies the evicted rows and their thresholds
// and has already cleared slot_of / slot_row; otherwise the rows come from slot_row and are unmapped here.  defer:
// the releases of rows going to M are left to call B (the Triton path's order), so this call counts none.
struct DirEvictCount {
  elr_dir_state st;
  elr_dir_params p;
  const int64_t* ev_slot;
  DevCount nev;
  const int64_t* ev_row_in;
  const int8_t* thr_in;
  int64_t* ev_row;
  uint8_t* rep;
  int64_t* ev_dyn;
  int64_t* bsum;
  int64_t nblk;
  DirHdr* hdr;
  bool defer;
  __device__ void operator()(int64_t blk, int64_t) const {
    dir_snapshot(blk, st, hdr);
    const int64_t i = (int64_t)blk * kDirBlock + threadIdx.x;
    const int64_t n_ev = nev.get();
    if (nev.p && blk * kDirBlock >= n_ev) return;   // device-driven: past the live blocks (nobody reads their counts)
    int v[3] = {0, 0, 0};
    if (i < n_ev) {
      const int64_t sl = ev_slot[i];
      const int64_t C = p.n0 + p.Cdyn;
      int64_t row = -1, c0 = -1, j = 0;
      bool rp = false;
      if (in_range(sl, C)) {
        row = ev_row_in ? ev_row_in[i] : st.slot_row[sl];
        c0 = st.adm_c0[sl];
        j = st.rj[sl];
        if (p.evl && in_range(row, p.R)) {
          const int64_t th = thr_in ? (int64_t)thr_in[i] : (int64_t)st.kthr[table_of(st.toff, st.T, row)];
          rp = st.rok[sl] != 0 && (c0 + j) <= th;
        }
        if (!ev_row_in) {
          if (in_range(row, p.R)) st.slot_of[row] = -1;
          st.slot_row[sl] = -1;
        }
      }
      if (!ev_row_in) ev_row[i] = row;
      rep[i] = rp ? 1 : 0;
      ev_dyn[i] = sl - p.n0;
      const EvCounts c = ev_counts(st, p, row, rp, c0, j);
      v[0] = c.nalloc;
      v[1] = c.nmat;
      v[2] = defer ? 0 : c.nrel;
    }
    int ex[3], tot[3];
    dir_block_scan<3>(v, ex, tot);
    if (threadIdx.x == 0)
      for (int c = 0; c < 3; ++c) bsum[c * nblk + blk] = tot[c];
  }
};

// A4: apply the eviction representation (elara_dir.cpp:79-93 except the stack pushes): log ids of rows going back
// to L (ent, lstep), MAT slots (loc, evf_slots), codes; records each item's release rank for A5.  fused: bsum holds
// the raw per-block counts (grid of at most kFusedScanBlocks blocks) and block 0 advances the counters; otherwise
// k_dir_scan has turned bsum into block offsets and advanced them.  With rel_cnt (deferred releases, no A5) each
// item's release count goes there instead: max(c0, 0) for a row going to M, 0 for one going back to L
// (srm2/elara_kernels.py:71-72, the release part of Directory.evict).
struct DirEvictApply {
  elr_dir_state st;
  elr_dir_params p;
  const int64_t* ev_slot;
  DevCount nev;
  const int64_t* ev_row;
  const uint8_t* rep;
  const int64_t* ev_dyn;
  int64_t* evl_ids;
  int64_t* evf_slots;
  const int64_t* boff;
  int64_t nblk;
  DirHdr* hdr;
  int64_t* rel_rank;
  bool fused;
  int64_t* rel_cnt;
  __device__ void operator()(int64_t blk, int64_t) const {
    const int64_t i = (int64_t)blk * kDirBlock + threadIdx.x;
    const int64_t K = p.K;
    const int64_t nev = this->nev.get();
    const int64_t nf0 = hdr->nf0, top0 = hdr->top0, mt0 = hdr->mt0;
    int64_t off[3], gtot[3];
    if (this->nev.p) {   // device-driven: block 0 (which always runs) advances the counters, blocks past the items exit
      const int64_t nlive = (nev + kDirBlock - 1) / kDirBlock;
      if (blk > 0 && blk >= nlive) return;
      live_offsets<3>(blk, boff, nblk, nlive, off, gtot);
      if (blk == 0 && threadIdx.x == 0) hdr->nf1 = dir_advance(st, nf0, top0, mt0, gtot[0], gtot[1], gtot[2]);
    } else if (fused) {
      fused_offsets<3>(blk, boff, nblk, off, gtot);
      if (blk == 0 && threadIdx.x == 0) hdr->nf1 = dir_advance(st, nf0, top0, mt0, gtot[0], gtot[1], gtot[2]);
    } else {
  #pragma unroll
      for (int c = 0; c < 3; ++c) off[c] = boff[c * nblk + blk];
    }
    int64_t row = -1, c0 = -1, j = 0;
    bool rp = false;
    EvCounts c{0, 0, 0};
    if (i < nev) {
      const int64_t sl = ev_slot[i];
      row = ev_row[i];
      rp = rep[i] != 0;
      if (in_range(sl, p.n0 + p.Cdyn)) {
        c0 = st.adm_c0[sl];
        j = st.rj[sl];
      }
      c = ev_counts(st, p, row, rp, c0, j);
      if (rel_cnt) c.nrel = 0;
    }
    int v[3] = {c.nalloc, c.nmat, c.nrel}, ex[3], tot[3];
    dir_block_scan<3>(v, ex, tot);
    if (i >= nev) return;
    // log ids for the resident history: ent[row, max(c0,0) + k] = id, lstep[id] = pstep[dyn, k]  (k < j)
    const int64_t rA = off[0] + ex[0];
    int64_t dyn = ev_dyn[i];
    if (!in_range(dyn, p.Cdyn)) dyn = p.Cdyn;
    const int64_t kb = c0 > 0 ? c0 : 0;
    for (int64_t k = 0; k < K; ++k) {
      int64_t id = -1;
      if (k < c.nalloc) {
        id = log_id_of_rank(st.lfree, p.Lcap, nf0, top0, rA + k);
        if (kb + k < K) st.ent[row * K + kb + k] = (int32_t)id;
        if (in_range(id, p.Lcap)) st.lstep[id] = st.pstep[dyn * K + k];
      }
      evl_ids[i * K + k] = id;
    }
    // MAT slot for rows going to M (elara_dir.cpp:36-44, 89-90); rows going back to L get the trash slot
    int64_t slot = -1;
    if (in_range(row, p.R)) {
      const int64_t cur = st.loc[row];
      slot = c.nmat ? mt0 + off[1] + ex[1] : cur;
      if (c.nmat) st.loc[row] = (int32_t)slot;
      const int64_t tj = c0 + j;
      st.code[row] = rp ? (int8_t)(tj < 127 ? tj : 127) : (int8_t)p.MAT;
    }
    evf_slots[i] = rp ? p.trash : slot;
    if (rel_cnt) rel_cnt[i] = rp ? 0 : (c0 > 0 ? c0 : 0);
    else rel_rank[i] = off[2] + ex[2];
  }
};

// Push the released entries of rows[i] (k < cnt, ent >= 0; `rank` = item's first push rank) and clear them
// (elara_dir.cpp:25-33).
__device__ __forceinline__ void release_row(const elr_dir_state& st, const elr_dir_params& p, int64_t row,
                                            int64_t cnt, int64_t push_at) {
  const int64_t K = p.K;
  int64_t q = 0;
  for (int64_t k = 0; k < K && k < cnt; ++k) {
    const int32_t e = st.ent[row * K + k];
    if (e >= 0) {
      const int64_t dst = push_at + q++;
      if (in_range(dst, p.Lcap)) st.lfree[dst] = e;
      st.ent[row * K + k] = -1;
    }
  }
}

// A5: releases of rows going to M (after every pop of this call).
struct DirEvictRelease {
  elr_dir_state st;
  elr_dir_params p;
  const int64_t* ev_slot;
  DevCount nev;
  const int64_t* ev_row;
  const uint8_t* rep;
  const int64_t* rel_rank;
  const DirHdr* hdr;
  __device__ void operator()(int64_t blk, int64_t) const {
    const int64_t i = (int64_t)blk * kDirBlock + threadIdx.x;
    if (i >= nev.get() || rep[i]) return;
    const int64_t row = ev_row[i], sl = ev_slot[i];
    if (!in_range(row, p.R) || !in_range(sl, p.n0 + p.Cdyn)) return;
    const int64_t c0 = st.adm_c0[sl];
    release_row(st, p, row, c0 > 0 ? c0 : 0, hdr->nf1 + rel_rank[i]);
  }
};

// Logged entries of `row` among its first cnt (elara_dir.cpp:27: the ones a release pushes).
__device__ __forceinline__ int live_entries(const elr_dir_state& st, const elr_dir_params& p, int64_t row,
                                            int64_t cnt) {
  int n = 0;
  for (int64_t k = 0; k < p.K && k < cnt; ++k) n += st.ent[row * p.K + k] >= 0 ? 1 : 0;
  return n;
}

// The items of call B after its appends: nr release items (the first r_cnt[i] entries of r_rows[i]) and then nc
// compactions (c_rows[i] with c_cnt[i] entries, released too when c_release).  Item q's counts: MAT slot needed and
// entries released, pushed in item order.  The reference's default order (elara_dir.cpp:107-108) is nr = 0,
// c_release; the Triton path's (srm2/elara_kernels.py:188-209) pushes the evictions' deferred part first.
struct DirBItems {
  const int64_t* c_rows;
  const int64_t* c_cnt;
  int64_t nc;
  const int64_t* r_rows;
  const int64_t* r_cnt;
  int64_t nr;
  bool c_release;
  // device-driven step: nc, nr are upper bounds and c_rows, c_cnt the class-ordered rows and codes, to be offset by
  // the compactions' first position; resolved() reads the descriptor
  const int64_t* desc;
  __device__ __forceinline__ DirBItems resolved() const {
    if (!desc) return *this;
    DirBItems r = *this;
    const int64_t at = clampi(desc[kDB + ELR_RANK_NCMP], 0, nc);
    r.c_rows = c_rows + at;
    r.c_cnt = c_cnt + at;
    r.nc = clampi(desc[kDNc], 0, nc - at);
    r.nr = clampi(desc[kDNr], 0, nr);
    r.desc = nullptr;
    return r;
  }
  __device__ __forceinline__ int64_t n() const { return nr + nc; }
  __device__ __forceinline__ bool is_rel(int64_t q) const { return q < nr; }
  __device__ __forceinline__ int64_t row(int64_t q) const { return q < nr ? r_rows[q] : c_rows[q - nr]; }
  __device__ __forceinline__ int64_t cnt(int64_t q) const { return q < nr ? r_cnt[q] : c_cnt[q - nr]; }
  __device__ __forceinline__ bool releases(int64_t q) const { return q < nr || c_release; }
};

// Counts of item q (MAT slot needed, entries released); cur = the row's MAT slot (-1: none or a release item).
__device__ __forceinline__ void b_item_counts(const elr_dir_state& st, const elr_dir_params& p, const DirBItems& it,
                                              int64_t q, int64_t& row, int64_t& cnt, int64_t& cur, int (&v)[2]) {
  row = it.row(q);
  cnt = it.cnt(q);
  cur = -1;
  if (!in_range(row, p.R)) return;
  if (!it.is_rel(q)) {
    cur = st.loc[row];
    v[0] = cur < 0 ? 1 : 0;
  }
  if (it.releases(q)) v[1] = live_entries(st, p, row, cnt);
}

// B1: appends (elara_dir.cpp:102-106; log id of append i has rank i) and per-block counts of the other items.
// Appended rows are disjoint from the compacted and the released ones.
struct DirBCount {
  elr_dir_state st;
  elr_dir_params p;
  const int64_t* a_rows;
  const int64_t* a_k;
  int64_t na;
  DirBItems it_in;
  int32_t s;
  int64_t* a_ids;
  int64_t* bsum;
  int64_t nblk_c;
  int64_t nblk_a;
  DirHdr* hdr;
  const int64_t* desc;   // device-driven step: na is an upper bound, a_rows / a_k the class-ordered rows and codes
  __device__ void operator()(int64_t blk, int64_t) const {
    dir_snapshot(blk, st, hdr);
    const int64_t K = p.K;
    if ((int64_t)blk < nblk_a) {
      const int64_t i = (int64_t)blk * kDirBlock + threadIdx.x;
      const int64_t at = desc ? clampi(desc[kDB + ELR_RANK_NAPP], 0, na) : 0;
      const int64_t* a_rows = this->a_rows + at;
      const int64_t* a_k = this->a_k + at;
      if (i >= (desc ? clampi(desc[kDNa], 0, na - at) : na)) return;
      const int64_t id = log_id_of_rank(st.lfree, p.Lcap, *st.n_lfree, *st.log_top, i);
      a_ids[i] = id;
      const int64_t row = a_rows[i], k = a_k[i];
      if (in_range(row, p.R) && in_range(k, K)) {
        st.ent[row * K + k] = (int32_t)id;
        st.code[row] = (int8_t)(k + 1);
      }
      if (in_range(id, p.Lcap)) st.lstep[id] = s;
      return;
    }
    const int64_t b = (int64_t)blk - nblk_a;
    const int64_t q = b * kDirBlock + threadIdx.x;
    const DirBItems it = it_in.resolved();
    if (desc && b * kDirBlock >= it.n()) return;   // device-driven: past the live blocks (nobody reads their counts)
    int v[2] = {0, 0};
    if (q < it.n()) {
      int64_t row, cnt, cur;
      b_item_counts(st, p, it, q, row, cnt, cur, v);
    }
    int ex[2], tot[2];
    dir_block_scan<2>(v, ex, tot);
    if (threadIdx.x == 0) {
      bsum[0 * nblk_c + b] = tot[0];
      bsum[1 * nblk_c + b] = tot[1];
    }
  }
};

// B3: compactions (elara_dir.cpp:107-108): MAT slot, release of their logs (c_release), code = MAT; release items:
// the push alone.  fused: bsum holds the raw per-block counts (grid of at most kFusedScanBlocks blocks, at least
// one) and block 0 advances the counters for the `na` appends and the items; otherwise k_dir_scan has turned bsum
// into block offsets and advanced them.
struct DirBCompact {
  elr_dir_state st;
  elr_dir_params p;
  DirBItems it_in;
  int64_t* c_slots;
  const int64_t* boff;
  int64_t nblk;
  DirHdr* hdr;
  bool fused;
  int64_t na;
  const int64_t* desc;   // device-driven step: the appends' count from the descriptor, live blocks only
  __device__ void operator()(int64_t blk, int64_t) const {
    const int64_t q = (int64_t)blk * kDirBlock + threadIdx.x;
    const int64_t mt0 = hdr->mt0;
    const DirBItems it = it_in.resolved();
    int64_t off[2], gtot[2], nf1;
    if (desc) {   // block 0 (which always runs) advances the counters, blocks past the items exit
      const int64_t nlive = (it.n() + kDirBlock - 1) / kDirBlock, na = clampi(desc[kDNa], 0, this->na);
      if (blk > 0 && blk >= nlive) return;
      live_offsets<2>(blk, boff, nblk, nlive, off, gtot);
      const int64_t nf0 = hdr->nf0;
      nf1 = nf_after_alloc(nf0, na);
      if (blk == 0 && threadIdx.x == 0) hdr->nf1 = dir_advance(st, nf0, hdr->top0, mt0, na, gtot[0], gtot[1]);
    } else if (fused) {
      fused_offsets<2>(blk, boff, nblk, off, gtot);
      const int64_t nf0 = hdr->nf0;
      nf1 = nf_after_alloc(nf0, na);
      if (blk == 0 && threadIdx.x == 0) hdr->nf1 = dir_advance(st, nf0, hdr->top0, mt0, na, gtot[0], gtot[1]);
    } else {
      off[0] = boff[blk];
      off[1] = boff[nblk + blk];
      nf1 = hdr->nf1;
    }
    int64_t row = -1, cnt = 0, cur = -1;
    int v[2] = {0, 0};
    if (q < it.n()) b_item_counts(st, p, it, q, row, cnt, cur, v);
    int ex[2], tot[2];
    dir_block_scan<2>(v, ex, tot);
    if (q >= it.n()) return;
    const bool rel = it.is_rel(q);
    if (!in_range(row, p.R)) {
      if (!rel) c_slots[q - it.nr] = -1;
      return;
    }
    if (it.releases(q)) release_row(st, p, row, cnt, nf1 + off[1] + ex[1]);
    if (rel) return;
    const int64_t slot = v[0] ? mt0 + off[0] + ex[0] : cur;
    if (v[0]) st.loc[row] = (int32_t)slot;
    c_slots[q - it.nr] = slot;
    st.code[row] = (int8_t)p.MAT;
  }
};

// Scratch layout: [DirHdr][bsum: nch * nblk int64][per-item release ranks: nev int64]
inline int64_t dir_nblocks(int64_t n) { return (n + kDirBlock - 1) / kDirBlock; }
inline int64_t dir_align(int64_t b) { return (b + 255) & ~int64_t(255); }
inline int64_t dir_a_scratch(int64_t nev) {
  return dir_align(sizeof(DirHdr)) + dir_align(3 * dir_nblocks(nev) * 8) + nev * 8;
}
inline int64_t dir_b_scratch(int64_t nitems) {
  return dir_align(sizeof(DirHdr)) + dir_align(2 * dir_nblocks(nitems) * 8);
}

// Host side (directory.hip).  The checks of elr_dir_a / elr_dir_b's arguments; the replay inputs and hit records
// (call A's first launch); the eviction part of call A and call B as functors with their grids, in launch order:
// count, then (not fused) the scan launch, then apply and release (call B: count, scan, compact).
int dir_a_check(const elr_dir_state* st, const elr_dir_params* p, const int64_t* hs, int64_t nh, const int64_t* L_row,
                const int32_t* L_cnt, int64_t nL, const int64_t* ev_slot, int64_t nev, int32_t* L_steps,
                int32_t* L_ids, int64_t* hrec_dyn, int64_t* hrec_j, int64_t* ev_row, uint8_t* rep, int64_t* evl_ids,
                int64_t* evf_slots, int64_t* ev_dyn, void* scratch, int64_t scratch_bytes);
int dir_b_check(const elr_dir_state* st, const elr_dir_params* p, const int64_t* a_rows, const int64_t* a_k,
                int64_t na, const int64_t* c_rows, const int64_t* c_cnt, int64_t nc, const int64_t* r_rows,
                const int64_t* r_cnt, int64_t nr, int64_t* a_ids, int64_t* c_slots, void* scratch,
                int64_t scratch_bytes);
// desc (a device-driven step): nh and nL are upper bounds that size the grid, the counts come from the descriptor.
void dir_lsteps_hits_launch(const elr_dir_state& S, const elr_dir_params& P, const int64_t* hs, int64_t nh,
                            const int64_t* L_row, const int32_t* L_cnt, int64_t nL, int64_t s, int32_t* L_steps,
                            int32_t* L_ids, int64_t* hrec_dyn, int64_t* hrec_j, hipStream_t strm,
                            const int64_t* desc = nullptr);
// The same as a functor and its block count, for a launch beside an independent body (the device-driven step pairs
// it with the segment sum's final kernel).
DirLstepsHits dir_lsteps_hits_prep(const elr_dir_state& S, const elr_dir_params& P, const int64_t* hs, int64_t nh,
                                   const int64_t* L_row, const int32_t* L_cnt, int64_t nL, int64_t s,
                                   int32_t* L_steps, int32_t* L_ids, int64_t* hrec_dyn, int64_t* hrec_j,
                                   const int64_t* desc, int64_t& blocks);

struct DirEvictPlan {
  DirEvictCount count;
  DirEvictApply apply;
  DirEvictRelease release;
  int64_t nblk;       // grid of each of the three
  int64_t rel_nblk;   // grid of the release launch (0 when the releases are deferred)
  bool fused;         // no scan launch
};
// rel_cnt: NULL for the reference's default order (the release launch pushes the host logs of rows going to M);
// otherwise those releases are deferred to call B and their counts written there (the release launch is empty).
// desc (a device-driven step): nev is an upper bound (the grid), the count comes from the descriptor, and the
// apply kernel sums the live blocks' counts itself (no scan launch).
DirEvictPlan dir_evict_plan(const elr_dir_state& S, const elr_dir_params& P, const int64_t* ev_slot, int64_t nev,
                            const int64_t* ev_row_in, const int8_t* thr_in, int64_t* ev_row_out, uint8_t* rep,
                            int64_t* evl_ids, int64_t* evf_slots, int64_t* ev_dyn, int64_t* rel_cnt, void* scratch,
                            const int64_t* desc = nullptr);
void dir_evict_scan(const DirEvictPlan& e, hipStream_t strm);

struct DirBPlan {
  DirBCount count;
  DirBCompact compact;
  int64_t count_blocks, compact_blocks, nblk_c, na;
  bool fused;
};
// Call B over its items (DirBItems: release items, then compactions).  desc (a device-driven step): na, it.nc and
// it.nr are upper bounds, a_rows / a_k and it.c_rows / c_cnt the rows and codes in class-rank order (offset on the
// device by the appends' and compactions' first positions), and no scan launch.
DirBPlan dir_b_plan(const elr_dir_state& S, const elr_dir_params& P, const int64_t* a_rows, const int64_t* a_k,
                    int64_t na, const DirBItems& it, int64_t s, int64_t* a_ids, int64_t* c_slots, void* scratch,
                    const int64_t* desc = nullptr);
void dir_b_scan(const DirBPlan& e, hipStream_t strm);

}  // namespace elr
