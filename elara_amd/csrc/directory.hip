// ELARA state directory on the GPU: row codes (I / L_c / M), log-entry ids and steps, sync-free allocators.
//
// Replaces srm2/csrc/elara_dir.cpp:13-110 (elara_dir_a / elara_dir_b, the reference's default directory
// implementation) with the same results and the same allocation order ("cpp" order):
//   call A:  replay inputs of L rows; resident-history recording of hits; eviction representation
//            (back to L: log ids for the resident history, MAT trash slot; to M: MAT slot, release host logs)
//   call B:  appends (stay L, one log id each), then compactions (to M: MAT slot, release all logs)
// and, as elr_dir_a_deferred / elr_dir_evict_deferred / elr_dir_b_release, in the order of the reference's Triton
// directory (srm2/elara_kernels.py), where every allocation of a step comes before any release: call A releases
// nothing, and call B pushes the evictions' releases after its appends' pops, ahead of the compacted rows' logs.
// Allocation ranks are exclusive prefix counts in row-major (item, k) order: the log allocator pops the free stack
// top-down and then bumps log_top (elara_dir.cpp:13-21), MAT slots bump mat_top (elara_dir.cpp:36-44), releases
// push onto the free stack at n_lfree + rank (elara_dir.cpp:23-34).
//
// The device counters n_lfree, log_top, mat_top, live stay in HBM; nothing is read back to the host.  Grid-wide
// ranks come from per-block counts (the count kernel also keeps the counters' old values in scratch) and an apply
// pass whose blocks add up the counts of the blocks before them and whose block 0 advances the counters; grids of
// more than kFusedScanBlocks blocks scan the counts in a single-block launch between the two instead.  Stack pops
// and pushes are separate launches, because a push may reuse a stack position that another block still has to pop.
//
// Trash conventions are the reference's (srm2/elara.py:119-123): loc/ent row R, pstep row Cdyn, MAT slot `trash`.
// The reference scatters values of invalid entries into lstep[Lcap] and lfree[Lcap] (which value lands there is
// unspecified on a GPU); this implementation does not write those two trash elements.
//
// Index safety: every gathered or scattered index is checked against its array's extent; an item whose slot, row
// or entry id is out of range is treated as carrying nothing (no writes).  The reference leaves such inputs
// undefined.
#include "elr_dir_dev.h"

namespace elr {

// Grids of more than kFusedScanBlocks blocks: single-block exclusive scan of the per-block counts of `nch`
// channels (in place) and the counter update, from the old counters that the count kernel kept in hdr.
// Channel roles: mode 0 (call A): 0 = log allocations, 1 = MAT allocations, 2 = releases.
//                mode 1 (call B): 0 = MAT allocations, 1 = releases; `nappend` log allocations (rank = item).
__global__ __launch_bounds__(kScanBlock) void k_dir_scan(elr_dir_state st, int mode, int64_t nappend,
                                                         int64_t* __restrict__ bsum, int64_t nblk, int nch,
                                                         DirHdr* __restrict__ hdr) {
  __shared__ int64_t chan_tot[3];
  if (threadIdx.x < 3) chan_tot[threadIdx.x] = 0;
  __syncthreads();
  scan_channels_block(bsum, nblk, nch, chan_tot);
  __syncthreads();
  if (threadIdx.x == 0) {
    const int64_t nalloc = mode == 0 ? chan_tot[0] : nappend;
    const int64_t nmat = mode == 0 ? chan_tot[1] : (nch > 0 ? chan_tot[0] : 0);
    const int64_t nrel = mode == 0 ? chan_tot[2] : (nch > 1 ? chan_tot[1] : 0);
    hdr->nf1 = dir_advance(st, hdr->nf0, hdr->top0, hdr->mt0, nalloc, nmat, nrel);
  }
}

inline bool params_ok(const elr_dir_state* st, const elr_dir_params* p) {
  return st && p && p->K >= 1 && p->K <= 126 && p->R >= 0 && p->Lcap >= 0 && p->n0 >= 0 && p->Cdyn >= 0 &&
         st->code && st->loc && st->ent && st->lstep && st->lfree && st->n_lfree && st->log_top && st->mat_top &&
         st->live && st->adm_c0 && st->rj && st->pstep && st->kthr && st->toff && st->slot_of && st->slot_row &&
         st->rok && st->T >= 1;
}

DirEvictPlan dir_evict_plan(const elr_dir_state& S, const elr_dir_params& P, const int64_t* ev_slot, int64_t nev,
                            const int64_t* ev_row_in, const int8_t* thr_in, int64_t* ev_row_out, uint8_t* rep,
                            int64_t* evl_ids, int64_t* evf_slots, int64_t* ev_dyn, int64_t* rel_cnt, void* scratch,
                            const int64_t* desc) {
  char* base = (char*)scratch;
  DirHdr* hdr = (DirHdr*)base;
  const int64_t nblk = dir_nblocks(nev);
  int64_t* bsum = (int64_t*)(base + dir_align(sizeof(DirHdr)));
  int64_t* rel_rank = (int64_t*)(base + dir_align(sizeof(DirHdr)) + dir_align(3 * nblk * 8));
  const int64_t* rows = ev_row_in ? ev_row_in : ev_row_out;
  DirEvictPlan e;
  e.nblk = nblk;
  e.rel_nblk = rel_cnt ? 0 : nblk;
  e.fused = desc || nblk <= kFusedScanBlocks;   // device-driven: the apply kernel's live blocks sum the counts
  const DevCount n = dcount(nev, desc, kDNev);
  e.count = DirEvictCount{S, P, ev_slot, n, ev_row_in, thr_in, ev_row_out, rep, ev_dyn, bsum, nblk, hdr,
                          rel_cnt != nullptr};
  e.apply = DirEvictApply{S, P, ev_slot, n, rows, rep, ev_dyn, evl_ids, evf_slots, bsum, nblk, hdr, rel_rank,
                          e.fused, rel_cnt};
  e.release = DirEvictRelease{S, P, ev_slot, n, rows, rep, rel_rank, hdr};
  return e;
}

void dir_evict_scan(const DirEvictPlan& e, hipStream_t strm) {
  if (!e.fused) k_dir_scan<<<1, kScanBlock, 0, strm>>>(e.count.st, 0, 0, e.count.bsum, e.nblk, 3, e.count.hdr);
}

DirBPlan dir_b_plan(const elr_dir_state& S, const elr_dir_params& P, const int64_t* a_rows, const int64_t* a_k,
                    int64_t na, const DirBItems& it, int64_t s, int64_t* a_ids, int64_t* c_slots, void* scratch,
                    const int64_t* desc) {
  char* base = (char*)scratch;
  DirHdr* hdr = (DirHdr*)base;
  const int64_t nblk_c = dir_nblocks(it.nr + it.nc), nblk_a = dir_nblocks(na);
  int64_t* bsum = (int64_t*)(base + dir_align(sizeof(DirHdr)));
  DirBPlan e;
  e.na = na;
  e.nblk_c = nblk_c;
  e.fused = desc || nblk_c <= kFusedScanBlocks;   // device-driven: the compaction kernel's live blocks sum the counts
  DirBItems itd = it;
  itd.desc = desc;
  e.count = DirBCount{S, P, a_rows, a_k, na, itd, (int32_t)s, a_ids, bsum, nblk_c, nblk_a, hdr, desc};
  e.count_blocks = nblk_a + nblk_c;
  e.compact = DirBCompact{S, P, itd, c_slots, bsum, nblk_c, hdr, e.fused, na, desc};
  // fused: at least one block, which advances the counters also when there are only appends
  e.compact_blocks = e.fused ? (nblk_c ? nblk_c : 1) : nblk_c;
  return e;
}

void dir_b_scan(const DirBPlan& e, hipStream_t strm) {
  if (!e.fused) k_dir_scan<<<1, kScanBlock, 0, strm>>>(e.count.st, 1, e.na, e.count.bsum, e.nblk_c, 2, e.count.hdr);
}

int dir_a_check(const elr_dir_state* st, const elr_dir_params* p, const int64_t* hs, int64_t nh, const int64_t* L_row,
                const int32_t* L_cnt, int64_t nL, const int64_t* ev_slot, int64_t nev, int32_t* L_steps,
                int32_t* L_ids, int64_t* hrec_dyn, int64_t* hrec_j, int64_t* ev_row, uint8_t* rep, int64_t* evl_ids,
                int64_t* evf_slots, int64_t* ev_dyn, void* scratch, int64_t scratch_bytes) {
  if (!params_ok(st, p) || nh < 0 || nL < 0 || nev < 0) return ELR_EINVAL;
  if ((nh && (!hs || !hrec_dyn || !hrec_j)) || (nL && (!L_row || !L_cnt || !L_steps || !L_ids)) ||
      (nev && (!ev_slot || !ev_row || !rep || !evl_ids || !evf_slots || !ev_dyn)))
    return ELR_EINVAL;
  if (nev && (!scratch || scratch_bytes < dir_a_scratch(nev))) return ELR_ECAPACITY;
  return ELR_OK;
}

DirLstepsHits dir_lsteps_hits_prep(const elr_dir_state& S, const elr_dir_params& P, const int64_t* hs, int64_t nh,
                                   const int64_t* L_row, const int32_t* L_cnt, int64_t nL, int64_t s,
                                   int32_t* L_steps, int32_t* L_ids, int64_t* hrec_dyn, int64_t* hrec_j,
                                   const int64_t* desc, int64_t& blocks) {
  const int64_t n1 = nL * P.K + nh;
  blocks = n1 ? dir_nblocks(n1) : 0;
  return DirLstepsHits{S, P, hs, dcount(nh, desc, kDNh), L_row, L_cnt, dcount(nL, desc, kDNL), (int32_t)s, L_steps,
                       L_ids, hrec_dyn, hrec_j};
}

void dir_lsteps_hits_launch(const elr_dir_state& S, const elr_dir_params& P, const int64_t* hs, int64_t nh,
                            const int64_t* L_row, const int32_t* L_cnt, int64_t nL, int64_t s, int32_t* L_steps,
                            int32_t* L_ids, int64_t* hrec_dyn, int64_t* hrec_j, hipStream_t strm,
                            const int64_t* desc) {
  int64_t blocks;
  const DirLstepsHits f = dir_lsteps_hits_prep(S, P, hs, nh, L_row, L_cnt, nL, s, L_steps, L_ids, hrec_dyn, hrec_j,
                                               desc, blocks);
  launch1(f, blocks, strm);
}

int dir_b_check(const elr_dir_state* st, const elr_dir_params* p, const int64_t* a_rows, const int64_t* a_k,
                int64_t na, const int64_t* c_rows, const int64_t* c_cnt, int64_t nc, const int64_t* r_rows,
                const int64_t* r_cnt, int64_t nr, int64_t* a_ids, int64_t* c_slots, void* scratch,
                int64_t scratch_bytes) {
  if (!params_ok(st, p) || na < 0 || nc < 0 || nr < 0) return ELR_EINVAL;
  if ((na && (!a_rows || !a_k || !a_ids)) || (nc && (!c_rows || !c_cnt || !c_slots)) || (nr && (!r_rows || !r_cnt)))
    return ELR_EINVAL;
  if (na == 0 && nc == 0 && nr == 0) return ELR_OK;
  if (!scratch || scratch_bytes < dir_b_scratch(nr + nc)) return ELR_ECAPACITY;
  return ELR_OK;
}

// The eviction part of call A (A2..A5) over nev slots; rows come from ev_row_in when given (then ev_row_out is
// not written and may be NULL).
static void launch_evict(const elr_dir_state& S, const elr_dir_params& P, const int64_t* ev_slot, int64_t nev,
                         const int64_t* ev_row_in, const int8_t* thr_in, int64_t* ev_row_out, uint8_t* rep,
                         int64_t* evl_ids, int64_t* evf_slots, int64_t* ev_dyn, int64_t* rel_cnt, void* scratch,
                         hipStream_t strm) {
  const DirEvictPlan e = dir_evict_plan(S, P, ev_slot, nev, ev_row_in, thr_in, ev_row_out, rep, evl_ids, evf_slots,
                                        ev_dyn, rel_cnt, scratch);
  launch1(e.count, e.nblk, strm);
  dir_evict_scan(e, strm);
  launch1(e.apply, e.nblk, strm);
  launch1(e.release, e.rel_nblk, strm);
}

static int dir_a_impl(const elr_dir_state* st, const elr_dir_params* p, const int64_t* hs, int64_t nh,
                      const int64_t* L_row, const int32_t* L_cnt, int64_t nL, const int64_t* ev_slot, int64_t nev,
                      int64_t s, int32_t* L_steps, int32_t* L_ids, int64_t* hrec_dyn, int64_t* hrec_j,
                      int64_t* ev_row, uint8_t* rep, int64_t* evl_ids, int64_t* evf_slots, int64_t* ev_dyn,
                      int64_t* rel_cnt, void* scratch, int64_t scratch_bytes, void* stream) {
  int rc = dir_a_check(st, p, hs, nh, L_row, L_cnt, nL, ev_slot, nev, L_steps, L_ids, hrec_dyn, hrec_j, ev_row, rep,
                       evl_ids, evf_slots, ev_dyn, scratch, scratch_bytes);
  if (rc) return rc;
  hipStream_t strm = (hipStream_t)stream;
  const elr_dir_state S = *st;
  const elr_dir_params P = *p;
  dir_lsteps_hits_launch(S, P, hs, nh, L_row, L_cnt, nL, s, L_steps, L_ids, hrec_dyn, hrec_j, strm);
  if (nev)
    launch_evict(S, P, ev_slot, nev, nullptr, nullptr, ev_row, rep, evl_ids, evf_slots, ev_dyn, rel_cnt, scratch,
                 strm);
  return launch_status();
}

static int dir_evict_impl(const elr_dir_state* st, const elr_dir_params* p, const int64_t* ev_slot,
                          const int64_t* ev_row, const int8_t* thr, int64_t nev, uint8_t* rep, int64_t* evl_ids,
                          int64_t* evf_slots, int64_t* ev_dyn, int64_t* rel_cnt, void* scratch,
                          int64_t scratch_bytes, void* stream) {
  if (!params_ok(st, p) || nev < 0) return ELR_EINVAL;
  if (nev == 0) return ELR_OK;
  if (!ev_slot || !ev_row || !thr || !rep || !evl_ids || !evf_slots || !ev_dyn) return ELR_EINVAL;
  if (!scratch || scratch_bytes < dir_a_scratch(nev)) return ELR_ECAPACITY;
  launch_evict(*st, *p, ev_slot, nev, ev_row, thr, nullptr, rep, evl_ids, evf_slots, ev_dyn, rel_cnt, scratch,
               (hipStream_t)stream);
  return launch_status();
}

}  // namespace elr

extern "C" int64_t elr_dir_scratch_bytes(int64_t nev, int64_t nc) {
  if (nev < 0 || nc < 0) return ELR_EINVAL;
  const int64_t a = elr::dir_a_scratch(nev), b = elr::dir_b_scratch(nc);
  return a > b ? a : b;
}

extern "C" int elr_dir_a(const elr_dir_state* st, const elr_dir_params* p, const int64_t* hs, int64_t nh,
                         const int64_t* L_row, const int32_t* L_cnt, int64_t nL, const int64_t* ev_slot, int64_t nev,
                         int64_t s, int32_t* L_steps, int32_t* L_ids, int64_t* hrec_dyn, int64_t* hrec_j,
                         int64_t* ev_row, uint8_t* rep, int64_t* evl_ids, int64_t* evf_slots, int64_t* ev_dyn,
                         void* scratch, int64_t scratch_bytes, void* stream) {
  return elr::dir_a_impl(st, p, hs, nh, L_row, L_cnt, nL, ev_slot, nev, s, L_steps, L_ids, hrec_dyn, hrec_j, ev_row,
                         rep, evl_ids, evf_slots, ev_dyn, nullptr, scratch, scratch_bytes, stream);
}

extern "C" int elr_dir_a_deferred(const elr_dir_state* st, const elr_dir_params* p, const int64_t* hs, int64_t nh,
                                  const int64_t* L_row, const int32_t* L_cnt, int64_t nL, const int64_t* ev_slot,
                                  int64_t nev, int64_t s, int32_t* L_steps, int32_t* L_ids, int64_t* hrec_dyn,
                                  int64_t* hrec_j, int64_t* ev_row, uint8_t* rep, int64_t* evl_ids,
                                  int64_t* evf_slots, int64_t* ev_dyn, int64_t* rel_cnt, void* scratch,
                                  int64_t scratch_bytes, void* stream) {
  if (nev && !rel_cnt) return ELR_EINVAL;
  return elr::dir_a_impl(st, p, hs, nh, L_row, L_cnt, nL, ev_slot, nev, s, L_steps, L_ids, hrec_dyn, hrec_j, ev_row,
                         rep, evl_ids, evf_slots, ev_dyn, rel_cnt, scratch, scratch_bytes, stream);
}

extern "C" int elr_dir_evict(const elr_dir_state* st, const elr_dir_params* p, const int64_t* ev_slot,
                             const int64_t* ev_row, const int8_t* thr, int64_t nev, uint8_t* rep, int64_t* evl_ids,
                             int64_t* evf_slots, int64_t* ev_dyn, void* scratch, int64_t scratch_bytes,
                             void* stream) {
  return elr::dir_evict_impl(st, p, ev_slot, ev_row, thr, nev, rep, evl_ids, evf_slots, ev_dyn, nullptr, scratch,
                             scratch_bytes, stream);
}

extern "C" int elr_dir_evict_deferred(const elr_dir_state* st, const elr_dir_params* p, const int64_t* ev_slot,
                                      const int64_t* ev_row, const int8_t* thr, int64_t nev, uint8_t* rep,
                                      int64_t* evl_ids, int64_t* evf_slots, int64_t* ev_dyn, int64_t* rel_cnt,
                                      void* scratch, int64_t scratch_bytes, void* stream) {
  if (nev > 0 && !rel_cnt) return ELR_EINVAL;
  return elr::dir_evict_impl(st, p, ev_slot, ev_row, thr, nev, rep, evl_ids, evf_slots, ev_dyn, rel_cnt, scratch,
                             scratch_bytes, stream);
}

extern "C" int elr_dir_b_release(const elr_dir_state* st, const elr_dir_params* p, const int64_t* a_rows,
                                 const int64_t* a_k, int64_t na, const int64_t* c_rows, const int64_t* c_cnt,
                                 int64_t nc, int c_release, const int64_t* r_rows, const int64_t* r_cnt, int64_t nr,
                                 int64_t s, int64_t* a_ids, int64_t* c_slots, void* scratch, int64_t scratch_bytes,
                                 void* stream) {
  using namespace elr;
  const int rc = dir_b_check(st, p, a_rows, a_k, na, c_rows, c_cnt, nc, r_rows, r_cnt, nr, a_ids, c_slots, scratch,
                             scratch_bytes);
  if (rc || (na == 0 && nc == 0 && nr == 0)) return rc;
  hipStream_t strm = (hipStream_t)stream;
  const DirBItems it{c_rows, c_cnt, nc, r_rows, r_cnt, nr, c_release != 0};
  const DirBPlan e = dir_b_plan(*st, *p, a_rows, a_k, na, it, s, a_ids, c_slots, scratch);
  launch1(e.count, e.count_blocks, strm);
  dir_b_scan(e, strm);
  launch1(e.compact, e.compact_blocks, strm);
  return launch_status();
}

extern "C" int elr_dir_b(const elr_dir_state* st, const elr_dir_params* p, const int64_t* a_rows, const int64_t* a_k,
                         int64_t na, const int64_t* c_rows, const int64_t* c_cnt, int64_t nc, int64_t s,
                         int64_t* a_ids, int64_t* c_slots, void* scratch, int64_t scratch_bytes, void* stream) {
  return elr_dir_b_release(st, p, a_rows, a_k, na, c_rows, c_cnt, nc, 1, nullptr, nullptr, 0, s, a_ids, c_slots,
                           scratch, scratch_bytes, stream);
}
