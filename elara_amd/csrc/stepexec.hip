// The rest of a planned ELARA step in one call (elr_step_exec): directory call A, the admissions with their
// pool-slot bookkeeping, directory call B, the fused assembly and the update (srm2/elara.py:271-414, 471-580), with
// every intermediate array carved from one workspace.  Each piece keeps its entry point's checks and kernels.
//
// The directory's eviction, admission and call-B kernels are small launches (a few dozen blocks each) that wait on
// one another.  Each of the first four shares its launch with a large row kernel that does not depend on it
// (elr_launch.h), in this order:
//   1. call A's replay inputs and hit records
//   2. eviction counts   + the hits' Adam pass
//   3. eviction apply    + the assembly of the work rows
//   4. eviction release  + the eviction moves (states to MAT, histories to the log arena)
//   5. admissions        + call B's appends and counts
//   6. call B's compactions
//   7. the admitted, compacted, transient and appended rows; 8. the S rows
// (and the directory's scan launches for grids above kFusedScanBlocks).  In the Triton path's order (dir_order 1)
// launch 4 holds no release: the host logs of rows going to M are pushed by call B's compaction launch, ahead of
// the compacted rows' logs and after the appends' pops.  The pairs touch disjoint data: the
// eviction kernels read and write only the directory, and their outputs feed later launches; the assembly reads the
// replay inputs of launch 1, the log and MAT rows of L and F rows and the F rows' MAT slots; the hits write their
// pool slots and history records, which the eviction moves read two launches later (a hit's slot may be evicted in
// the same step); the moves read evf_slots and evl_ids of launch 3; the admissions write the slots the eviction
// kernels of launches 2-4 read, and call B pops the log ids that launch 4 pushed.  (Pairing the apply kernel, the
// largest of the eviction kernels in registers, with the assembly rather than the Adam pass keeps both pairs at the
// occupancy of their row kernel.)  In the device-driven step (elr_step_dev) launch 1 shares its launch with the
// segment sum's final kernel: both read only the plan's scatter and the sum writes only the per-row gradients G,
// which neither launch 1 nor the directory reads, while launch 1 writes the replay inputs, the hits' history records
// and the directory's pstep / rj / rok, which the sum does not touch.
#include "elr_admit_dev.h"
#include "elr_asm_dev.h"
#include "elr_dir_dev.h"
#include "elr_exec_dev.h"
#include "elr_seg_dev.h"

namespace {

struct ExecLayout {
  elr_exec_out o;
  int64_t rel_cnt;  // the evictions' deferred release counts (Triton order only)
  int64_t stage_mat, stage_log;  // with a link stream: the evicted states and histories staged in HBM
  int64_t dir_a_scratch, dir_a_scratch_bytes, dir_b_scratch, dir_b_scratch_bytes, total;
};

int64_t al256(int64_t b) { return (b + 255) & ~int64_t(255); }
int64_t cap(int64_t blocks, int64_t lim) { return blocks < lim ? blocks : lim; }

// Byte layout of the workspace for args; false when the bounds are inconsistent.
bool exec_layout(const elr_exec_args& a, ExecLayout& L) {
  const int64_t* b = a.b;
  for (int r = 0; r < ELR_NRANK; ++r)
    if (b[r] < 0 || b[r + 1] < b[r]) return false;
  const int64_t K = a.pv.K, D = a.upd.D;
  if (K < 1 || D < 1 || a.slots.nev < 0 || (a.dir_order != 0 && a.dir_order != 1)) return false;
  const int64_t nh = b[ELR_RANK_HIT + 1] - b[ELR_RANK_HIT];
  const int64_t nL = (b[ELR_RANK_LADM + 1] - b[ELR_RANK_LADM]) + (b[ELR_RANK_LAPP + 1] - b[ELR_RANK_LAPP]) +
                     (b[ELR_RANK_LCMP + 1] - b[ELR_RANK_LCMP]);
  const int64_t nev = a.slots.nev, n_adm = b[ELR_RANK_FADM + 1] - b[ELR_RANK_NADM];
  const int64_t na = b[ELR_RANK_LAPP + 1] - b[ELR_RANK_NAPP], nc = b[ELR_RANK_LCMP + 1] - b[ELR_RANK_NCMP];
  const int64_t nw = b[ELR_RANK_S] - b[ELR_RANK_NADM];
  int64_t o = 0;
  auto take = [&](int64_t bytes) {
    const int64_t at = o;
    o += al256(bytes);
    return at;
  };
  L.o.L_steps = take(nL * K * 4);
  L.o.L_ids = take(nL * K * 4);
  L.o.hrec_dyn = take(nh * 8);
  L.o.hrec_j = take(nh * 8);
  L.o.ev_row = take(nev * 8);
  L.o.rep = take(nev);
  L.o.evl_ids = take(nev * K * 8);
  L.o.evf_slots = take(nev * 8);
  L.o.ev_dyn = take(nev * 8);
  L.o.adm_slots = take(n_adm * 8);
  L.o.a_ids = take(na * 8);
  L.o.c_slots = take(nc * 8);
  L.o.work = take(nw * 3 * D * 4);
  const int64_t nr = a.dir_order ? nev : 0;
  L.rel_cnt = take(nr * 8);
  L.dir_a_scratch_bytes = elr_dir_scratch_bytes(nev, 0);
  L.dir_b_scratch_bytes = elr_dir_scratch_bytes(0, nc + nr);
  if (L.dir_a_scratch_bytes < 0 || L.dir_b_scratch_bytes < 0) return false;
  L.dir_a_scratch = take(L.dir_a_scratch_bytes > 0 ? L.dir_a_scratch_bytes : 1);
  L.dir_b_scratch = take(L.dir_b_scratch_bytes > 0 ? L.dir_b_scratch_bytes : 1);
  L.stage_mat = take(a.link_stream ? nev * 3 * D * 4 : 0);
  L.stage_log = take(a.link_stream ? nev * K * D * 4 : 0);
  L.total = o;
  return true;
}

}  // namespace

extern "C" int64_t elr_step_exec_bytes(const elr_exec_args* args) {
  if (!args) return ELR_EINVAL;
  ExecLayout L;
  if (!exec_layout(*args, L)) return ELR_EINVAL;
  return L.total;
}

extern "C" int elr_step_exec(const elr_exec_args* args, void* ws, int64_t ws_bytes, elr_exec_out* out, void* stream) {
  using namespace elr;
  if (!args || !out) return ELR_EINVAL;
  const elr_exec_args& a = *args;
  ExecLayout L;
  if (!exec_layout(a, L) || (a.link_stream && (!a.link_start || !a.link_done))) return ELR_EINVAL;
  if (!ws || ws_bytes < L.total || (reinterpret_cast<uintptr_t>(ws) & 255)) return ELR_ECAPACITY;
  *out = L.o;
  char* w = static_cast<char*>(ws);
  auto at = [&](int64_t off) { return static_cast<void*>(w + off); };
  const int64_t* b = a.b;
  const int64_t K = a.pv.K, D = a.upd.D, s = a.s;
  const int64_t nh = b[ELR_RANK_HIT + 1] - b[ELR_RANK_HIT];
  const int64_t nLa = b[ELR_RANK_LADM + 1] - b[ELR_RANK_LADM], nLp = b[ELR_RANK_LAPP + 1] - b[ELR_RANK_LAPP],
                nLc = b[ELR_RANK_LCMP + 1] - b[ELR_RANK_LCMP], nL = nLa + nLp + nLc;
  const int64_t nNa = b[ELR_RANK_NADM + 1] - b[ELR_RANK_NADM];
  const int64_t nev = a.slots.nev, n_adm = b[ELR_RANK_FADM + 1] - b[ELR_RANK_NADM];
  const int64_t na = b[ELR_RANK_LAPP + 1] - b[ELR_RANK_NAPP], nc = b[ELR_RANK_LCMP + 1] - b[ELR_RANK_NCMP];
  const int64_t w0 = b[ELR_RANK_NADM], nw = b[ELR_RANK_S] - w0;
  const int64_t lazy_n = nNa + nLa;
  const bool evl = a.pv.evl != 0;
  // Triton order: the host logs of rows going to M are released by call B, after its appends
  const int64_t nr = a.dir_order ? nev : 0;
  int64_t* rel_cnt = a.dir_order ? static_cast<int64_t*>(at(L.rel_cnt)) : nullptr;
  int32_t* L_steps = static_cast<int32_t*>(at(L.o.L_steps));
  int32_t* L_ids = static_cast<int32_t*>(at(L.o.L_ids));
  int64_t* hrec_dyn = static_cast<int64_t*>(at(L.o.hrec_dyn));
  int64_t* hrec_j = static_cast<int64_t*>(at(L.o.hrec_j));
  int64_t* evl_ids = static_cast<int64_t*>(at(L.o.evl_ids));
  int64_t* evf_slots = static_cast<int64_t*>(at(L.o.evf_slots));
  int64_t* ev_dyn = static_cast<int64_t*>(at(L.o.ev_dyn));
  int64_t* adm_slots = static_cast<int64_t*>(at(L.o.adm_slots));
  int64_t* a_ids = static_cast<int64_t*>(at(L.o.a_ids));
  int64_t* c_slots = static_cast<int64_t*>(at(L.o.c_slots));
  float* work = static_cast<float*>(at(L.o.work));
  int rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  int64_t* ev_row = static_cast<int64_t*>(at(L.o.ev_row));
  uint8_t* rep = static_cast<uint8_t*>(at(L.o.rep));
  // call A: replay inputs of the L rows, history records of the hits, the evictions
  if ((rc = dir_a_check(&a.dir, &a.pv, a.sl_ord + b[ELR_RANK_HIT], nh, a.L_row, a.L_cnt, nL, a.slots.ev_slot, nev,
                        L_steps, L_ids, hrec_dyn, hrec_j, ev_row, rep, evl_ids, evf_slots, ev_dyn,
                        at(L.dir_a_scratch), L.dir_a_scratch_bytes)))
    return rc;
  // admissions: the evicted slots pushed on the free stack, the admitted rows' slots popped from its top
  elr_slots_args sl = a.slots;
  sl.adm_slots = adm_slots;
  const int64_t C = a.pv.n0 + a.pv.Cdyn;
  if ((rc = admit_slots_check(sl, a.u_ord + w0, n_adm, lazy_n, a.pv.n0, C, a.pv.R, (int)K, a.dir.code, a.dir.slot_of,
                              a.dir.slot_row, a.dir.adm_c0, a.dir.rj, a.dir.rok, a.dir.pstep)))
    return rc;
  const PlanAdmitSlots admit{sl, a.u_ord + w0, n_adm, lazy_n, evl ? 1 : 0, s, a.pv.n0, C, a.pv.R, (int)K,
                             a.dir.code, a.dir.slot_of, a.dir.slot_row, a.dir.adm_c0, a.dir.rj, a.dir.rok,
                             a.dir.pstep};
  // call B: appends (entry index = the row's current count) and compactions of the non-resident lazy rows
  const int64_t* a_rows = a.u_ord + b[ELR_RANK_NAPP];
  const int64_t* a_k = a.c_ord + b[ELR_RANK_NAPP];
  const int64_t* c_rows = a.u_ord + b[ELR_RANK_NCMP];
  const int64_t* c_cnt = a.c_ord + b[ELR_RANK_NCMP];
  if ((rc = dir_b_check(&a.dir, &a.pv, a_rows, a_k, na, c_rows, c_cnt, nc, ev_row, rel_cnt, nr, a_ids, c_slots,
                        at(L.dir_b_scratch), L.dir_b_scratch_bytes)))
    return rc;
  // the work rows in class-rank order: admitted N / L / F, appended N / L, compacted N / L, transient F
  elr_assemble_args g{};
  g.work = work;
  g.rows = a.u_ord + w0;
  g.n = nw;
  g.D = D;
  g.K = (int)K;
  const int rank_of[8] = {ELR_RANK_NADM, ELR_RANK_LADM, ELR_RANK_FADM, ELR_RANK_NAPP,
                          ELR_RANK_LAPP, ELR_RANK_NCMP, ELR_RANK_LCMP, ELR_RANK_FN};
  const int kind_of[8] = {ELR_ASM_INIT, ELR_ASM_REPLAY, ELR_ASM_GATHER, ELR_ASM_INIT,
                          ELR_ASM_REPLAY, ELR_ASM_INIT, ELR_ASM_REPLAY, ELR_ASM_GATHER};
  const int64_t aux_of[8] = {0, 0, 0, 0, nLa, 0, nLa + nLp, 0};
  g.nseg = 8;
  for (int q = 0; q < 8; ++q) {
    g.seg_end[q] = b[rank_of[q] + 1] - w0;
    g.seg_kind[q] = kind_of[q];
    g.seg_aux[q] = aux_of[q];
  }
  g.seed = a.seed;
  g.bound = a.bound;
  g.L_ids = L_ids;
  g.L_steps = L_steps;
  g.L_cnt = a.L_cnt;
  g.nL = nL;
  g.logs = a.upd.logs;
  g.nlogs = a.upd.log_rows;
  g.table = a.table;
  g.recip = a.recip;
  g.table_rows = a.table_rows;
  g.mat = a.upd.mat;
  g.mat_rows = a.upd.mat_rows;
  g.loc = a.dir.loc;
  g.R = a.pv.R;
  if (nw > 0 && (rc = assemble_check(g))) return rc;
  // the update: hits, evictions, admissions, compactions, transient and S rows, log appends
  elr_update_args u = a.upd;
  for (int r = 0; r <= ELR_NRANK; ++r) u.b[r] = b[r];
  u.K = K;
  u.work = work;
  u.step = s;
  u.evl = evl ? 1 : 0;
  u.hit_slot = a.sl_ord + b[ELR_RANK_HIT];
  u.hrec_dyn = evl ? hrec_dyn : nullptr;
  u.hrec_j = evl ? hrec_j : nullptr;
  u.nev = nev;
  u.ev_slot = a.slots.ev_slot;
  u.evf_slots = evf_slots;
  u.evl_ids = evl_ids;
  u.ev_dyn = ev_dyn;
  u.adm_slots = adm_slots;
  u.lazy_n = lazy_n;
  u.n0 = a.pv.n0;
  u.c_slots = c_slots;
  u.a_ids = a_ids;
  u.fn_slot = a.loc_ord + b[ELR_RANK_FN];
  u.s_slot = a.loc_ord + b[ELR_RANK_S];
  u.part = ELR_UPDATE_ALL;
  u.link_blocks = a.link_stream ? a.upd.link_blocks : 0;
  UpdatePrep up;
  if ((rc = update_prep(&u, up))) return rc;
  ExecMulti hx;
  int64_t hblocks;
  exec_multi({up.hits}, int64_t(1) << 20, hx, hblocks);

  // 1.
  const elr_dir_state S = a.dir;
  const elr_dir_params P = a.pv;
  dir_lsteps_hits_launch(S, P, a.sl_ord + b[ELR_RANK_HIT], nh, a.L_row, a.L_cnt, nL, s, L_steps, L_ids, hrec_dyn,
                         hrec_j, st);
  // 2-4. (without evictions: the assembly, the hits and no moves)
  const int64_t ev_blocks = nev ? dir_nblocks(nev) : 0;
  DirEvictPlan ep{};
  if (nev)
    ep = dir_evict_plan(S, P, a.slots.ev_slot, nev, nullptr, nullptr, ev_row, rep, evl_ids, evf_slots, ev_dyn,
                        rel_cnt, at(L.dir_a_scratch));
  exec_visit(up.vpl, D, hx, hblocks, up.s, [&](const auto& f, int64_t nb) { launch2(ep.count, ev_blocks, f, nb, st); });
  if (nev) dir_evict_scan(ep, st);
  if (a.link_wait && (rc = hip_rc(hipStreamWaitEvent(st, static_cast<hipEvent_t>(a.link_wait), 0)))) return rc;
  if (nw > 0) assemble_visit(g, [&](const auto& f, int64_t nb) { launch2(ep.apply, ev_blocks, f, nb, st); });
  else launch1(ep.apply, ev_blocks, st);
  hipStream_t lk = static_cast<hipStream_t>(a.link_stream);
  // with a link stream, the evicted states and histories are staged in HBM here (before the admissions reuse their
  // slots) and written to the host arenas on the link stream, with the update's other host-arena writes
  float* stage_mat = lk ? static_cast<float*>(at(L.stage_mat)) : nullptr;
  float* stage_log = lk ? static_cast<float*>(at(L.stage_log)) : nullptr;
  const EvictMove& mv = up.move;
  const EvictMove stage{{stage_mat, nev, IxList{nullptr}, mv.c1.src, mv.c1.src_rows, mv.c1.six, nev, 3 * D, nullptr,
                         1},
                        {stage_log, nev * K, IxList{nullptr}, mv.c2.src, mv.c2.src_rows, mv.c2.six, nev * K, D,
                         nullptr, K},
                        mv.nb1, mv.nb2, mv.v4 && aligned16(stage_mat) && aligned16(stage_log)};
  if (nev)
    evict_move_visit(lk ? stage : mv,
                     [&](const auto& f, int64_t nb) { launch2(ep.release, ep.rel_nblk, f, nb, st); });
  // 5-6.
  const int64_t adm_blocks = admit_slots_blocks(sl, n_adm);
  if (na || nc || nr) {
    const DirBItems it{c_rows, c_cnt, nc, ev_row, rel_cnt, nr, true};
    const DirBPlan bp = dir_b_plan(S, P, a_rows, a_k, na, it, s, a_ids, c_slots, at(L.dir_b_scratch));
    launch2(admit, adm_blocks, bp.count, bp.count_blocks, st);
    dir_b_scan(bp, st);
    launch1(bp.compact, bp.compact_blocks, st);
  } else {
    launch1(admit, adm_blocks, st);
  }
  // 7-8.
  if ((rc = launch_status())) return rc;
  if (!lk) {
    if ((rc = adam_exec(up, {up.adm, up.tail, up.app}, st))) return rc;
    return update_s_rows(up, st);
  }
  // the host-arena writes on the link stream, after everything above
  if ((rc = adam_exec(up, {up.adm}, st))) return rc;
  if ((rc = hip_rc(hipEventRecord(static_cast<hipEvent_t>(a.link_start), st))) ||
      (rc = hip_rc(hipStreamWaitEvent(lk, static_cast<hipEvent_t>(a.link_start), 0))))
    return rc;
  if (nev) {   // the staged evictions into the host arenas
    const CopyPart<IxList, IxList> o1{mv.c1.dst, mv.c1.dst_rows, mv.c1.dix, stage_mat, nev, IxList{nullptr}, nev,
                                      3 * D, nullptr, 1};
    const CopyPart<IxList, IxList> o2{mv.c2.dst, mv.c2.dst_rows, mv.c2.dix, stage_log, nev * K, IxList{nullptr},
                                      nev * K, D, nullptr, K};
    const int64_t nb1 = cap(mv.nb1, up.lb), nb = nb1 + cap(mv.nb2, up.lb);
    if (stage.v4) launch1(CopyRows2<true, IxList, IxList, IxList, IxList>{o1, o2, nb1}, nb, lk);
    else launch1(CopyRows2<false, IxList, IxList, IxList, IxList>{o1, o2, nb1}, nb, lk);
  }
  if ((rc = adam_exec(up, {up.tail}, lk, up.lb)) || (rc = adam_exec(up, {up.app}, lk, up.lb)) ||
      (rc = update_s_rows(up, lk)))
    return rc;
  return hip_rc(hipEventRecord(static_cast<hipEvent_t>(a.link_done), lk));
}

// ---- the device-driven form (elr_step_exec_dev) ------------------------------------------------------------------
// The same launches with every count and class-order offset read from the step descriptor that elr_plan_step wrote:
// b[ELR_NRANK] of the arguments bounds the batch's rows, slots.nev the evictions (and the admissions and kept slots
// with it), and the workspace is laid out for those bounds.  Row kernels run on grids capped at kDevRowBlocks blocks
// whose waves loop over the rows; the directory kernels' grids cover the bounds and their blocks past the items exit
// at once.  The S rows' Adam is the fourth part of the last launch.

namespace {

constexpr int64_t kDevRowBlocks = 4096;
// The assembly keeps one work row per wave for the rows of a large batch (C5: about 37k rows; 65k waves here): its
// rows' loads are then all in flight at once, where a looping wave would wait for its stores before the next
// row's loads.
constexpr int64_t kDevAsmBlocks = 16384;

struct DevBounds {
  int64_t n, nev, nadm, nkeep, nfree;
};

bool dev_bounds(const elr_exec_args& a, DevBounds& v) {
  v.n = a.b[ELR_NRANK];
  v.nev = a.slots.nev;
  v.nkeep = a.slots.nkeep;
  v.nfree = a.slots.n_free;
  const int64_t C = a.pv.n0 + a.pv.Cdyn;
  v.nadm = v.n < C ? v.n : C;
  return v.n >= 1 && v.nev >= 0 && v.nkeep >= 0 && v.nfree >= 0 && v.nev <= a.pv.Cdyn && v.nkeep <= a.pv.Cdyn &&
         v.nfree <= C && a.pv.K >= 1 && a.upd.D >= 1 && (a.dir_order == 0 || a.dir_order == 1);
}

// Byte layout of the device-driven workspace: every array at its bound.
bool exec_layout_dev(const elr_exec_args& a, ExecLayout& L) {
  DevBounds v;
  if (!dev_bounds(a, v)) return false;
  const int64_t K = a.pv.K, D = a.upd.D, n = v.n, nev = v.nev;
  int64_t o = 0;
  auto take = [&](int64_t bytes) {
    const int64_t at = o;
    o += al256(bytes);
    return at;
  };
  L.o.L_steps = take(n * K * 4);
  L.o.L_ids = take(n * K * 4);
  L.o.hrec_dyn = take(n * 8);
  L.o.hrec_j = take(n * 8);
  L.o.ev_row = take(nev * 8);
  L.o.rep = take(nev);
  L.o.evl_ids = take(nev * K * 8);
  L.o.evf_slots = take(nev * 8);
  L.o.ev_dyn = take(nev * 8);
  L.o.adm_slots = take(v.nadm * 8);
  L.o.a_ids = take(n * 8);
  L.o.c_slots = take(n * 8);
  L.o.work = take(n * 3 * D * 4);
  const int64_t nr = a.dir_order ? nev : 0;
  L.rel_cnt = take(nr * 8);
  L.dir_a_scratch_bytes = elr_dir_scratch_bytes(nev, 0);
  L.dir_b_scratch_bytes = elr_dir_scratch_bytes(0, n + nr);
  if (L.dir_a_scratch_bytes < 0 || L.dir_b_scratch_bytes < 0) return false;
  L.dir_a_scratch = take(L.dir_a_scratch_bytes > 0 ? L.dir_a_scratch_bytes : 1);
  L.dir_b_scratch = take(L.dir_b_scratch_bytes > 0 ? L.dir_b_scratch_bytes : 1);
  L.total = o;
  return true;
}

}  // namespace

extern "C" int64_t elr_step_exec_dev_bytes(const elr_exec_args* args) {
  if (!args) return ELR_EINVAL;
  ExecLayout L;
  if (!exec_layout_dev(*args, L)) return ELR_EINVAL;
  return L.total;
}

// The device-driven executor; with lsteps_done its first launch (call A's replay inputs and hit records) was issued
// by the caller already (elr_step_dev runs it beside the segment sum's final kernel).  With mark, the lookahead's
// mark of a batch loaded ahead runs in the compaction's launch, after the stream waits for mark_event (if any).
static int step_exec_dev(const elr_exec_args* args, const int64_t* desc, void* ws, int64_t ws_bytes,
                         elr_exec_out* out, void* stream, bool lsteps_done, const elr::MarkRows* mark = nullptr,
                         hipEvent_t mark_event = nullptr) {
  using namespace elr;
  if (!args || !out || !desc) return ELR_EINVAL;
  const elr_exec_args& a = *args;
  ExecLayout L;
  DevBounds v;
  if (!exec_layout_dev(a, L) || !dev_bounds(a, v) || a.link_stream || a.link_wait) return ELR_EINVAL;
  if (!ws || ws_bytes < L.total || (reinterpret_cast<uintptr_t>(ws) & 255)) return ELR_ECAPACITY;
  *out = L.o;
  char* w = static_cast<char*>(ws);
  auto at = [&](int64_t off) { return static_cast<void*>(w + off); };
  const int64_t K = a.pv.K, D = a.upd.D, s = a.s, n = v.n, nev = v.nev;
  const bool evl = a.pv.evl != 0;
  const int64_t nr = a.dir_order ? nev : 0;
  int64_t* rel_cnt = a.dir_order ? static_cast<int64_t*>(at(L.rel_cnt)) : nullptr;
  int32_t* L_steps = static_cast<int32_t*>(at(L.o.L_steps));
  int32_t* L_ids = static_cast<int32_t*>(at(L.o.L_ids));
  int64_t* hrec_dyn = static_cast<int64_t*>(at(L.o.hrec_dyn));
  int64_t* hrec_j = static_cast<int64_t*>(at(L.o.hrec_j));
  int64_t* evl_ids = static_cast<int64_t*>(at(L.o.evl_ids));
  int64_t* evf_slots = static_cast<int64_t*>(at(L.o.evf_slots));
  int64_t* ev_dyn = static_cast<int64_t*>(at(L.o.ev_dyn));
  int64_t* adm_slots = static_cast<int64_t*>(at(L.o.adm_slots));
  int64_t* a_ids = static_cast<int64_t*>(at(L.o.a_ids));
  int64_t* c_slots = static_cast<int64_t*>(at(L.o.c_slots));
  float* work = static_cast<float*>(at(L.o.work));
  int64_t* ev_row = static_cast<int64_t*>(at(L.o.ev_row));
  uint8_t* rep = static_cast<uint8_t*>(at(L.o.rep));
  hipStream_t st = static_cast<hipStream_t>(stream);
  int rc;
  // the argument checks of the host-count form, at the bounds
  if ((rc = dir_a_check(&a.dir, &a.pv, a.sl_ord, n, a.L_row, a.L_cnt, n, a.slots.ev_slot, nev, L_steps, L_ids,
                        hrec_dyn, hrec_j, ev_row, rep, evl_ids, evf_slots, ev_dyn, at(L.dir_a_scratch),
                        L.dir_a_scratch_bytes)))
    return rc;
  if ((rc = dir_b_check(&a.dir, &a.pv, a.u_ord, a.c_ord, n, a.u_ord, a.c_ord, n, ev_row, rel_cnt, nr, a_ids, c_slots,
                        at(L.dir_b_scratch), L.dir_b_scratch_bytes)))
    return rc;
  const int64_t C = a.pv.n0 + a.pv.Cdyn;
  elr_slots_args sl = a.slots;
  sl.adm_slots = adm_slots;
  if (!sl.free_stack || !sl.ev_slot || !sl.keep || !sl.dyn_out || !a.u_ord || !a.c_ord || !a.sl_ord || !a.loc_ord ||
      !a.upd.grad || !a.upd.pool || !a.upd.mat || !a.upd.logs || !a.upd.glog || a.upd.glog_slots < 1)
    return ELR_EINVAL;
  const PlanAdmitSlots admit{sl, a.u_ord, v.nadm, v.nadm, evl ? 1 : 0, s, a.pv.n0, C, a.pv.R, (int)K,
                             a.dir.code, a.dir.slot_of, a.dir.slot_row, a.dir.adm_c0, a.dir.rj, a.dir.rok,
                             a.dir.pstep, desc, n};
  // the assembly: the rows and the kind of each from the descriptor (one nominal segment for the host checks)
  elr_assemble_args g{};
  g.work = work;
  g.rows = a.u_ord;
  g.n = n;
  g.D = D;
  g.K = (int)K;
  g.nseg = 1;
  g.seg_end[0] = n;
  g.seg_kind[0] = ELR_ASM_INIT;
  g.seed = a.seed;
  g.bound = a.bound;
  g.L_ids = L_ids;
  g.L_steps = L_steps;
  g.L_cnt = a.L_cnt;
  g.nL = n;
  g.logs = a.upd.logs;
  g.nlogs = a.upd.log_rows;
  g.table = a.table;
  g.recip = a.recip;
  g.table_rows = a.table_rows;
  g.mat = a.upd.mat;
  g.mat_rows = a.upd.mat_rows;
  g.loc = a.dir.loc;
  g.R = a.pv.R;
  if ((rc = assemble_check(g))) return rc;
  // the update's parts at their bounds
  const elr_update_args& U = a.upd;
  float sc[8];
  elr_adam_scalars(U.lr, U.b1, U.b2, U.eps, s, sc);
  const AdamScalars scal = make_scalars(sc);
  const float* G = U.grad;
  const int64_t nd = U.glog_slots;
  const bool al = aligned16(U.pool) && aligned16(U.mat) && aligned16(U.glog) && aligned16(work) && aligned16(G) &&
                  aligned16(U.logs);
  const int vpl = al ? wpr_vpl(D) : 0;
  const ExecAdam hits{U.pool, U.pool_rows, a.sl_ord, n, nullptr, nullptr, 0, 0, G, 0, n, U.glog, nd, K, hrec_dyn,
                      hrec_j, 0, evl ? n : 0, 0, kExecHits, desc, n};
  const ExecAdam adm{U.pool, U.pool_rows, adm_slots, v.nadm, nullptr, work, n, 0, G, 0, v.nadm, U.glog, nd, K,
                     nullptr, nullptr, a.pv.n0, evl ? v.nadm : 0, 0, kExecAdm, desc, n};
  const ExecAdam tail{U.mat, U.mat_rows, c_slots, n, a.loc_ord, work, n, 0, G, 0, n, U.glog, nd, K, nullptr, nullptr,
                      0, 0, 0, kExecTail, desc, n};
  const ExecAdam app{U.logs, U.log_rows, a_ids, n, nullptr, nullptr, 0, 0, G, 0, n, nullptr, 0, K, nullptr, nullptr,
                     0, 0, 1, kExecApp, desc, n};
  const ExecAdam srows{U.mat, U.mat_rows, a.loc_ord, n, nullptr, nullptr, 0, 0, G, 0, n, nullptr, 0, K, nullptr,
                       nullptr, 0, 0, 0, kExecS, desc, n};
  ExecMulti hx, tx;
  int64_t hblocks, tblocks;
  if (!exec_multi({hits}, kDevRowBlocks, hx, hblocks) || !exec_multi({adm, tail, app, srows}, kDevRowBlocks, tx, tblocks))
    return ELR_EINVAL;
  const EvictMove move = evict_move_prep(U.mat, U.mat_rows, evf_slots, U.pool, U.pool_rows, a.slots.ev_slot, U.logs,
                                         U.log_rows, evl_ids, U.glog, nd, K, ev_dyn, nev, D, desc);

  // 1. call A's replay inputs and hit records
  const elr_dir_state S = a.dir;
  const elr_dir_params P = a.pv;
  if (!lsteps_done)
    dir_lsteps_hits_launch(S, P, a.sl_ord, n, a.L_row, a.L_cnt, n, s, L_steps, L_ids, hrec_dyn, hrec_j, st, desc);
  // 2-4. eviction counts + the hits; eviction apply + the assembly; eviction release + the eviction moves
  const int64_t ev_blocks = dir_nblocks(nev > 0 ? nev : 1);
  const DirEvictPlan ep = dir_evict_plan(S, P, a.slots.ev_slot, nev, nullptr, nullptr, ev_row, rep, evl_ids,
                                         evf_slots, ev_dyn, rel_cnt, at(L.dir_a_scratch), desc);
  exec_visit(vpl, D, hx, hblocks, scal, [&](const auto& f, int64_t nb) { launch2(ep.count, ev_blocks, f, nb, st); });
  assemble_visit(g, [&](const auto& f, int64_t nb) { launch2(ep.apply, ev_blocks, f, nb, st); }, desc,
                 kDevAsmBlocks);
  evict_move_visit(move, [&](const auto& f, int64_t nb) { launch2(ep.release, ep.rel_nblk ? ev_blocks : 0, f, nb, st); });
  // 5-6. admissions + call B's appends and counts; call B's compactions
  const DirBItems it{a.u_ord, a.c_ord, n, ev_row, rel_cnt, nr, true};
  const DirBPlan bp = dir_b_plan(S, P, a.u_ord, a.c_ord, n, it, s, a_ids, c_slots, at(L.dir_b_scratch), desc);
  launch2(admit, admit_slots_blocks(sl, v.nadm), bp.count, bp.count_blocks, st);
  // no kernel after this step's plan reads last_seen or next_bits, and the next step's plan comes after this; if the
  // wait for the batch's sort cannot be queued, the step is still issued whole and the error returned at its end
  const bool waited = mark && (!mark_event || hipStreamWaitEvent(st, mark_event, 0) == hipSuccess);
  if (waited) launch2(bp.compact, bp.compact_blocks, *mark, mark_rows_blocks(mark->n_max), st);
  else launch1(bp.compact, bp.compact_blocks, st);
  // 7. the admitted, compacted, transient, appended and S rows
  exec_visit(vpl, D, tx, tblocks, scal, [&](const auto& f, int64_t nb) { launch1(f, nb, st); });
  if (mark && !waited) return ELR_EINVAL;
  return launch_status();
}

// ---- the whole device-driven step (elr_step_dev) -------------------------------------------------------------------

namespace {

struct StepDevLayout {
  elr_step_dev_out o;
  int64_t plan_scratch, plan_scratch_bytes, exec_bytes, total;
};

extern "C" int elr_step_exec_dev(const elr_exec_args* args, const int64_t* desc, void* ws, int64_t ws_bytes,
                                 elr_exec_out* out, void* stream) {
  return step_exec_dev(args, desc, ws, ws_bytes, out, stream, false);
}

// Workspace: the plan's outputs at their bounds (n rows, nd dynamic slots), its scratch, G [n, D], then the
// executor's workspace.
bool step_dev_layout(const elr_step_dev_args& a, StepDevLayout& L) {
  const int64_t n = a.plan.n, nd = a.plan.nd, D = a.exec.upd.D;
  if (n < 1 || nd < 0 || D < 1) return false;
  int64_t o = 0;
  auto take = [&](int64_t bytes) {
    const int64_t at = o;
    o += al256(bytes);
    return at;
  };
  L.o.cls = take(n);
  L.o.flags = take(n);
  L.o.sl = take(n * 4);
  L.o.c = take(n);
  L.o.order = take(n * 8);
  L.o.rank = take(n * 8);
  L.o.dyn_out = take(2 * nd * 8);
  L.o.counts = take(17 * 8);
  L.o.u_ord = take(n * 8);
  L.o.c_ord = take(n * 8);
  L.o.sl_ord = take(n * 8);
  L.o.L_row = take(n * 8);
  L.o.L_cnt = take(n * 4);
  L.o.loc_ord = take(n * 8);
  L.plan_scratch_bytes = elr_plan_step_scratch_bytes(n, nd);
  if (L.plan_scratch_bytes < 0) return false;
  L.plan_scratch = take(L.plan_scratch_bytes);
  L.o.grad_rows = take(n * D * 4);
  elr_exec_args e = a.exec;
  e.b[ELR_NRANK] = n;
  L.exec_bytes = elr_step_exec_dev_bytes(&e);
  if (L.exec_bytes < 0) return false;
  L.o.exec_ws = take(L.exec_bytes);
  L.total = o;
  return true;
}

}  // namespace

extern "C" int64_t elr_step_dev_bytes(const elr_step_dev_args* args) {
  if (!args) return ELR_EINVAL;
  StepDevLayout L;
  if (!step_dev_layout(*args, L)) return ELR_EINVAL;
  return L.total;
}

extern "C" int elr_step_dev(const elr_step_dev_args* args, void* ws, int64_t ws_bytes, elr_step_dev_out* out,
                            void* stream) {
  if (!args || !out) return ELR_EINVAL;
  const elr_step_dev_args& a = *args;
  if (a.mark_rows && (!a.mark_n || !a.plan.last_seen || a.mark_nmax < 0 || a.mark_value < INT32_MIN ||
                      a.mark_value > INT32_MAX || a.mark_bit < 0 || a.mark_bit > (int64_t)UINT32_MAX))
    return ELR_EINVAL;
  StepDevLayout L;
  if (!step_dev_layout(a, L)) return ELR_EINVAL;
  if (!ws || ws_bytes < L.total || (reinterpret_cast<uintptr_t>(ws) & 255)) return ELR_ECAPACITY;
  char* w = static_cast<char*>(ws);
  const int64_t n = a.plan.n, D = a.exec.upd.D;
  elr_plan_out po;
  po.cls = reinterpret_cast<int8_t*>(w + L.o.cls);
  po.flags = reinterpret_cast<uint8_t*>(w + L.o.flags);
  po.sl = reinterpret_cast<int32_t*>(w + L.o.sl);
  po.c = reinterpret_cast<int8_t*>(w + L.o.c);
  po.order = reinterpret_cast<int64_t*>(w + L.o.order);
  po.rank = reinterpret_cast<int64_t*>(w + L.o.rank);
  po.dyn_out = reinterpret_cast<int64_t*>(w + L.o.dyn_out);
  po.counts = reinterpret_cast<int64_t*>(w + L.o.counts);
  po.u_ord = reinterpret_cast<int64_t*>(w + L.o.u_ord);
  po.c_ord = reinterpret_cast<int64_t*>(w + L.o.c_ord);
  po.sl_ord = reinterpret_cast<int64_t*>(w + L.o.sl_ord);
  po.L_row = reinterpret_cast<int64_t*>(w + L.o.L_row);
  po.L_cnt = reinterpret_cast<int32_t*>(w + L.o.L_cnt);
  po.loc_ord = reinterpret_cast<int64_t*>(w + L.o.loc_ord);
  if (!a.plan.loc) return ELR_EINVAL;   // the executor needs the rows' MAT slots in class order
  int rc = elr_plan_step(&a.plan, &po, &a.ctl, w + L.plan_scratch, L.plan_scratch_bytes, a.grad, a.n_occ, D,
                         (int)a.key_bits, a.dplan, a.dplan_bytes, stream);
  if (rc) return rc;
  float* G = reinterpret_cast<float*>(w + L.o.grad_rows);
  elr_exec_args e = a.exec;
  e.b[ELR_NRANK] = n;
  e.u_ord = po.u_ord;
  e.c_ord = po.c_ord;
  e.sl_ord = po.sl_ord;
  e.loc_ord = po.loc_ord;
  e.L_row = po.L_row;
  e.L_cnt = po.L_cnt;
  e.slots.ev_slot = po.dyn_out;
  e.slots.keep = po.dyn_out;
  e.upd.grad = G;
  // the segment sum's final kernel, with the executor's first launch (call A's replay inputs and hit records, which
  // need the plan's scatter and nothing of the sum) beside it in one launch where the final kernel allows it
  bool lsteps_done = false;
  ExecLayout EL;
  if (a.n_occ > 0 && exec_layout_dev(e, EL)) {
    char* ew = w + L.o.exec_ws;
    int64_t lblocks = 0;
    const elr::DirLstepsHits lh = elr::dir_lsteps_hits_prep(
        e.dir, e.pv, e.sl_ord, n, e.L_row, e.L_cnt, n, e.s, reinterpret_cast<int32_t*>(ew + EL.o.L_steps),
        reinterpret_cast<int32_t*>(ew + EL.o.L_ids), reinterpret_cast<int64_t*>(ew + EL.o.hrec_dyn),
        reinterpret_cast<int64_t*>(ew + EL.o.hrec_j), a.ctl.desc, lblocks);
    rc = elr::segment_sum_plan_final_with(a.grad, a.n_occ, D, (int)a.key_bits, a.dplan, a.dplan_bytes, po.rank, G, n,
                                          lh, lblocks, stream);
    if (rc == ELR_OK) lsteps_done = true;
    else if (rc != ELR_EUNSUPPORTED) return rc;
  }
  if (a.n_occ > 0 && !lsteps_done &&
      (rc = elr_segment_sum_plan_final(a.grad, a.n_occ, D, (int)a.key_bits, a.dplan, a.dplan_bytes, po.rank, G, n,
                                       stream)))
    return rc;
  elr::MarkRows mark{a.mark_rows, a.mark_n, a.mark_nmax, (int32_t)a.mark_value, const_cast<int32_t*>(a.plan.last_seen),
                     a.plan.R, a.plan.next_bits, (uint32_t)a.mark_bit};
  if ((rc = step_exec_dev(&e, a.ctl.desc, w + L.o.exec_ws, L.exec_bytes, &L.o.exec, stream, lsteps_done,
                          a.mark_rows ? &mark : nullptr, (hipEvent_t)a.mark_event)))
    return rc;
  *out = L.o;
  return ELR_OK;
}

extern "C" int elr_abi_sizes(int64_t* out, int n) {
  if (!out || n < 0) return ELR_EINVAL;
  const int64_t sz[] = {(int64_t)sizeof(elr_dir_state), (int64_t)sizeof(elr_dir_params), (int64_t)sizeof(elr_plan_in),
                        (int64_t)sizeof(elr_plan_out), (int64_t)sizeof(elr_assemble_args),
                        (int64_t)sizeof(elr_slots_args), (int64_t)sizeof(elr_update_args),
                        (int64_t)sizeof(elr_exec_args), (int64_t)sizeof(elr_exec_out), (int64_t)sizeof(elr_plan_ctl),
                        (int64_t)sizeof(elr_step_dev_args), (int64_t)sizeof(elr_step_dev_out)};
  const int m = (int)(sizeof(sz) / sizeof(sz[0]));
  const int k = n < m ? n : m;
  for (int i = 0; i < k; ++i) out[i] = sz[i];
  return k;
}
