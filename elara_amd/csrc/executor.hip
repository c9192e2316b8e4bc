// The executor's update of one step (srm2/elara.py:491-542 ELARAExecutor.update, plus the host worker's arena
// writes 544-580), issued from native code: one C-ABI call per step instead of a dozen from Python.
//
// The planner has sorted the batch's unique rows by class rank (hits; admitted N, L, F; appended N, L; compacted
// N, L; transient F; S), so every group is a contiguous range of the per-row gradients G [n, D] and, from the
// admitted N rows to the transient F rows, of the assembled work rows W [*, 3, D].  The launches, in the order
// the reference's update performs its writes:
//   1. hits: their gradient into their resident history (evl) and Adam in place on their pool slots, one pass;
//   2. evictions: full states of rows going to M into their MAT slots, and the resident histories of rows going
//      back to L into their new log ids -- both read the evicted pool slots and glog rows before step 3 reuses
//      them for admissions;
//   3. admitted rows: Adam from the work array straight into their pool slots, with the admission record of the N
//      and L rows (entry 0 of their resident history);
//   4. compacted rows: Adam from the work array into their new MAT slots; transient F rows back into theirs;
//   5. appended rows: their gradient into their new log ids;
//   6. S rows: Adam in place in the MAT arena.
// Steps 1, 3 and 4 are Adam passes of k_adam_exec: the row moves and history records ride on them, and the work
// array is never written back (no later kernel reads it).  Step 2 is one launch (both copies), and steps 3-5 share
// one k_adam_exec launch, block ranges per part (their rows, slots and log ids are disjoint); step 1 stays a launch
// of its own, since a hit's slot can be evicted in the same step (elara.py:226-227: the eviction copies the state
// after this step's update).  Steps 1-3 are the device part and 4-6 the link part (elr_update_args.part): a caller
// with the arenas in host memory runs the link part on a second stream, with each of its steps a launch of its own.
// D = 64, 128, 256 or 512 with 16-byte aligned arrays: wave-per-row kernels (elr_rowio.h); any other D or alignment:
// the same launches with the generic kernel, a wave per row whose lanes step through the row one float at a time.
#include "elr_exec_dev.h"

namespace elr {

// One launch over the parts with rows (vpl = 0: the generic kernel for D), each part on at most max_blocks
// blocks; without any rows, no launch.
int adam_exec(int vpl, int64_t D, std::initializer_list<ExecAdam> parts, const AdamScalars& s, hipStream_t st,
              int64_t max_blocks) {
  ExecMulti x;
  int64_t blocks;
  if (!exec_multi(parts, max_blocks, x, blocks)) return ELR_EINVAL;
  if (!blocks) return ELR_OK;
  exec_visit(vpl, D, x, blocks, s, [&](const auto& f, int64_t nb) { launch1(f, nb, st); });
  return launch_status();
}

int update_prep(const elr_update_args* a, UpdatePrep& u) {
  if (!a) return ELR_EINVAL;
  const int64_t D = a->D, K = a->K;
  const int64_t* b = a->b;
  if (D <= 0 || K < 1 || a->pool_rows < 0 || a->mat_rows < 0 || a->log_rows < 0 || a->glog_slots < 0)
    return ELR_EINVAL;
  for (int r = 0; r < ELR_NRANK; ++r)
    if (b[r] < 0 || b[r + 1] < b[r]) return ELR_EINVAL;
  auto cnt = [&](int r0, int r1) { return b[r1 + 1] - b[r0]; };
  const int64_t n_hit = cnt(ELR_RANK_HIT, ELR_RANK_HIT), n_adm = cnt(ELR_RANK_NADM, ELR_RANK_FADM),
                n_app = cnt(ELR_RANK_NAPP, ELR_RANK_LAPP), n_cmp = cnt(ELR_RANK_NCMP, ELR_RANK_LCMP),
                n_fn = cnt(ELR_RANK_FN, ELR_RANK_FN), n_s = cnt(ELR_RANK_S, ELR_RANK_S),
                n_tail = cnt(ELR_RANK_NCMP, ELR_RANK_FN), n_work = b[ELR_RANK_S] - b[ELR_RANK_NADM];
  if (a->nev < 0 || a->lazy_n < 0 || a->lazy_n > n_adm) return ELR_EINVAL;
  const bool rec = a->evl != 0;
  if ((n_hit && (!a->pool || !a->hit_slot || (rec && (!a->hrec_dyn || !a->hrec_j || !a->glog)))) ||
      (a->nev && (!a->mat || !a->pool || !a->ev_slot || !a->evf_slots || !a->evl_ids || !a->ev_dyn || !a->glog ||
                  !a->logs)) ||
      (n_work && !a->work) || (b[ELR_NRANK] && !a->grad) || (n_adm && (!a->pool || !a->adm_slots)) ||
      (rec && a->lazy_n && !a->glog) || (n_cmp && (!a->mat || !a->c_slots)) || (n_app && (!a->logs || !a->a_ids)) ||
      (n_fn && (!a->mat || !a->fn_slot)) || (n_s && (!a->mat || !a->s_slot)))
    return ELR_EINVAL;
  if (a->part < ELR_UPDATE_ALL || a->part > ELR_UPDATE_LINK || a->link_blocks < 0) return ELR_EINVAL;
  if (a->nev && a->glog_slots < 1) return ELR_EINVAL;
  elr_adam_scalars(a->lr, a->b1, a->b2, a->eps, a->step, u.sc);
  const float* G = a->grad;
  float* Wk = a->work;
  const int64_t w0 = b[ELR_RANK_NADM];
  const bool al = aligned16(a->pool) && aligned16(a->mat) && aligned16(a->glog) && aligned16(Wk) && aligned16(G) &&
                  aligned16(a->logs);
  u.vpl = al ? wpr_vpl(D) : 0;
  u.D = D;
  u.lb = a->link_blocks > 0 ? a->link_blocks : int64_t(1) << 20;
  u.s = make_scalars(u.sc);
  const int64_t nd = a->glog_slots;
  u.dev_part = a->part != ELR_UPDATE_LINK;
  u.link_part = a->part != ELR_UPDATE_DEVICE;
  // 1. hits: history record and Adam in place
  u.hits = ExecAdam{a->pool, a->pool_rows, a->hit_slot, n_hit, nullptr, nullptr, 0, 0, G, b[ELR_RANK_HIT], n_hit,
                    a->glog, nd, K, a->hrec_dyn, a->hrec_j, 0, rec ? n_hit : 0};
  // 2. evictions (before admissions reuse the slots)
  u.nev = a->nev;
  if (a->nev)
    u.move = evict_move_prep(a->mat, a->mat_rows, a->evf_slots, a->pool, a->pool_rows, a->ev_slot, a->logs,
                             a->log_rows, a->evl_ids, a->glog, nd, K, a->ev_dyn, a->nev, D);
  // 3. admitted rows: Adam from the work array into their pool slots, admission record of the N and L rows
  u.adm = ExecAdam{a->pool, a->pool_rows, a->adm_slots, n_adm, nullptr, Wk, n_work, 0, G, w0,
                   n_adm, a->glog, nd, K, nullptr, nullptr, a->n0, rec ? a->lazy_n : 0};
  // 4. compacted rows into their new MAT slots, transient F rows back into theirs
  u.tail = ExecAdam{a->mat, a->mat_rows, a->c_slots, n_cmp, a->fn_slot, Wk, n_work, b[ELR_RANK_NCMP] - w0, G,
                    b[ELR_RANK_NCMP], n_tail, a->glog, nd, K, nullptr, nullptr, 0, 0};
  // 5. appended rows log their gradient
  u.app = ExecAdam{a->logs, a->log_rows, a->a_ids, n_app, nullptr, nullptr, 0, 0, G, b[ELR_RANK_NAPP], n_app,
                   nullptr, 0, K, nullptr, nullptr, 0, 0, 1};
  // 6. S rows: Adam in place in the MAT arena
  u.n_s = n_s;
  u.mat = a->mat;
  u.mat_rows = a->mat_rows;
  u.s_slot = a->s_slot;
  u.s_grad = G ? G + b[ELR_RANK_S] * D : nullptr;
  return ELR_OK;
}

int adam_exec(const UpdatePrep& u, std::initializer_list<ExecAdam> parts, hipStream_t st, int64_t max_blocks) {
  return adam_exec(u.vpl, u.D, parts, u.s, st, max_blocks);
}

int update_s_rows(const UpdatePrep& u, hipStream_t st) {
  if (!u.n_s) return ELR_OK;
  return elr_adam_rows(u.mat, u.mat_rows, u.s_slot, 1, u.s_grad, u.n_s, u.D, u.sc, st);
}

}  // namespace elr

extern "C" int elr_step_update(const elr_update_args* a, void* stream) {
  using namespace elr;
  UpdatePrep u;
  int rc = update_prep(a, u);
  if (rc) return rc;
  hipStream_t st = (hipStream_t)stream;
  if (u.dev_part) {
    if ((rc = adam_exec(u, {u.hits}, st))) return rc;
    if (u.nev) {
      evict_move_visit(u.move, [&](const auto& f, int64_t blocks) { launch1(f, blocks, st); });
      if ((rc = launch_status())) return rc;
    }
    // 3, with 4 and 5 when the whole update runs here
    if ((rc = u.link_part ? adam_exec(u, {u.adm, u.tail, u.app}, st) : adam_exec(u, {u.adm}, st))) return rc;
  } else {
    if ((rc = adam_exec(u, {u.tail}, st, u.lb))) return rc;
    if ((rc = adam_exec(u, {u.app}, st, u.lb))) return rc;
  }
  if (!u.link_part) return ELR_OK;
  return update_s_rows(u, st);
}

