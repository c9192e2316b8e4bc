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
#include <initializer_list>

#include "elr_rowio.h"

#ifndef ELR_EXEC_U
#define ELR_EXEC_U 2   // rows per wave in flight
#endif

namespace elr {

// One part of an Adam launch of the executor with the row moves fused in.  Row i < n reads gradient row
// g_base + i; with i < n_rec it stores that gradient into entry rec_j[i] (0 when rec_j is NULL) of resident-history
// slot (rec_dyn ? rec_dyn[i] : its destination row) - rec_off; it reads its state from work row src_base + i (src
// NULL: in place, from its destination row), applies Adam, and writes the state to destination row dst_a[i]
// (i < na) or dst_b[i - na].  So the hits record their history and update in place in one pass, and the
// admitted, compacted and transient rows go from the work array straight to their pool or MAT slots.  With
// copy set, the part only stores gradient row g_base + i into row dst_a[i] of dst, rows of D floats (the appended
// rows' log entries).
struct ExecAdam {
  float* dst;
  int64_t dst_rows;
  const int64_t* dst_a;
  int64_t na;
  const int64_t* dst_b;
  const float* src;
  int64_t src_rows, src_base;
  const float* grad;
  int64_t g_base, n;
  float* glog;
  int64_t nd, K;
  const int64_t* rec_dyn;
  const int64_t* rec_j;
  int64_t rec_off, n_rec;
  int copy;
};

// Up to kExecParts parts in one launch: part q takes the blocks [bbeg[q], bbeg[q+1]) (a grid-stride loop over
// its rows inside them).
constexpr int kExecParts = 3;
struct ExecMulti {
  ExecAdam part[kExecParts];
  int64_t bbeg[kExecParts + 1];
};

// The part of this block (block-uniform) and the block's wave index and wave count within it.
__device__ __forceinline__ int exec_part(const ExecMulti& x, int64_t& wid, int64_t& wcount) {
  const int64_t b = blockIdx.x;
  int q = 0;
#pragma unroll
  for (int r = 1; r < kExecParts; ++r) q += b >= x.bbeg[r] ? 1 : 0;
  const int64_t b0 = x.bbeg[q], nb = x.bbeg[q + 1] - b0;
  wid = (b - b0) * (blockDim.x >> 6) + (threadIdx.x >> 6);
  wcount = nb * (blockDim.x >> 6);
  return q;
}

template <int VPL, int U>
__global__ __launch_bounds__(256) void k_adam_exec(ExecMulti x, AdamScalars s) {
  constexpr int64_t D = 64 * VPL;
  const int lane = threadIdx.x & 63;
  int64_t wid, wcount;
  const ExecAdam& a = x.part[exec_part(x, wid, wcount)];
  if (a.copy) {
    for (int64_t i = wid; i < a.n; i += wcount) {
      const int64_t d = a.dst_a[i];
      if (d < 0 || d >= a.dst_rows) continue;
      frag_store<VPL>(a.dst + d * D + lane * VPL, frag_load<VPL, true>(a.grad + (a.g_base + i) * D + lane * VPL));
    }
    return;
  }
  for (int64_t i0 = wid * U; i0 < a.n; i0 += wcount * U) {
    int64_t d[U];
    bool ok[U];
    RowFrag<VPL> g[U], w[U], m[U], v[U];
    // every row's loads first, so that U rows are in flight per wave
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = i0 + u;
      ok[u] = i < a.n;
      if (!ok[u]) continue;
      d[u] = i < a.na ? a.dst_a[i] : a.dst_b[i - a.na];
      g[u] = frag_load<VPL, true>(a.grad + (a.g_base + i) * D + lane * VPL);
      ok[u] = d[u] >= 0 && d[u] < a.dst_rows && !(a.src && a.src_base + i >= a.src_rows);
      if (!ok[u]) continue;
      const float* sp = (a.src ? a.src + (a.src_base + i) * 3 * D : a.dst + d[u] * 3 * D) + lane * VPL;
      w[u] = frag_load<VPL, false>(sp);
      m[u] = frag_load<VPL, false>(sp + D);
      v[u] = frag_load<VPL, false>(sp + 2 * D);
    }
    // history records (also for a row whose destination is out of range)
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = i0 + u;
      if (i >= a.n || i >= a.n_rec) continue;
      const int64_t slot = (a.rec_dyn ? a.rec_dyn[i] : d[u]) - a.rec_off, e = a.rec_j ? a.rec_j[i] : 0;
      if (slot >= 0 && slot < a.nd && e >= 0 && e < a.K)
        frag_store<VPL>(a.glog + (slot * a.K + e) * D + lane * VPL, g[u]);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (!ok[u]) continue;
      frag_adam<VPL>(w[u], m[u], v[u], g[u], s);
      float* o = a.dst + d[u] * 3 * D + lane * VPL;
      frag_store<VPL>(o, w[u]);
      frag_store<VPL>(o + D, m[u]);
      frag_store<VPL>(o + 2 * D, v[u]);
    }
  }
}

// k_adam_exec for any D: a wave per row, lane l handling elements l, l + 64, ... (same rows, same writes).
__global__ __launch_bounds__(256) void k_adam_exec_gen(ExecMulti x, AdamScalars s, int64_t D) {
  const int lane = threadIdx.x & 63;
  int64_t wid, wcount;
  const ExecAdam& a = x.part[exec_part(x, wid, wcount)];
  if (a.copy) {
    for (int64_t i = wid; i < a.n; i += wcount) {
      const int64_t d = a.dst_a[i];
      if (d < 0 || d >= a.dst_rows) continue;
      const float* g = a.grad + (a.g_base + i) * D;
      float* o = a.dst + d * D;
      for (int64_t j = lane; j < D; j += 64) o[j] = g[j];
    }
    return;
  }
  for (int64_t i = wid; i < a.n; i += wcount) {
    const int64_t d = i < a.na ? a.dst_a[i] : a.dst_b[i - a.na];
    const float* g = a.grad + (a.g_base + i) * D;
    if (i < a.n_rec) {   // history record (also for a row whose destination is out of range)
      const int64_t slot = (a.rec_dyn ? a.rec_dyn[i] : d) - a.rec_off, e = a.rec_j ? a.rec_j[i] : 0;
      if (slot >= 0 && slot < a.nd && e >= 0 && e < a.K) {
        float* h = a.glog + (slot * a.K + e) * D;
        for (int64_t j = lane; j < D; j += 64) h[j] = g[j];
      }
    }
    if (d < 0 || d >= a.dst_rows || (a.src && a.src_base + i >= a.src_rows)) continue;
    const float* sp = a.src ? a.src + (a.src_base + i) * 3 * D : a.dst + d * 3 * D;
    float* o = a.dst + d * 3 * D;
    for (int64_t j = lane; j < D; j += 64) {
      float w = sp[j], m = sp[D + j], v = sp[2 * D + j];
      adam_elem(w, m, v, g[j], s);
      o[j] = w;
      o[D + j] = m;
      o[2 * D + j] = v;
    }
  }
}

// One launch over the parts with rows (vpl = 0: the generic kernel for D), each part on at most max_blocks
// blocks; without any rows, no launch.
static int adam_exec(int vpl, int64_t D, std::initializer_list<ExecAdam> parts, const AdamScalars& s,
                     hipStream_t st, int64_t max_blocks = int64_t(1) << 20) {
  constexpr int U = ELR_EXEC_U;
  ExecMulti x{};
  int q = 0;
  int64_t blocks = 0;
  for (const ExecAdam& a : parts) {
    if (a.n <= 0) continue;
    if (q == kExecParts) return ELR_EINVAL;
    int64_t nb = (a.n + (a.copy ? 4 : 4 * U) - 1) / (a.copy ? 4 : 4 * U);
    if (nb > max_blocks) nb = max_blocks;
    x.part[q] = a;
    x.bbeg[q++] = blocks;
    blocks += nb;
  }
  if (!q) return ELR_OK;
  for (int r = q; r <= kExecParts; ++r) x.bbeg[r] = blocks;
  switch (vpl) {
    case 0: k_adam_exec_gen<<<(unsigned)blocks, 256, 0, st>>>(x, s, D); break;
    case 1: k_adam_exec<1, U><<<(unsigned)blocks, 256, 0, st>>>(x, s); break;
    case 2: k_adam_exec<2, U><<<(unsigned)blocks, 256, 0, st>>>(x, s); break;
    case 4: k_adam_exec<4, U><<<(unsigned)blocks, 256, 0, st>>>(x, s); break;
    default: k_adam_exec<8, U><<<(unsigned)blocks, 256, 0, st>>>(x, s); break;
  }
  return launch_status();
}

}  // namespace elr

extern "C" int elr_step_update(const elr_update_args* a, void* stream) {
  using namespace elr;
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
  hipStream_t st = (hipStream_t)stream;
  float sc[8];
  elr_adam_scalars(a->lr, a->b1, a->b2, a->eps, a->step, sc);
  const float* G = a->grad;
  float* Wk = a->work;
  const int64_t w0 = b[ELR_RANK_NADM];
  int rc;
  const bool al = aligned16(a->pool) && aligned16(a->mat) && aligned16(a->glog) && aligned16(Wk) && aligned16(G) &&
                  aligned16(a->logs);
  const int vpl = al ? wpr_vpl(D) : 0;
  if (a->part < ELR_UPDATE_ALL || a->part > ELR_UPDATE_LINK || a->link_blocks < 0) return ELR_EINVAL;
  const int64_t lb = a->link_blocks > 0 ? a->link_blocks : int64_t(1) << 20;
  const AdamScalars s = make_scalars(sc);
  const int64_t nd = a->glog_slots;
  const bool dev_part = a->part != ELR_UPDATE_LINK, link_part = a->part != ELR_UPDATE_DEVICE;
  // 3. admitted rows: Adam from the work array into their pool slots, admission record of the N and L rows
  const ExecAdam adm{a->pool, a->pool_rows, a->adm_slots, n_adm, nullptr, Wk, n_work, 0, G, w0,
                     n_adm, a->glog, nd, K, nullptr, nullptr, a->n0, rec ? a->lazy_n : 0};
  // 4. compacted rows into their new MAT slots, transient F rows back into theirs
  const ExecAdam tail{a->mat, a->mat_rows, a->c_slots, n_cmp, a->fn_slot, Wk, n_work, b[ELR_RANK_NCMP] - w0, G,
                      b[ELR_RANK_NCMP], n_tail, a->glog, nd, K, nullptr, nullptr, 0, 0};
  // 5. appended rows log their gradient
  const ExecAdam app{a->logs, a->log_rows, a->a_ids, n_app, nullptr, nullptr, 0, 0, G, b[ELR_RANK_NAPP], n_app,
                     nullptr, 0, K, nullptr, nullptr, 0, 0, 1};
  if (dev_part) {
    // 1. hits: history record and Adam in place
    if ((rc = adam_exec(vpl, D, {ExecAdam{a->pool, a->pool_rows, a->hit_slot, n_hit, nullptr, nullptr, 0, 0, G,
                                          b[ELR_RANK_HIT], n_hit, a->glog, nd, K, a->hrec_dyn, a->hrec_j, 0,
                                          rec ? n_hit : 0}}, s, st)))
      return rc;
    // 2. evictions (before admissions reuse the slots)
    if (a->nev && (rc = evict_move(a->mat, a->mat_rows, a->evf_slots, a->pool, a->pool_rows, a->ev_slot, a->logs,
                                   a->log_rows, a->evl_ids, a->glog, nd, K, a->ev_dyn, a->nev, D, st)))
      return rc;
    // 3, with 4 and 5 when the whole update runs here
    if ((rc = link_part ? adam_exec(vpl, D, {adm, tail, app}, s, st) : adam_exec(vpl, D, {adm}, s, st))) return rc;
  } else {
    if ((rc = adam_exec(vpl, D, {tail}, s, st, lb))) return rc;
    if ((rc = adam_exec(vpl, D, {app}, s, st, lb))) return rc;
  }
  if (!link_part) return ELR_OK;
  // 6. S rows: Adam in place in the MAT arena
  if (n_s && (rc = elr_adam_rows(a->mat, a->mat_rows, a->s_slot, 1, G + b[ELR_RANK_S] * D, n_s, D, sc, st)))
    return rc;
  return ELR_OK;
}
