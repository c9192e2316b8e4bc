// Device side of the executor's update (executor.hip): the Adam passes with their row moves as functors
// (elr_launch.h), so that the step's executor can launch them beside the directory's eviction kernels.
#pragma once

#include <initializer_list>

#include "elr_copy_dev.h"
#include "elr_desc.h"
#include "elr_launch.h"
#include "elr_rowio.h"


namespace elr {

constexpr int kExecRowsPerWave = 2;   // rows per wave in flight

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
  // device-driven step: which of the update's parts this is (kExecHits ...), its counts and class-order offsets
  // then come from the descriptor (n, na and n_rec hold upper bounds; n_rec 0: no records); g_rows: the rows of
  // grad (and of the class-ordered slot arrays the tail and S parts index)
  int kind;
  const int64_t* desc;
  int64_t g_rows;
};

enum : int { kExecPlain = 0, kExecHits, kExecAdm, kExecTail, kExecApp, kExecS };

// The part's counts and offsets in a device-driven step (positions b[r] of the class order, executor.hip's update
// order): the hits in place; the admitted rows from the work array into their pool slots with the N and L rows'
// admission records; the compacted rows into their new MAT slots and the transient F rows into theirs (dst_b: the
// class-ordered MAT slots, from b[FN]); the appended rows' gradients into their log ids; the S rows in place in
// the MAT arena (dst_a: the class-ordered MAT slots, from b[S]).
// Every value is kept within the part's bounds: in.n (its rows and its slot array), in.g_rows (the gradient rows)
// and in.src_rows (the work rows).
__device__ __forceinline__ ExecAdam exec_resolve(const ExecAdam& in) {
  if (!in.desc) return in;
  const int64_t* d = in.desc;
  const int64_t gr = in.g_rows;
  ExecAdam a = in;
  switch (in.kind) {
    case kExecHits:
      a.g_base = clampi(d[kDB + ELR_RANK_HIT], 0, gr);
      a.n = clampi(d[kDNh], 0, in.n < gr - a.g_base ? in.n : gr - a.g_base);
      a.n_rec = in.n_rec ? a.n : 0;
      break;
    case kExecAdm:
      a.g_base = clampi(d[kDW0], 0, gr);
      a.n = clampi(d[kDNAdm], 0, in.n < gr - a.g_base ? in.n : gr - a.g_base);
      a.n_rec = in.n_rec ? clampi(d[kDLazy], 0, a.n) : 0;
      break;
    case kExecTail: {
      a.g_base = clampi(d[kDB + ELR_RANK_NCMP], 0, gr);
      a.n = clampi(d[kDNTail], 0, in.n < gr - a.g_base ? in.n : gr - a.g_base);
      a.na = clampi(d[kDNc], 0, a.n);
      a.src_base = clampi(d[kDB + ELR_RANK_NCMP] - d[kDW0], 0, in.src_rows);
      a.dst_b = in.dst_b + a.g_base + a.na;   // the transient rows' MAT slots follow the compacted rows'
      break;
    }
    case kExecApp:
      a.g_base = clampi(d[kDB + ELR_RANK_NAPP], 0, gr);
      a.n = clampi(d[kDNa], 0, in.n < gr - a.g_base ? in.n : gr - a.g_base);
      break;
    case kExecS:
      a.g_base = clampi(d[kDB + ELR_RANK_S], 0, gr);
      a.n = clampi(d[kDNs], 0, in.n < gr - a.g_base ? in.n : gr - a.g_base);
      a.dst_a = in.dst_a + a.g_base;
      break;
    default:
      break;
  }
  if (a.na > a.n) a.na = a.n;
  return a;
}

// Up to kExecParts parts in one launch: part q takes the blocks [bbeg[q], bbeg[q+1]) (a grid-stride loop over
// its rows inside them).
constexpr int kExecParts = 4;
struct ExecMulti {
  ExecAdam part[kExecParts];
  int64_t bbeg[kExecParts + 1];
};

// The part of this block (block-uniform) and the block's wave index and wave count within it.
__device__ __forceinline__ int exec_part(const ExecMulti& x, int64_t b, int64_t& wid, int64_t& wcount) {
  int q = 0;
#pragma unroll
  for (int r = 1; r < kExecParts; ++r) q += b >= x.bbeg[r] ? 1 : 0;
  const int64_t b0 = x.bbeg[q], nb = x.bbeg[q + 1] - b0;
  wid = body_wave(b - b0);
  wcount = body_waves(nb);
  return q;
}

template <int VPL, int U>
struct AdamExec {
  ExecMulti x;
  AdamScalars s;
  __device__ void operator()(int64_t blk, int64_t) const;
};

template <int VPL, int U>
__device__ void AdamExec<VPL, U>::operator()(int64_t blk, int64_t) const {
  constexpr int64_t D = 64 * VPL;
  const int lane = threadIdx.x & 63;
  int64_t wid, wcount;
  const ExecAdam a = exec_resolve(x.part[exec_part(x, blk, wid, wcount)]);
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

// AdamExec for any D: a wave per row, lane l handling elements l, l + 64, ... (same rows, same writes).
struct AdamExecGen {
  ExecMulti x;
  AdamScalars s;
  int64_t D;
  __device__ void operator()(int64_t blk, int64_t) const;
};

__device__ inline void AdamExecGen::operator()(int64_t blk, int64_t) const {
  const int lane = threadIdx.x & 63;
  int64_t wid, wcount;
  const ExecAdam a = exec_resolve(x.part[exec_part(x, blk, wid, wcount)]);
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

// The parts with rows of one launch, each part on at most max_blocks blocks; false when there are more than
// kExecParts of them.
inline bool exec_multi(std::initializer_list<ExecAdam> parts, int64_t max_blocks, ExecMulti& x, int64_t& blocks) {
  constexpr int U = kExecRowsPerWave;
  x = ExecMulti{};
  int q = 0;
  blocks = 0;
  for (const ExecAdam& a : parts) {
    if (a.n <= 0) continue;
    if (q == kExecParts) return false;
    int64_t nb = (a.n + (a.copy ? 4 : 4 * U) - 1) / (a.copy ? 4 : 4 * U);
    if (nb > max_blocks) nb = max_blocks;
    x.part[q] = a;
    x.bbeg[q++] = blocks;
    blocks += nb;
  }
  for (int r = q; r <= kExecParts; ++r) x.bbeg[r] = blocks;
  return true;
}

// The Adam functor for vpl (0: the generic one for D), passed to visit(functor, blocks).
template <class Visit>
inline void exec_visit(int vpl, int64_t D, const ExecMulti& x, int64_t blocks, const AdamScalars& s, Visit&& visit) {
  constexpr int U = kExecRowsPerWave;
  switch (vpl) {
    case 0: visit(AdamExecGen{x, s, D}, blocks); break;
    case 1: visit(AdamExec<1, U>{x, s}, blocks); break;
    case 2: visit(AdamExec<2, U>{x, s}, blocks); break;
    case 4: visit(AdamExec<4, U>{x, s}, blocks); break;
    default: visit(AdamExec<8, U>{x, s}, blocks); break;
  }
}

// elr_step_update's checks and launch arguments (executor.hip): the hits, the eviction moves, the admitted,
// compacted, transient and appended rows, the S rows.
struct UpdatePrep {
  int vpl;
  int64_t D, lb, nev, n_s, mat_rows;
  float sc[8];
  AdamScalars s;
  bool dev_part, link_part;
  ExecAdam hits, adm, tail, app, srows;   // srows: the S rows as an Adam part (device-driven step)
  EvictMove move;
  float* mat;
  const int64_t* s_slot;
  const float* s_grad;
};
int update_prep(const elr_update_args* a, UpdatePrep& u);
// One launch of the parts with rows (each on at most max_blocks blocks); the S rows' Adam (elr_adam_rows).
int adam_exec(int vpl, int64_t D, std::initializer_list<ExecAdam> parts, const AdamScalars& s, hipStream_t st,
              int64_t max_blocks = int64_t(1) << 20);
int adam_exec(const UpdatePrep& u, std::initializer_list<ExecAdam> parts, hipStream_t st,
              int64_t max_blocks = int64_t(1) << 20);
int update_s_rows(const UpdatePrep& u, hipStream_t st);

}  // namespace elr
