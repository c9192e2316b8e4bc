/*
 * CPU oracle for the ELARA sparse-update path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker that the HIP product path is compared against; it is
 * loaded by tests/, by __graft_entry__.smoke() and by the cpu_baseline leg of bench.py, and by nothing else.
 * The product library (elara_amd/libelara_amd.so) never links, loads or calls it.
 *
 * Built by oracle/Makefile with  -O3 -ffp-contract=off -fno-fast-math  so that every float operation below
 * is a separately rounded IEEE-754 binary32 operation (round to nearest even), as in the reference's CPU
 * extension (srm2/ops.py:24 passes the same flags).
 *
 * Each function names the reference lines it restates.  How each one is pinned (checked against something
 * other than itself) is listed in oracle/__init__.py.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------------------------------------------------
 * Adam scalars.  srm2/csrc/srm2_cpu.cpp:13-20: fp64 arithmetic (std::pow) cast to fp32, in the order
 * (lr, b1, 1-b1, b2, 1-b2, 1-b1^t, 1-b2^t, eps).
 * ------------------------------------------------------------------------------------------------------- */
void orc_adam_scalars(double lr, double b1, double b2, double eps, int64_t step, float out[8]) {
  out[0] = (float)lr;
  out[1] = (float)b1;
  out[2] = (float)(1.0 - b1);
  out[3] = (float)b2;
  out[4] = (float)(1.0 - b2);
  out[5] = (float)(1.0 - pow(b1, (double)step));
  out[6] = (float)(1.0 - pow(b2, (double)step));
  out[7] = (float)eps;
}

/* One Adam update of a D-vector (w, m, v) with gradient g.  srm2/csrc/srm2_cpu.cpp:22-34, op for op:
 *   mj = b1*m; t1 = omb1*g; mj = mj+t1; vj = b2*v; t2 = omb2*g; t2 = t2*g; vj = vj+t2;
 *   mh = mj/bc1; vh = vj/bc2; den = sqrt(vh); den = den+eps; num = lr*mh; up = num/den; w = w-up.      */
static void adam_vec(float* w, float* m, float* v, const float* g, int64_t D, const float* s) {
  const float lr = s[0], b1 = s[1], omb1 = s[2], b2 = s[3], omb2 = s[4], bc1 = s[5], bc2 = s[6], eps = s[7];
  for (int64_t j = 0; j < D; ++j) {
    float gj = g[j];
    float mj = b1 * m[j];
    float t1 = omb1 * gj;
    mj = mj + t1;
    float vj = b2 * v[j];
    float t2 = omb2 * gj;
    t2 = t2 * gj;
    vj = vj + t2;
    float mh = mj / bc1;
    float vh = vj / bc2;
    float den = sqrtf(vh);
    den = den + eps;
    float num = lr * mh;
    float up = num / den;
    w[j] = w[j] - up;
    m[j] = mj;
    v[j] = vj;
  }
}

/* ---------------------------------------------------------------------------------------------------------
 * Contiguous-chunk thread split.  srm2/csrc/srm2_cpu.cpp:49-55: one thread when nthreads <= 1 or n < minpar,
 * else chunk = ceil(n / nthreads) rows per std::thread.
 * ------------------------------------------------------------------------------------------------------- */
typedef void (*orc_range_fn)(void* ctx, int64_t lo, int64_t hi);
typedef struct { orc_range_fn fn; void* ctx; int64_t lo, hi; } orc_task;

static void* orc_task_main(void* p) {
  orc_task* t = (orc_task*)p;
  t->fn(t->ctx, t->lo, t->hi);
  return NULL;
}

static void orc_pfor(int64_t n, int nthreads, int64_t minpar, orc_range_fn fn, void* ctx) {
  if (nthreads <= 1 || n < minpar) { fn(ctx, 0, n); return; }
  int64_t chunk = (n + nthreads - 1) / nthreads;
  pthread_t* th = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)nthreads);
  orc_task* tk = (orc_task*)malloc(sizeof(orc_task) * (size_t)nthreads);
  int started = 0;
  for (int t = 0; t < nthreads; ++t) {
    int64_t lo = (int64_t)t * chunk, hi = lo + chunk < n ? lo + chunk : n;
    if (lo >= hi) break;
    tk[started] = (orc_task){fn, ctx, lo, hi};
    if (pthread_create(&th[started], NULL, orc_task_main, &tk[started]) != 0) { fn(ctx, lo, hi); continue; }
    ++started;
  }
  for (int t = 0; t < started; ++t) pthread_join(th[t], NULL);
  free(th);
  free(tk);
}

/* ---------------------------------------------------------------------------------------------------------
 * Row-sparse Adam on an interleaved [R,3,D] (w,m,v) table.  srm2/csrc/srm2_cpu.cpp:36-56.
 * rows: int64 [n] (unique), grad: [n,D]; row i of grad updates record rows[i].
 * ------------------------------------------------------------------------------------------------------- */
typedef struct { float* S; const int64_t* r; const float* G; int64_t D; const float* s; } adam_ctx;

static void adam_range(void* p, int64_t lo, int64_t hi) {
  adam_ctx* c = (adam_ctx*)p;
  for (int64_t i = lo; i < hi; ++i) {
    float* base = c->S + c->r[i] * 3 * c->D;
    adam_vec(base, base + c->D, base + 2 * c->D, c->G + i * c->D, c->D, c->s);
  }
}

int orc_cpu_adam(float* state, const int64_t* rows, const float* grad, int64_t n, int64_t D, const float sc[8],
                 int nthreads) {
  if (n < 0 || D <= 0) return -1;
  adam_ctx c = {state, rows, grad, D, sc};
  orc_pfor(n, nthreads, 256, adam_range, &c);
  return 0;
}

/* ---------------------------------------------------------------------------------------------------------
 * Counter-hash initial weights.  srm2/gpu_ops.py:15-23 (_hash32 = MurmurHash3 fmix32 on uint32) and
 * gpu_ops.py:26-38 (_init_rows):
 *   key = u32(r*D + j) ^ fmix32(u32(r >> 32) + u32(seed));  h = fmix32(key ^ u32(seed));
 *   u = f32(h >> 8) * 2^-24;  w0 = (u*2 - 1) * bound;  m = v = 0.
 * ------------------------------------------------------------------------------------------------------- */
uint32_t orc_fmix32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x85EBCA6Bu;
  x ^= x >> 13;
  x *= 0xC2B2AE35u;
  x ^= x >> 16;
  return x;
}

static void init_vec(float* w, int64_t r, int64_t D, uint32_t seed, float bound) {
  uint32_t hi = orc_fmix32((uint32_t)((uint64_t)r >> 32) + seed);
  for (int64_t j = 0; j < D; ++j) {
    uint32_t key = (uint32_t)((uint64_t)r * (uint64_t)D + (uint64_t)j) ^ hi;
    uint32_t h = orc_fmix32(key ^ seed);
    float u = (float)(h >> 8) * (1.0f / 16777216.0f);
    float t = u * 2.0f;
    t = t - 1.0f;
    w[j] = t * bound;
  }
}

void orc_init_rows(float* out, const int64_t* rows, int64_t n, int64_t D, uint32_t seed, float bound) {
  for (int64_t i = 0; i < n; ++i) {
    float* base = out + i * 3 * D;
    init_vec(base, rows[i], D, seed, bound);
    memset(base + D, 0, sizeof(float) * (size_t)(2 * D));
  }
}

/* ---------------------------------------------------------------------------------------------------------
 * Exact replay.  srm2/gpu_ops.py:51-79: state = init(row); for k < cnt[i]: Adam with the scalars of logical
 * step steps[i,k] (table row, gpu_ops.py:82-88) and gradient logs[offs[i] + k].  Returns -1 if an index is out
 * of range (the reference leaves that undefined).
 * ------------------------------------------------------------------------------------------------------- */
typedef struct {
  float* out; const int64_t* rows; const float* logs; const int64_t* offs; const int32_t* steps; const int32_t* cnt;
  int64_t D; int K; uint32_t seed; float bound; const float* table; int64_t table_rows; int64_t nlogs; int bad;
} replay_ctx;

static void replay_range(void* p, int64_t lo, int64_t hi) {
  replay_ctx* c = (replay_ctx*)p;
  const int64_t D = c->D;
  for (int64_t i = lo; i < hi; ++i) {
    float* w = c->out + i * 3 * D;
    init_vec(w, c->rows[i], D, c->seed, c->bound);
    memset(w + D, 0, sizeof(float) * (size_t)(2 * D));
    for (int k = 0; k < c->K && k < c->cnt[i]; ++k) {
      int64_t st = c->steps[i * c->K + k], e = c->offs[i] + k;
      if (st < 0 || st >= c->table_rows || e < 0 || e >= c->nlogs) { c->bad = 1; continue; }
      adam_vec(w, w + D, w + 2 * D, c->logs + e * D, D, c->table + st * 8);
    }
  }
}

int orc_replay_rows(float* out, const int64_t* rows, const float* logs, int64_t nlogs, const int64_t* offs,
                    const int32_t* steps, const int32_t* cnt, int64_t n, int64_t D, int K, uint32_t seed, float bound,
                    const float* table, int64_t table_rows, int nthreads) {
  replay_ctx c = {out, rows, logs, offs, steps, cnt, D, K, seed, bound, table, table_rows, nlogs, 0};
  orc_pfor(n, nthreads, 256, replay_range, &c);
  return c.bad ? -1 : 0;
}

/* ---------------------------------------------------------------------------------------------------------
 * Duplicate-id reduction (dedup + per-id gradient sum), the step before Adam for a batch with repeated ids
 * (srm2/train.py:352 torch.unique(..., return_inverse=True) and train.py:429 embedding_dense_backward).
 * Unique ids come out ascending (torch.unique's definition).  The sums follow ATen's
 * embedding_dense_backward as its ROCm build runs on the GPU (PyTorch 2.10 / 2.11, third-party code the reference
 * calls; aten/src/ATen/native/cuda/Embedding.cu embedding_dense_backward_cuda), restated kernel by kernel:
 *  - at most ORC_ATEN_SMALL indices (embedding_backward_feature_kernel): the indices are taken in windows of
 *    ORC_ATEN_WINDOW consecutive positions (the kernel's blockDim.y: 16 in the ROCm build, 32 in the CUDA build);
 *    in a window the first position of each id sums that id's gradients of the window left to right, starting
 *    from its own, and adds the sum into the id's output row, which starts at zero;
 *  - more indices (EmbeddingBackwardKernel.cu embedding_backward_cuda_kernel): a stable sort of the indices
 *    groups each id's occurrences in ascending position; they are cut into partial segments of
 *    NROWS_PER_THREAD = 10 from the id's first, each summed from zero (compute_grad_weight), and an id's partial
 *    sums are added from zero in order (sum_and_scatter).
 * Returns the number of unique ids.
 * ------------------------------------------------------------------------------------------------------- */
#define ORC_ATEN_SMALL 3072
#define ORC_ATEN_WINDOW 16
#define ORC_ATEN_NROWS 10

/* Occurrences sorted by (id, position): a stable sort by id.  The pairs carry their own key, so the comparator
 * reads no global and concurrent calls are safe. */
typedef struct orc_occ {
  int64_t id, pos;
} orc_occ;
static int cmp_occ(const void* a, const void* b) {
  const orc_occ* p = (const orc_occ*)a;
  const orc_occ* q = (const orc_occ*)b;
  if (p->id != q->id) return p->id < q->id ? -1 : 1;
  return p->pos < q->pos ? -1 : (p->pos > q->pos);
}

int64_t orc_segment_sum(const int64_t* ids, const float* grad, int64_t nocc, int64_t D, int64_t* uniq,
                        float* gsum, int64_t* inverse) {
  orc_occ* occ = (orc_occ*)malloc(sizeof(orc_occ) * (size_t)(nocc > 0 ? nocc : 1));
  int64_t* ord = (int64_t*)malloc(sizeof(int64_t) * (size_t)(nocc > 0 ? nocc : 1));
  int64_t* inv = (int64_t*)malloc(sizeof(int64_t) * (size_t)(nocc > 0 ? nocc : 1));
  float* part = (float*)malloc(sizeof(float) * (size_t)(D > 0 ? D : 1));
  float* tot = (float*)malloc(sizeof(float) * (size_t)(D > 0 ? D : 1));
  for (int64_t i = 0; i < nocc; ++i) {
    occ[i].id = ids[i];
    occ[i].pos = i;
  }
  qsort(occ, (size_t)nocc, sizeof(orc_occ), cmp_occ);   /* ties by position: a stable sort */
  for (int64_t i = 0; i < nocc; ++i) ord[i] = occ[i].pos;
  free(occ);
  int64_t U = 0;
  for (int64_t q0 = 0; q0 < nocc;) {
    int64_t q1 = q0 + 1;
    while (q1 < nocc && ids[ord[q1]] == ids[ord[q0]]) ++q1;
    uniq[U] = ids[ord[q0]];
    for (int64_t q = q0; q < q1; ++q) inv[ord[q]] = U;
    if (nocc > ORC_ATEN_SMALL) {
      /* sort path: partial segments of ORC_ATEN_NROWS, each summed from zero; partial sums added from zero */
      for (int64_t j = 0; j < D; ++j) tot[j] = 0.0f;
      for (int64_t c0 = q0; c0 < q1; c0 += ORC_ATEN_NROWS) {
        const int64_t c1 = c0 + ORC_ATEN_NROWS < q1 ? c0 + ORC_ATEN_NROWS : q1;
        for (int64_t j = 0; j < D; ++j) part[j] = 0.0f;
        for (int64_t q = c0; q < c1; ++q) {
          const float* g = grad + ord[q] * D;
          for (int64_t j = 0; j < D; ++j) part[j] = part[j] + g[j];
        }
        for (int64_t j = 0; j < D; ++j) tot[j] = tot[j] + part[j];
      }
      memcpy(gsum + U * D, tot, sizeof(float) * (size_t)D);
    }
    ++U;
    q0 = q1;
  }
  if (nocc <= ORC_ATEN_SMALL) {
    /* windowed path, window by window in position order */
    for (int64_t u = 0; u < U * D; ++u) gsum[u] = 0.0f;
    for (int64_t w0 = 0; w0 < nocc; w0 += ORC_ATEN_WINDOW) {
      const int64_t w1 = w0 + ORC_ATEN_WINDOW < nocc ? w0 + ORC_ATEN_WINDOW : nocc;
      for (int64_t p = w0; p < w1; ++p) {
        int leader = 1;
        for (int64_t q = w0; q < p; ++q) leader &= ids[q] != ids[p];
        if (!leader) continue;
        memcpy(part, grad + p * D, sizeof(float) * (size_t)D);
        for (int64_t q = p + 1; q < w1; ++q)
          if (ids[q] == ids[p]) {
            const float* g = grad + q * D;
            for (int64_t j = 0; j < D; ++j) part[j] = part[j] + g[j];
          }
        float* s = gsum + inv[p] * D;
        for (int64_t j = 0; j < D; ++j) s[j] = s[j] + part[j];
      }
    }
  }
  if (inverse) memcpy(inverse, inv, sizeof(int64_t) * (size_t)nocc);
  free(ord);
  free(inv);
  free(part);
  free(tot);
  return U;
}

/* =========================================================================================================
 * GPU state directory, restated sequentially from srm2/csrc/elara_dir.cpp:13-110 (which is line-for-line the
 * torch path of srm2/elara.py:171-206, 285-343, 379-386).  Layout (elara_dir.cpp:8-11):
 *   code i8[R]  loc i32[R+1]  ent i32[(R+1)K]  lstep i32[Lcap+1]  lfree i32[Lcap+1]  n_lfree/log_top/mat_top/live
 *   i64[1]  adm_c0 i8[C]  rj i8[C]  pstep i32[Cdyn+1,K]  kthr i8[T]  toff i64[T]  slot_of i32[R]  slot_row i64[C]
 *   rok i8[C];  params (R, K, Lcap, n0, Cdyn, MAT, trash, evl).
 * Every tensor op of the reference reads its inputs before it writes, in program order; the loops below keep
 * that order (a gather loop completes before the scatter loop that follows it).
 * ========================================================================================================= */
typedef struct {
  int8_t* code; int32_t* loc; int32_t* ent; int32_t* lstep; int32_t* lfree;
  int64_t* n_lfree; int64_t* log_top; int64_t* mat_top; int64_t* live;
  int8_t* adm_c0; int8_t* rj; int32_t* pstep; const int8_t* kthr; const int64_t* toff;
  int32_t* slot_of; int64_t* slot_row; int8_t* rok; int64_t T;
} orc_dir;

typedef struct { int64_t R, K, Lcap, n0, Cdyn, MAT, trash, evl; } orc_dir_params;

/* elara_dir.cpp:13-21: ids for flags valid[0..m) in order; free stack first (top down), then bump. */
static void orc_alloc_logs(orc_dir* d, const uint8_t* valid, int64_t m, int64_t* ids) {
  const int64_t nf = *d->n_lfree, top = *d->log_top;
  int64_t rank = -1;
  for (int64_t i = 0; i < m; ++i) {
    if (valid[i]) ++rank;
    int64_t fi = nf - 1 - rank;
    if (fi < 0) fi = 0;
    ids[i] = rank < nf ? (int64_t)d->lfree[fi] : top + rank - nf;
  }
  int64_t k = rank + 1, used = k < nf ? k : nf;
  *d->log_top += k - used;
  *d->n_lfree -= used;
  *d->live += k;
}

/* elara_dir.cpp:23-34: release the first cnt[i] live entries of rows[i] onto the free stack, clear them. */
static void orc_free_logs(orc_dir* d, const orc_dir_params* p, const int64_t* rows, const int64_t* cnt, int64_t n) {
  if (n == 0) return;
  const int64_t K = p->K, nf = *d->n_lfree;
  int64_t rank = 0;
  int64_t* clr = (int64_t*)malloc(sizeof(int64_t) * (size_t)(n * K));
  int64_t nclr = 0;
  for (int64_t i = 0; i < n; ++i)
    for (int64_t k = 0; k < K; ++k) {
      int64_t pos = rows[i] * K + k;
      int32_t e = d->ent[pos];
      if (k < cnt[i] && e >= 0) { d->lfree[nf + rank] = e; ++rank; clr[nclr++] = pos; }
    }
  *d->n_lfree += rank;
  *d->live -= rank;
  for (int64_t q = 0; q < nclr; ++q) d->ent[clr[q]] = -1;
  free(clr);
}

/* elara_dir.cpp:36-44: MAT slots for rows without one (restricted to mask), in order; loc written for all. */
static void orc_alloc_mat(orc_dir* d, const int64_t* rows, const uint8_t* mask, int64_t n, int64_t* sl) {
  const int64_t top = *d->mat_top;
  int64_t rank = 0;
  for (int64_t i = 0; i < n; ++i) {
    int64_t cur = d->loc[rows[i]];
    int nw = cur < 0 && (mask ? mask[i] : 1);
    sl[i] = nw ? top + rank : cur;
    rank += nw;
  }
  for (int64_t i = 0; i < n; ++i) d->loc[rows[i]] = (int32_t)sl[i];
  *d->mat_top += rank;
}

/* elara_dir.cpp:46-48: searchsorted(toff, row, right=True) - 1. */
static int64_t orc_table_of(const orc_dir* d, int64_t row) {
  int64_t lo = 0, hi = d->T;
  while (lo < hi) { int64_t mid = (lo + hi) / 2; if (d->toff[mid] <= row) lo = mid + 1; else hi = mid; }
  return lo - 1;
}

/* elara_dir.cpp:50-96 (call A).  Outputs: L_steps i32[nL,K], L_ids i32[nL,K], hrec_dyn i64[nh], hrec_j i64[nh],
 * ev_row i64[nev], rep u8[nev], evl_ids i64[nev,K], evf_slots i64[nev], ev_dyn i64[nev].
 * rel_cnt != NULL: the order of the reference's Triton path (srm2/elara_kernels.py:63-75, 152-171: Directory.evict
 * allocates and assigns MAT slots but releases nothing; its release part (ev_row, counts[1]) with counts[1] =
 * rep ? 0 : max(c0, 0) is pushed by Directory.release after the step's appends): the host logs of rows going to M
 * stay, and rel_cnt i64[nev] receives those counts for orc_dir_b. */
int orc_dir_a(orc_dir* d, const orc_dir_params* p, const int64_t* hs, int64_t nh, const int64_t* L_row,
              const int32_t* L_cnt, int64_t nL, const int64_t* ev_slot, int64_t nev, int64_t s,
              int32_t* L_steps, int32_t* L_ids, int64_t* hrec_dyn, int64_t* hrec_j, int64_t* ev_row, uint8_t* rep,
              int64_t* evl_ids, int64_t* evf_slots, int64_t* ev_dyn, int64_t* rel_cnt) {
  const int64_t K = p->K;
  /* replay inputs (elara_dir.cpp:56-59) */
  for (int64_t i = 0; i < nL; ++i)
    for (int64_t k = 0; k < K; ++k) {
      int32_t e = d->ent[L_row[i] * K + k];
      L_steps[i * K + k] = e >= 0 ? d->lstep[e] : 0;
      L_ids[i * K + k] = k < L_cnt[i] ? e : -1;
    }
  /* hits (elara_dir.cpp:60-71): all reads, then pstep, rj, rok writes */
  uint8_t* rec = (uint8_t*)malloc((size_t)(nh > 0 ? nh : 1));
  int64_t* jh = (int64_t*)malloc(sizeof(int64_t) * (size_t)(nh > 0 ? nh : 1));
  uint8_t* okh = (uint8_t*)malloc((size_t)(nh > 0 ? nh : 1));
  for (int64_t i = 0; i < nh; ++i) {
    int64_t sl = hs[i];
    int dyn = sl >= p->n0;
    int64_t c0 = d->adm_c0[sl];
    jh[i] = d->rj[sl];
    okh[i] = d->rok[sl] != 0;
    rec[i] = p->evl && dyn && okh[i] && (c0 + jh[i] < K);
    hrec_dyn[i] = rec[i] ? sl - p->n0 : p->Cdyn;
    hrec_j[i] = rec[i] ? jh[i] : 0;
  }
  for (int64_t i = 0; i < nh; ++i) d->pstep[hrec_dyn[i] * K + hrec_j[i]] = (int32_t)s;
  for (int64_t i = 0; i < nh; ++i) {
    int dyn = hs[i] >= p->n0;
    d->rj[hs[i]] = (int8_t)(jh[i] + rec[i]);
    d->rok[hs[i]] = (int8_t)(okh[i] && !(dyn && !rec[i]));
  }
  free(rec); free(jh); free(okh);
  /* evictions (elara_dir.cpp:72-94) */
  int64_t* c0 = (int64_t*)malloc(sizeof(int64_t) * (size_t)(nev > 0 ? nev : 1));
  int64_t* jj = (int64_t*)malloc(sizeof(int64_t) * (size_t)(nev > 0 ? nev : 1));
  for (int64_t i = 0; i < nev; ++i) {
    int64_t sl = ev_slot[i];
    ev_row[i] = d->slot_row[sl];
    c0[i] = d->adm_c0[sl];
    jj[i] = d->rj[sl];
    rep[i] = (p->evl && nev) ? (d->rok[sl] != 0 && c0[i] + jj[i] <= d->kthr[orc_table_of(d, ev_row[i])]) : 0;
    ev_dyn[i] = sl - p->n0;
  }
  for (int64_t i = 0; i < nev; ++i) d->slot_of[ev_row[i]] = -1;
  for (int64_t i = 0; i < nev; ++i) d->slot_row[ev_slot[i]] = -1;
  uint8_t* valid = (uint8_t*)malloc((size_t)(nev * K > 0 ? nev * K : 1));
  for (int64_t i = 0; i < nev; ++i)
    for (int64_t k = 0; k < K; ++k) valid[i * K + k] = rep[i] && k < jj[i];
  orc_alloc_logs(d, valid, nev * K, evl_ids);
  for (int64_t q = 0; q < nev * K; ++q)
    if (!valid[q]) evl_ids[q] = -1;
  for (int64_t i = 0; i < nev; ++i)
    for (int64_t k = 0; k < K; ++k)
      if (valid[i * K + k]) d->ent[ev_row[i] * K + (c0[i] > 0 ? c0[i] : 0) + k] = (int32_t)evl_ids[i * K + k];
  for (int64_t i = 0; i < nev; ++i)
    for (int64_t k = 0; k < K; ++k)
      if (valid[i * K + k]) d->lstep[evl_ids[i * K + k]] = d->pstep[ev_dyn[i] * K + k];
  uint8_t* notrep = (uint8_t*)malloc((size_t)(nev > 0 ? nev : 1));
  for (int64_t i = 0; i < nev; ++i) notrep[i] = !rep[i];
  orc_alloc_mat(d, ev_row, notrep, nev, evf_slots);
  for (int64_t i = 0; i < nev; ++i)
    if (rep[i]) evf_slots[i] = p->trash;
  if (nev) {
    int64_t* cnt = rel_cnt ? rel_cnt : (int64_t*)malloc(sizeof(int64_t) * (size_t)nev);
    for (int64_t i = 0; i < nev; ++i) cnt[i] = rep[i] ? 0 : (c0[i] > 0 ? c0[i] : 0);
    if (!rel_cnt) {
      orc_free_logs(d, p, ev_row, cnt, nev);
      free(cnt);
    }
    for (int64_t i = 0; i < nev; ++i) {
      int64_t t = c0[i] + jj[i];
      d->code[ev_row[i]] = rep[i] ? (int8_t)(t < 127 ? t : 127) : (int8_t)p->MAT;
    }
  }
  free(c0); free(jj); free(valid); free(notrep);
  return 0;
}

/* elara_dir.cpp:98-110 (call B): appends (stay L), then compactions (to M).  Outputs a_ids i64[na], c_slots
 * i64[nc].  Releases: those of r_rows[0..nr) (the first r_cnt[i] entries each), then, when c_release, those of the
 * compacted rows, as one push sequence.  The reference's default order is nr = 0, c_release = 1; its Triton path
 * (srm2/elara_kernels.py:173-209: appends, compact without release, then release([ev part, (c_rows, c_cnt)])) is
 * the evictions' deferred part as r with c_release = 1.  Directory.release places entry k of item i at n_lfree +
 * (counts before i) + k; every counted entry exists there by construction (elara_kernels.py:208), so that equals
 * the packed push of orc_free_logs. */
int orc_dir_b(orc_dir* d, const orc_dir_params* p, const int64_t* a_rows, const int64_t* a_k, int64_t na,
              const int64_t* c_rows, const int64_t* c_cnt, int64_t nc, int64_t s, int64_t* a_ids, int64_t* c_slots,
              int c_release, const int64_t* r_rows, const int64_t* r_cnt, int64_t nr) {
  const int64_t K = p->K;
  uint8_t* ones = (uint8_t*)malloc((size_t)(na > 0 ? na : 1));
  memset(ones, 1, (size_t)(na > 0 ? na : 1));
  orc_alloc_logs(d, ones, na, a_ids);
  free(ones);
  for (int64_t i = 0; i < na; ++i) d->ent[a_rows[i] * K + a_k[i]] = (int32_t)a_ids[i];
  for (int64_t i = 0; i < na; ++i) d->lstep[a_ids[i]] = (int32_t)s;
  for (int64_t i = 0; i < na; ++i) d->code[a_rows[i]] = (int8_t)(a_k[i] + 1);
  orc_alloc_mat(d, c_rows, NULL, nc, c_slots);
  const int64_t nrel = nr + (c_release ? nc : 0);
  if (nrel) {
    int64_t* rows = (int64_t*)malloc(sizeof(int64_t) * (size_t)nrel);
    int64_t* cnt = (int64_t*)malloc(sizeof(int64_t) * (size_t)nrel);
    for (int64_t i = 0; i < nr; ++i) { rows[i] = r_rows[i]; cnt[i] = r_cnt[i]; }
    for (int64_t i = nr; i < nrel; ++i) { rows[i] = c_rows[i - nr]; cnt[i] = c_cnt[i - nr]; }
    orc_free_logs(d, p, rows, cnt, nrel);
    free(rows);
    free(cnt);
  }
  for (int64_t i = 0; i < nc; ++i) d->code[c_rows[i]] = (int8_t)p->MAT;
  return 0;
}
