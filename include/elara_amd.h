/*
 * elara_amd — C-ABI of the MI355X (gfx950) sparse-update path of ELARA.
 *
 * Conventions
 *   - extern "C", plain pointers and int64 sizes; no C++ types or exceptions cross the boundary.
 *   - All memory is owned by the caller.  Device pointers point to HBM; host pointers are marked "host".
 *   - Every entry point that touches the GPU takes an explicit hipStream_t (passed as void*, so this header
 *     needs no HIP include) and is asynchronous on that stream; nothing uses the legacy default stream.
 *   - Return value: ELR_OK (0) on success, a negative ELR_E* code for an invalid argument detected on the
 *     host, or a positive hipError_t from the launch.  elr_error_string() describes a code.
 *   - The library keeps no mutable global state (re-entrant; callable from several host threads), except the
 *     per-device scratch array of elr_adam_dedup_noalloc and the cache of its device addresses.
 *   - Device-side index checks: a row whose index (slot, log offset, step) is out of range is skipped and left
 *     unwritten instead of faulting.  The reference leaves such inputs undefined; callers must not rely on it.
 *
 * Layouts (the reference's, srm2/ops.py:47, srm2/csrc/srm2_cpu.cpp:36):
 *   state  fp32 [C, 3, D]   interleaved record (w, m, v) per row, row stride 12*D bytes
 *   grad   fp32 [n, D]      row i belongs to slots[i]
 *   logs   fp32 [L, D]      gradient-log entries; row i of a replay owns logs[offs[i] .. offs[i]+cnt[i])
 *   table  fp32 [S, 8]      Adam scalars per logical step (lr, b1, 1-b1, b2, 1-b2, 1-b1^t, 1-b2^t, eps)
 */
#ifndef ELARA_AMD_H
#define ELARA_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ELR_OK 0
#define ELR_EINVAL (-1)      /* null pointer, negative size or inconsistent shape */
#define ELR_EUNSUPPORTED (-2) /* valid for the reference but outside this build's limits (e.g. K > 8) */
#define ELR_ECAPACITY (-3)   /* caller-provided scratch or output too small */

/* Text for a return code (static storage). */
const char* elr_error_string(int code);

/* Library version as MAJOR*10000 + MINOR*100 + PATCH. */
int elr_version(void);

/* Device-visible address of pinned host memory (no counterpart in the reference, whose host arenas are reached
 * through CPU gathers and staging copies): *dev receives the address the kernels use for host, or the HIP error is
 * returned if the memory is not pinned and mapped.  Every entry point below accepts such addresses for its arena
 * arguments (the MAT and log arenas of the capacity tier), which the kernels then read and write over the host
 * link. */
int elr_host_device_ptr(const void* host, void** dev);

/* ---------------------------------------------------------------------------------------------------------
 * Adam scalars for logical step `step` (host only).
 * Replaces: srm2/csrc/srm2_cpu.cpp:13-20 make_scalars and its binding adam_scalars (srm2_cpu.cpp:255-257),
 * called from srm2/ops.py:64 and srm2/gpu_ops.py:86.  out = (lr, b1, 1-b1, b2, 1-b2, 1-b1^t, 1-b2^t, eps),
 * each computed in fp64 and rounded to fp32.
 * ------------------------------------------------------------------------------------------------------- */
void elr_adam_scalars(double lr, double b1, double b2, double eps, int64_t step, float out[8]);

/* Fill a host table [max_step+1, 8]: row 0 zeros, row t = elr_adam_scalars(t).
 * Replaces: srm2/gpu_ops.py:82-88 ScalarTable (host part; the caller copies it to HBM). */
int elr_scalar_table(double lr, double b1, double b2, double eps, int64_t max_step, float* table_host);

/* Fill a host array [table_rows, 2] with RN_f64(1 / bc1), RN_f64(1 / bc2) of each table row (columns 5 and 6;
 * row 0's zeros give inf).  elr_replay_rows uses them for its divisions by the bias corrections (no counterpart in
 * the reference: the reciprocals only make those correctly rounded divisions cheaper). */
int elr_scalar_recip(const float* table_host, int64_t table_rows, double* recip_host);

/* ---------------------------------------------------------------------------------------------------------
 * Row-sparse Adam, in place.
 * Replaces: srm2/ops.py:42-67 gpu_adam / _adam_rows.  For i < n: Adam(state[slots[i]], grad[i]) with the
 * scalars sc (host array, from elr_adam_scalars).  Slots must be unique within a call (as in the reference).
 *   state  device fp32 [C,3,D];  slots device int32 (idx64 = 0) or int64 (idx64 = 1) [n];  grad device [n,D].
 *   slots == NULL (an extension): grad row i updates state row i (contiguous work arrays of the executor).
 * ------------------------------------------------------------------------------------------------------- */
int elr_adam_rows(float* state, int64_t C, const void* slots, int idx64, const float* grad, int64_t n, int64_t D,
                  const float sc[8], void* stream);

/* elr_adam_rows with kernel timing (no counterpart in the reference): start_event / stop_event (hipEvent_t, either
 * may be NULL) are recorded by the launches themselves at the start of the first and the end of the last kernel
 * (hipExtLaunchKernelGGL), with no marker packet between launches -- a kernel's duration as a profiler reports it.
 * With n == 0 nothing is launched and the events are not recorded. */
int elr_adam_rows_timed(float* state, int64_t C, const void* slots, int idx64, const float* grad, int64_t n,
                        int64_t D, const float sc[8], void* start_event, void* stop_event, void* stream);

/* Row-sparse Adam on the host (no GPU involved), for rows held in host memory.
 * Replaces: srm2/csrc/srm2_cpu.cpp:37-56 cpu_adam (bound as ext().cpu_adam, srm2_cpu.cpp:249; called by the host
 * update worker, srm2/elara.py:567, and srm2/store.py:67, 181).  Same arithmetic and order as elr_adam_rows, on
 * nthreads host threads over contiguous ranges of `rows` (one thread below 256 rows).  All pointers host memory:
 *   state fp32 [R,3,D]; rows int64 [n] (unique within a call; rows outside [0, R) are skipped); grad fp32 [n,D];
 *   sc from elr_adam_scalars.  Blocks until done. */
int elr_cpu_adam(float* state, int64_t R, const int64_t* rows, const float* grad, int64_t n, int64_t D,
                 const float sc[8], int nthreads);

/* ---------------------------------------------------------------------------------------------------------
 * Counter-hash initial state.
 * Replaces: srm2/gpu_ops.py:41-48 init_rows / _init_rows (hash gpu_ops.py:15-23).  out[i] = (w0(rows[i]), 0, 0)
 * with w0[j] = ((h >> 8) * 2^-24 * 2 - 1) * bound, h = fmix32(u32(r*D + j) ^ fmix32(u32(r >> 32) + seed) ^ seed).
 *   out device fp32 [n,3,D];  rows device int64 [n];  seed = low 32 bits of the reference's seed;
 *   bound = the reference's bound rounded to fp32.
 * ------------------------------------------------------------------------------------------------------- */
int elr_init_rows(float* out, const int64_t* rows, int64_t n, int64_t D, uint32_t seed, float bound, void* stream);

/* ---------------------------------------------------------------------------------------------------------
 * Exact replay of logged gradients.
 * Replaces: srm2/gpu_ops.py:91-99 replay_rows / _replay (gpu_ops.py:51-79).  out[i] = init(rows[i]) followed by
 * Adam with gradient logs[offs[i] + k] and scalars table[steps[i*K + k]] for k < cnt[i].  1 <= K <= 8.
 *   out device fp32 [n,3,D]; rows int64 [n]; logs fp32 [nlogs,D]; offs int64 [n]; steps int32 [n,K];
 *   cnt int32 [n]; table fp32 [table_rows, 8]; recip fp64 [table_rows, 2] from elr_scalar_recip (copied to the
 *   device), or NULL (then the kernel computes the reciprocals itself, at some cost).  All device pointers.
 * ------------------------------------------------------------------------------------------------------- */
int elr_replay_rows(float* out, const int64_t* rows, const float* logs, int64_t nlogs, const int64_t* offs,
                    const int32_t* steps, const int32_t* cnt, int64_t n, int64_t D, int K, uint32_t seed, float bound,
                    const float* table, const double* recip, int64_t table_rows, void* stream);

/* elr_replay_rows with kernel timing (no counterpart in the reference), as elr_adam_rows_timed. */
int elr_replay_rows_timed(float* out, const int64_t* rows, const float* logs, int64_t nlogs, const int64_t* offs,
                          const int32_t* steps, const int32_t* cnt, int64_t n, int64_t D, int K, uint32_t seed,
                          float bound, const float* table, const double* recip, int64_t table_rows,
                          void* start_event, void* stop_event, void* stream);

/* ---------------------------------------------------------------------------------------------------------
 * State directory.
 * Replaces: srm2/csrc/elara_dir.cpp (state layout 8-11; elara_dir_a 50-96; elara_dir_b 98-110), the reference's
 * default directory implementation, with the same results and allocation order.  All pointers in the two
 * structs are device pointers (the structs themselves are host memory, read at the call).  Row codes: 0 = I,
 * 1..K = L_c, MAT = K + 1 = M.  Trash: loc/ent row R, lstep/lfree index Lcap, pstep row Cdyn.
 * ------------------------------------------------------------------------------------------------------- */
typedef struct elr_dir_state {
  int8_t* code;         /* [R]          row codes */
  int32_t* loc;         /* [R+1]        MAT slot of each row (-1: none) */
  int32_t* ent;         /* [(R+1)*K]    log-entry ids of each row (-1: none) */
  int32_t* lstep;       /* [Lcap+1]     logical step of each log entry */
  int32_t* lfree;       /* [Lcap+1]     free stack of log ids */
  int64_t* n_lfree;     /* [1]          free-stack depth */
  int64_t* log_top;     /* [1]          bump pointer of the log arena */
  int64_t* mat_top;     /* [1]          bump pointer of the MAT arena */
  int64_t* live;        /* [1]          live log entries */
  int8_t* adm_c0;       /* [C]          host log entries of the slot's row at admission (-1: admitted from M) */
  int8_t* rj;           /* [C]          gradients recorded while resident */
  int32_t* pstep;       /* [Cdyn+1, K]  steps of the resident history */
  const int8_t* kthr;   /* [T]          per-table materialisation threshold */
  const int64_t* toff;  /* [T]          first row of each table (ascending) */
  int32_t* slot_of;     /* [R]          pool slot of each row (-1: not resident) */
  int64_t* slot_row;    /* [C]          row held by each pool slot (-1: empty) */
  int8_t* rok;          /* [C]          resident history still representable as logs */
  int64_t T;            /* number of tables */
} elr_dir_state;

/* The reference's parameter vector pv (elara_dir.cpp:11, srm2/elara.py:277): C = n0 + Cdyn pool slots. */
typedef struct elr_dir_params {
  int64_t R, K, Lcap, n0, Cdyn, MAT, trash, evl;
} elr_dir_params;

/* Bytes of device scratch elr_dir_a (nev evictions) and elr_dir_b (nc compactions) need (max of both), or a
 * negative code. */
int64_t elr_dir_scratch_bytes(int64_t nev, int64_t nc);

/* Call A (elara_dir.cpp:50-96): replay inputs of the L rows L_row [nL] (counts L_cnt int32 [nL]) ->
 * L_steps int32 [nL,K], L_ids int32 [nL,K]; resident-history recording of the hit slots hs [nh] -> hrec_dyn,
 * hrec_j int64 [nh]; eviction of the pool slots ev_slot [nev] -> ev_row int64 [nev], rep uint8 [nev] (1: back to
 * L), evl_ids int64 [nev,K], evf_slots int64 [nev], ev_dyn int64 [nev].  Mutates the directory.  Inputs hs,
 * L_row, ev_slot int64.  `scratch` (device, >= elr_dir_scratch_bytes(nev, 0) bytes) is needed when nev > 0. */
int elr_dir_a(const elr_dir_state* st, const elr_dir_params* p, const int64_t* hs, int64_t nh, const int64_t* L_row,
              const int32_t* L_cnt, int64_t nL, const int64_t* ev_slot, int64_t nev, int64_t s, int32_t* L_steps,
              int32_t* L_ids, int64_t* hrec_dyn, int64_t* hrec_j, int64_t* ev_row, uint8_t* rep, int64_t* evl_ids,
              int64_t* evf_slots, int64_t* ev_dyn, void* scratch, int64_t scratch_bytes, void* stream);

/* The eviction part of call A in the form of srm2/elara_kernels.py:152-171 Directory.evict: the caller has unmapped
 * the evicted slots (slot_of / slot_row) itself and passes their rows ev_row int64 [nev] and thresholds thr int8
 * [nev] (kthr of each row's table).  Outputs as elr_dir_a's rep, evl_ids, evf_slots, ev_dyn.  Allocation order:
 * elr_dir_a's (the released host logs of rows going to M are pushed at once); elr_dir_evict_deferred below keeps
 * the Triton path's. */
int elr_dir_evict(const elr_dir_state* st, const elr_dir_params* p, const int64_t* ev_slot, const int64_t* ev_row,
                  const int8_t* thr, int64_t nev, uint8_t* rep, int64_t* evl_ids, int64_t* evf_slots,
                  int64_t* ev_dyn, void* scratch, int64_t scratch_bytes, void* stream);

/* Call B (elara_dir.cpp:98-110): appends of rows a_rows [na] at entry a_k [na] -> a_ids int64 [na]; compactions of
 * rows c_rows [nc] with c_cnt [nc] logged entries -> c_slots int64 [nc].  All inputs int64.  Mutates the
 * directory.  `scratch` (device, >= elr_dir_scratch_bytes(0, nc) bytes) is needed when na + nc > 0. */
int elr_dir_b(const elr_dir_state* st, const elr_dir_params* p, const int64_t* a_rows, const int64_t* a_k, int64_t na,
              const int64_t* c_rows, const int64_t* c_cnt, int64_t nc, int64_t s, int64_t* a_ids, int64_t* c_slots,
              void* scratch, int64_t scratch_bytes, void* stream);

/* The reference's Triton directory path (srm2/elara.py:279-318, 374-378 with srm2/elara_kernels.py), whose log ids
 * follow another allocation order: every log id of a step is allocated before any of its releases.  States other
 * than the log ids (and the free stack holding them) are the same under both orders.
 *
 * Replaces: lsteps + hits + Directory.evict (elara_kernels.py:16-60, 152-171) in the planner's call sequence.  As
 * elr_dir_a, except that the host logs of rows going to M are not released: rel_cnt int64 [nev] receives each
 * evicted row's release count (max(c0, 0) for a row going to M, 0 for one going back to L; the release part of
 * elara_kernels.py:171), for elr_dir_b_release. */
int elr_dir_a_deferred(const elr_dir_state* st, const elr_dir_params* p, const int64_t* hs, int64_t nh,
                       const int64_t* L_row, const int32_t* L_cnt, int64_t nL, const int64_t* ev_slot, int64_t nev,
                       int64_t s, int32_t* L_steps, int32_t* L_ids, int64_t* hrec_dyn, int64_t* hrec_j,
                       int64_t* ev_row, uint8_t* rep, int64_t* evl_ids, int64_t* evf_slots, int64_t* ev_dyn,
                       int64_t* rel_cnt, void* scratch, int64_t scratch_bytes, void* stream);

/* Replaces: Directory.evict (elara_kernels.py:152-171): elr_dir_evict with the releases deferred as in
 * elr_dir_a_deferred (rel_cnt int64 [nev]). */
int elr_dir_evict_deferred(const elr_dir_state* st, const elr_dir_params* p, const int64_t* ev_slot,
                           const int64_t* ev_row, const int8_t* thr, int64_t nev, uint8_t* rep, int64_t* evl_ids,
                           int64_t* evf_slots, int64_t* ev_dyn, int64_t* rel_cnt, void* scratch,
                           int64_t scratch_bytes, void* stream);

/* Replaces: Directory.appends, .compact and .release (elara_kernels.py:173-209).  Appends of a_rows [na] at entry a_k
 * -> a_ids (log ids popped as elr_dir_b pops them); MAT slots and code = MAT of the compacted rows c_rows [nc] ->
 * c_slots; then the releases, pushed onto the free stack in this order: the first r_cnt[i] logged entries of each
 * r_rows[i] (i < nr), then -- when c_release -- the first c_cnt[i] of each compacted row.  elr_dir_b is this call
 * with c_release = 1 and nr = 0.  The planner's Triton path: the evictions' (ev_row, rel_cnt) as r and c_release =
 * 1, after elr_dir_a_deferred.  All inputs int64.  `scratch` (device, >= elr_dir_scratch_bytes(0, nc + nr) bytes)
 * is needed when na + nc + nr > 0. */
int elr_dir_b_release(const elr_dir_state* st, const elr_dir_params* p, const int64_t* a_rows, const int64_t* a_k,
                      int64_t na, const int64_t* c_rows, const int64_t* c_cnt, int64_t nc, int c_release,
                      const int64_t* r_rows, const int64_t* r_cnt, int64_t nr, int64_t s, int64_t* a_ids,
                      int64_t* c_slots, void* scratch, int64_t scratch_bytes, void* stream);

/* ---------------------------------------------------------------------------------------------------------
 * Batch dedup and duplicate-id gradient reduction.
 * Summation order: ATen's embedding_dense_backward on this GPU (aten/src/ATen/native/cuda/Embedding.cu,
 * EmbeddingBackwardKernel.cu), equal bits.  n <= 3072: per window of 16 consecutive indices an id's gradients are
 * summed left to right and the window sums added into a zeroed row; n > 3072: an id's occurrences in ascending
 * index are cut into runs of 10, each run summed from zero, and the run sums added from zero.  n < 2^31.
 * ------------------------------------------------------------------------------------------------------- */

/* Bytes of device scratch elr_unique / elr_segment_sum / elr_adam_dedup need for n occurrences of width D
 * (D = 1 for elr_unique), or a negative code. */
int64_t elr_dedup_scratch_bytes(int64_t n, int64_t D);

/* Replaces: torch.unique(ids, return_inverse=True) at srm2/train.py:352.  ids int64 [n] in [0, 2^key_bits)
 * -> uniq int64 [>= U] ascending (first U valid), inverse int64 [n] (uniq[inverse[i]] == ids[i]; may be NULL),
 * n_unique int64 [1] = U.  All device pointers; nothing is read back to the host. */
int elr_unique(const int64_t* ids, int64_t n, int key_bits, int64_t* uniq, int64_t* inverse, int64_t* n_unique,
               void* scratch, int64_t scratch_bytes, void* stream);

/* Replaces: aten.embedding_dense_backward(grad, inv, num_rows, -1, False) at srm2/train.py:429.  out[k] = sum of
 * grad[i] (fp32 [n, D]) over i with idx[i] == k (idx int64 [n] in [0, num_rows)), in the order above; rows of out
 * without an index are not written (the caller zero-fills).  D <= 512. */
int elr_segment_sum(const float* grad, const int64_t* idx, int64_t n, int64_t D, int64_t num_rows, float* out,
                    void* scratch, int64_t scratch_bytes, void* stream);

/* Duplicate-id row-sparse Adam (config C3; the dedup of srm2/train.py:352 and 429 followed by srm2/ops.py:59-67
 * gpu_adam on the unique rows): state fp32 [C,3,D]; ids int64 [n] in [0, C), repeats allowed; grad fp32 [n,D].
 * Each unique id gets one Adam step (scalars sc) with the sum of its gradients.  D <= 512. */
int elr_adam_dedup(float* state, int64_t C, const int64_t* ids, const float* grad, int64_t n, int64_t D,
                   const float sc[8], void* scratch, int64_t scratch_bytes, void* stream);

/* Duplicate-id row-sparse Adam that allocates nothing (no counterpart in the reference; for callers that cannot
 * allocate device memory: code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments and results as elr_adam_dedup, without the scratch arguments: the scratch is a device array of
 * ELR_NOALLOC_SCRATCH_BYTES inside the library, one per GPU it runs on, held until the process ends.  Calls with
 * elr_dedup_scratch_bytes(n, D) > ELR_NOALLOC_SCRATCH_BYTES return ELR_ECAPACITY before any launch (at D = 128:
 * n up to about 558,000 occurrences).  No hipMalloc / hipFree or allocating library call is made.  Every call on
 * one GPU uses that GPU's array: calls that overlap in time on one GPU (two streams or threads) race.  The device
 * is the current one (hipGetDevice); a `stream` of another device returns ELR_EINVAL before any launch. */
#define ELR_NOALLOC_SCRATCH_BYTES (64ll << 20)
int elr_adam_dedup_noalloc(float* state, int64_t C, const int64_t* ids, const float* grad, int64_t n, int64_t D,
                           const float sc[8], void* stream);

/* Dedup plan (no counterpart in the reference; the reference sorts each batch twice, in torch.unique and in the
 * embedding backward): elr_dedup_plan is elr_unique that keeps its sort -- sorted positions, segment starts, first
 * occurrences, the chunk plan and U -- in `plan` (elr_dedup_plan_bytes(n, D) bytes, the width D of the gradients to
 * be summed later).  elr_segment_sum_plan then sums a gradient batch grad [n, D] over that plan, segment u (the
 * u-th smallest id) into out[perm ? perm[u] : u] (out_rows rows; rows out of range are skipped), in the same
 * order as elr_segment_sum for n indices.  key_bits must be the value given to elr_dedup_plan. */
int64_t elr_dedup_plan_bytes(int64_t n, int64_t D);
int elr_dedup_plan(const int64_t* ids, int64_t n, int key_bits, int64_t* uniq, int64_t* inverse, int64_t* n_unique,
                   void* plan, int64_t plan_bytes, int64_t D, void* stream);
/* elr_dedup_plan for a batch laid out by field, as the reference's one-hot batches are (srm2/train.py:187-214:
 * global id = local id + the field's table offset, flattened in (sample, field) order): ids [nrows * nfields],
 * field c of sample i at ids[i * nfields + c], and field c's ids in [field_lo[c], field_lo[c + 1]) (field_lo: host
 * array of nfields + 1 ascending bounds, field_lo[0] >= 0).  The whole batch sorted is then each field's column
 * sorted, one after the other, and one block per field sorts its column in LDS: three launches in place of
 * elr_dedup_plan's three per radix pass and four more.  The plan, uniq, inverse and n_unique are bitwise
 * elr_dedup_plan's (the order of the hot-segment list aside, which no result depends on).  An id outside its
 * field's rows breaks that contract: it comes out as -1 in uniq, a row out of range for the caller.  Shapes the
 * per-field sort does not take (nrows > 16,384, nfields > 128, nrows * nfields <= 3,072, a field of more than
 * 2^31 - 2 rows) go to elr_dedup_plan with the same arguments.  ELR_EINVAL for bounds that are not ascending. */
int elr_dedup_plan_fields(const int64_t* ids, int64_t nrows, int64_t nfields, const int64_t* field_lo, int key_bits,
                          int64_t* uniq, int64_t* inverse, int64_t* n_unique, void* plan, int64_t plan_bytes,
                          int64_t D, void* stream);
int elr_segment_sum_plan(const float* grad, int64_t n, int64_t D, int key_bits, const void* plan, int64_t plan_bytes,
                         const int64_t* perm, float* out, int64_t out_rows, void* stream);
/* elr_segment_sum_plan in two parts, for a caller that queues the first beside other work: the partial chunks of
 * the long segments (written into `plan`; elr_plan_classify_seg computes them with the planner's count pass), then
 * this call, the rest of the sum.  Same arguments and results as elr_segment_sum_plan once the partial chunks of
 * the same plan and gradients are in place. */
int elr_segment_sum_plan_final(const float* grad, int64_t n, int64_t D, int key_bits, const void* plan,
                               int64_t plan_bytes, const int64_t* perm, float* out, int64_t out_rows, void* stream);
/* elr_adam_dedup over a dedup plan made earlier (elr_dedup_plan of the same ids, possibly on another stream and
 * ahead of time; no counterpart in the reference, where each step sorts its batch where it updates): uniq is that
 * call's unique-id output (its first U entries, U on the device in the plan, are the rows updated).  Bitwise what
 * elr_adam_dedup gives for those ids and gradients; rows outside [0, C) are skipped. */
int elr_adam_dedup_plan(float* state, int64_t C, const int64_t* uniq, const float* grad, int64_t n, int64_t D,
                        int key_bits, const void* plan, int64_t plan_bytes, const float sc[8], void* stream);

/* ---------------------------------------------------------------------------------------------------------
 * Planner classification of one step: srm2/elara.py:214-267 (ELARAPlanner.plan up to the class counts) -- the
 * per-row class of the batch's unique rows, the stable class order, the expired / preemptible / protected split of
 * the dynamic pool slots, and the counts the host needs, in three launches.
 *
 * Classes (srm2/elara.py:31-32): 0 HIT, 1 N admitted, 2 N append, 3 N compact, 4 L admitted, 5 L append,
 * 6 L compact, 7 F admitted, 8 F not admitted (transient), 9 S.  `order` sorts the positions stably by class rank:
 * HIT, N admitted, L admitted, F admitted, N append, L append, N compact, L compact, F transient, S -- so the
 * admissions, the appends and the compactions are contiguous ranges.  A row hits when slot_of[u] >= 0; a missing row is
 * admitted when last_seen[u] > s; N rows have code 0, L rows 1..K, F/S rows code K+1; "append" when
 * code < kthr[table]; F rows that are not admitted are transient with want_t, else S.
 * ------------------------------------------------------------------------------------------------------- */
#define ELR_PLAN_HIT 1
#define ELR_PLAN_N 2
#define ELR_PLAN_L 4
#define ELR_PLAN_APP 8
#define ELR_PLAN_ADMIT 16
#define ELR_PLAN_NEXT 32   /* the row appears in one of the next batches */

typedef struct elr_plan_in {
  const int64_t* u;           /* [n] the batch's unique rows, ascending */
  int64_t n;
  const int64_t* next[4];     /* unique rows of the next batches, each ascending */
  int64_t n_next[4];
  int nnext;                  /* 0..4 */
  const int32_t* slot_of;     /* [R] pool slot of each row or -1 */
  const int32_t* last_seen;   /* [R] last logical step each row is known to appear at */
  const int8_t* code;         /* [R] row codes */
  const int8_t* kthr;         /* [T] */
  const int64_t* toff;        /* [T] first row of each table */
  int64_t T;
  const int64_t* dyn;         /* [nd] occupied dynamic pool slots */
  int64_t nd;
  const int64_t* slot_row;    /* [C] row held by each slot or -1 */
  const int64_t* mat_top;     /* device counters copied into counts[13], counts[14] (may be NULL) */
  const int64_t* log_top;
  int64_t s;                  /* logical step */
  int K;
  int want_t;                 /* transient updates of non-admitted F rows (st_mode 'T') */
  const int32_t* loc;         /* [R + 1] MAT slot of each row (only read when out->loc_ord is set) */
  int64_t R;                  /* rows: a row of u outside [0, R) is classified S with slot -1, code K+1 and MAT
                                 slot -1, which every later copy and update skips (0: no check) */
  uint32_t* next_bits;        /* [R] optional ring of loaded batches: bit t % 32 of next_bits[r] is set while the
                                 batch of logical step t holds row r (elr_mark_rows with bits).  When given, "appears in
                                 one of the next batches" is next_bits[r] & next_mask != 0 (one load in place of the
                                 searches of next[]), and the scatter pass clears bit s % 32 of the batch's rows: no
                                 later plan asks about step s */
  uint32_t next_mask;         /* the bits of the next batches' steps (s+1, s+2, ...), none equal to bit s % 32 */
  int carry;                  /* residency 'carry' (srm2/elara.py:221, 231-233): a missing row is admitted when it
                                 appears in one of the next batches, and every unprotected dynamic slot is expired;
                                 0: 'ttl' (admitted when last_seen > s; expired when last_seen of its row <= s) */
  const int64_t* live;        /* device counter copied into counts[15] (may be NULL) */
  const int64_t* n_dev;       /* device int64 [1] or NULL: the row count is min(*n_dev, n), n then the upper bound
                                 that sizes the grids (the batch's unique count, read on the device) */
  const int64_t* nd_dev;      /* device int64 [1] or NULL: the dynamic slot count is min(*nd_dev, nd) */
} elr_plan_in;

typedef struct elr_plan_out {
  int8_t* cls;                /* [n] class of each position */
  uint8_t* flags;             /* [n] ELR_PLAN_* bits */
  int32_t* sl;                /* [n] slot_of[u] */
  int8_t* c;                  /* [n] code[u] */
  int64_t* order;             /* [n] positions sorted stably by class rank */
  int64_t* rank;              /* [n] inverse of order (may be NULL) */
  int64_t* dyn_out;           /* [2 nd]: slots as [expired | preemptible | protected], then [expired | the rest],
                                 each part in dyn order */
  int64_t* counts;            /* [17] device: 10 class counts, expired, preemptible, protected, mat_top, log_top,
                                 live, rows of u outside [0, R) (0 when R is 0) */
  /* Optional outputs in class-rank order (each may be NULL), so that the caller needs no gathers: */
  int64_t* u_ord;             /* [n] u[order[r]] */
  int64_t* c_ord;             /* [n] code of u[order[r]] */
  int64_t* sl_ord;            /* [n] slot_of of u[order[r]] (the hit slots are the first counts[0]) */
  int64_t* L_row;             /* [n] the L rows as the reference lists them: admitted, append, compact (first
                                 counts[4] + counts[5] + counts[6] entries) */
  int32_t* L_cnt;             /* [n] their codes (logged entries), same order */
  int64_t* loc_ord;           /* [n] loc of u[order[r]]: the MAT slots of the transient F and S rows, which the
                                 step's directory calls do not move (they change only resident and N/L rows) */
} elr_plan_out;

int64_t elr_plan_scratch_bytes(int64_t n, int64_t nd);
int elr_plan_classify(const elr_plan_in* in, const elr_plan_out* out, void* scratch, int64_t scratch_bytes,
                      void* stream);
/* elr_plan_classify whose first launch also computes the partial chunks of the segment sum of grad [n_occ, D] over
 * the dedup plan `dplan` (elr_dedup_plan of the same batch; no counterpart in the reference): the two are
 * independent, and the count pass's small latency-bound blocks then cost no launch of their own.  The segment sum
 * is completed by elr_segment_sum_plan_final with the same grad and plan.  Errors of either part's arguments are
 * reported before any launch. */
int elr_plan_classify_seg(const elr_plan_in* in, const elr_plan_out* out, void* scratch, int64_t scratch_bytes,
                          const float* grad, int64_t n_occ, int64_t D, int key_bits, const void* dplan,
                          int64_t dplan_bytes, void* stream);

/* ---------------------------------------------------------------------------------------------------------
 * The device-driven step (no counterpart in the reference, whose planner reads the class counts and the host work
 * lists on the host every step, srm2/elara.py:242, 406).  elr_plan_step is elr_plan_classify_seg whose scan launch
 * also resolves the step on the device: the preemption and the overflow decisions (srm2/elara.py:234-258: the
 * un-admitted rows are dropped in the reference's priority order and reclassified, and the carry barrier noted),
 * the class-rank bounds, the evicted and kept slot ranges, the capacity bound of the step's allocations and the
 * count of rows out of range.  It writes them into the step descriptor `desc` (ELR_DESC_WORDS int64, device), which
 * elr_step_exec_dev reads, and keeps the dynamic pool's counters, sticky errors and accumulated statistics in
 * `state` (ELR_CTL_WORDS int64, device, zero-initialised by the caller except the free-stack depth and the slot
 * count).  A step that would run past an arena or holds rows outside [0, R) records the error in state and does
 * nothing (every count of its descriptor is 0), nor does any later step: the caller raises when it next reads
 * state.  No host synchronisation anywhere.
 * ------------------------------------------------------------------------------------------------------- */
#define ELR_DESC_WORDS 40
#define ELR_CTL_WORDS 32
#define ELR_STEP_ERR_ROWS 1        /* rows of the batch outside [0, R): state[4] holds how many */
#define ELR_STEP_ERR_CAPACITY 2    /* the step could allocate past an arena: state[4], state[5] = MAT and log bounds */
typedef struct elr_plan_ctl {
  int64_t* state;             /* [ELR_CTL_WORDS] device: 0 free-stack depth, 1 dynamic slots held, 2 error bits,
                                 3 step of the first error, 4-6 its figures (rows out of range, MAT bound, log
                                 bound), 7 unused, 8-20 statistics (hits, N, L, F, S, admitted,
                                 evicted, preempted, overflow, compactions, appends, barriers, steps) */
  int64_t* desc;              /* [ELR_DESC_WORDS] device: the step descriptor */
  int64_t mat_cap;            /* largest MAT row the step may allocate (capacity - 1: the last row is trash) */
  int64_t log_cap;            /* largest log id */
  int64_t triton;             /* 1: the Triton directory's order (the evictions' releases go to call B) */
} elr_plan_ctl;
int64_t elr_plan_step_scratch_bytes(int64_t n, int64_t nd);
int elr_plan_step(const elr_plan_in* in, const elr_plan_out* out, const elr_plan_ctl* ctl, void* scratch,
                  int64_t scratch_bytes, const float* grad, int64_t n_occ, int64_t D, int key_bits, const void* dplan,
                  int64_t dplan_bytes, void* stream);

/* Admissions of one step (srm2/elara.py:352-367): row adm_rows[i] takes dynamic pool slot adm_slots[i]
 * (slot_of, slot_row); the first lazy_n rows are N/L rows (adm_c0 = their code; with evl their resident history
 * starts: rj = rok = 1, pstep[slot - n0][0] = s), the others F rows (adm_c0 = -1, rj = rok = 0).  Rows or slots
 * out of range are skipped. */
int elr_plan_admit(const int64_t* adm_rows, const int64_t* adm_slots, int64_t n_adm, int64_t lazy_n, int evl,
                   int64_t s, int64_t n0, int64_t C, int64_t R, int K, const int8_t* code, int32_t* slot_of,
                   int64_t* slot_row, int8_t* adm_c0, int8_t* rj, int8_t* rok, int32_t* pstep, void* stream);

/* The admissions with the pool-slot bookkeeping that precedes them (srm2/elara.py:345-347, 368), in one launch:
 * the evicted slots ev_slot [nev] are pushed on the free stack free_stack[0, n_free), the top n_adm entries of the
 * result become adm_slots (bottom first) and are admitted as elr_plan_admit does, the entries below them stay on
 * the stack (free_stack is updated in place; its new depth is n_free + nev - n_adm), and dyn_out receives keep
 * [nkeep] followed by adm_slots: the occupied dynamic slots after the step.  dyn_out must not overlap keep or
 * free_stack.  n_adm <= n_free + nev <= C. */
typedef struct elr_slots_args {
  int64_t* free_stack;        /* [>= n_free + nev] free pool slots, bottom first */
  int64_t n_free;
  const int64_t* ev_slot;     /* [nev] evicted slots, pushed in this order */
  int64_t nev;
  const int64_t* keep;        /* [nkeep] occupied dynamic slots the step keeps */
  int64_t nkeep;
  int64_t* adm_slots;         /* [n_adm] out */
  int64_t* dyn_out;           /* [nkeep + n_adm] out */
} elr_slots_args;

int elr_plan_admit_slots(const elr_slots_args* slots, const int64_t* adm_rows, int64_t n_adm, int64_t lazy_n, int evl,
                         int64_t s, int64_t n0, int64_t C, int64_t R, int K, const int8_t* code, int32_t* slot_of,
                         int64_t* slot_row, int8_t* adm_c0, int8_t* rj, int8_t* rok, int32_t* pstep, void* stream);

/* ---------------------------------------------------------------------------------------------------------
 * Fused weight assembly: srm2/elara.py:471-489 (ELARAExecutor.assemble) -- the full states [n, 3, D] of the
 * step's non-resident rows in one launch.  Work row k (row rows[k]) lies in segment g (positions
 * [seg_end[g-1], seg_end[g])) of kind seg_kind[g]:
 *   ELR_ASM_INIT    counter-hash initial state (as elr_init_rows);
 *   ELR_ASM_REPLAY  initial state plus the row's logged Adam steps (as elr_replay_rows), entry q of L row
 *                   j = seg_aux[g] + (k - seg_start) read from logs[L_ids[j*K + q]] at step L_steps[j*K + q] for
 *                   q < L_cnt[j] (elr_dir_a's replay inputs);
 *   ELR_ASM_GATHER  the state held in the MAT arena at mat[loc[row]].
 * Any D >= 1 (wave-per-row kernels for D = 64, 128, 256, 512 with 16-byte aligned arrays, generic ones otherwise);
 * 1 <= K <= 8 (ELR_EUNSUPPORTED above).  Rows with out-of-range inputs are skipped.
 * ------------------------------------------------------------------------------------------------------- */
#define ELR_ASM_INIT 0
#define ELR_ASM_REPLAY 1
#define ELR_ASM_GATHER 2
#define ELR_ASM_MAX_SEG 16

typedef struct elr_assemble_args {
  float* work;                /* [n, 3, D] output */
  const int64_t* rows;        /* [n] */
  int64_t n;
  int64_t D;
  int K;
  int nseg;
  int64_t seg_end[ELR_ASM_MAX_SEG];
  int seg_kind[ELR_ASM_MAX_SEG];
  int64_t seg_aux[ELR_ASM_MAX_SEG];
  uint32_t seed;              /* counter-hash init: seed (low 32 bits) and bound */
  float bound;
  const int32_t* L_ids;       /* [nL, K] log entry ids (-1 unused) */
  const int32_t* L_steps;     /* [nL, K] logical steps */
  const int32_t* L_cnt;       /* [nL] */
  int64_t nL;
  const float* logs;          /* [nlogs, D] log arena */
  int64_t nlogs;
  const float* table;         /* [table_rows, 8] Adam scalars per step */
  const double* recip;        /* [table_rows, 2] elr_scalar_recip */
  int64_t table_rows;
  const float* mat;           /* [mat_rows, 3, D] MAT arena */
  int64_t mat_rows;
  const int32_t* loc;         /* [R + 1] MAT slot of each row */
  int64_t R;
} elr_assemble_args;

int elr_assemble(const elr_assemble_args* args, void* stream);

/* ---------------------------------------------------------------------------------------------------------
 * The executor's update of one step.
 * Replaces: srm2/elara.py:491-542 (ELARAExecutor.update: Adam on the hits and on the admitted, compacted and
 * transient rows, the resident-history records, the pool scatter of admissions) and the arena writes of the host
 * worker, srm2/elara.py:544-580 (evictions to MAT, history entries back to the log arena, compactions and
 * transient rows to MAT, log appends, the S rows' Adam), all on the device and in one call.
 *
 * The batch's unique rows are in class-rank order (elr_plan_classify's `order`): rank r holds positions
 * b[r] .. b[r+1] of grad [b[ELR_NRANK], D].  The work rows [b[ELR_RANK_S] - b[ELR_RANK_NADM], 3, D] (elr_assemble)
 * hold the admitted, appended, compacted and transient rows in the same order.  The launches follow the
 * reference's order of writes: the evicted slots and their glog rows are read before the admissions reuse them.
 * The row moves and history records ride on the Adam launches: the hits record and update in place, and the
 * admitted, compacted and transient rows go from the work array straight into their pool / MAT slots (the work
 * array is not written back).  Any D >= 1: wave-per-row kernels for D = 64, 128, 256 or 512 with every array
 * 16-byte aligned, generic kernels otherwise.  Index arrays are int64; arenas may be device or mapped pinned host
 * memory (elr_host_device_ptr).  Items whose index is out of range are skipped.  ELR_EINVAL for inconsistent
 * bounds or a NULL array that a nonzero count needs.
 * ------------------------------------------------------------------------------------------------------- */
#define ELR_RANK_HIT 0
#define ELR_RANK_NADM 1
#define ELR_RANK_LADM 2
#define ELR_RANK_FADM 3
#define ELR_RANK_NAPP 4
#define ELR_RANK_LAPP 5
#define ELR_RANK_NCMP 6
#define ELR_RANK_LCMP 7
#define ELR_RANK_FN 8
#define ELR_RANK_S 9
#define ELR_NRANK 10

typedef struct elr_update_args {
  int64_t D, K;
  float* pool;                /* [pool_rows, 3, D] resident states */
  int64_t pool_rows;
  float* mat;                 /* [mat_rows, 3, D] MAT arena */
  int64_t mat_rows;
  float* logs;                /* [log_rows, D] log arena */
  int64_t log_rows;
  float* glog;                /* [glog_slots, K, D] resident histories of the dynamic slots */
  int64_t glog_slots;
  const float* grad;          /* [b[ELR_NRANK], D] per-row gradients in class-rank order */
  float* work;                /* assembled work rows (updated in place) */
  int64_t b[ELR_NRANK + 1];   /* class-rank bounds */
  int64_t step;               /* logical step of the Adam scalars (elr_adam_scalars) */
  double lr, b1, b2, eps;
  int32_t evl;                /* resident histories recorded (evl on) */
  const int64_t* hit_slot;    /* [n_hit] pool slots of the hits */
  const int64_t* hrec_dyn;    /* [n_hit] history record of the hits: glog slot and entry (elr_dir_a) */
  const int64_t* hrec_j;
  int64_t nev;                /* evicted slots */
  const int64_t* ev_slot;     /* [nev] pool slots */
  const int64_t* evf_slots;   /* [nev] MAT slots of rows going to M (others: out of range) */
  const int64_t* evl_ids;     /* [nev, K] new log ids of the history entries of rows going back to L (-1: none) */
  const int64_t* ev_dyn;      /* [nev] their glog slots */
  const int64_t* adm_slots;   /* [n_adm] pool slots of the admitted N, L, F rows */
  int64_t lazy_n;             /* admitted N and L rows: their gradient is entry 0 of glog slot adm_slots[i] - n0 */
  int64_t n0;                 /* static pool slots */
  const int64_t* c_slots;     /* [n_cmp] new MAT slots of the compacted rows (elr_dir_b) */
  const int64_t* a_ids;       /* [n_app] log ids of the appended gradients (elr_dir_b) */
  const int64_t* fn_slot;     /* [n_fn] MAT slots of the transient F rows */
  const int64_t* s_slot;      /* [n_s] MAT slots of the S rows */
  int32_t part;               /* ELR_UPDATE_ALL, or one of the two parts below, each in its own call */
  int64_t link_blocks;        /* > 0: at most this many blocks per launch of the link part (its waves mostly wait on
                                 the host link; a small grid leaves the GPU to the other stream); 0: no cap */
} elr_update_args;

/* elr_update_args.part: the whole update, or its two halves for a caller that runs them on two streams (the
 * capacity tier: the link part writes the arenas in host memory while the device part's stream goes on).
 * ELR_UPDATE_DEVICE: the hits, the evictions (reading the evicted pool slots and glog rows, which the admissions
 * then reuse) and the admissions.  ELR_UPDATE_LINK: the compacted and transient rows into MAT, the log appends and
 * the S rows' Adam; it reads only the work array, the gradients and its index arrays, and writes MAT and log rows
 * that no row of the device part touches. */
#define ELR_UPDATE_ALL 0
#define ELR_UPDATE_DEVICE 1
#define ELR_UPDATE_LINK 2

int elr_step_update(const elr_update_args* args, void* stream);


/* ---------------------------------------------------------------------------------------------------------
 * The rest of a planned step in one call: srm2/elara.py:271-414 after the class-count synchronisation (call A of
 * the directory, the admissions with the pool-slot bookkeeping, call B), the fused assembly (elara.py:471-489) and
 * the executor's update with the host worker's arena writes (elara.py:491-580), issued from C++ on the caller's
 * stream: the kernels of elr_dir_a, elr_plan_admit_slots, elr_dir_b, elr_assemble and elr_step_update, with the
 * directory's small eviction and admission launches each sharing a launch with an independent row kernel (seven
 * launches in all when no directory scan needs a launch of its own).  No counterpart in the reference, whose
 * planner issues these as separate torch and extension calls; it is the same work with the per-call host cost of
 * one call.  The caller has classified the batch (elr_plan_classify) and read its counts;
 * `ws` (device, >= elr_step_exec_bytes(args) bytes, 256-byte aligned) receives every intermediate array, at the
 * offsets elr_step_exec reports in `out` (bytes from ws).
 * ------------------------------------------------------------------------------------------------------- */
typedef struct elr_exec_args {
  elr_dir_state dir;          /* the directory (as elr_dir_a) */
  elr_dir_params pv;          /* R, K, Lcap, n0, Cdyn, MAT, trash, evl */
  int64_t s;                  /* logical step */
  int64_t b[ELR_NRANK + 1];   /* class-rank bounds of the batch */
  const int64_t* u_ord;       /* [b[ELR_NRANK]] rows, codes, pool slots, MAT slots in class-rank order */
  const int64_t* c_ord;
  const int64_t* sl_ord;
  const int64_t* loc_ord;
  const int64_t* L_row;       /* [nL] the L rows as admitted, append, compact (nL = the three L ranks' rows) */
  const int32_t* L_cnt;
  elr_slots_args slots;       /* free stack, evicted and kept slots, dyn_out (adm_slots: filled from ws) */
  uint32_t seed;              /* counter-hash init */
  float bound;
  const float* table;         /* [table_rows, 8] Adam scalars, [table_rows, 2] reciprocals */
  const double* recip;
  int64_t table_rows;
  elr_update_args upd;        /* D, K, the arenas and their rows, grad, lr, b1, b2, eps, n0 (the other fields are set
                                 by the call) */
  int64_t dir_order;          /* log-id allocation order: 0 = elara_dir.cpp's (the reference's default directory,
                                 equal to its torch path), 1 = its Triton path's (as elr_dir_a_deferred followed by
                                 elr_dir_b_release) */
  void* link_stream;          /* elr_step_exec only (host arenas), or NULL: the update's host-arena writes -- the
                                 compacted and transient rows into MAT, the log appends, the S rows -- go to this
                                 hipStream_t, ordered after the rest by link_start (recorded on the call's stream,
                                 waited on by link_stream), and link_done is recorded after them.  The caller keeps
                                 the workspace and G until link_done. */
  void* link_start;           /* hipEvent_t (with link_stream) */
  void* link_done;            /* hipEvent_t (with link_stream) */
  void* link_wait;            /* hipEvent_t or NULL: waited on by the call's stream just before the assembly (the
                                 first launch that reads the arenas), e.g. the link_done of a step whose writes the
                                 assembly may read */
} elr_exec_args;

/* Offsets (bytes from ws) of the arrays elr_step_exec writes: elr_dir_a's nine outputs (L_steps, L_ids, hrec_dyn,
 * hrec_j, ev_row, rep, evl_ids, evf_slots, ev_dyn), the admitted slots, elr_dir_b's a_ids and c_slots, and the work
 * rows [b[ELR_RANK_S] - b[ELR_RANK_NADM], 3, D]. */
typedef struct elr_exec_out {
  int64_t L_steps, L_ids, hrec_dyn, hrec_j, ev_row, rep, evl_ids, evf_slots, ev_dyn, adm_slots, a_ids, c_slots, work;
} elr_exec_out;

int64_t elr_step_exec_bytes(const elr_exec_args* args);
int elr_step_exec(const elr_exec_args* args, void* ws, int64_t ws_bytes, elr_exec_out* out, void* stream);

/* elr_step_exec for the device-driven step (no counterpart in the reference): every count and class-order offset
 * comes from the descriptor `desc` that elr_plan_step wrote on the same stream, so the host issues the rest of the
 * step without reading the GPU.  args as for elr_step_exec except: b[ELR_NRANK] bounds the batch's rows (the other
 * bounds are ignored); u_ord, c_ord, sl_ord, loc_ord, L_row, L_cnt are elr_plan_step's outputs (class order, from
 * position 0); slots.ev_slot and slots.keep are its dyn_out, slots.nev bounds the evictions and slots.nkeep the kept
 * slots (both at most Cdyn), slots.n_free the free stack's depth.  The workspace (elr_step_exec_dev_bytes) holds
 * every array at its bound; the arrays' valid prefixes have the descriptor's counts.  The S rows are updated too.
 * link_stream and link_wait must be NULL (every launch on the call's stream). */
int64_t elr_step_exec_dev_bytes(const elr_exec_args* args);
int elr_step_exec_dev(const elr_exec_args* args, const int64_t* desc, void* ws, int64_t ws_bytes, elr_exec_out* out,
                      void* stream);

/* A whole device-driven step in one call (no counterpart in the reference): elr_plan_step, the rest of the batch's
 * segment sum (elr_segment_sum_plan_final, in the class order the plan resolves) and elr_step_exec_dev, with every
 * array in one workspace that the caller keeps from step to step (elr_step_dev_bytes, 256-byte aligned).  Where the
 * sum's final kernel is the single wave-per-row launch (D = 64, 128, 256 or 512, 16-byte aligned rows, more than
 * 3072 occurrences), the executor's first launch (call A's replay inputs and hit records) runs in the same launch. 
 *   plan:  as for elr_plan_step; its u, n, n_dev, s and next_mask change per step, nd bounds the dynamic slots;
 *          the output pointers are ignored (the call places them in ws).
 *   ctl:   as for elr_plan_step (desc is where this step's descriptor goes).
 *   grad [n_occ, D], key_bits, dplan, dplan_bytes: the batch's occurrence gradients and dedup plan (elr_dedup_plan).
 *   exec:  as for elr_step_exec_dev; its class-ordered arrays and slot lists are taken from the plan's outputs in
 *          ws, exec.b[ELR_NRANK] from plan.n and exec.upd.grad from the segment sum in ws.
 *   mark_*: optional (mark_rows NULL: none): the TTL lookahead's mark of a batch loaded ahead, elr_mark_rows(
 *          mark_rows, mark_n, mark_nmax, mark_value, plan.last_seen, plan.R, plan.next_bits, mark_bit), done in one
 *          launch with the directory's compaction -- after this step's plan has read last_seen and next_bits and
 *          before the next step's -- once the stream has waited for mark_event (a hipEvent_t recorded after the
 *          batch's dedup plan on another stream, or NULL).  The mark does not depend on this step's results and
 *          happens also when the step itself does nothing (an error).  If the wait cannot be queued, the step is
 *          issued without the mark and the call returns ELR_EINVAL.
 * out receives the byte offsets in ws of the plan's outputs (elr_plan_out order), of the per-row gradients G and
 * of the executor's outputs; they hold this step's values until the next call. */
typedef struct elr_step_dev_args {
  elr_plan_in plan;
  elr_plan_ctl ctl;
  const float* grad;
  int64_t n_occ;
  int64_t key_bits;
  const void* dplan;
  int64_t dplan_bytes;
  elr_exec_args exec;
  const int64_t* mark_rows;
  const int64_t* mark_n;
  int64_t mark_nmax;
  int64_t mark_value;
  int64_t mark_bit;
  void* mark_event;
} elr_step_dev_args;
typedef struct elr_step_dev_out {
  int64_t cls, flags, sl, c, order, rank, dyn_out, counts, u_ord, c_ord, sl_ord, L_row, L_cnt, loc_ord;
  int64_t grad_rows;          /* G [plan.n, D]: the per-row gradients in class-rank order */
  int64_t exec_ws;            /* the executor's workspace; out.exec's offsets are relative to it */
  elr_exec_out exec;
} elr_step_dev_out;
int64_t elr_step_dev_bytes(const elr_step_dev_args* args);
int elr_step_dev(const elr_step_dev_args* args, void* ws, int64_t ws_bytes, elr_step_dev_out* out, void* stream);

/* sizeof of this header's structs, for a binding to check its layouts (no counterpart in the reference): out[0..11] =
 * elr_dir_state, elr_dir_params, elr_plan_in, elr_plan_out, elr_assemble_args, elr_slots_args, elr_update_args,
 * elr_exec_args, elr_exec_out, elr_plan_ctl, elr_step_dev_args, elr_step_dev_out (at most n of them); returns the
 * number written. */
int elr_abi_sizes(int64_t* out, int n);

/* ---------------------------------------------------------------------------------------------------------
 * Row copies: dst[dst_idx[i]] = src[src_idx[i]], i < n, rows of W floats (NULL index = identity).
 * Replaces: the gradient-log append logs[A_ids] = g (srm2/elara.py:569-570 with srm2/csrc/srm2_cpu.cpp:167-180
 * cs_append semantics; here the log arena is in HBM), the resident-history record glog.index_put_((dyn, j), g)
 * (srm2/elara.py:501, 524) and the executor's index_select / index_copy_ of rows (srm2/elara.py:480-488,
 * 506-531).  Rows with an index outside [0, dst_rows) / [0, src_rows) are skipped.  Device pointers.
 * ------------------------------------------------------------------------------------------------------- */
int elr_copy_rows(float* dst, int64_t dst_rows, const int64_t* dst_idx, const float* src, int64_t src_rows,
                  const int64_t* src_idx, int64_t n, int64_t W, void* stream);

/* Resident-history record glog.index_put_((dyn - dyn_off, j), g) (srm2/elara.py:501, 524): glog [nd, K, W],
 * g [n, W], dyn and j int64 [n] (j NULL: entry 0, the admission record of srm2/elara.py:521-524, with dyn the pool
 * slots and dyn_off the static slot count).  Items whose slot or entry is out of range are skipped. */
int elr_glog_put(float* glog, int64_t nd, int64_t K, const int64_t* dyn, int64_t dyn_off, const int64_t* j,
                 const float* g, int64_t n, int64_t W, void* stream);

/* The history entries of evicted rows going back to L, moved into the log arena at their new log ids
 * (srm2/elara.py:396, 507 gather them from glog; elara.py:569-570 append them): logs[ids[r*K + k]] =
 * glog[clamp(dyn[r], 0, nd-1), k] for r < n, k < K; ids out of [0, nlogs) (-1: no entry) are skipped. */
int elr_glog_take(float* logs, int64_t nlogs, const int64_t* ids, const float* glog, int64_t nd, int64_t K,
                  const int64_t* dyn, int64_t n, int64_t W, void* stream);

/* out[rows[i]] = value for i < min(*n_dev, n_max), with the count read on the device (no counterpart in the
 * reference, which reads the batch's unique count on the host first): the TTL lookahead's record of when rows
 * appear next (srm2/elara.py:160-161) for a batch whose unique count the host reads later.  With bits (may be
 * NULL), also bits[rows[i]] |= bit: the planner's ring of loaded batches (elr_plan_in.next_bits).  rows must be
 * distinct.  Rows out of range are skipped. */
int elr_mark_rows(const int64_t* rows, const int64_t* n_dev, int64_t n_max, int32_t value, int32_t* out,
                  int64_t out_rows, uint32_t* bits, uint32_t bit, void* stream);

/* ---------------------------------------------------------------------------------------------------------
 * Exhaustive check of the step-constant division (no counterpart in the reference).  The Adam kernels compute
 * a / b for b = 1 - b1^t and b = 1 - b2^t as RN_f32((double)a * RN_f64(1/b)); for all 2^32 float bit patterns a
 * this compares that with the correctly rounded fp32 quotient a / b, adds the number of mismatches to
 * *mismatches (device uint64, caller zeroes it) and the lowest mismatching pattern to *first_bad (device uint32
 * atomic min; caller sets it to 0xFFFFFFFF).  Asynchronous; a few milliseconds.
 * ------------------------------------------------------------------------------------------------------- */
int elr_selfcheck_div(float b, unsigned long long* mismatches, unsigned int* first_bad, void* stream);

/* The same for the square root (no counterpart in the reference): the Adam kernels' fp32 square root against the
 * correctly rounded one, for all 2^32 bit patterns x. */
int elr_selfcheck_sqrt(unsigned long long* mismatches, unsigned int* first_bad, void* stream);

/* The same for the division by den (no counterpart in the reference): the Adam kernels' fast fp32 division core
 * against the correctly rounded division n / d, for one d in [2^-48, 2^65) (else ELR_EINVAL) and every bit pattern
 * n with 2^-60 <= |n| < 2^40; *tested (device uint64, caller zeroes it) receives the number of n compared. */
int elr_selfcheck_quot(float d, unsigned long long* mismatches, unsigned long long* tested, unsigned int* first_bad,
                       void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ELARA_AMD_H */
