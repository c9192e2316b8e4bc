// The device-driven step: the step's counts live in a small device array (the step descriptor) that the planner's
// scan launch writes, and every later kernel of the step reads its item counts and range offsets there instead of
// taking them from the host.  Grids are sized from upper bounds the host knows without reading the GPU (the batch's
// occurrence count, the dynamic pool size); blocks and waves past a device count do nothing.  So the host issues a
// whole step -- plan, segment sum, directory calls, admissions, assembly and update -- without waiting for the GPU
// (the reference reads its class counts on the host every step, srm2/elara.py:242, 406).
#pragma once

#include "elr_common.h"

namespace elr {

// Descriptor fields (int64 each; ELR_DESC_WORDS in the C header).
enum : int {
  kDB = 0,            // [0, 11): class-rank bounds b[r] (positions of rank r in the class order: b[r] .. b[r+1])
  kDNev = 11,         // evicted dynamic slots: dyn_out[0, nev)
  kDKeepOff = 12,     // kept dynamic slots: dyn_out[keep_off, keep_off + nkeep)
  kDNKeep = 13,
  kDNFree = 14,       // free-stack depth before this step's pushes
  kDNAdm = 15,        // admitted rows (ranks NADM, LADM, FADM)
  kDLazy = 16,        // admitted N and L rows (the first lazy of the admitted)
  kDNL = 17,          // L rows (admitted, appended, compacted), their replay inputs
  kDNLa = 18,         // admitted L rows
  kDNLp = 19,         // appended L rows
  kDNa = 20,          // appends (N and L)
  kDNc = 21,          // compactions (N and L)
  kDNr = 22,          // deferred release items of call B (the evictions, Triton order; else 0)
  kDNh = 23,          // hits
  kDW0 = 24,          // first work position (= b[NADM])
  kDNw = 25,          // work rows (b[S] - b[NADM])
  kDNs = 26,          // S rows
  kDNTail = 27,       // compacted and transient rows (b[FN + 1] - b[NCMP])
  kDSkip = 28,        // 1: the step does nothing (an error of this or an earlier step; every count above is 0)
  kDOverflow = 29,    // admissions dropped for want of pool slots (srm2/elara.py:246-256)
  kDTake = 30,        // preempted slots
  kDBarrier = 31,     // 1: a dropped row appears in the next batches (the exactness barrier, elara.py:252-258)
  kDNRows = 32,       // the batch's unique rows
  kDNd = 33,          // dynamic slots held before the step
  kDMatHi = 34,       // bounds of the step's allocations (capacity check)
  kDLogHi = 35,
  kDWords = 40
};

// The persistent control state of a device-driven ElaraStep (int64 each; ELR_CTL_WORDS in the C header).
enum : int {
  kSNFree = 0,     // free-stack depth
  kSNd = 1,        // dynamic slots held (the list's length)
  kSErr = 2,       // sticky error bits: ELR_STEP_ERR_ROWS, ELR_STEP_ERR_CAPACITY
  kSErrStep = 3,   // logical step of the first error
  kSErrA = 4,      // its figures: rows out of range, the MAT bound, the log bound
  kSErrB = 5,
  kSErrC = 6,
  kSReserved = 7,  // unused
  kSStats = 8,     // [8, 8 + kNumStats): accumulated per-step statistics (the ElaraStep.stats keys below)
  kSWords = 32
};

// Accumulated statistics, in this order: hits, N, L, F, S, adm, ev, preempt, overflow, compactions, appends,
// barriers, steps.
enum : int {
  kStHits = 0, kStN, kStL, kStF, kStS, kStAdm, kStEv, kStPreempt, kStOverflow, kStCompactions, kStAppends,
  kStBarriers, kStSteps, kNumStats
};

// x clamped to [lo, hi]: every value a kernel takes from the descriptor is kept within the bounds its arrays were
// sized for, so that no count or offset can carry an access outside them.
__device__ __forceinline__ int64_t clampi(int64_t x, int64_t lo, int64_t hi) { return x < lo ? lo : (x > hi ? hi : x); }

// A count a kernel takes from its argument (v) or, in a device-driven step, from the descriptor (p[0] * mul).  In
// a device-driven step v holds the host's upper bound, which sizes the grid (and bounds the count).
struct DevCount {
  int64_t v;
  const int64_t* p;
  int64_t mul;
  __device__ __forceinline__ int64_t get() const { return p ? clampi(*p * mul, 0, v) : v; }
};

__host__ __device__ inline DevCount dcount(int64_t v) { return DevCount{v, nullptr, 1}; }
__host__ __device__ inline DevCount dcount(int64_t hi, const int64_t* desc, int field, int64_t mul = 1) {
  return desc ? DevCount{hi, desc + field, mul} : DevCount{hi, nullptr, 1};
}

// A pointer a kernel offsets by a descriptor field in a device-driven step (base + p[0] * mul), else base itself.
template <class T>
struct DevPtr {
  T* base;
  const int64_t* p;
  int64_t mul;
  __device__ __forceinline__ T* get() const { return p ? base + (*p < 0 ? 0 : *p) * mul : base; }
};

template <class T>
__host__ __device__ inline DevPtr<T> dptr_at(T* base) {
  return DevPtr<T>{base, nullptr, 1};
}
template <class T>
__host__ __device__ inline DevPtr<T> dptr_at(T* base, const int64_t* desc, int field, int64_t mul = 1) {
  return DevPtr<T>{base, desc ? desc + field : nullptr, mul};
}

}  // namespace elr
