// Device side of the admissions (planner.hip): one admitted row's directory fields, and the admissions with their
// pool-slot bookkeeping as a functor (elr_launch.h), which the step's executor launches beside call B's count kernel.
#pragma once

#include "elr_desc.h"
#include "elr_launch.h"

namespace elr {

// Admissions of one step (srm2/elara.py:352-367): row adm_rows[i] takes pool slot adm_slots[i]; the first lazy_n
// rows are N/L rows (they keep their code as c0 and, with evl, start a resident history whose step 0 is s), the rest
// are F rows (c0 = -1).
__device__ __forceinline__ void admit_one(int64_t i, int64_t r, int64_t a, int64_t lazy_n, int evl, int64_t s,
                                          int64_t n0, int64_t C, int64_t R, int K, const int8_t* __restrict__ code,
                                          int32_t* __restrict__ slot_of, int64_t* __restrict__ slot_row,
                                          int8_t* __restrict__ adm_c0, int8_t* __restrict__ rj,
                                          int8_t* __restrict__ rok, int32_t* __restrict__ pstep) {
  if (r < 0 || r >= R || a < n0 || a >= C) return;
  const bool il = i < lazy_n, lazy = il && evl;
  slot_of[r] = (int32_t)a;
  slot_row[a] = r;
  adm_c0[a] = il ? code[r] : (int8_t)-1;
  rj[a] = lazy ? 1 : 0;
  rok[a] = lazy ? 1 : 0;
  if (lazy) pstep[(a - n0) * K] = (int32_t)s;
}

// The pool-slot bookkeeping of the admissions (srm2/elara.py:345-347, 368) together with the admissions: the stack
// is free_stack[0, n_free) followed by ev_slot[0, nev); its top n_adm entries are the admitted rows' slots (bottom
// first), the evicted slots below them are written above n_free in place (the stack's reads at positions < n_free
// and its writes at positions >= n_free never meet), and dyn_out = keep, then the admitted slots.
struct PlanAdmitSlots {
  elr_slots_args sl;
  const int64_t* adm_rows;
  int64_t n_adm, lazy_n;
  int evl;
  int64_t s, n0, C, R;
  int K;
  const int8_t* code;
  int32_t* slot_of;
  int64_t* slot_row;
  int8_t* adm_c0;
  int8_t* rj;
  int8_t* rok;
  int32_t* pstep;
  // device-driven step: sl.n_free, sl.nev, sl.nkeep, n_adm and lazy_n are upper bounds (the grid), and sl.keep and
  // adm_rows the planner's slot partition (2 nkeep entries) and the rows in class-rank order (rows_bound of them),
  // offset on the device
  const int64_t* desc;
  int64_t rows_bound;
  __device__ void operator()(int64_t blk, int64_t) const {
    elr_slots_args sl = this->sl;
    int64_t n_adm = this->n_adm, lazy_n = this->lazy_n;
    const int64_t* adm_rows = this->adm_rows;
    if (desc) {   // each within the bound the grid and the arrays were sized for
      sl.n_free = clampi(desc[kDNFree], 0, sl.n_free);
      sl.nev = clampi(desc[kDNev], 0, sl.nev);
      sl.nkeep = clampi(desc[kDNKeep], 0, sl.nkeep);
      sl.keep += clampi(desc[kDKeepOff], 0, 2 * this->sl.nkeep - sl.nkeep);
      n_adm = clampi(desc[kDNAdm], 0, this->n_adm);
      lazy_n = clampi(desc[kDLazy], 0, n_adm);
      adm_rows += clampi(desc[kDW0], 0, rows_bound - n_adm);
    }
    const int64_t i = blk * kFunctorBlock + threadIdx.x;
    const int64_t nf = sl.n_free + sl.nev, rest = nf - n_adm;
    if (i < n_adm) {
      const int64_t pos = rest + i;
      const int64_t a = pos < sl.n_free ? sl.free_stack[pos] : sl.ev_slot[pos - sl.n_free];
      sl.adm_slots[i] = a;
      sl.dyn_out[sl.nkeep + i] = a;
      admit_one(i, adm_rows[i], a, lazy_n, evl, s, n0, C, R, K, code, slot_of, slot_row, adm_c0, rj, rok, pstep);
    }
    if (i < sl.nkeep) sl.dyn_out[i] = sl.keep[i];
    if (i < sl.nev && sl.n_free + i < rest) sl.free_stack[sl.n_free + i] = sl.ev_slot[i];
  }
};

// Blocks of a PlanAdmitSlots launch: one thread per admitted row, kept slot and evicted slot.
inline int64_t admit_slots_blocks(const elr_slots_args& sl, int64_t n_adm) {
  int64_t m = n_adm > sl.nkeep ? n_adm : sl.nkeep;
  if (sl.nev > m) m = sl.nev;
  return (m + kFunctorBlock - 1) / kFunctorBlock;
}

// The checks of elr_plan_admit_slots's arguments (planner.hip).
int admit_slots_check(const elr_slots_args& sl, const int64_t* adm_rows, int64_t n_adm, int64_t lazy_n, int64_t n0,
                      int64_t C, int64_t R, int K, const int8_t* code, int32_t* slot_of, int64_t* slot_row,
                      int8_t* adm_c0, int8_t* rj, int8_t* rok, int32_t* pstep);

}  // namespace elr
