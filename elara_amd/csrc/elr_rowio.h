// Wave-per-row access helpers: a row of D = 64*VPL floats is spread over the 64 lanes of one wavefront, lane l
// holding the VPL consecutive floats [l*VPL, l*VPL + VPL).  One wave therefore reads or writes a whole row with a
// single coalesced vector instruction (VPL = 1, 2, 4: dword, dwordx2, dwordx4; VPL = 8: two dwordx4).
//
// Why a wave per row: every per-row quantity (row id, slot, log offset, count, logical steps, Adam scalars) is
// then uniform across the wave.  Reading it through a readfirstlane'd index lets the compiler use scalar loads
// (s_load, through the scalar cache) and scalar branches, so the vector pipe only moves the D-wide payload.
#pragma once

#include "elr_common.h"

namespace elr {

template <int VPL>
struct RowFrag {
  float v[VPL];
};

template <int VPL, bool NT>
__device__ __forceinline__ RowFrag<VPL> frag_load(const float* __restrict__ p) {
  RowFrag<VPL> r;
  if constexpr (VPL == 1) {
    r.v[0] = NT ? __builtin_nontemporal_load(p) : *p;
  } else if constexpr (VPL == 2) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    const f2 t = NT ? __builtin_nontemporal_load(reinterpret_cast<const f2*>(p)) : *reinterpret_cast<const f2*>(p);
    r.v[0] = t.x;
    r.v[1] = t.y;
  } else {
    static_assert(VPL % 4 == 0, "VPL must be 1, 2 or a multiple of 4");
#pragma unroll
    for (int q = 0; q < VPL / 4; ++q) {
      const f32x4 t = NT ? __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p) + q)
                         : reinterpret_cast<const f32x4*>(p)[q];
      r.v[4 * q + 0] = t.x;
      r.v[4 * q + 1] = t.y;
      r.v[4 * q + 2] = t.z;
      r.v[4 * q + 3] = t.w;
    }
  }
  return r;
}

// Stores are marked non-temporal: every row written here (updated Adam state, replayed rows, fresh rows) is read
// again only by a later kernel, after far more than the caches hold has streamed through.  Measured on the C2 Adam
// step (d=128): 158 us with ordinary stores, 140 us with non-temporal ones.
template <int VPL, bool NT = true>
__device__ __forceinline__ void frag_store(float* __restrict__ p, const RowFrag<VPL>& r) {
  if constexpr (VPL == 1) {
    if constexpr (NT) __builtin_nontemporal_store(r.v[0], p);
    else *p = r.v[0];
  } else if constexpr (VPL == 2) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    f2 t;
    t.x = r.v[0];
    t.y = r.v[1];
    if constexpr (NT) __builtin_nontemporal_store(t, reinterpret_cast<f2*>(p));
    else *reinterpret_cast<f2*>(p) = t;
  } else {
#pragma unroll
    for (int q = 0; q < VPL / 4; ++q) {
      f32x4 t;
      t.x = r.v[4 * q + 0];
      t.y = r.v[4 * q + 1];
      t.z = r.v[4 * q + 2];
      t.w = r.v[4 * q + 3];
      if constexpr (NT) __builtin_nontemporal_store(t, reinterpret_cast<f32x4*>(p) + q);
      else reinterpret_cast<f32x4*>(p)[q] = t;
    }
  }
}

// adam_elem over the lane's fragment, with one range check and one branch for all its elements: the moments and the
// bias-corrected quotients of every element first, then either the cores (sqrt_core, div_core) for all of them, when
// every element of every active lane is in their range, or the general sequences.  Same operations, same bits.
template <int VPL>
__device__ __forceinline__ void frag_adam(RowFrag<VPL>& w, RowFrag<VPL>& m, RowFrag<VPL>& v, const RowFrag<VPL>& g,
                                          const AdamScalars& s) {
  float vh[VPL], num[VPL];
  uint64_t ok = __builtin_amdgcn_read_exec();
#pragma unroll
  for (int e = 0; e < VPL; ++e) {
    float mj = s.b1 * m.v[e];
    float t1 = s.omb1 * g.v[e];
    mj = mj + t1;
    float vj = s.b2 * v.v[e];
    float t2 = s.omb2 * g.v[e];
    t2 = t2 * g.v[e];
    vj = vj + t2;
    m.v[e] = mj;
    v.v[e] = vj;
    const float mh = div_by_recip(mj, s.r1);
    vh[e] = div_by_recip(vj, s.r2);
    num[e] = s.lr * mh;
    ok &= sqrt_core_lanes(vh[e]) & quot_num_lanes(num[e]);
  }
  if (eps_ok(s.eps) && ok == __builtin_amdgcn_read_exec()) {
#pragma unroll
    for (int e = 0; e < VPL; ++e) {
      float den = sqrt_core(vh[e]);
      den = den + s.eps;
      w.v[e] = w.v[e] - div_core(num[e], den);
    }
  } else {
#pragma unroll
    for (int e = 0; e < VPL; ++e) {
      float den = __builtin_sqrtf(vh[e]);
      den = den + s.eps;
      w.v[e] = w.v[e] - num[e] / den;
    }
  }
}

// Range check of the Adam cores, deferred: per lane, the smallest and largest vh and |num| of every element and
// step the fast path computed.  The cores' operand ranges hold for all of them exactly when vmin >= 2^-96,
// vmax < inf, nmin >= 2^-60 and nmax < 2^40 (min / max ignore a NaN operand; a NaN vh or num gives NaN through the
// cores as through the general sequences, so a NaN needs no recompute).  Two min3 / max3 instructions per two
// elements instead of four compares per element.
struct RangeAcc {
  float vmin, vmax, nmin, nmax;
};
__device__ __forceinline__ RangeAcc range_acc_init() {
  return RangeAcc{__builtin_inff(), 0.0f, __builtin_inff(), 0.0f};
}
__device__ __forceinline__ bool range_acc_ok(const RangeAcc& a) {
  return a.vmin >= 0x1.0p-96f && a.vmax < __builtin_inff() && a.nmin >= 0x1.0p-60f && a.nmax < 0x1.0p40f;
}

// One Adam step of the lane's fragment on the fast path only (the cores sqrt_core and div_core), with the operand
// ranges folded into acc; the caller recomputes the row on the general path when range_acc_ok(acc) fails on some
// lane.
template <int VPL>
__device__ __forceinline__ void frag_adam_fast(RowFrag<VPL>& w, RowFrag<VPL>& m, RowFrag<VPL>& v,
                                               const RowFrag<VPL>& g, const AdamScalars& s, RangeAcc& acc) {
  float vh[VPL], num[VPL];
#pragma unroll
  for (int e = 0; e < VPL; ++e) {
    float mj = s.b1 * m.v[e];
    const float t1 = s.omb1 * g.v[e];
    mj = mj + t1;
    float vj = s.b2 * v.v[e];
    float t2 = s.omb2 * g.v[e];
    t2 = t2 * g.v[e];
    vj = vj + t2;
    m.v[e] = mj;
    v.v[e] = vj;
    const float mh = div_by_recip(mj, s.r1);
    vh[e] = div_by_recip(vj, s.r2);
    num[e] = s.lr * mh;
  }
#pragma unroll
  for (int e = 0; e < VPL; e += 2) {
    if (e + 1 < VPL) {
      acc.vmin = __builtin_fminf(acc.vmin, __builtin_fminf(vh[e], vh[e + 1]));
      acc.vmax = __builtin_fmaxf(acc.vmax, __builtin_fmaxf(vh[e], vh[e + 1]));
      acc.nmin = __builtin_fminf(acc.nmin, __builtin_fminf(__builtin_fabsf(num[e]), __builtin_fabsf(num[e + 1])));
      acc.nmax = __builtin_fmaxf(acc.nmax, __builtin_fmaxf(__builtin_fabsf(num[e]), __builtin_fabsf(num[e + 1])));
    } else {
      acc.vmin = __builtin_fminf(acc.vmin, vh[e]);
      acc.vmax = __builtin_fmaxf(acc.vmax, vh[e]);
      acc.nmin = __builtin_fminf(acc.nmin, __builtin_fabsf(num[e]));
      acc.nmax = __builtin_fmaxf(acc.nmax, __builtin_fabsf(num[e]));
    }
  }
#pragma unroll
  for (int e = 0; e < VPL; ++e) {
    float den = sqrt_core(vh[e]);
    den = den + s.eps;
    w.v[e] = w.v[e] - div_core(num[e], den);
  }
}

// Initial weights of the lane's fragment of row r (D = 64*VPL): elements j = lane*VPL + e.
template <int VPL>
__device__ __forceinline__ RowFrag<VPL> frag_init(int64_t r, int lane, uint32_t seed, float bound) {
  constexpr uint32_t D = 64u * VPL;
  const uint32_t rk = init_row_key(r, seed);
  const uint32_t base = (uint32_t)((uint64_t)r * (uint64_t)D) + (uint32_t)(lane * VPL);
  RowFrag<VPL> w;
#pragma unroll
  for (int e = 0; e < VPL; ++e) w.v[e] = init_elem(base + (uint32_t)e, rk, seed, bound);
  return w;
}

template <int VPL>
__device__ __forceinline__ RowFrag<VPL> frag_zero() {
  RowFrag<VPL> z;
#pragma unroll
  for (int e = 0; e < VPL; ++e) z.v[e] = 0.0f;
  return z;
}

// Scalars of one table row, read through the scalar cache when `step` is wave-uniform.  recip [S, 2] holds
// RN_f64(1/bc1), RN_f64(1/bc2) per row (elr_scalar_recip).
__device__ __forceinline__ AdamScalars table_scalars(const float* __restrict__ table,
                                                     const double* __restrict__ recip, int64_t step) {
  const float* t = table + step * 8;
  return AdamScalars{t[0], t[1], t[2], t[3], t[4], t[5], t[6], t[7], recip[2 * step], recip[2 * step + 1]};
}

// The same without a reciprocal table (recip may be NULL): the reciprocals are then computed here with the
// correctly rounded double division.
__device__ __forceinline__ AdamScalars table_scalars_any(const float* __restrict__ table,
                                                         const double* __restrict__ recip, int64_t step) {
  const float* t = table + step * 8;
  const double r1 = recip ? recip[2 * step] : 1.0 / (double)t[5];
  const double r2 = recip ? recip[2 * step + 1] : 1.0 / (double)t[6];
  return AdamScalars{t[0], t[1], t[2], t[3], t[4], t[5], t[6], t[7], r1, r2};
}

// Index of this wave in the grid and the number of waves, both wave-uniform (SGPR) values.
__device__ __forceinline__ int64_t wave_id() {
  return (int64_t)__builtin_amdgcn_readfirstlane((int)(blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)));
}
__device__ __forceinline__ int64_t wave_count() { return (int64_t)gridDim.x * (blockDim.x >> 6); }

// Launch `kern` on grid g; with timing events (either may be NULL), hipExtLaunchKernelGGL has the dispatch itself
// record them at the kernel's start and end, as a profiler times a kernel (no marker packets between launches).
template <typename Kern, typename... Args>
inline void launch_timed(Kern kern, unsigned g, hipStream_t st, hipEvent_t e0, hipEvent_t e1, Args... args) {
  if (e0 || e1) hipExtLaunchKernelGGL(kern, dim3(g), dim3(256), 0, st, e0, e1, 0, args...);
  else kern<<<g, 256, 0, st>>>(args...);
}

// VPL for D if the wave-per-row kernels handle it (D = 64, 128, 256, 512), else 0.
inline int wpr_vpl(int64_t D) {
  switch (D) {
    case 64: return 1;
    case 128: return 2;
    case 256: return 4;
    case 512: return 8;
    default: return 0;
  }
}

}  // namespace elr
