// Shared device code of the elara_amd HIP kernels (gfx950, wave64).
//
// Bit-exactness rules for every fp32 expression in this library:
//   - no contraction into FMA (the build passes -ffp-contract=off; the pragma below enforces it per file);
//   - division and square root correctly rounded (-fhip-fp32-correctly-rounded-divide-sqrt; plain '/' and
//     __builtin_sqrtf, never the native/approximate intrinsics);
//   - fp32 denormals kept (no -fgpu-flush-denormals-to-zero).
// Under those rules each statement below is one IEEE-754 binary32 operation rounded to nearest even, which is
// what the reference's CPU Adam computes (srm2/csrc/srm2_cpu.cpp:22-34, built with -ffp-contract=off).
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#pragma clang fp contract(off)

#include "../../include/elara_amd.h"

namespace elr {

// The 8 fp32 scalars of one logical step (srm2/csrc/srm2_cpu.cpp:13-20) and the double reciprocals of the two
// bias corrections, r1 = RN_f64(1 / bc1) and r2 = RN_f64(1 / bc2), which make the divisions by them cheap.
struct AdamScalars {
  float lr, b1, omb1, b2, omb2, bc1, bc2, eps;
  double r1, r2;
};

inline AdamScalars make_scalars(const float sc[8]) {
  return AdamScalars{sc[0], sc[1], sc[2], sc[3], sc[4], sc[5], sc[6], sc[7], 1.0 / (double)sc[5],
                     1.0 / (double)sc[6]};
}

// Correctly rounded fp32 quotient a / b from y = RN_f64(1 / b): RN_f32((double)a * y).  The double product is
// within (2^-53 + 2^-53 + 2^-106) |a/b| < 2^-51 |a/b| of a/b.  Write the distance from a/b to a midpoint mu between
// consecutive floats as |a - mu*b| / |b| and bound the numerator below by the granularity of a and of mu*b: when
// it is not zero, the distance exceeds the product's error, for normal and subnormal results alike.  It is zero
// only if a/b is itself a midpoint, which needs a subnormal quotient and b an even integer other than a power of
// two; the divisors here are bias corrections in (0, 1], so rounding the product to float yields RN_f32(a / b) for
// every finite a (and inf/NaN propagate as in the division).  Three instructions instead of the eleven of the
// general correctly rounded fp32 division; checked over all 2^32 values of a by elr_selfcheck_div.
__device__ __forceinline__ float div_by_recip(float a, double y) { return (float)((double)a * y); }

// True on every active lane: a wave-uniform condition for choosing between a fast and a general code path.
__device__ __forceinline__ bool wave_all(bool p) {
  return __builtin_amdgcn_ballot_w64(p) == __builtin_amdgcn_read_exec();
}

// Lanes (as a wave mask) whose x lies in [lo, hi): two compares, each ballot taken on a single compare so that the
// mask is the compare's result itself.  NaN is in no range.
__device__ __forceinline__ uint64_t lanes_in(float x, float lo, float hi) {
  return __builtin_amdgcn_ballot_w64(x >= lo) & __builtin_amdgcn_ballot_w64(x < hi);
}

// Correctly rounded fp32 square root.  The compiler's IEEE sequence wraps a core -- the hardware estimate s and a
// choice among s - 1 ulp, s, s + 1 ulp by the signs of the residuals x - s'*s -- in a rescaling of small inputs and
// a special-case selection for 0, inf and NaN.  For a normal x >= 2^-96 neither wrapper changes anything, so when
// every lane of the wave has such an x (a wave-uniform branch) the core alone is used; otherwise the full
// sequence.  Checked over all 2^32 inputs by elr_selfcheck_sqrt.
__device__ __forceinline__ float sqrt_core(float x) {
  const float s = __builtin_amdgcn_sqrtf(x);
  const float sm = __uint_as_float(__float_as_uint(s) - 1u);
  const float sp = __uint_as_float(__float_as_uint(s) + 1u);
  const float rm = __builtin_fmaf(-sm, s, x);
  const float rp = __builtin_fmaf(-sp, s, x);
  const float r = rm <= 0.0f ? sm : s;
  return rp > 0.0f ? sp : r;
}

// x is finite, normal and >= 2^-96; then 2^-48 <= sqrt(x) < 2^64.
__device__ __forceinline__ bool sqrt_core_ok(float x) { return x >= 0x1.0p-96f && x < __builtin_inff(); }
__device__ __forceinline__ uint64_t sqrt_core_lanes(float x) { return lanes_in(x, 0x1.0p-96f, __builtin_inff()); }

__device__ __forceinline__ float sqrt_rn(float x) {
  if (sqrt_core_lanes(x) == __builtin_amdgcn_read_exec()) return sqrt_core(x);
  return __builtin_sqrtf(x);
}

// Correctly rounded fp32 division n / d for operands in a range.  The compiler's IEEE sequence is a scaling step
// (v_div_scale on d and on n), the Newton-refined reciprocal r, the quotient n*r, two remainder corrections (the
// last one, v_div_fmas, rescales when the scaling step asked for it) and a fixup (v_div_fixup) that handles zero,
// infinite and NaN operands and results out of range.  For 2^-48 <= d < 2^65 and 2^-60 <= |n| < 2^40 the scaling
// step changes neither operand and asks for no rescale (d and n/d are normal, 1/d is normal, the exponents differ
// by less than 96, n is far from the denormal range), and the fixup returns the quotient as it is (no special
// operand, a normal quotient whose sign is sign(n)).  There the core below -- the same instructions without
// scaling and fixup -- gives the same bits as n / d.  Checked over all 2^32 values of n for a set of d by
// elr_selfcheck_quot.
__device__ __forceinline__ bool quot_num_ok(float n) {  // 2^-60 <= |n| < 2^40
  return __builtin_fabsf(n) >= 0x1.0p-60f && __builtin_fabsf(n) < 0x1.0p40f;
}
__device__ __forceinline__ uint64_t quot_num_lanes(float n) {
  return lanes_in(__builtin_fabsf(n), 0x1.0p-60f, 0x1.0p40f);
}
__device__ __forceinline__ bool quot_den_ok(float d) { return d >= 0x1.0p-48f && d < 0x1.0p65f; }
__device__ __forceinline__ float div_core(float n, float d) {
  float r = __builtin_amdgcn_rcpf(d);
  const float e = __builtin_fmaf(-d, r, 1.0f);
  r = __builtin_fmaf(e, r, r);
  float q = n * r;
  float rem = __builtin_fmaf(-d, q, n);
  q = __builtin_fmaf(rem, r, q);
  rem = __builtin_fmaf(-d, q, n);
  return __builtin_fmaf(rem, r, q);
}

// eps in [+0, 2^60] (a test of the bit pattern, done on the scalar unit for a wave-uniform eps).  With
// sqrt_core_ok(vh) it puts den = sqrt(vh) + eps in [2^-48, 2^65), the range of div_core.
__device__ __forceinline__ bool eps_ok(float eps) { return __float_as_uint(eps) <= 0x5D800000u; }

// One Adam update of one element, in the reference's operation order (srm2/csrc/srm2_cpu.cpp:26-32).  Each
// statement is one correctly rounded fp32 operation; the two divisions by the step's bias corrections use
// div_by_recip.  When every lane of the wave has vh and num in range (and eps is), the square root and the
// division by den take their cores sqrt_core and div_core; otherwise the compiler's general sequences.  Both
// branches give the same bits.
__device__ __forceinline__ void adam_elem(float& w, float& m, float& v, float g, const AdamScalars& s) {
  float mj = s.b1 * m;
  float t1 = s.omb1 * g;
  mj = mj + t1;
  float vj = s.b2 * v;
  float t2 = s.omb2 * g;
  t2 = t2 * g;
  vj = vj + t2;
  float mh = div_by_recip(mj, s.r1);
  float vh = div_by_recip(vj, s.r2);
  float num = s.lr * mh;
  float up;
  if (eps_ok(s.eps) && (sqrt_core_lanes(vh) & quot_num_lanes(num)) == __builtin_amdgcn_read_exec()) {
    float den = sqrt_core(vh);
    den = den + s.eps;
    up = div_core(num, den);
  } else {
    float den = __builtin_sqrtf(vh);
    den = den + s.eps;
    up = num / den;
  }
  w = w - up;
  m = mj;
  v = vj;
}

__device__ __forceinline__ void adam_vec4(float4& w, float4& m, float4& v, const float4& g, const AdamScalars& s) {
  adam_elem(w.x, m.x, v.x, g.x, s);
  adam_elem(w.y, m.y, v.y, g.y, s);
  adam_elem(w.z, m.z, v.z, g.z, s);
  adam_elem(w.w, m.w, v.w, g.w, s);
}

// MurmurHash3 32-bit finalizer (fmix32), as srm2/gpu_ops.py:15-23 applies it to uint32 values.
__device__ __forceinline__ uint32_t fmix32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x85EBCA6Bu;
  x ^= x >> 13;
  x *= 0xC2B2AE35u;
  x ^= x >> 16;
  return x;
}

// Per-row part of the counter hash: fmix32(u32(r >> 32) + seed)  (srm2/gpu_ops.py:33).
__device__ __forceinline__ uint32_t init_row_key(int64_t r, uint32_t seed) {
  return fmix32((uint32_t)((uint64_t)r >> 32) + seed);
}

// Initial weight of element j of row r (srm2/gpu_ops.py:33-36):
//   key = u32(r*D + j) ^ rowkey;  h = fmix32(key ^ seed);  u = f32(h >> 8) * 2^-24;  w0 = (u*2 - 1) * bound.
// With k = h >> 8 < 2^24, f32(k), u = k*2^-24 and u*2 = k*2^-23 are exact, and so is u*2 - 1 = (k - 2^23)*2^-23
// (|k - 2^23| <= 2^23 fits the significand); one fma(f32(k), 2^-23, -1) computes that exact value.  The product with
// bound is the only rounding.
__device__ __forceinline__ float init_elem(uint32_t rlo_times_d_plus_j, uint32_t rowkey, uint32_t seed, float bound) {
  uint32_t h = fmix32((rlo_times_d_plus_j ^ rowkey) ^ seed);
  const float t = __builtin_fmaf((float)(h >> 8), 0x1.0p-23f, -1.0f);
  return t * bound;
}

// Four consecutive initial weights starting at element j0 (j0 % 4 == 0).
__device__ __forceinline__ float4 init_vec4(int64_t r, int64_t D, int64_t j0, uint32_t rowkey, uint32_t seed,
                                            float bound) {
  uint32_t base = (uint32_t)((uint64_t)r * (uint64_t)D + (uint64_t)j0);
  float4 w;
  w.x = init_elem(base + 0u, rowkey, seed, bound);
  w.y = init_elem(base + 1u, rowkey, seed, bound);
  w.z = init_elem(base + 2u, rowkey, seed, bound);
  w.w = init_elem(base + 3u, rowkey, seed, bound);
  return w;
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

// 16-byte load marked non-temporal (data read once, e.g. gradients and log entries).
__device__ __forceinline__ float4 ldg_stream(const float4* p) {
  const f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
  return make_float4(v.x, v.y, v.z, v.w);
}

// Lanes of a 64-wide wave that share one row when a row holds `nchunk` 16-byte chunks: the smallest power of two
// >= nchunk, capped at 64 (a lane then loops over nchunk/64 chunks).
inline int lanes_per_row_log2(int64_t nchunk) {
  int l = 0;
  while ((1 << l) < nchunk && l < 6) ++l;
  return l;
}

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Wave-per-row kernels launch one wave per group of rows (no loop iteration in practice): on gfx9 stores count in
// vmcnt, so a second grid-stride iteration would wait for the first iteration's stores before its loads.  The
// grid-stride loop remains only as a fallback past this many blocks (gridDim.x * 256 stays below 2^31).
constexpr int64_t kOneShotBlocks = int64_t(1) << 22;

// Rows per launch of a loop-free wave-per-row kernel with U rows per wave and 4 waves per block.
constexpr int64_t wpr_rows_per_launch(int U) { return kOneShotBlocks * 4 * U; }

// Grid size for a grid-stride loop over `units` work units of `per_block` units per block: enough blocks to
// cover the work, capped (by default at a few full waves of the 256-CU chip) so very large calls loop.
inline unsigned grid_for(int64_t units, int64_t per_block, int64_t cap_blocks = 256 * 64) {
  int64_t b = (units + per_block - 1) / per_block;
  if (b < 1) b = 1;
  if (b > cap_blocks) b = cap_blocks;
  return (unsigned)b;
}

inline int hip_rc(hipError_t e) { return e == hipSuccess ? ELR_OK : (int)e; }

inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? ELR_OK : (int)e;
}

}  // namespace elr
