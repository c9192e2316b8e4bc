// Exhaustive checks of this library's fp32 arithmetic shortcuts: the division by a step-constant divisor, the
// square root (sqrt_rn) and the division core (div_core).
//
// The Adam kernels compute the correctly rounded quotient a / b for the two per-step divisors b = 1 - b1^t and
// b = 1 - b2^t as RN_f32((double)a * y) with y = RN_f64(1 / b).  Why that is exact for every finite a: the double
// product is within 2^-51 |a/b| of a/b, while a quotient of two floats lies at least 2^-49 |a/b| away from every
// midpoint between consecutive floats (normal and subnormal results alike), so rounding the product to float
// gives the float nearest to a/b.  This kernel confirms it on the GPU for one divisor over all 2^32 bit patterns
// of a, against the compiler's correctly rounded fp32 division (NaN results compare equal when both are NaN).
#include "elr_common.h"

namespace elr {

constexpr int kCheckThreads = 256;
constexpr int kCheckPerThread = 16;

__global__ __launch_bounds__(kCheckThreads) void k_check_div(float b, double y, uint64_t base,
                                                             unsigned long long* __restrict__ bad,
                                                             unsigned int* __restrict__ first_bad) {
  const uint64_t t0 = base + ((uint64_t)blockIdx.x * kCheckThreads + threadIdx.x) * kCheckPerThread;
  int nbad = 0;
  uint32_t firstv = 0xFFFFFFFFu;
  for (int k = 0; k < kCheckPerThread; ++k) {
    const uint64_t ab = t0 + k;
    if (ab > 0xFFFFFFFFull) break;
    const float a = __uint_as_float((uint32_t)ab);
    const float want = a / b;
    const float got = div_by_recip(a, y);
    const bool same = __float_as_uint(want) == __float_as_uint(got) || (want != want && got != got);
    if (!same) {
      ++nbad;
      if ((uint32_t)ab < firstv) firstv = (uint32_t)ab;
    }
  }
  if (nbad) {
    atomicAdd(bad, (unsigned long long)nbad);
    atomicMin(first_bad, firstv);
  }
}

// sqrt_rn against the compiler's correctly rounded fp32 square root, for all 2^32 bit patterns x (consecutive
// patterns share a wave, so waves with special or small values take sqrt_rn's full path and the others its core).
__global__ __launch_bounds__(kCheckThreads) void k_check_sqrt(uint64_t base, unsigned long long* __restrict__ bad,
                                                              unsigned int* __restrict__ first_bad) {
  const uint64_t t0 = base + ((uint64_t)blockIdx.x * kCheckThreads + threadIdx.x);
  int nbad = 0;
  uint32_t firstv = 0xFFFFFFFFu;
  const uint64_t stride = (uint64_t)gridDim.x * kCheckThreads;
  for (uint64_t xb = t0; xb <= 0xFFFFFFFFull; xb += stride) {
    const float x = __uint_as_float((uint32_t)xb);
    const float want = __builtin_sqrtf(x);
    const float got = sqrt_rn(x);
    const bool same = __float_as_uint(want) == __float_as_uint(got) || (want != want && got != got);
    if (!same) {
      ++nbad;
      if ((uint32_t)xb < firstv) firstv = (uint32_t)xb;
    }
  }
  if (nbad) {
    atomicAdd(bad, (unsigned long long)nbad);
    atomicMin(first_bad, firstv);
  }
}

// div_core(n, d) against the compiler's correctly rounded fp32 division n / d, for one d in div_core's range and
// every bit pattern n in it (quot_num_ok); `tested` counts the patterns compared.
__global__ __launch_bounds__(kCheckThreads) void k_check_quot(float d, uint64_t base,
                                                              unsigned long long* __restrict__ bad,
                                                              unsigned long long* __restrict__ tested,
                                                              unsigned int* __restrict__ first_bad) {
  const uint64_t t0 = base + ((uint64_t)blockIdx.x * kCheckThreads + threadIdx.x) * kCheckPerThread;
  int nbad = 0, ntested = 0;
  uint32_t firstv = 0xFFFFFFFFu;
  for (int k = 0; k < kCheckPerThread; ++k) {
    const uint64_t nb = t0 + k;
    if (nb > 0xFFFFFFFFull) break;
    const float n = __uint_as_float((uint32_t)nb);
    if (!quot_num_ok(n)) continue;
    ++ntested;
    const float want = n / d;
    const float got = div_core(n, d);
    if (__float_as_uint(want) != __float_as_uint(got)) {
      ++nbad;
      if ((uint32_t)nb < firstv) firstv = (uint32_t)nb;
    }
  }
  if (ntested) atomicAdd(tested, (unsigned long long)ntested);
  if (nbad) {
    atomicAdd(bad, (unsigned long long)nbad);
    atomicMin(first_bad, firstv);
  }
}

}  // namespace elr

extern "C" int elr_selfcheck_sqrt(unsigned long long* mismatches, unsigned int* first_bad, void* stream) {
  using namespace elr;
  if (!mismatches || !first_bad) return ELR_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  const uint64_t blocks = 1ull << 18;                               // 2^26 threads, 64 patterns each
  k_check_sqrt<<<(unsigned)blocks, kCheckThreads, 0, st>>>(0, mismatches, first_bad);
  return launch_status();
}

extern "C" int elr_selfcheck_div(float b, unsigned long long* mismatches, unsigned int* first_bad, void* stream) {
  using namespace elr;
  if (!mismatches || !first_bad) return ELR_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  const double y = 1.0 / (double)b;
  const uint64_t per_block = (uint64_t)kCheckThreads * kCheckPerThread;
  const uint64_t blocks_per_launch = 1ull << 18;
  for (uint64_t base = 0; base < (1ull << 32); base += blocks_per_launch * per_block)
    k_check_div<<<(unsigned)blocks_per_launch, kCheckThreads, 0, st>>>(b, y, base, mismatches, first_bad);
  return launch_status();
}

extern "C" int elr_selfcheck_quot(float d, unsigned long long* mismatches, unsigned long long* tested,
                                  unsigned int* first_bad, void* stream) {
  using namespace elr;
  if (!mismatches || !tested || !first_bad) return ELR_EINVAL;
  if (!(d >= 0x1.0p-48f && d < 0x1.0p65f)) return ELR_EINVAL;  // the range of div_core's denominators
  hipStream_t st = (hipStream_t)stream;
  const uint64_t per_block = (uint64_t)kCheckThreads * kCheckPerThread;
  const uint64_t blocks_per_launch = 1ull << 18;
  for (uint64_t base = 0; base < (1ull << 32); base += blocks_per_launch * per_block)
    k_check_quot<<<(unsigned)blocks_per_launch, kCheckThreads, 0, st>>>(d, base, mismatches, tested, first_bad);
  return launch_status();
}
