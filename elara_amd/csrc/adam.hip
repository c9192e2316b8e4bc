// Row-sparse Adam on an interleaved [C,3,D] fp32 (w,m,v) table, in place (HBM-bound, no MFMA).
//
// Replaces srm2/ops.py:42-67 (_adam_rows / gpu_adam).  Per element the arithmetic is elr::adam_elem, the
// reference's CPU operation order (srm2/csrc/srm2_cpu.cpp:22-34), so results are bitwise those of cpu_adam.
//
// Launch shape: a row of D floats is D/4 16-byte chunks; 2^lg lanes of a wave share one row (lg from
// lanes_per_row_log2), so a wave updates 64 >> lg rows at a time with one global_load_dwordx4 per lane for each
// of w, m, v, g and one global_store_dwordx4 for each of w, m, v.  The gradient is read once, with a
// non-temporal load.  A grid-stride loop over row groups keeps the grid bounded for very large calls.
#include "elr_common.h"

#include <cmath>

namespace elr {

template <typename Idx>
__global__ __launch_bounds__(256) void k_adam_rows_v4(float* __restrict__ state, int64_t C,
                                                      const Idx* __restrict__ slots, const float* __restrict__ grad,
                                                      int64_t n, int nchunk, int lg, AdamScalars s) {
  const int lane = threadIdx.x & 63;
  const int l = lane & ((1 << lg) - 1);
  const int64_t rpw = 64 >> lg;
  const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int64_t nwave = ((int64_t)gridDim.x * blockDim.x) >> 6;
  for (int64_t i = wave * rpw + (lane >> lg); i < n; i += nwave * rpw) {
    const int64_t slot = (int64_t)slots[i];
    if (slot < 0 || slot >= C) continue;
    float4* rec = reinterpret_cast<float4*>(state) + slot * 3 * (int64_t)nchunk;
    const float4* g = reinterpret_cast<const float4*>(grad) + i * (int64_t)nchunk;
    for (int c = l; c < nchunk; c += (1 << lg)) {
      float4 w = rec[c];
      float4 m = rec[nchunk + c];
      float4 v = rec[2 * nchunk + c];
      float4 gg = ldg_stream(g + c);
      adam_vec4(w, m, v, gg, s);
      rec[c] = w;
      rec[nchunk + c] = m;
      rec[2 * nchunk + c] = v;
    }
  }
}

// Fallback for D % 4 != 0 or buffers not 16-byte aligned: one wave per row, one float per lane.
template <typename Idx>
__global__ __launch_bounds__(256) void k_adam_rows_scalar(float* __restrict__ state, int64_t C,
                                                          const Idx* __restrict__ slots,
                                                          const float* __restrict__ grad, int64_t n, int64_t D,
                                                          AdamScalars s) {
  const int lane = threadIdx.x & 63;
  const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int64_t nwave = ((int64_t)gridDim.x * blockDim.x) >> 6;
  for (int64_t i = wave; i < n; i += nwave) {
    const int64_t slot = (int64_t)slots[i];
    if (slot < 0 || slot >= C) continue;
    float* w = state + slot * 3 * D;
    const float* g = grad + i * D;
    for (int64_t j = lane; j < D; j += 64) {
      float wj = w[j], mj = w[D + j], vj = w[2 * D + j];
      adam_elem(wj, mj, vj, g[j], s);
      w[j] = wj;
      w[D + j] = mj;
      w[2 * D + j] = vj;
    }
  }
}

template <typename Idx>
static int launch_adam(float* state, int64_t C, const Idx* slots, const float* grad, int64_t n, int64_t D,
                       const AdamScalars& s, hipStream_t st) {
  if (D % 4 == 0 && D / 4 <= INT32_MAX && aligned16(state) && aligned16(grad)) {
    const int64_t nchunk = D / 4;
    const int lg = lanes_per_row_log2(nchunk);
    const int64_t rpw = 64 >> lg;
    const int64_t waves = (n + rpw - 1) / rpw;
    k_adam_rows_v4<Idx><<<grid_for(waves, 4), 256, 0, st>>>(state, C, slots, grad, n, (int)nchunk, lg, s);
  } else {
    k_adam_rows_scalar<Idx><<<grid_for(n, 4), 256, 0, st>>>(state, C, slots, grad, n, D, s);
  }
  return launch_status();
}

}  // namespace elr

extern "C" void elr_adam_scalars(double lr, double b1, double b2, double eps, int64_t step, float out[8]) {
  // fp64 arithmetic rounded to fp32, srm2/csrc/srm2_cpu.cpp:15-20.
  out[0] = (float)lr;
  out[1] = (float)b1;
  out[2] = (float)(1.0 - b1);
  out[3] = (float)b2;
  out[4] = (float)(1.0 - b2);
  out[5] = (float)(1.0 - std::pow(b1, (double)step));
  out[6] = (float)(1.0 - std::pow(b2, (double)step));
  out[7] = (float)eps;
}

extern "C" int elr_scalar_table(double lr, double b1, double b2, double eps, int64_t max_step, float* table_host) {
  if (max_step < 0 || !table_host) return ELR_EINVAL;
  for (int j = 0; j < 8; ++j) table_host[j] = 0.0f;  // row 0: no step (srm2/gpu_ops.py:87)
  for (int64_t t = 1; t <= max_step; ++t) elr_adam_scalars(lr, b1, b2, eps, t, table_host + t * 8);
  return ELR_OK;
}

extern "C" int elr_adam_rows(float* state, int64_t C, const void* slots, int idx64, const float* grad, int64_t n,
                             int64_t D, const float sc[8], void* stream) {
  if (n < 0 || D <= 0 || C < 0 || !sc) return ELR_EINVAL;
  if (n == 0) return ELR_OK;
  if (!state || !slots || !grad) return ELR_EINVAL;
  const elr::AdamScalars s = {sc[0], sc[1], sc[2], sc[3], sc[4], sc[5], sc[6], sc[7]};
  hipStream_t st = (hipStream_t)stream;
  if (idx64) return elr::launch_adam(state, C, (const int64_t*)slots, grad, n, D, s, st);
  return elr::launch_adam(state, C, (const int32_t*)slots, grad, n, D, s, st);
}
