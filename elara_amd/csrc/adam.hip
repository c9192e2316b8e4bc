// Row-sparse Adam on an interleaved [C,3,D] fp32 (w,m,v) table, in place (HBM-bound, no MFMA).
//
// Replaces srm2/ops.py:42-67 (_adam_rows / gpu_adam).  Per element the arithmetic is elr::adam_elem, the
// reference's CPU operation order (srm2/csrc/srm2_cpu.cpp:22-34), so results are bitwise those of cpu_adam.
//
// Launch shapes.  D in {64,128,256,512}: one wave per row (elr_rowio.h), U rows per wave, slot ids read as scalars.
// Other D divisible by 4: 2^lg lanes share one row (lg from lanes_per_row_log2), one 16-byte chunk per lane per
// pass, a grid-stride loop over row groups.  Otherwise one float per lane.  The gradient is read once, with a
// non-temporal load.
#include "elr_rowio.h"

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
    const int64_t slot = slots ? (int64_t)slots[i] : i;
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
    const int64_t slot = slots ? (int64_t)slots[i] : i;
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

// Wave-per-row variant for D = 64*VPL: the slot of each row is a wave-uniform (scalar) load; the U rows of a wave
// issue all their w, m, v, g loads before the first update.  No loop (see init_replay.hip): one row group per
// wave, large calls split into several launches on the host.
constexpr int kAdamRowsPerWave = 1;

template <int VPL, typename Idx, int U>
__global__ __launch_bounds__(256) void k_adam_rows_wpr(float* __restrict__ state, int64_t C,
                                                       const Idx* __restrict__ slots, int64_t base,
                                                       const float* __restrict__ grad, int64_t n, AdamScalars s) {
  constexpr int64_t D = 64 * VPL;
  const int lane = threadIdx.x & 63;
  const int64_t i0 = wave_id() * U;
  int64_t sl[U];
  RowFrag<VPL> w[U], m[U], v[U], g[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t i = i0 + u;
    sl[u] = i < n ? (slots ? (int64_t)slots[i] : base + i) : -1;
    if (sl[u] >= C) sl[u] = -1;
    if (sl[u] >= 0) {
      const float* rec = state + sl[u] * 3 * D + lane * VPL;
      w[u] = frag_load<VPL, false>(rec);
      m[u] = frag_load<VPL, false>(rec + D);
      v[u] = frag_load<VPL, false>(rec + 2 * D);
      g[u] = frag_load<VPL, true>(grad + i * D + lane * VPL);
    }
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (sl[u] < 0) continue;
    frag_adam<VPL>(w[u], m[u], v[u], g[u], s);
    float* rec = state + sl[u] * 3 * D + lane * VPL;
    frag_store<VPL>(rec, w[u]);
    frag_store<VPL>(rec + D, m[u]);
    frag_store<VPL>(rec + 2 * D, v[u]);
  }
}

template <int VPL, typename Idx>
static void launch_adam_wpr(float* state, int64_t C, const Idx* slots, const float* grad, int64_t n,
                            const AdamScalars& s, hipStream_t st, hipEvent_t e0, hipEvent_t e1) {
  constexpr int U = kAdamRowsPerWave;
  constexpr int64_t D = 64 * VPL;
  constexpr int64_t per = wpr_rows_per_launch(U);
  for (int64_t a = 0; a < n; a += per) {
    const int64_t m = n - a < per ? n - a : per;
    launch_timed(k_adam_rows_wpr<VPL, Idx, U>, grid_for((m + U - 1) / U, 4, kOneShotBlocks), st,
                 a == 0 ? e0 : nullptr, a + m >= n ? e1 : nullptr, state, C, slots ? slots + a : nullptr, a,
                 grad + a * D, m, s);
  }
}

// D = 64, four rows per wave: a quarter wave (16 lanes of 16 bytes) per row, so that each load and store
// instruction moves 1 KB instead of the 256 bytes of a wave-per-row pass (C1: 22.0 us per launch against 23.0 with
// two rows per wave of 8-byte lanes and 25.5 with a wave per row).  Same per-element operations as every other Adam
// kernel here; frag_adam's range check then covers the lanes of all four rows.
template <typename Idx>
__global__ __launch_bounds__(256) void k_adam_rows_d64_quad(float* __restrict__ state, int64_t C,
                                                            const Idx* __restrict__ slots, int64_t base,
                                                            const float* __restrict__ grad, int64_t n,
                                                            AdamScalars s) {
  constexpr int64_t D = 64;
  const int lane = threadIdx.x & 63;
  const int64_t i = wave_id() * 4 + (lane >> 4);
  const int off = (lane & 15) * 4;
  int64_t sl = i < n ? (slots ? (int64_t)slots[i] : base + i) : -1;
  if (sl >= C) sl = -1;
  if (sl < 0) return;
  float* rec = state + sl * 3 * D + off;
  RowFrag<4> w = frag_load<4, false>(rec), m = frag_load<4, false>(rec + D), v = frag_load<4, false>(rec + 2 * D);
  const RowFrag<4> g = frag_load<4, true>(grad + i * D + off);
  frag_adam<4>(w, m, v, g, s);
  frag_store<4>(rec, w);
  frag_store<4>(rec + D, m);
  frag_store<4>(rec + 2 * D, v);
}

template <typename Idx>
static void launch_adam_d64_quad(float* state, int64_t C, const Idx* slots, const float* grad, int64_t n,
                                 const AdamScalars& s, hipStream_t st, hipEvent_t e0, hipEvent_t e1) {
  constexpr int64_t per = wpr_rows_per_launch(4);
  for (int64_t a = 0; a < n; a += per) {
    const int64_t m = n - a < per ? n - a : per;
    launch_timed(k_adam_rows_d64_quad<Idx>, grid_for((m + 3) / 4, 4, kOneShotBlocks), st, a == 0 ? e0 : nullptr,
                 a + m >= n ? e1 : nullptr, state, C, slots ? slots + a : nullptr, a, grad + a * 64, m, s);
  }
}

template <typename Idx>
static int launch_adam(float* state, int64_t C, const Idx* slots, const float* grad, int64_t n, int64_t D,
                       const AdamScalars& s, hipStream_t st, hipEvent_t e0, hipEvent_t e1) {
  const int vpl = wpr_vpl(D);
  if (vpl && aligned16(state) && aligned16(grad)) {
    switch (vpl) {
      case 1: launch_adam_d64_quad<Idx>(state, C, slots, grad, n, s, st, e0, e1); break;
      case 2: launch_adam_wpr<2, Idx>(state, C, slots, grad, n, s, st, e0, e1); break;     // wave per row
      case 4: launch_adam_wpr<4, Idx>(state, C, slots, grad, n, s, st, e0, e1); break;
      default: launch_adam_wpr<8, Idx>(state, C, slots, grad, n, s, st, e0, e1); break;
    }
    return launch_status();
  }
  if (D % 4 == 0 && D / 4 <= INT32_MAX && aligned16(state) && aligned16(grad)) {
    const int64_t nchunk = D / 4;
    const int lg = lanes_per_row_log2(nchunk);
    const int64_t rpw = 64 >> lg;
    const int64_t waves = (n + rpw - 1) / rpw;
    launch_timed(k_adam_rows_v4<Idx>, grid_for(waves, 4), st, e0, e1, state, C, slots, grad, n, (int)nchunk, lg, s);
  } else {
    launch_timed(k_adam_rows_scalar<Idx>, grid_for(n, 4), st, e0, e1, state, C, slots, grad, n, D, s);
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

extern "C" int elr_scalar_recip(const float* table_host, int64_t table_rows, double* recip_host) {
  if (table_rows < 0 || (table_rows && (!table_host || !recip_host))) return ELR_EINVAL;
  for (int64_t t = 0; t < table_rows; ++t) {
    recip_host[2 * t] = 1.0 / (double)table_host[8 * t + 5];
    recip_host[2 * t + 1] = 1.0 / (double)table_host[8 * t + 6];
  }
  return ELR_OK;
}

extern "C" int elr_adam_rows(float* state, int64_t C, const void* slots, int idx64, const float* grad, int64_t n,
                             int64_t D, const float sc[8], void* stream) {
  return elr_adam_rows_timed(state, C, slots, idx64, grad, n, D, sc, nullptr, nullptr, stream);
}

extern "C" int elr_adam_rows_timed(float* state, int64_t C, const void* slots, int idx64, const float* grad, int64_t n,
                                   int64_t D, const float sc[8], void* start_event, void* stop_event, void* stream) {
  if (n < 0 || D <= 0 || C < 0 || !sc) return ELR_EINVAL;
  if (n == 0) return ELR_OK;
  if (!state || !grad) return ELR_EINVAL;   // slots == NULL: row i of grad updates state row i
  const elr::AdamScalars s = elr::make_scalars(sc);
  hipStream_t st = (hipStream_t)stream;
  hipEvent_t e0 = (hipEvent_t)start_event, e1 = (hipEvent_t)stop_event;
  if (idx64) return elr::launch_adam(state, C, (const int64_t*)slots, grad, n, D, s, st, e0, e1);
  return elr::launch_adam(state, C, (const int32_t*)slots, grad, n, D, s, st, e0, e1);
}
