// Counter-hash row initialisation and exact replay of short gradient logs (HBM-bound, no MFMA).
//
// init   replaces srm2/gpu_ops.py:26-48:  out[i] = (w0(rows[i]), 0, 0)
// replay replaces srm2/gpu_ops.py:51-99:  out[i] = init(rows[i]); then for k < cnt[i], one Adam step with the
//        scalars of logical step steps[i,k] and the gradient logs[offs[i]+k].  The Adam arithmetic is
//        elr::adam_elem, so replay(init, log) is bitwise equal to eager Adam applied at those steps.
//
// D in {64, 128, 256, 512}: wave-per-row kernels (elr_rowio.h).  A wave owns U rows; their ids, counts, log offsets
// and steps are scalar loads, all their log-entry loads are issued before the first update, the Adam scalars of each
// step come through the scalar cache, the initial weights are computed in registers while the loads are in
// flight, and each record is written once.  The kernels have no loop: a loop back-edge makes the compiler guard the
// next iteration's loads with vmcnt(0) waits that also drain this iteration's stores, so very large calls are split
// into several launches on the host instead.
// Other D, or no reciprocal table: the generic kernels below (2^lg lanes per row with 16-byte chunks, or one float
// per lane).
#include "elr_rowio.h"

namespace elr {

// ---- generic kernels (any D) --------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_init_rows_v4(float* __restrict__ out, const int64_t* __restrict__ rows,
                                                      int64_t n, int nchunk, int lg, uint32_t seed, float bound) {
  const int lane = threadIdx.x & 63;
  const int l = lane & ((1 << lg) - 1);
  const int64_t rpw = 64 >> lg;
  const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int64_t nwave = ((int64_t)gridDim.x * blockDim.x) >> 6;
  const int64_t D = 4 * (int64_t)nchunk;
  const float4 zero = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int64_t i = wave * rpw + (lane >> lg); i < n; i += nwave * rpw) {
    const int64_t r = rows[i];
    const uint32_t rk = init_row_key(r, seed);
    float4* dst = reinterpret_cast<float4*>(out) + i * 3 * (int64_t)nchunk;
    for (int c = l; c < nchunk; c += (1 << lg)) {
      dst[c] = init_vec4(r, D, 4 * (int64_t)c, rk, seed, bound);
      dst[nchunk + c] = zero;
      dst[2 * nchunk + c] = zero;
    }
  }
}

__global__ __launch_bounds__(256) void k_init_rows_scalar(float* __restrict__ out, const int64_t* __restrict__ rows,
                                                          int64_t n, int64_t D, uint32_t seed, float bound) {
  const int lane = threadIdx.x & 63;
  const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int64_t nwave = ((int64_t)gridDim.x * blockDim.x) >> 6;
  for (int64_t i = wave; i < n; i += nwave) {
    const int64_t r = rows[i];
    const uint32_t rk = init_row_key(r, seed);
    float* dst = out + i * 3 * D;
    for (int64_t j = lane; j < D; j += 64) {
      dst[j] = init_elem((uint32_t)((uint64_t)r * (uint64_t)D + (uint64_t)j), rk, seed, bound);
      dst[D + j] = 0.f;
      dst[2 * D + j] = 0.f;
    }
  }
}

__device__ __forceinline__ AdamScalars load_scalars(const float* __restrict__ table, const double* __restrict__ recip,
                                                    int64_t step) {
  const float4* t = reinterpret_cast<const float4*>(table + step * 8);
  const float4 a = t[0], b = t[1];
  const double r1 = recip ? recip[2 * step] : 1.0 / (double)b.y;
  const double r2 = recip ? recip[2 * step + 1] : 1.0 / (double)b.z;
  return AdamScalars{a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w, r1, r2};
}

// Row i is valid when every used step indexes the table and every used log entry exists.
template <int K>
__device__ __forceinline__ bool replay_row_inputs(const int32_t* __restrict__ steps, int64_t i, int c, int64_t o,
                                                  int64_t nlogs, int64_t table_rows, int32_t (&st)[K]) {
  bool ok = true;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    st[k] = 0;
    if (k < c) {
      st[k] = steps[i * K + k];
      ok = ok && st[k] >= 0 && st[k] < table_rows && o + k >= 0 && o + k < nlogs;
    }
  }
  return ok;
}

template <int K>
__global__ __launch_bounds__(256) void k_replay_v4(float* __restrict__ out, const int64_t* __restrict__ rows,
                                                   const float* __restrict__ logs, int64_t nlogs,
                                                   const int64_t* __restrict__ offs,
                                                   const int32_t* __restrict__ steps, const int32_t* __restrict__ cnt,
                                                   int64_t n, int nchunk, int lg, uint32_t seed, float bound,
                                                   const float* __restrict__ table, const double* __restrict__ recip,
                                                   int64_t table_rows) {
  const int lane = threadIdx.x & 63;
  const int l = lane & ((1 << lg) - 1);
  const int64_t rpw = 64 >> lg;
  const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int64_t nwave = ((int64_t)gridDim.x * blockDim.x) >> 6;
  const int64_t D = 4 * (int64_t)nchunk;
  const float4* lg4 = reinterpret_cast<const float4*>(logs);
  const float4 zero = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int64_t i = wave * rpw + (lane >> lg); i < n; i += nwave * rpw) {
    const int64_t r = rows[i];
    const int c = cnt[i];
    const int64_t o = offs[i];
    int32_t st[K];
    if (!replay_row_inputs<K>(steps, i, c, o, nlogs, table_rows, st)) continue;
    const uint32_t rk = init_row_key(r, seed);
    float4* dst = reinterpret_cast<float4*>(out) + i * 3 * (int64_t)nchunk;
    for (int ch = l; ch < nchunk; ch += (1 << lg)) {
      float4 g[K];
#pragma unroll
      for (int k = 0; k < K; ++k)
        if (k < c) g[k] = ldg_stream(lg4 + (o + k) * (int64_t)nchunk + ch);
      float4 w = init_vec4(r, D, 4 * (int64_t)ch, rk, seed, bound);
      float4 m = zero, v = zero;
#pragma unroll
      for (int k = 0; k < K; ++k)
        if (k < c) adam_vec4(w, m, v, g[k], load_scalars(table, recip, st[k]));
      dst[ch] = w;
      dst[nchunk + ch] = m;
      dst[2 * nchunk + ch] = v;
    }
  }
}

template <int K>
__global__ __launch_bounds__(256) void k_replay_scalar(float* __restrict__ out, const int64_t* __restrict__ rows,
                                                       const float* __restrict__ logs, int64_t nlogs,
                                                       const int64_t* __restrict__ offs,
                                                       const int32_t* __restrict__ steps,
                                                       const int32_t* __restrict__ cnt, int64_t n, int64_t D,
                                                       uint32_t seed, float bound, const float* __restrict__ table,
                                                       const double* __restrict__ recip, int64_t table_rows) {
  const int lane = threadIdx.x & 63;
  const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int64_t nwave = ((int64_t)gridDim.x * blockDim.x) >> 6;
  for (int64_t i = wave; i < n; i += nwave) {
    const int64_t r = rows[i];
    const int c = cnt[i];
    const int64_t o = offs[i];
    int32_t st[K];
    if (!replay_row_inputs<K>(steps, i, c, o, nlogs, table_rows, st)) continue;
    const uint32_t rk = init_row_key(r, seed);
    float* dst = out + i * 3 * D;
    for (int64_t j = lane; j < D; j += 64) {
      float w = init_elem((uint32_t)((uint64_t)r * (uint64_t)D + (uint64_t)j), rk, seed, bound), m = 0.f, v = 0.f;
      for (int k = 0; k < K; ++k) {
        if (k >= c) break;
        adam_elem(w, m, v, logs[(o + k) * D + j], table_scalars_any(table, recip, st[k]));
      }
      dst[j] = w;
      dst[D + j] = m;
      dst[2 * D + j] = v;
    }
  }
}

// ---- wave-per-row kernels (D = 64*VPL) ------------------------------------------------------------------------------
// Rows per wave of the replay: one (at C2, 262,144 x 128: 0.3-1% faster per launch than two, same box and run;
// four is 4-5% slower).  Its loads are issued before its arithmetic either way.
constexpr int kReplayRowsPerWave = 1;
constexpr int kInitRowsPerWave = 2;

template <int VPL, int U>
__global__ __launch_bounds__(256) void k_init_rows_wpr(float* __restrict__ out, const int64_t* __restrict__ rows,
                                                       int64_t n, uint32_t seed, float bound) {
  constexpr int64_t D = 64 * VPL;
  const int lane = threadIdx.x & 63;
  const RowFrag<VPL> z = frag_zero<VPL>();
  const int64_t i0 = wave_id() * U;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t i = i0 + u;
    if (i < n) {
      float* dst = out + i * 3 * D + lane * VPL;
      frag_store<VPL>(dst, frag_init<VPL>(rows[i], lane, seed, bound));
      frag_store<VPL>(dst + D, z);
      frag_store<VPL>(dst + 2 * D, z);
    }
  }
}

template <int VPL, int K, int U>
__global__ __launch_bounds__(256) void k_replay_wpr(float* __restrict__ out, const int64_t* __restrict__ rows,
                                                    const float* __restrict__ logs, int64_t nlogs,
                                                    const int64_t* __restrict__ offs,
                                                    const int32_t* __restrict__ steps,
                                                    const int32_t* __restrict__ cnt, int64_t n, uint32_t seed,
                                                    float bound, const float* __restrict__ table,
                                                    const double* __restrict__ recip, int64_t table_rows) {
  constexpr int64_t D = 64 * VPL;
  const int lane = threadIdx.x & 63;
  const int64_t i0 = wave_id() * U;
  int64_t r[U], o[U];
  int c[U];
  int32_t st[U][K];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t i = i0 + u;
    c[u] = -1;  // -1: past the end, or invalid inputs (the row is skipped)
    r[u] = 0;
    o[u] = 0;
    if (i < n) {
      r[u] = rows[i];
      o[u] = offs[i];
      const int ci = cnt[i];
      const int cc = ci < 0 ? 0 : (ci > K ? K : ci);
      // every used step indexes the table and every used log entry exists (branch-free)
      int bad = (o[u] < 0) | (o[u] + cc > nlogs);
#pragma unroll
      for (int k = 0; k < K; ++k) {
        st[u][k] = steps[i * K + k];
        bad |= (k < cc) & ((st[u][k] < 0) | (st[u][k] >= table_rows));
      }
      c[u] = bad ? -1 : cc;
    }
  }
  RowFrag<VPL> g[U][K];
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int k = 0; k < K; ++k)
      if (k < c[u]) g[u][k] = frag_load<VPL, true>(logs + (o[u] + k) * D + lane * VPL);
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (c[u] < 0) continue;
    RowFrag<VPL> w = frag_init<VPL>(r[u], lane, seed, bound), m = frag_zero<VPL>(), v = frag_zero<VPL>();
    // the cores for every step, their operand ranges checked once per row (deferred: a min / max per lane, one
    // vote per row); a row that fails the check is recomputed on the general path, which gives the same bits
    RangeAcc acc = range_acc_init();
    bool eps_all = true;
#pragma unroll
    for (int k = 0; k < K; ++k)
      if (k < c[u]) {
        const AdamScalars sc = table_scalars(table, recip, st[u][k]);
        eps_all = eps_all && eps_ok(sc.eps);
        frag_adam_fast<VPL>(w, m, v, g[u][k], sc, acc);
      }
    if (!(eps_all && wave_all(range_acc_ok(acc)))) {
      w = frag_init<VPL>(r[u], lane, seed, bound);
      m = frag_zero<VPL>();
      v = frag_zero<VPL>();
#pragma unroll
      for (int k = 0; k < K; ++k)
        if (k < c[u]) frag_adam<VPL>(w, m, v, g[u][k], table_scalars(table, recip, st[u][k]));
    }
    float* dst = out + (i0 + u) * 3 * D + lane * VPL;
    frag_store<VPL>(dst, w);
    frag_store<VPL>(dst + D, m);
    frag_store<VPL>(dst + 2 * D, v);
  }
}

template <int VPL, int K>
static void launch_replay_wpr(float* out, const int64_t* rows, const float* logs, int64_t nlogs, const int64_t* offs,
                              const int32_t* steps, const int32_t* cnt, int64_t n, uint32_t seed, float bound,
                              const float* table, const double* recip, int64_t table_rows, hipStream_t st,
                              hipEvent_t e0, hipEvent_t e1) {
  constexpr int U = kReplayRowsPerWave;
  constexpr int64_t D = 64 * VPL;
  constexpr int64_t per = wpr_rows_per_launch(U);
  for (int64_t a = 0; a < n; a += per) {
    const int64_t m = n - a < per ? n - a : per;
    launch_timed(k_replay_wpr<VPL, K, U>, grid_for((m + U - 1) / U, 4, kOneShotBlocks), st, a == 0 ? e0 : nullptr,
                 a + m >= n ? e1 : nullptr, out + a * 3 * D, rows + a, logs, nlogs, offs + a, steps + a * K, cnt + a,
                 m, seed, bound, table, recip, table_rows);
  }
}

template <int VPL>
static void launch_init_wpr(float* out, const int64_t* rows, int64_t n, uint32_t seed, float bound, hipStream_t st) {
  constexpr int U = kInitRowsPerWave;
  constexpr int64_t D = 64 * VPL;
  constexpr int64_t per = wpr_rows_per_launch(U);
  for (int64_t a = 0; a < n; a += per) {
    const int64_t m = n - a < per ? n - a : per;
    k_init_rows_wpr<VPL, U><<<grid_for((m + U - 1) / U, 4, kOneShotBlocks), 256, 0, st>>>(out + a * 3 * D, rows + a,
                                                                                          m, seed, bound);
  }
}

template <int K>
static int launch_replay(float* out, const int64_t* rows, const float* logs, int64_t nlogs, const int64_t* offs,
                         const int32_t* steps, const int32_t* cnt, int64_t n, int64_t D, uint32_t seed, float bound,
                         const float* table, const double* recip, int64_t table_rows, hipStream_t st, hipEvent_t e0,
                         hipEvent_t e1) {
  const int vpl = wpr_vpl(D);
  if (K <= 4 && vpl && recip && aligned16(out) && aligned16(logs)) {
#define ELR_WPR_REPLAY(V) \
  launch_replay_wpr<V, K>(out, rows, logs, nlogs, offs, steps, cnt, n, seed, bound, table, recip, table_rows, st, \
                          e0, e1)
    switch (vpl) {
      case 1: ELR_WPR_REPLAY(1); break;
      case 2: ELR_WPR_REPLAY(2); break;
      case 4: ELR_WPR_REPLAY(4); break;
      default: ELR_WPR_REPLAY(8); break;
    }
#undef ELR_WPR_REPLAY
    return launch_status();
  }
  if (D % 4 == 0 && D / 4 <= INT32_MAX && aligned16(out) && aligned16(logs) && aligned16(table)) {
    const int64_t nchunk = D / 4;
    const int lg = lanes_per_row_log2(nchunk);
    const int64_t rpw = 64 >> lg;
    launch_timed(k_replay_v4<K>, grid_for((n + rpw - 1) / rpw, 4), st, e0, e1, out, rows, logs, nlogs, offs, steps,
                 cnt, n, (int)nchunk, lg, seed, bound, table, recip, table_rows);
  } else {
    launch_timed(k_replay_scalar<K>, grid_for(n, 4), st, e0, e1, out, rows, logs, nlogs, offs, steps, cnt, n, D, seed,
                 bound, table, recip, table_rows);
  }
  return launch_status();
}

}  // namespace elr

extern "C" int elr_init_rows(float* out, const int64_t* rows, int64_t n, int64_t D, uint32_t seed, float bound,
                             void* stream) {
  if (n < 0 || D <= 0) return ELR_EINVAL;
  if (n == 0) return ELR_OK;
  if (!out || !rows) return ELR_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  const int vpl = elr::wpr_vpl(D);
  if (vpl && elr::aligned16(out)) {
    switch (vpl) {
      case 1: elr::launch_init_wpr<1>(out, rows, n, seed, bound, st); break;
      case 2: elr::launch_init_wpr<2>(out, rows, n, seed, bound, st); break;
      case 4: elr::launch_init_wpr<4>(out, rows, n, seed, bound, st); break;
      default: elr::launch_init_wpr<8>(out, rows, n, seed, bound, st); break;
    }
  } else if (D % 4 == 0 && D / 4 <= INT32_MAX && elr::aligned16(out)) {
    const int64_t nchunk = D / 4;
    const int lg = elr::lanes_per_row_log2(nchunk);
    const int64_t rpw = 64 >> lg;
    elr::k_init_rows_v4<<<elr::grid_for((n + rpw - 1) / rpw, 4), 256, 0, st>>>(out, rows, n, (int)nchunk, lg, seed,
                                                                                bound);
  } else {
    elr::k_init_rows_scalar<<<elr::grid_for(n, 4), 256, 0, st>>>(out, rows, n, D, seed, bound);
  }
  return elr::launch_status();
}

extern "C" int elr_replay_rows(float* out, const int64_t* rows, const float* logs, int64_t nlogs, const int64_t* offs,
                               const int32_t* steps, const int32_t* cnt, int64_t n, int64_t D, int K, uint32_t seed,
                               float bound, const float* table, const double* recip, int64_t table_rows,
                               void* stream) {
  return elr_replay_rows_timed(out, rows, logs, nlogs, offs, steps, cnt, n, D, K, seed, bound, table, recip,
                               table_rows, nullptr, nullptr, stream);
}

extern "C" int elr_replay_rows_timed(float* out, const int64_t* rows, const float* logs, int64_t nlogs,
                                     const int64_t* offs, const int32_t* steps, const int32_t* cnt, int64_t n,
                                     int64_t D, int K, uint32_t seed, float bound, const float* table,
                                     const double* recip, int64_t table_rows, void* start_event, void* stop_event,
                                     void* stream) {
  if (n < 0 || D <= 0 || nlogs < 0 || table_rows < 0) return ELR_EINVAL;
  if (K < 1 || K > 8) return ELR_EUNSUPPORTED;
  if (n == 0) return ELR_OK;
  if (!out || !rows || !offs || !steps || !cnt || !table || (nlogs > 0 && !logs)) return ELR_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  switch (K) {
#define ELR_REPLAY_CASE(KK) \
  case KK:                  \
    return elr::launch_replay<KK>(out, rows, logs, nlogs, offs, steps, cnt, n, D, seed, bound, table, recip, \
                                  table_rows, st, (hipEvent_t)start_event, (hipEvent_t)stop_event);
    ELR_REPLAY_CASE(1)
    ELR_REPLAY_CASE(2)
    ELR_REPLAY_CASE(3)
    ELR_REPLAY_CASE(4)
    ELR_REPLAY_CASE(5)
    ELR_REPLAY_CASE(6)
    ELR_REPLAY_CASE(7)
    ELR_REPLAY_CASE(8)
#undef ELR_REPLAY_CASE
  }
  return ELR_EUNSUPPORTED;
}
