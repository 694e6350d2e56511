// wt_kernels.hip — MI355X (gfx950) kernels of the conductance-LIF hot path and their
// C-ABI (include/wiretorch_amd.h).
//
// Forward (wt_cond_run): one persistent launch runs all T steps.
//   * Workgroups form `groups` groups of R (workgroup i is in group i % groups, slot
//     i / groups; with a multiple of 8 groups each group lies on one XCD, since the
//     dispatcher places workgroup i on XCD i % 8). Group g owns trials g, g + groups, ...; slot r owns the
//     targets [r * range_n, (r + 1) * range_n) of those trials, for the whole run.
//   * Step t, per workgroup: (A) update the owned neurons — inject step t-1's
//     activations, spike, membrane, refractory — and decide their spikes of step t+1,
//     set in an LDS bitmap published to the group (agent-scope stores); (P) walk the
//     nonzero inputs of step t and the group's fired bitmap of step t (published one
//     step earlier), list each event's edges onto the workgroup's own targets, and add
//     their weights into an LDS accumulator; then the group barrier.
//   * Accumulation is exact: int64 multiples of 2^-frac_bits (LDS 64-bit atomic adds),
//     converted to float32 once, so the sum is the exactly rounded one whatever order
//     the events arrive in — deterministic without float atomics, and only active
//     synapses are touched.
//   * Cross-workgroup data (fired bitmaps, the barrier counter) is moved with agent-scope
//     atomic loads/stores (coherent at device scope); each thread waits for its stores
//     to complete before its workgroup arrives at the barrier.
//     Per-XCD groups keep the barrier to R arrivals per counter (≈0.8 µs measured for 32
//     workgroups, against ≈3.7 µs for one device-wide counter of 256).
// Backward (wt_cond_scan_backward): one thread per (trial, neuron), reverse time loop,
// the adjoint state in registers.
// Weight gradient (wt_weight_gradient): one thread per synapse, summing over the
// (trial, step) events of its source.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include "../../include/wiretorch_amd.h"
#include "wt_math.h"

#include "wt_back.h"
#include "wt_philox.h"
#include "wt_run.h"

namespace wt {

// The nonzero inputs of each (trial, step) row of x: one workgroup per row; at most
// kInCap listed (count above kInCap: the row is scanned in place by the run kernel).
__global__ __launch_bounds__(256) void compact_input_kernel(const float* x, int64_t rows,
                                                            int64_t n_in, int32_t* count,
                                                            int32_t* idx, float* val) {
  __shared__ int32_t s_n;
  const int64_t row = blockIdx.x;
  if (row >= rows) return;
  if (threadIdx.x == 0) s_n = 0;
  __syncthreads();
  const float* xr = x + row * n_in;
  for (int64_t j = threadIdx.x; j < n_in; j += blockDim.x) {
    const float xv = xr[j];
    if (xv != 0.0f) {
      const int32_t pos = atomicAdd(&s_n, 1);
      if (pos < kInCap) {
        idx[row * kInCap + pos] = (int32_t)j;
        val[row * kInCap + pos] = xv;
      }
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) count[row] = s_n;
}

// The same lists for on-device Poisson input: row (b, t) draws channel j's spike from
// the counter-based stream (wt_philox.h) instead of reading x.
__global__ __launch_bounds__(256) void poisson_lists_kernel(const float* prob, int64_t n_in,
                                                            uint64_t seed, int64_t t0,
                                                            int64_t T, int64_t rows,
                                                            int32_t* count, int32_t* idx,
                                                            float* val) {
  __shared__ int32_t s_n;
  const int64_t row = blockIdx.x;
  if (row >= rows) return;
  if (threadIdx.x == 0) s_n = 0;
  __syncthreads();
  const uint32_t b = (uint32_t)(row / T), t = (uint32_t)(t0 + row % T);
  for (int64_t j = threadIdx.x; j < n_in; j += blockDim.x) {
    if (poisson_fires(seed, b, t, (uint32_t)j, prob[j])) {
      const int32_t pos = atomicAdd(&s_n, 1);
      if (pos < kInCap) {
        idx[row * kInCap + pos] = (int32_t)j;
        val[row * kInCap + pos] = 1.0f;
      }
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) count[row] = s_n;
}

__global__ void poisson_fill_kernel(const float* prob, int64_t n_in, uint64_t seed, int64_t t0,
                                    int64_t B, int64_t T, float* x) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= B * T * n_in) return;
  const int64_t j = i % n_in, bt = i / n_in, b = bt / T, t = bt - b * T;
  x[i] = poisson_fires(seed, (uint32_t)b, (uint32_t)(t0 + t), (uint32_t)j, prob[j]) ? 1.0f : 0.0f;
}

// ---------------------------------------------------------------------------------
// Ranges of each source's ascending targets: split[j][r] = first edge with target >=
// r * range_n (r = 0..R), by binary search.
__global__ void split_ranges_kernel(const int64_t* indptr, const int32_t* targets,
                                    int64_t n_src, int64_t R, int64_t range_n,
                                    int64_t* split) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n_src * (R + 1)) return;
  const int64_t j = i / (R + 1), rr = i - j * (R + 1);
  const int64_t bound = rr * range_n;
  int64_t a = indptr[j], z = indptr[j + 1];
  while (a < z) {
    int64_t m = (a + z) >> 1;
    if ((int64_t)targets[m] < bound) a = m + 1; else z = m;
  }
  split[i] = a;
}

// ---------------------------------------------------------------------------------
// Weight gradient on the support: one thread per synapse; it walks its source's
// events (the (trial, step) where the source was active, ascending) and sums the
// target's dL/da of that step, times the event's value (1 for every event without
// ev_val: spikes).
__global__ void weight_gradient_kernel(wt_side side, const int64_t* edge_src, int64_t E,
                                       const int64_t* ev_indptr, const int32_t* ev_bt,
                                       const float* ev_val, const float* grad_A, int64_t BT,
                                       int64_t N, int64_t k0, float* grad_w) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= E) return;
  const int64_t j = edge_src[e];
  const int32_t k = side.pathway[j];
  float sum = 0.0f;
  if (k >= 0) {
    const int64_t n = side.targets[e];
    const float* gA = grad_A + (k0 + k) * BT * N + n;
    for (int64_t i = ev_indptr[j]; i < ev_indptr[j + 1]; ++i)
      sum += (ev_val ? ev_val[i] : 1.0f) * gA[(int64_t)ev_bt[i] * N];
  }
  grad_w[e] = sum;
}

// The same sums, grouped by (pathway, target): workgroup kn = k * N + n holds the
// target's dL/da_k over every (trial, step), row kn of grad_A_T (k, n, b*T+t), in LDS —
// read once, contiguously — and each wave takes its incoming synapses one at a time: its
// 64 lanes read 64 consecutive events of the synapse's source (one coalesced load) and
// add the row's entries; the lanes' partial sums are then added in a fixed tree (the sum
// is deterministic). The synapses' lookups are made 64 at a time, one per lane. Rows longer than the LDS chunk are taken a chunk at a time, each
// synapse's running sum kept in grad_w.
constexpr int kWgBlock = 1024;
constexpr int64_t kWgChunk = 32768;  // floats of a row in LDS (128 KB)

// dL/da (K, BT, N) -> rows (K * N, BT), through 64 x 64 LDS tiles (coalesced both ways).
__global__ __launch_bounds__(256) void transpose_rows_kernel(const float* src, float* dst,
                                                             int64_t BT, int64_t N) {
  __shared__ float tile[64][65];
  const int64_t k = blockIdx.z, n0 = (int64_t)blockIdx.x * 64, bt0 = (int64_t)blockIdx.y * 64;
  const float* s = src + k * BT * N;
  float* d = dst + k * N * BT;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;  // 64 x 4
  for (int r = ty; r < 64; r += 4) {
    const int64_t bt = bt0 + r, n = n0 + tx;
    if (bt < BT && n < N) tile[r][tx] = s[bt * N + n];
  }
  __syncthreads();
  for (int r = ty; r < 64; r += 4) {
    const int64_t n = n0 + r, bt = bt0 + tx;
    if (bt < BT && n < N) d[n * BT + bt] = tile[tx][r];
  }
}

// Lane k's 64-bit value, in every lane (k wave-uniform).
__device__ inline int64_t readlane64(int64_t v, int k) {
  const uint64_t u = (uint64_t)v;
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, k);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), k);
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

// VALUES: each event's value multiplies its term (otherwise every value is 1: spikes,
// and the value list is not read).
template <bool VALUES>
__global__ __launch_bounds__(kWgBlock) void weight_gradient_target_kernel(
    const int64_t* in_indptr, const int64_t* in_edge, const int64_t* edge_src,
    const int64_t* ev_indptr, const int32_t* ev_bt, const float* ev_val,
    const float* grad_A_T, int64_t BT, float* grad_w) {
  extern __shared__ float row[];
  const int64_t kn = blockIdx.x;
  const int64_t e0 = in_indptr[kn], e1 = in_indptr[kn + 1];
  if (e0 == e1) return;  // uniform
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, n_waves = blockDim.x >> 6;
  const float* src = grad_A_T + kn * BT;
  const bool vec = (BT & 3) == 0 && ((uintptr_t)grad_A_T & 15) == 0;
  for (int64_t c0 = 0; c0 < BT; c0 += kWgChunk) {
    const int64_t len = BT - c0 < kWgChunk ? BT - c0 : kWgChunk;
    __syncthreads();  // the previous chunk is no longer read
    if (vec) {
      const float4* s4 = reinterpret_cast<const float4*>(src + c0);
      float4* r4 = reinterpret_cast<float4*>(row);
      const int64_t n4 = len >> 2;
      int64_t i = threadIdx.x;
      for (; i + 3 * kWgBlock < n4; i += 4 * kWgBlock) {  // four loads in flight
        const float4 a = s4[i], b = s4[i + kWgBlock], c = s4[i + 2 * kWgBlock],
                     d = s4[i + 3 * kWgBlock];
        r4[i] = a;
        r4[i + kWgBlock] = b;
        r4[i + 2 * kWgBlock] = c;
        r4[i + 3 * kWgBlock] = d;
      }
      for (; i < n4; i += kWgBlock) r4[i] = s4[i];
    } else {
      for (int64_t i = threadIdx.x; i < len; i += blockDim.x) row[i] = src[c0 + i];
    }
    __syncthreads();
    // Wave w takes in-edges e0 + w, e0 + w + n_waves, ... (as one at a time would), 64 at
    // a time: lane l looks up edge l's synapse, source and event range (and, past the
    // first chunk, its first event in the chunk) for all 64 together, and keeps edge l's
    // sum; the sums are stored after the 64. Done one edge after another, each edge's
    // dependent lookups cost four round trips to memory, and its store made the next
    // edge's loads wait (one counter covers a wave's loads and stores).
    for (int64_t base = e0 + wave; base < e1; base += 64 * (int64_t)n_waves) {
      const int64_t my_ei = base + (int64_t)lane * n_waves;
      int64_t my_e = 0, my_i0 = 0, my_i1 = 0;
      if (my_ei < e1) {
        my_e = in_edge[my_ei];
        const int64_t j = edge_src[my_e];
        my_i0 = ev_indptr[j];
        my_i1 = ev_indptr[j + 1];
        if (c0 > 0) {  // the first event at or past the chunk (events ascend in b*T+t)
          int64_t lo = my_i0, hi = my_i1;
          while (lo < hi) {
            const int64_t mid = (lo + hi) >> 1;
            if (ev_bt[mid] < c0) lo = mid + 1; else hi = mid;
          }
          my_i0 = lo;
        }
      }
      const int64_t left = (e1 - base + n_waves - 1) / n_waves;
      const int cnt = left < 64 ? (int)left : 64;
      float mine = 0.0f;
      for (int k = 0; k < cnt; ++k) {
        const int64_t i0 = readlane64(my_i0, k), i1 = readlane64(my_i1, k);
        float part = 0.0f;
        int64_t i = i0 + lane;
        for (; i + 192 < i1; i += 256) {  // four events per lane in flight
          int64_t bt[4];
          float val[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            bt[u] = (int64_t)ev_bt[i + 64 * u] - c0;
            val[u] = VALUES ? ev_val[i + 64 * u] : 1.0f;
          }
          bool past = false;
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            if (bt[u] >= len) past = true;
            if (!past) part += VALUES ? val[u] * row[bt[u]] : row[bt[u]];
          }
          if (past) {  // this lane's later events are past the chunk too
            i = i1;
            break;
          }
        }
        for (; i < i1; i += 64) {
          const int64_t bt = (int64_t)ev_bt[i] - c0;
          if (bt >= len) break;
          part += VALUES ? ev_val[i] * row[bt] : row[bt];
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) part += __shfl_xor(part, off);
        if (lane == k) mine = part;
      }
      if (my_ei < e1) grad_w[my_e] = (c0 > 0 ? grad_w[my_e] : 0.0f) + mine;
    }
  }
}

__global__ void edge_source_kernel(const int64_t* indptr, int64_t n_src, int64_t* edge_src) {
  const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= n_src) return;
  for (int64_t e = indptr[j]; e < indptr[j + 1]; ++e) edge_src[e] = j;
}

// ---- Events by source: the nonzero entries of a (BT, n) activity, per column j in
// ascending row order. Rows are taken in chunks of kEvChunk; thread (chunk c, column j)
// counts, then writes, its chunk's entries of column j (a wave reads 64 consecutive
// columns of one row at a time). The count also records which rows of the chunk are
// nonzero, as 8 words of bits (word w of chunk c, column j at bits[(c * 8 + w) * n + j]):
// a fill that wants no values (spikes) reads those instead of the activity again.
constexpr int64_t kEvChunk = 256;
constexpr int kEvBlock = 256;
constexpr int kEvWords = (int)kEvChunk / 32;

__global__ void events_count_kernel(const float* __restrict__ act, int64_t BT, int64_t n,
                                    int32_t* __restrict__ chunk, uint32_t* __restrict__ bits) {
  const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= n) return;
  const int64_t r0 = (int64_t)blockIdx.y * kEvChunk;
  const int64_t r1 = r0 + kEvChunk < BT ? r0 + kEvChunk : BT;
  // Every load before the first store (one counter covers a wave's loads and stores: a
  // store between them would make the later loads' use wait for it).
  const float* p = act + r0 * n + j;  // row r0 of column j; rows n floats apart
  const int rows = (int)(r1 - r0);
  uint32_t words[kEvWords];
  if (rows == (int)kEvChunk) {  // a whole chunk: no branch around the loads
#pragma unroll
    for (int w = 0; w < kEvWords; ++w) {
      uint32_t word = 0u;
#pragma unroll 8
      for (int u = 0; u < 32; ++u)
        word |= (p[(int64_t)(32 * w + u) * n] != 0.0f ? 1u : 0u) << u;
      words[w] = word;
    }
  } else {
#pragma unroll
    for (int w = 0; w < kEvWords; ++w) {
      uint32_t word = 0u;
      for (int u = 0; u < 32; ++u) {
        const int r = 32 * w + u;
        if (r < rows && p[(int64_t)r * n] != 0.0f) word |= 1u << u;
      }
      words[w] = word;
    }
  }
  int32_t count = 0;
#pragma unroll
  for (int w = 0; w < kEvWords; ++w) {
    count += __builtin_popcount(words[w]);
    bits[((int64_t)blockIdx.y * kEvWords + w) * n + j] = words[w];
  }
  chunk[blockIdx.y * n + j] = count;
}

// The fill of a value-free list (every value 1) from the count's bits.
__global__ void events_fill_bits_kernel(const uint32_t* __restrict__ bits, int64_t n,
                                        const int32_t* __restrict__ chunk,
                                        const int64_t* __restrict__ indptr,
                                        int32_t* __restrict__ bt, int64_t T, int64_t T_pad) {
  const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= n) return;
  const int64_t r0 = (int64_t)blockIdx.y * kEvChunk;
  int64_t pos = indptr[j] + chunk[blockIdx.y * n + j];
  uint32_t words[kEvWords];
#pragma unroll
  for (int w = 0; w < kEvWords; ++w) words[w] = bits[((int64_t)blockIdx.y * kEvWords + w) * n + j];
#pragma unroll
  for (int w = 0; w < kEvWords; ++w) {
    uint32_t word = words[w];
    while (word) {
      const int64_t row = r0 + 32 * w + __builtin_ctz(word);  // b*T + t, as b*T_pad + t
      word &= word - 1u;
      bt[pos++] = (int32_t)(T_pad == T ? row : row + (row / T) * (T_pad - T));
    }
  }
}

// Per column: each chunk's count becomes its offset within the column; the column's
// total goes to totals[j].
__global__ void events_column_kernel(int32_t* __restrict__ chunk, int64_t n_chunks, int64_t n,
                                     int64_t* __restrict__ totals) {
  const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= n) return;
  int32_t sum = 0;
  for (int64_t c = 0; c < n_chunks; ++c) {
    const int32_t v = chunk[c * n + j];
    chunk[c * n + j] = sum;
    sum += v;
  }
  totals[j] = sum;
}

// indptr[0] = 0, indptr[j + 1] = totals[0] + ... + totals[j]; one workgroup, each thread
// a contiguous segment. totals may alias indptr + 1.
__global__ __launch_bounds__(kRunBlock) void events_indptr_kernel(const int64_t* totals,
                                                                 int64_t n, int64_t* indptr) {
  using Scan64 = rocprim::block_scan<int64_t, kRunBlock>;
  __shared__ typename Scan64::storage_type storage;
  const int64_t per = (n + kRunBlock - 1) / kRunBlock;
  const int64_t j0 = threadIdx.x * per, j1 = j0 + per < n ? j0 + per : n;
  int64_t local = 0;
  for (int64_t j = j0; j < j1; ++j) local += totals[j];
  int64_t before = 0, all = 0;
  Scan64().exclusive_scan(local, before, (int64_t)0, all, storage);
  __syncthreads();  // every total is read before any is overwritten (aliasing)
  int64_t run = before;
  for (int64_t j = j0; j < j1; ++j) {  // totals[j] is read before indptr[j + 1] (its
    const int64_t v = totals[j];         // alias) is written, by this thread alone
    indptr[j + 1] = run + v;
    run += v;
  }
  if (threadIdx.x == 0) indptr[0] = 0;
}

__global__ void events_fill_kernel(const float* __restrict__ act, int64_t BT, int64_t n,
                                   const int32_t* __restrict__ chunk,
                                   const int64_t* __restrict__ indptr, int32_t* __restrict__ bt,
                                   float* __restrict__ value, int64_t T, int64_t T_pad) {
  const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= n) return;
  const int64_t r0 = (int64_t)blockIdx.y * kEvChunk;
  const int64_t r1 = r0 + kEvChunk < BT ? r0 + kEvChunk : BT;
  int64_t pos = indptr[j] + chunk[blockIdx.y * n + j];
  for (int64_t rb = r0; rb < r1; rb += 16) {  // sixteen rows loaded at once, then written
    float a[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) a[u] = rb + u < r1 ? act[(rb + u) * n + j] : 0.0f;
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      if (a[u] != 0.0f) {
        const int64_t row = rb + u;  // b*T + t, written as b*T_pad + t
        bt[pos] = (int32_t)(T_pad == T ? row : row + (row / T) * (T_pad - T));
        if (value) value[pos] = a[u];
        ++pos;
      }
    }
  }
}

// ---- Presynaptic dynamics of a feedforward pathway (network_simulators/network.py:
// 186-250): one thread per (trial, source row), the chunk's steps in order. Each
// operation is rounded as torch rounds it on the CPU (-ffp-contract=off, left to right).
__global__ void gate_scan_kernel(const float* __restrict__ x, int64_t B, int64_t T,
                                 int64_t n_in, const int64_t* __restrict__ rows, int64_t n,
                                 const float* __restrict__ params, float* __restrict__ gating,
                                 int64_t R, int64_t stp_col, int64_t sat_col,
                                 float* __restrict__ factors) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= B * n) return;
  const int64_t b = idx / n, i = idx - b * n;
  const int64_t row = rows[i];
  float* base = gating + b * R;
  const float c = params[0], d = params[1], U = params[2], d_D = params[3], d_F = params[4];
  const bool stp = stp_col >= 0, sat = sat_col >= 0;
  float u = stp ? base[stp_col + i] : 0.0f, r = stp ? base[stp_col + n + i] : 0.0f;
  float g = sat ? base[sat_col + i] : 0.0f;
  for (int64_t t = 0; t < T; ++t) {
    const float s = x[(b * T + t) * n_in + row];
    float f = 1.0f;
    if (stp) {  // resources recover, facilitation relaxes; a spike releases u r
      r = 1.0f - (1.0f - r) * d_D;
      u = U + (u - U) * d_F;
      const float release = u * r;
      f = release / U;
      r = r - s * release;
      u = u + s * U * (1.0f - u);
    }
    if (sat) {  // the receptors' gating decays; a release opens c f of the closed
      g = g * d;
      const float closed = 1.0f - g;
      f = stp ? fminf(c * f * closed, closed) : c * closed;
      g = fminf(g + s * f, 1.0f);
    }
    factors[(b * T + t) * n + i] = f;
  }
  if (stp) {
    base[stp_col + i] = u;
    base[stp_col + n + i] = r;
  }
  if (sat) base[sat_col + i] = g;
}

}  // namespace wt

// ===================================================================================
// C-ABI
// ===================================================================================
using namespace wt;

// RunLaunch<S>::run is compiled in wt_run_s<S>.hip.
extern template struct wt::RunLaunch<1>;
extern template struct wt::RunLaunch<2>;
extern template struct wt::RunLaunch<3>;
extern template struct wt::RunLaunch<4>;
extern template struct wt::RunLaunch<5>;
extern template struct wt::RunLaunch<6>;
extern template struct wt::RunLaunch<7>;
extern template struct wt::RunLaunch<8>;
extern template struct wt::BackLaunch<1>;
extern template struct wt::BackLaunch<2>;
extern template struct wt::BackLaunch<3>;
extern template struct wt::BackLaunch<4>;
extern template struct wt::BackLaunch<5>;
extern template struct wt::BackLaunch<6>;
extern template struct wt::BackLaunch<7>;
extern template struct wt::BackLaunch<8>;

// The two backward drivers as dispatch targets.
template <int S>
struct BackRun {
  static hipError_t run(BackArgs& a, hipStream_t stream) { return BackLaunch<S>::run(a, stream); }
};
template <int S>
struct BackRecurrent {
  static hipError_t run(BackArgs& a, hipStream_t stream) {
    return BackLaunch<S>::recurrent(a, stream);
  }
};

template <template <int> class F, typename... Args>
static hipError_t dispatch_S(int64_t S, Args&&... args) {
  switch (S) {
    case 1: return F<1>::run(args...);
    case 2: return F<2>::run(args...);
    case 3: return F<3>::run(args...);
    case 4: return F<4>::run(args...);
    case 5: return F<5>::run(args...);
    case 6: return F<6>::run(args...);
    case 7: return F<7>::run(args...);
    case 8: return F<8>::run(args...);
    default: return hipErrorInvalidValue;
  }
}

static int64_t run_tpg_max(const wt_geometry* geo, int64_t B) {
  return (B + geo->groups - 1) / geo->groups;
}

// Scratch: [0, zeroed) must be zero at launch (error flags, barrier counters); the rest
// (fired bitmaps, the input lists) is written before it is read.
static int64_t scratch_zeroed(const wt_geometry* geo) { return 256 + geo->groups * 128; }

// Fired bitmaps: three buffers of [groups][tpg_max][R * words] words (step t in buffer
// t % 3: a workgroup still reads step t's bits after it has arrived at the barrier that
// lets the others publish step t+1's).
static int64_t bitmap_words(const wt_geometry* geo, int64_t B) {
  return geo->groups * run_tpg_max(geo, B) * geo->R * (geo->range_n / 32);
}

extern "C" int64_t wt_cond_run_scratch_bytes(const wt_geometry* geo, int64_t B, int64_t T) {
  int64_t bytes = scratch_zeroed(geo);
  bytes += 3 * bitmap_words(geo, B) * 4;                  // fired bitmaps
  bytes = (bytes + 255) / 256 * 256;
  bytes += B * T * 4;                                     // input counts
  bytes += B * T * kInCap * 8;                            // input indices and values
  return bytes;
}

extern "C" int64_t wt_cond_run_scratch_zeroed(const wt_geometry* geo) {
  return scratch_zeroed(geo);
}

static int run_impl(const wt_tables* tab, const wt_side* rec, const wt_side* ff,
                    const wt_geometry* geo, const wt_run_io* io, void* scratch,
                    uint64_t* timing, wt_stream_t stream) {
  if (!tab || !rec || !ff || !geo || !io || !scratch || !io->spikes || !io->v || !io->g)
    return hipErrorInvalidValue;
  if (tab->n_ref && !io->counter) return hipErrorInvalidValue;
  if (tab->adapt && (!tab->adapt_decay || !tab->E_adapt || !io->adaptation))
    return hipErrorInvalidValue;
  if (tab->S < 1 || tab->S > WT_MAX_S || tab->K < 0 || tab->K > WT_MAX_K || tab->K_rec > tab->K)
    return hipErrorInvalidValue;
  if (geo->groups < 1 || geo->groups > kMaxGroups || geo->R < 1 || geo->R > 256 ||
      geo->range_n < 32 || geo->range_n % 32 != 0 || geo->R * geo->range_n < tab->N ||
      (!geo->bound && (geo->frac_bits < 0 || geo->frac_bits > 60)) || geo->max_list < 0 ||
      geo->max_list > kMaxList || geo->max_list % kRunBlock != 0)
    return hipErrorInvalidValue;
  const int64_t tpg = run_tpg_max(geo, io->B);
  if (io->B < 1 || io->T < 0) return hipErrorInvalidValue;
  if ((io->v_saved != nullptr) != (io->G_saved != nullptr)) return hipErrorInvalidValue;
  if (io->track_v && (!io->track_I || !io->track_g)) return hipErrorInvalidValue;
  if (rec->n_src > 0 && rec->n_src != tab->N) return hipErrorInvalidValue;
  if (ff->n_src > 0 && ff->n_src != io->n_in) return hipErrorInvalidValue;
  if (io->T == 0) return hipSuccess;

  RunArgs a;
  a.tab = *tab;
  a.rec = *rec;
  a.ff = *ff;
  a.geo = *geo;
  a.io = *io;
  a.words = geo->range_n / 32;
  char* base = static_cast<char*>(scratch);
  a.err = reinterpret_cast<uint32_t*>(base);
  a.barrier = reinterpret_cast<uint32_t*>(base + 256);
  a.bitmap = reinterpret_cast<uint32_t*>(base + scratch_zeroed(geo));
  a.tpg_max = tpg;
  int64_t off = scratch_zeroed(geo) + 3 * bitmap_words(geo, io->B) * 4;
  off = (off + 255) / 256 * 256;
  int32_t* in_count = reinterpret_cast<int32_t*>(base + off);
  off += io->B * io->T * 4;
  int32_t* in_idx = reinterpret_cast<int32_t*>(base + off);
  float* in_val = reinterpret_cast<float*>(base + off + io->B * io->T * kInCap * 4);
  a.in_count = in_count;
  a.in_idx = in_idx;
  a.in_val = in_val;
  a.timing = timing;
  if (!tab->types || !tab->type_of || tab->n_types < 1) return hipErrorInvalidValue;
  if (tab->n_types > kMaxLdsTypes) return hipErrorInvalidValue;
  // descriptors pack the target within the range in 16 bits, the trial in 8
  if (geo->range_n > 65535 || tpg > 255) return hipErrorInvalidValue;
  // the fired list packs a source in 24 bits
  if (tab->N >= (1 << 24)) return hipErrorInvalidValue;

  if (tpg * geo->range_n > kMaxItemsPerWg) return hipErrorInvalidValue;
  const int64_t acc_len = (tab->K > 0 ? tab->K : 1) * tpg * geo->range_n;
  const size_t lds = (size_t)acc_len * sizeof(double);
  int dev = 0, max_lds = 0;
  hipError_t qe = hipGetDevice(&dev);
  if (qe == hipSuccess)
    qe = hipDeviceGetAttribute(&max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev);
  if (qe != hipSuccess) return qe;
  // static LDS besides the event list (+ 64 for alignment)
  const size_t static_lds = kRunBlock * 4 + sizeof(BlockScan::storage_type) +
                            (kPhases + 1) * 8 + 64 + kMaxLdsTypes * kRow * 4 +
                            kMaxOwnWords * 4 + kMaxItemsPerWg + 64;
  const int64_t per_thread = (tpg * geo->range_n + kRunBlock - 1) / kRunBlock;
  // the kMaxList-entry list where the accumulator leaves room for it (and the workgroup
  // has at most kBigMaxi items per thread); else kRunBlock entries
  // (a timed launch keeps it, and so does an adapting network's: their kernels have this
  // list only)
  int32_t cap = kRunBlock;
  if (!timing && !tab->adapt && per_thread <= kBigMaxi && (geo->max_list == 0 || geo->max_list >= kMaxList) &&
      static_lds + (size_t)list_bytes(kMaxList) + lds <= (size_t)max_lds)
    cap = kMaxList;
  if (static_lds + (size_t)list_bytes(cap) + lds > (size_t)max_lds) return hipErrorInvalidValue;
  a.list_cap = cap;
  const size_t dyn = lds;
  if (ff->n_src > 0 && io->x) {
    const int64_t rows = io->B * io->T;
    hipLaunchKernelGGL(compact_input_kernel, dim3((unsigned)rows), dim3(256), 0,
                       (hipStream_t)stream, io->x, rows, io->n_in, in_count, in_idx, in_val);
    hipError_t ce = hipGetLastError();
    if (ce != hipSuccess) return ce;
  } else if (ff->n_src > 0 && io->in_prob) {  // on-device Poisson input: no x at all
    const int64_t rows = io->B * io->T;
    hipLaunchKernelGGL(poisson_lists_kernel, dim3((unsigned)rows), dim3(256), 0,
                       (hipStream_t)stream, io->in_prob, io->n_in, io->in_seed, io->in_t0,
                       io->T, rows, in_count, in_idx, in_val);
    hipError_t ce = hipGetLastError();
    if (ce != hipSuccess) return ce;
  } else if (ff->n_src > 0) {
    return hipErrorInvalidValue;  // a feed-forward side needs x or in_prob
  }
  const bool coop = tab->K_rec > 0 && rec->n_src > 0 && geo->R > 1;
  return dispatch_S<RunLaunch>(tab->S, a, dyn, per_thread, (hipStream_t)stream, coop);
}

extern "C" int wt_cond_run(const wt_tables* tab, const wt_side* rec, const wt_side* ff,
                           const wt_geometry* geo, const wt_run_io* io, void* scratch,
                           wt_stream_t stream) {
  return run_impl(tab, rec, ff, geo, io, scratch, nullptr, stream);
}

extern "C" int wt_poisson_fill(const float* prob, int64_t n_in, uint64_t seed, int64_t t0,
                               int64_t B, int64_t T, float* x, wt_stream_t stream) {
  if (n_in < 0 || B < 0 || T < 0 || t0 < 0 || n_in > UINT32_MAX || B > UINT32_MAX ||
      t0 + T > (int64_t)UINT32_MAX)
    return hipErrorInvalidValue;
  const int64_t n = B * T * n_in;
  if (n == 0) return hipSuccess;
  if (!prob || !x) return hipErrorInvalidValue;
  hipLaunchKernelGGL(poisson_fill_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, prob, n_in, seed, t0, B, T, x);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------
// wt_cond_run_noalloc: wt_cond_run with its workspace in a file-scope device array, for
// callers that cannot allocate. The array's host-side name is not a device address:
// each device's copy is located once with hipGetSymbolAddress and only that pointer is
// handed to kernels.
// ---------------------------------------------------------------------------------
namespace noalloc {

__device__ __align__(256) unsigned char scratch[WT_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex lock;
void* device_scratch[kMaxDevices] = {};

// Zero `words` 32-bit words (a kernel, not hipMemsetAsync, so that the call may be
// captured into a graph).
__global__ void zero_words(uint32_t* p, int64_t words) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < words;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0u;
}

__global__ void copy_word(const uint32_t* from, uint32_t* to) {
  if (threadIdx.x == 0) *to = *from;
}

// This device's copy of the array (looked up on the device's first call).
hipError_t locate(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> guard(lock);
  if (!device_scratch[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    device_scratch[dev] = p;
  }
  *out = device_scratch[dev];
  return hipSuccess;
}

}  // namespace noalloc

extern "C" int wt_cond_run_noalloc(const wt_tables* tab, const wt_side* rec, const wt_side* ff,
                                   const wt_geometry* geo, const wt_run_io* io,
                                   uint32_t* flags, wt_stream_t stream) {
  if (!tab || !rec || !ff || !geo || !io) return hipErrorInvalidValue;
  if (geo->groups < 1 || geo->groups > kMaxGroups || geo->R < 1 || geo->range_n < 32 ||
      io->B < 1 || io->T < 0)
    return hipErrorInvalidValue;
  const int64_t bytes = wt_cond_run_scratch_bytes(geo, io->B, io->T);
  if (bytes > WT_NOALLOC_SCRATCH_BYTES) return hipErrorOutOfMemory;
  void* work = nullptr;
  hipError_t e = noalloc::locate(&work);
  if (e != hipSuccess) return e;
  const int64_t words = scratch_zeroed(geo) / 4;
  hipLaunchKernelGGL(noalloc::zero_words, dim3((unsigned)((words + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, static_cast<uint32_t*>(work), words);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  e = (hipError_t)run_impl(tab, rec, ff, geo, io, work, nullptr, stream);
  if (e != hipSuccess || !flags) return e;
  hipLaunchKernelGGL(noalloc::copy_word, dim3(1), dim3(64), 0, (hipStream_t)stream,
                     static_cast<const uint32_t*>(work), flags);
  return hipGetLastError();
}

extern "C" int wt_cond_run_timed(const wt_tables* tab, const wt_side* rec, const wt_side* ff,
                                 const wt_geometry* geo, const wt_run_io* io, void* scratch,
                                 uint64_t* timing, wt_stream_t stream) {
  if (!timing) return hipErrorInvalidValue;
  return run_impl(tab, rec, ff, geo, io, scratch, timing, stream);
}

extern "C" int wt_split_ranges(const int64_t* indptr, const int32_t* targets, int64_t n_src,
                               int64_t R, int64_t range_n, int64_t* split, wt_stream_t stream) {
  if (n_src < 0 || R < 1 || range_n < 1) return hipErrorInvalidValue;
  const int64_t total = n_src * (R + 1);
  if (total == 0) return hipSuccess;
  if (!split || !indptr || !targets) return hipErrorInvalidValue;
  const int block = 256;
  hipLaunchKernelGGL(split_ranges_kernel, dim3((unsigned)((total + block - 1) / block)),
                     dim3(block), 0, (hipStream_t)stream, indptr, targets, n_src, R,
                     range_n, split);
  return hipGetLastError();
}

extern "C" int wt_cond_scan_backward(const wt_tables* tab, const wt_backward_io* io,
                                     wt_stream_t stream) {
  if (!tab || !io || !io->grad_spikes || !io->spikes || !io->v_saved || !io->G_saved)
    return hipErrorInvalidValue;
  if (tab->S < 1 || tab->S > WT_MAX_S || tab->K < 0 || tab->K > WT_MAX_K)
    return hipErrorInvalidValue;
  if ((io->grad_decay || io->grad_jump || io->grad_scale) && !io->A) return hipErrorInvalidValue;
  if (io->grad_decay && !io->g_init) return hipErrorInvalidValue;
  if (tab->adapt && (!tab->adapt_decay || !tab->E_adapt || !io->a_saved))
    return hipErrorInvalidValue;
  if (io->grad_A_rows &&
      (io->T_pad < io->T || io->T_pad % 16 || io->B * io->T_pad > INT32_MAX || tab->K < 1))
    return hipErrorInvalidValue;
  if (io->B * tab->N == 0 || io->T == 0) return hipSuccess;
  BackArgs a = {};
  a.tab = *tab;
  a.io = *io;
  return dispatch_S<BackRun>(tab->S, a, (hipStream_t)stream);
}

static int64_t back_fields_of(int64_t S) { return 1 + 9 * S + WT_MAX_K + 5 + 4; }

extern "C" int64_t wt_cond_recurrent_backward_scratch_bytes(int64_t S, int64_t K_rec, int64_t B,
                                                            int64_t N) {
  const int64_t state = (back_fields_of(S) * B * N * 4 + 255) / 256 * 256;
  const int64_t grad_now = (K_rec * N * B * 4 + 255) / 256 * 256;
  return state + grad_now + B * N * 4;
}

extern "C" int wt_cond_recurrent_backward(const wt_tables* tab, const wt_side* rec,
                                          const wt_backward_io* io, void* scratch,
                                          wt_stream_t stream) {
  if (!tab || !rec || !io || !scratch || !io->grad_spikes || !io->spikes || !io->v_saved ||
      !io->G_saved)
    return hipErrorInvalidValue;
  if (tab->S < 1 || tab->S > WT_MAX_S || tab->K < 0 || tab->K > WT_MAX_K ||
      tab->K_rec < 1 || tab->K_rec > tab->K)
    return hipErrorInvalidValue;
  if ((io->grad_decay || io->grad_jump || io->grad_scale) && !io->A) return hipErrorInvalidValue;
  if (io->grad_decay && !io->g_init) return hipErrorInvalidValue;
  if (tab->adapt && (!tab->adapt_decay || !tab->E_adapt || !io->a_saved))
    return hipErrorInvalidValue;
  if (rec->n_src != tab->N || io->grad_A_rows) return hipErrorInvalidValue;
  if (io->B * tab->N == 0 || io->T == 0) return hipSuccess;
  if (!rec->indptr || !rec->pathway) return hipErrorInvalidValue;
  BackArgs a = {};
  a.tab = *tab;
  a.io = *io;
  a.rec = *rec;
  a.state = static_cast<float*>(scratch);
  const int64_t state_bytes = (back_fields_of(tab->S) * io->B * tab->N * 4 + 255) / 256 * 256;
  const int64_t grad_bytes = (tab->K_rec * tab->N * io->B * 4 + 255) / 256 * 256;
  a.grad_now = reinterpret_cast<float*>(static_cast<char*>(scratch) + state_bytes);
  a.R = reinterpret_cast<float*>(static_cast<char*>(scratch) + state_bytes + grad_bytes);
  return dispatch_S<BackRecurrent>(tab->S, a, (hipStream_t)stream);
}

extern "C" int wt_edge_sources(const int64_t* indptr, int64_t n_src, int64_t* edge_src,
                               wt_stream_t stream) {
  if (!indptr || !edge_src || n_src < 0) return hipErrorInvalidValue;
  if (n_src == 0) return hipSuccess;
  const int block = 256;
  hipLaunchKernelGGL(edge_source_kernel, dim3((unsigned)((n_src + block - 1) / block)),
                     dim3(block), 0, (hipStream_t)stream, indptr, n_src, edge_src);
  return hipGetLastError();
}

extern "C" int64_t wt_events_scratch_bytes(int64_t BT, int64_t n) {
  if (BT < 0 || n < 0) return 0;
  return ((BT + kEvChunk - 1) / kEvChunk) * n * 4 * (1 + kEvWords);  // counts, then bits
}

extern "C" int wt_events_count(const float* activity, int64_t BT, int64_t n, void* scratch,
                               int64_t* indptr, wt_stream_t stream) {
  if (!indptr || BT < 0 || n < 0 || BT > INT32_MAX) return hipErrorInvalidValue;
  const int64_t n_chunks = (BT + kEvChunk - 1) / kEvChunk;
  if (n_chunks > 65535) return hipErrorInvalidValue;
  if (n > 0 && BT > 0 && (!activity || !scratch)) return hipErrorInvalidValue;
  int32_t* chunk = static_cast<int32_t*>(scratch);
  const dim3 cols((unsigned)((n + kEvBlock - 1) / kEvBlock));
  if (n > 0 && BT > 0) {
    hipLaunchKernelGGL(events_count_kernel, dim3(cols.x, (unsigned)n_chunks), dim3(kEvBlock), 0,
                       (hipStream_t)stream, activity, BT, n, chunk,
                       reinterpret_cast<uint32_t*>(chunk + n_chunks * n));
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (n > 0) {  // column totals into indptr[1 .. n], then scanned in place
    hipLaunchKernelGGL(events_column_kernel, cols, dim3(kEvBlock), 0, (hipStream_t)stream,
                       chunk, n_chunks, n, indptr + 1);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(events_indptr_kernel, dim3(1), dim3(kRunBlock), 0, (hipStream_t)stream,
                     indptr + 1, n, indptr);
  return hipGetLastError();
}

extern "C" int wt_events_fill(const float* activity, int64_t BT, int64_t n, const void* scratch,
                              const int64_t* indptr, int32_t* bt, float* value, int64_t T,
                              int64_t T_pad, wt_stream_t stream) {
  if (BT < 0 || n < 0 || T < 1 || T_pad < T || BT % T) return hipErrorInvalidValue;
  if ((BT / T) * T_pad > INT32_MAX) return hipErrorInvalidValue;
  if (BT == 0 || n == 0) return hipSuccess;
  if (!activity || !scratch || !indptr || !bt) return hipErrorInvalidValue;
  const int64_t n_chunks = (BT + kEvChunk - 1) / kEvChunk;
  if (n_chunks > 65535) return hipErrorInvalidValue;
  const int32_t* chunk = static_cast<const int32_t*>(scratch);
  const dim3 grid((unsigned)((n + kEvBlock - 1) / kEvBlock), (unsigned)n_chunks);
  if (value)
    hipLaunchKernelGGL(events_fill_kernel, grid, dim3(kEvBlock), 0, (hipStream_t)stream,
                       activity, BT, n, chunk, indptr, bt, value, T, T_pad);
  else  // positions only: from the count's bits
    hipLaunchKernelGGL(events_fill_bits_kernel, grid, dim3(kEvBlock), 0, (hipStream_t)stream,
                       reinterpret_cast<const uint32_t*>(chunk + n_chunks * n), n, chunk, indptr,
                       bt, T, T_pad);
  return hipGetLastError();
}

extern "C" int wt_gate_scan(const float* x, int64_t B, int64_t T, int64_t n_in,
                            const int64_t* rows, int64_t n, const float* params,
                            float* gating, int64_t R, int64_t stp_col, int64_t sat_col,
                            float* factors, wt_stream_t stream) {
  if (B < 0 || T < 0 || n_in < 0 || n < 0 || R < 0) return hipErrorInvalidValue;
  if (stp_col < 0 && sat_col < 0) return hipErrorInvalidValue;  // no dynamics to step
  if ((stp_col >= 0 && stp_col + 2 * n > R) || (sat_col >= 0 && sat_col + n > R))
    return hipErrorInvalidValue;
  if (B * n == 0 || T == 0) return hipSuccess;
  if (!x || !rows || !params || !gating || !factors || n_in == 0) return hipErrorInvalidValue;
  const int block = 256;
  hipLaunchKernelGGL(gate_scan_kernel, dim3((unsigned)((B * n + block - 1) / block)),
                     dim3(block), 0, (hipStream_t)stream, x, B, T, n_in, rows, n, params,
                     gating, R, stp_col, sat_col, factors);
  return hipGetLastError();
}

extern "C" int wt_weight_gradient(const wt_side* side, const int64_t* edge_src, int64_t n_edges,
                                  const int64_t* ev_indptr, const int32_t* ev_bt,
                                  const float* ev_val, const float* grad_A, int64_t B,
                                  int64_t T, int64_t N, int64_t pathway_offset, float* grad_w,
                                  wt_stream_t stream) {
  if (pathway_offset < 0 || n_edges < 0) return hipErrorInvalidValue;
  if (n_edges == 0) return hipSuccess;  // nothing to write (pointers of empty tensors may be null)
  if (!side || !edge_src || !ev_indptr || !ev_bt || !grad_A || !grad_w)
    return hipErrorInvalidValue;
  const int block = 256;
  hipLaunchKernelGGL(weight_gradient_kernel, dim3((unsigned)((n_edges + block - 1) / block)),
                     dim3(block), 0, (hipStream_t)stream, *side, edge_src, n_edges, ev_indptr,
                     ev_bt, ev_val, grad_A, B * T, N, pathway_offset, grad_w);
  return hipGetLastError();
}

extern "C" int wt_weight_gradient_by_target(const int64_t* edge_src, int64_t n_edges,
                                            const int64_t* in_indptr, const int64_t* in_edge,
                                            int64_t n_pathways, int64_t N,
                                            const int64_t* ev_indptr, const int32_t* ev_bt,
                                            const float* ev_val, const float* grad_A,
                                            int64_t BT, float* rows, float* grad_w,
                                            wt_stream_t stream) {
  if (n_edges < 0 || n_pathways < 0 || N < 0 || BT < 0 || BT > INT32_MAX)
    return hipErrorInvalidValue;
  const int64_t n_rows = n_pathways * N;
  if (n_edges == 0 || n_rows == 0) return hipSuccess;
  if (!edge_src || !in_indptr || !in_edge || !ev_indptr || !ev_bt || !rows || !grad_w ||
      BT == 0)
    return hipErrorInvalidValue;
  if (n_rows > 0x7fffffff || (N + 63) / 64 > 0x7fffffff || (BT + 63) / 64 > 65535 ||
      n_pathways > 65535)
    return hipErrorInvalidValue;
  if (grad_A)  // (else rows holds them already)
    hipLaunchKernelGGL(transpose_rows_kernel,
                       dim3((unsigned)((N + 63) / 64), (unsigned)((BT + 63) / 64),
                            (unsigned)n_pathways),
                       dim3(256), 0, (hipStream_t)stream, grad_A, rows, BT, N);
  const int64_t chunk = BT < kWgChunk ? BT : kWgChunk;
  const void* fn = ev_val ? (const void*)weight_gradient_target_kernel<true>
                          : (const void*)weight_gradient_target_kernel<false>;
  const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)(chunk * sizeof(float)));
  if (e != hipSuccess) return e;
  if (ev_val)
    hipLaunchKernelGGL(weight_gradient_target_kernel<true>, dim3((unsigned)n_rows),
                       dim3(kWgBlock), (size_t)chunk * sizeof(float), (hipStream_t)stream,
                       in_indptr, in_edge, edge_src, ev_indptr, ev_bt, ev_val, rows, BT, grad_w);
  else
    hipLaunchKernelGGL(weight_gradient_target_kernel<false>, dim3((unsigned)n_rows),
                       dim3(kWgBlock), (size_t)chunk * sizeof(float), (hipStream_t)stream,
                       in_indptr, in_edge, edge_src, ev_indptr, ev_bt, ev_val, rows, BT, grad_w);
  return hipGetLastError();
}

extern "C" int wt_device_info(int64_t* n_cu, int64_t* max_lds_bytes) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  int cu = 0, lds = 0;
  e = hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev);
  if (e != hipSuccess) return e;
  if (n_cu) *n_cu = cu;
  if (max_lds_bytes) *max_lds_bytes = lds;
  return hipSuccess;
}
