// wt_run.h — the persistent forward kernel of wt_cond_run (see wt_kernels.hip) and its
// launcher, instantiated per synapse count S in wt_run_s<S>.hip (compiled in parallel).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/wiretorch_amd.h"
#include "wt_math.h"

namespace wt {

constexpr int kRunBlock = 1024;
constexpr int kMaxGroups = 64;

struct RunArgs {
  wt_tables tab;
  wt_side rec, ff;
  wt_geometry geo;
  wt_run_io io;
  // scratch
  uint32_t* err;        // [0]: error flags
  uint32_t* barrier;    // one counter per group, 128 bytes apart
  uint32_t* bitmap;     // [2][B][R * words]: which neurons fired, per trial
  const int32_t* in_count;  // [B*T]: nonzero inputs of each (trial, step), or > kInCap
  const int32_t* in_idx;    // [B*T][kInCap]
  const float* in_val;      // [B*T][kInCap]
  uint64_t* timing;     // [wgs][kPhases] wall-clock ticks per phase, or null
  int64_t words;        // bitmap words per workgroup range (range_n / 32)
  int64_t table_in_lds; // the per-type table fits the LDS copy
};

constexpr int kPhases = 5;  // update, publish, feedforward events, barrier wait, recurrent push
constexpr int kInCap = 64;  // inputs listed per (trial, step); denser rows are scanned
constexpr int kMaxLdsTypes = 256;
constexpr int kTypeCols = 6;  // theta, U_reset, E_L, C_m, beta, n_ref; then scale[K]

__device__ inline void store_agent(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline uint32_t load_agent(const uint32_t* p) {
  return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Split group barrier. arrive(): every thread's stores complete, then one arrival per
// workgroup on the group's counter. wait(): bounded (2 s of wall clock), giving up as
// soon as any workgroup has flagged an error. Work placed between the two overlaps
// the other workgroups' progress.
__device__ inline void barrier_arrive(uint32_t* counter) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0)
    __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ inline bool barrier_wait(uint32_t* counter, uint32_t target, uint32_t* err,
                                    uint32_t* s_flag) {
  if (threadIdx.x == 0) {
    uint32_t bad = 0;
    uint64_t start = wall_clock64();
    uint32_t polls = 0;
    while (__hip_atomic_load(counter, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
      __builtin_amdgcn_s_sleep(1);
      if ((++polls & 63u) == 0) {
        if (__hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) { bad = 1; break; }
        if (wall_clock64() - start > 200000000ull) {  // 2 s at the 100 MHz wall clock
          __hip_atomic_fetch_or(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          bad = 1;
          break;
        }
      }
    }
    *s_flag = bad;
  }
  __syncthreads();
  return *s_flag == 0;
}

template <int S>
__device__ inline void load_synapses(const wt_tables& tab, Synapses<S>& syn) {
#pragma unroll
  for (int s = 0; s < S; ++s) {
    syn.E[s] = tab.E_syn[s];
    syn.clip[s] = tab.g_clip[s];
    syn.decay_r[s] = tab.decay[s];
    syn.decay_d[s] = tab.decay[S + s];
    syn.jump_r[s] = tab.jump[s];
    syn.jump_d[s] = tab.jump[S + s];
  }
}

__device__ inline void add_fixed(long long* cell, float x, float fscale) {
  atomicAdd(reinterpret_cast<unsigned long long*>(cell), (unsigned long long)to_fixed(x, fscale));
}

// Serial fallback for an event that did not fit the work list.
__device__ inline void push_edges(long long* row, const wt_side& side, int64_t e0, int64_t e1,
                                  int64_t lo, float value, float fscale) {
  for (int64_t e = e0; e < e1; ++e) {
    const float w = side.weights[e];
    add_fixed(row + (side.targets[e] - lo), value == 1.0f ? w : value * w, fscale);
  }
}

__device__ inline void tick(uint64_t* acc_t, uint64_t& last, int phase) {
  if (acc_t && threadIdx.x == 0) {
    const uint64_t now = wall_clock64();
    acc_t[phase] += now - last;
    last = now;
  }
}

// An item index the compiler cannot see through: recomputed each step instead of
// hoisted out of the time loop (which would keep every item's derived indices live in
// registers for the whole launch).
__device__ inline uint32_t opaque(uint32_t x) {
  asm volatile("" : "+v"(x));
  return x;
}

// The workgroup's list of this step's events: a source whose synapses onto the
// workgroup's targets are edges [e0, e0 + count) of `side` (0 recurrent, 1 input), to be
// added times `value` to the accumulator row at `row`.
struct EventList {
  int64_t* e0;
  int32_t* count;  // becomes the exclusive prefix of the counts
  int32_t* row;
  float* value;
  uint8_t* side;
  int32_t* n;      // entries appended (may exceed the capacity: the rest ran serially)
  int32_t* wave_sum;
  int cap;
};

__device__ inline void append_event(const EventList& L, long long* acc, const wt_side& side,
                                    int side_id, int64_t e0, int64_t e1, int64_t row,
                                    int64_t lo, float value, float fscale) {
  if (e1 <= e0) return;
  const int pos = atomicAdd(L.n, 1);
  if (pos < L.cap) {
    L.e0[pos] = e0;
    L.count[pos] = (int32_t)(e1 - e0);
    L.row[pos] = (int32_t)(row - lo);
    L.value[pos] = value;
    L.side[pos] = (uint8_t)side_id;
  } else {
    push_edges(acc + row, side, e0, e1, lo, value, fscale);
  }
}

// Exclusive prefix of L.count[0 .. m) in place; returns the total. Two levels in LDS:
// 64 threads sum contiguous chunks, one thread scans the 64 chunk sums, the 64 threads
// rewrite their chunks.
__device__ inline int32_t scan_counts(const EventList& L, int m) {
  const int tid = threadIdx.x;
  const int chunk = (m + 63) / 64;
  if (tid < 64) {
    int32_t sum = 0;
    const int end = (tid + 1) * chunk < m ? (tid + 1) * chunk : m;
    for (int i = tid * chunk; i < end; ++i) sum += L.count[i];
    L.wave_sum[tid] = sum;
  }
  __syncthreads();
  if (tid == 0) {
    int32_t run = 0;
    for (int w = 0; w < 64; ++w) {
      const int32_t v = L.wave_sum[w];
      L.wave_sum[w] = run;
      run += v;
    }
    L.wave_sum[64] = run;
  }
  __syncthreads();
  if (tid < 64) {
    int32_t run = L.wave_sum[tid];
    const int end = (tid + 1) * chunk < m ? (tid + 1) * chunk : m;
    for (int i = tid * chunk; i < end; ++i) {
      const int32_t c = L.count[i];
      L.count[i] = run;
      run += c;
    }
  }
  __syncthreads();
  return L.wave_sum[64];
}

// Every listed synapse, spread evenly over the workgroup (four per thread per round,
// loads issued before the atomics), added to the accumulator.
__device__ inline void run_events(const EventList& L, int m, int32_t total, long long* acc,
                                  const wt_side& rec, const wt_side& ff, int64_t lo,
                                  float fscale) {
  const int stride = blockDim.x;
  for (int32_t base = threadIdx.x; base < total; base += 4 * stride) {
    int32_t tgt[4], rows[4];
    float x[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int32_t f = base + u * stride;
      if (f < total) {
        int a = 0, z = m;  // entry a with prefix[a] <= f < prefix[a + 1]
        while (z - a > 1) {
          const int mid = (a + z) >> 1;
          if (L.count[mid] <= f) a = mid; else z = mid;
        }
        const wt_side& side = L.side[a] ? ff : rec;
        const int64_t e = L.e0[a] + (f - L.count[a]);
        tgt[u] = side.targets[e];
        const float w = side.weights[e];
        const float v = L.value[a];
        x[u] = v == 1.0f ? w : v * w;
        rows[u] = L.row[a];  // may be negative: rows are relative to the range start
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (base + u * stride < total) add_fixed(acc + rows[u] + tgt[u], x[u], fscale);
  }
}

// The persistent forward. Each thread owns up to MAXI (trial, neuron) items — item
// threadIdx.x + i * blockDim.x of its workgroup — whose state stays in registers for
// the whole launch.
template <int S, int MAXI, bool EXTRA>
__global__ __launch_bounds__(kRunBlock) void cond_run_kernel(RunArgs A) {
  extern __shared__ long long acc[];  // [K][tpg][range_n], the fired bitmap, the type table
  __shared__ uint32_t s_flag;
  __shared__ uint64_t s_time[kPhases];
  __shared__ int64_t s_e0[kRunBlock];
  __shared__ int32_t s_count[kRunBlock];
  __shared__ int32_t s_row[kRunBlock];
  __shared__ float s_value[kRunBlock];
  __shared__ uint8_t s_side[kRunBlock];
  __shared__ int32_t s_nev;
  __shared__ int32_t s_wave[65];

  const wt_tables& tab = A.tab;
  const wt_run_io& io = A.io;
  const int64_t groups = A.geo.groups, R = A.geo.R, range_n = A.geo.range_n;
  const int64_t N = tab.N, K = tab.K, K_rec = tab.K_rec, B = io.B, T = io.T;
  // Optional outputs exist only in the EXTRA variant (the lean one writes spikes only).
  float* const o_prob = EXTRA ? io.prob : nullptr;
  float* const o_v_saved = EXTRA ? io.v_saved : nullptr;
  float* const o_G_saved = EXTRA ? io.G_saved : nullptr;
  int8_t* const o_held = EXTRA ? io.held : nullptr;
  float* const o_A_saved = EXTRA ? io.A_saved : nullptr;
  float* const o_track_v = EXTRA ? io.track_v : nullptr;
  float* const o_track_I = EXTRA ? io.track_I : nullptr;
  float* const o_track_g = EXTRA ? io.track_g : nullptr;
  const int64_t wg = blockIdx.x;
  const int64_t g = wg % groups, r = wg / groups;
  const int64_t tpg = g < B ? (B - g + groups - 1) / groups : 0;
  if (tpg == 0) return;  // no trial in this group: it takes part in nothing
  const int64_t lo = r * range_n;
  const int64_t nr = lo < N ? (N - lo < range_n ? N - lo : range_n) : 0;
  const int64_t items = tpg * nr;
  const int64_t acc_len = K * tpg * range_n;
  const int64_t words = A.words;
  const uint32_t nr32 = (uint32_t)(nr > 0 ? nr : 1), items32 = (uint32_t)items;
  uint32_t* s_bits = reinterpret_cast<uint32_t*>(acc + acc_len);  // [tpg][words]
  const int64_t cols = kTypeCols + K;      // columns of a type row (global table)
  const int64_t lcols = cols + 2;          // LDS rows add rate and g_L
  float* s_types = reinterpret_cast<float*>(s_bits + tpg * words);
  const bool refractory = tab.n_ref != nullptr;
  const bool recurrent = K_rec > 0 && A.rec.n_src > 0;
  const float dt = *tab.dt;
  const float fscale = ldexpf(1.0f, (int)A.geo.frac_bits);
  const float inv_fscale = ldexpf(1.0f, -(int)A.geo.frac_bits);
  const EventList EL{s_e0, s_count, s_row, s_value, s_side, &s_nev, s_wave, (int)blockDim.x};
  Synapses<S> syn;
  load_synapses<S>(tab, syn);
  uint64_t* my_time = A.timing ? s_time : nullptr;
  if (threadIdx.x < kPhases) s_time[threadIdx.x] = 0;
  uint64_t last = wall_clock64();

  for (int64_t i = threadIdx.x; i < acc_len; i += blockDim.x) acc[i] = 0;
  {
    for (int64_t ty = threadIdx.x; ty < tab.n_types; ty += blockDim.x) {
      const float* src = tab.types + ty * cols;
      float* dst = s_types + ty * lcols;
      for (int64_t c = 0; c < cols; ++c) dst[c] = src[c];
      const Leak lk = leak(src[3], src[4], dt);
      dst[cols] = lk.rate;
      dst[cols + 1] = lk.g_L;
    }
  }

  // Registers: the owned items' state.
  float v[MAXI], gr[MAXI][S], gd[MAXI][S];
  int32_t counter[MAXI];
  uint32_t type_pack[(MAXI + 3) / 4];  // each item's row of the type table, one byte each
#pragma unroll
  for (int i = 0; i < MAXI; ++i) {
    const uint32_t it = threadIdx.x + (uint32_t)i * blockDim.x;
    if (i % 4 == 0) type_pack[i / 4] = 0;
    if (it < items32) {
      const uint32_t q = it / nr32;
      const int64_t n = lo + (it - q * nr32), b = g + (int64_t)q * groups;
      v[i] = io.v[b * N + n];
      counter[i] = refractory ? io.counter[b * N + n] : 0;
      type_pack[i / 4] |= ((uint32_t)tab.type_of[n] & 0xffu) << (8 * (i % 4));
#pragma unroll
      for (int s = 0; s < S; ++s) {
        gr[i][s] = io.g[(b * 2 * S + s) * N + n];
        gd[i][s] = io.g[(b * 2 * S + S + s) * N + n];
      }
    }
  }
  uint32_t* my_barrier = A.barrier + g * 32;
  uint32_t phase = 0;  // barriers passed
  // Per item, as bit masks: the spike s_t of the step about to be integrated, and
  // whether the neuron is held (refractory) during it.
  uint32_t masks = 0;  // bit i: item i spikes at the current step; bit 8 + i: it is held
  const int64_t total_words = R * words;  // one trial's bitmap

  // Spikes of step 0, from the entering state.
  for (int64_t w = threadIdx.x; w < tpg * words; w += blockDim.x) s_bits[w] = 0;
  __syncthreads();
#pragma unroll
  for (int i = 0; i < MAXI; ++i) {
    const uint32_t it = opaque(threadIdx.x + (uint32_t)i * blockDim.x);
    if (it >= items32) continue;
    const uint32_t q = it / nr32, ln = it - q * nr32;
    const int64_t n = lo + ln, b = g + (int64_t)q * groups;
    const int64_t ty0 = (type_pack[i / 4] >> (8 * (i % 4))) & 0xffu;
    const float theta = s_types[ty0 * lcols];
    float r_hold, held;
    const float s0 = spike_step(v[i], theta, counter[i], (int32_t)s_types[ty0 * lcols + 5],
                                refractory, r_hold, held);
    if (s0 != 0.0f) {
      masks |= 1u << i;
      if (recurrent) atomicOr(&s_bits[q * words + (ln >> 5)], 1u << (ln & 31));
    }
    if (held != 0.0f) masks |= 256u << i;
    if (o_prob) {
      const float pr = 1.0f / (1.0f + expf(-(*tab.surr * (v[i] - theta))));
      o_prob[b * T * N + n] = refractory ? pr * (1.0f - held) : pr;
    }
  }
  if (recurrent) {
    __syncthreads();
    for (int64_t w = threadIdx.x; w < tpg * words; w += blockDim.x) {
      const int64_t q = w / words, b = g + q * groups;
      store_agent(A.bitmap + b * total_words + r * words + (w - q * words), s_bits[w]);
    }
    barrier_arrive(my_barrier);
    if (!barrier_wait(my_barrier, (uint32_t)(++phase * R), A.err, &s_flag)) return;
  }

  constexpr int kPre = MAXI;  // bitmap words preloaded per thread (one per item at R = 32)
  for (int64_t t = 0; t < T; ++t) {
    const int64_t cur = t & 1, nxt = (t + 1) & 1;
    const bool more = t + 1 < T;
    // ---- preload this step's fired bitmap (published one phase ago) ----
    uint32_t pre[kPre];
    const uint32_t* in_bits = A.bitmap + cur * B * total_words;
#pragma unroll
    for (int u = 0; u < kPre; ++u) {
      const int64_t w = threadIdx.x + (int64_t)u * blockDim.x;
      pre[u] = (recurrent && w < tpg * total_words)
                   ? load_agent(in_bits + (g + (w / total_words) * groups) * total_words + w % total_words)
                   : 0u;
    }
    for (int64_t w = threadIdx.x; w < tpg * words; w += blockDim.x) s_bits[w] = 0;
    if (threadIdx.x == 0) s_nev = 0;
    __syncthreads();

    // ---------------- (A) integrate step t for the owned neurons ----------------
    uint32_t masks_next = 0;
#pragma unroll
    for (int i = 0; i < MAXI; ++i) {
      const uint32_t it = opaque(threadIdx.x + (uint32_t)i * blockDim.x);
      if (it >= items32) continue;
      const uint32_t q = it / nr32, ln = it - q * nr32;
      const int64_t n = lo + ln;
      const int64_t b = g + (int64_t)q * groups;
      // opaque: the row's values are re-read from LDS each step, not held in registers
      const int64_t ty = opaque((type_pack[i / 4] >> (8 * (i % 4))) & 0xffu);
      auto P = [&](int64_t c) -> float { return s_types[ty * lcols + c]; };
      if (t > 0) {
        // g <- g * decay, then each pathway's activation times its kernel, in order
        // (dynamics.py:206-208; kernel = jump * scale * made, dynamics.py:95-100).
#pragma unroll
        for (int s = 0; s < S; ++s) {
          gr[i][s] = gr[i][s] * syn.decay_r[s];
          gd[i][s] = gd[i][s] * syn.decay_d[s];
        }
        for (int64_t k = 0; k < K; ++k) {
          long long* cell = acc + (k * tpg + (int64_t)q) * range_n + ln;
          const float a = from_fixed(*cell, inv_fscale);
          *cell = 0;
          if (o_A_saved) o_A_saved[((k * B + b) * T + (t - 1)) * N + n] = a;
          const float sc = P(kTypeCols + k);
#pragma unroll
          for (int s = 0; s < S; ++s) {
            const float mk = tab.made[k * S + s];
            if (mk != 0.0f) {
              gr[i][s] = gr[i][s] + a * (syn.jump_r[s] * sc * mk);
              gd[i][s] = gd[i][s] + a * (syn.jump_d[s] * sc * mk);
            }
          }
        }
        if (o_track_g && (io.track_b < 0 || io.track_b == b)) {
          const int64_t bt = io.track_b < 0 ? b : 0;
          float* out = o_track_g + ((bt * T + (t - 1)) * N + n) * 2 * S;
#pragma unroll
          for (int s = 0; s < S; ++s) {
            out[s] = gr[i][s];
            out[S + s] = gd[i][s];
          }
        }
      }
      const float s_t = (float)((masks >> i) & 1u);
      const float held_t = (float)((masks >> (8 + i)) & 1u);
      const float r_hold = refractory ? fmaxf(s_t, held_t) : s_t;
      const int64_t out = (b * T + t) * N + n;
      io.spikes[out] = s_t;
      float G[S], I[S], I_leak;
      const float v_next = membrane<S>(v[i], r_hold, gr[i], gd[i], syn, P(2), P(3), P(1),
                                       Leak{P(cols), P(cols + 1)}, dt, G, I, I_leak);
      if (o_v_saved) {
        o_v_saved[out] = v[i];
#pragma unroll
        for (int s = 0; s < S; ++s) o_G_saved[out * S + s] = G[s];
        if (refractory && o_held) o_held[out] = (int8_t)(held_t != 0.0f);
      }
      if (o_track_v && (io.track_b < 0 || io.track_b == b)) {
        const int64_t bt = io.track_b < 0 ? b : 0;
        const int64_t row = (bt * T + t) * N + n;
        o_track_v[row] = v_next;
#pragma unroll
        for (int s = 0; s < S; ++s) o_track_I[row * (S + 1) + s] = I[s];
        o_track_I[row * (S + 1) + S] = I_leak;
      }
      v[i] = v_next;
      if (more) {  // the spike of step t+1 depends on v_{t+1} only: decide it now
        const float theta = P(0);
        float r_next, held;
        const float s_next = spike_step(v_next, theta, counter[i], (int32_t)P(5), refractory,
                                        r_next, held);
        if (s_next != 0.0f) {
          masks_next |= 1u << i;
          if (recurrent) atomicOr(&s_bits[q * words + (ln >> 5)], 1u << (ln & 31));
        }
        if (held != 0.0f) masks_next |= 256u << i;
        if (o_prob) {
          const float pr = 1.0f / (1.0f + expf(-(*tab.surr * (v_next - theta))));
          o_prob[out + N] = refractory ? pr * (1.0f - held) : pr;
        }
      }
      // items one after another: interleaving them only raises register pressure (the
      // workgroup's 16 waves hide the latency)
      __builtin_amdgcn_sched_barrier(0);
    }
    masks = masks_next;
    tick(my_time, last, 0);
    __syncthreads();  // the accumulator is read and cleared: events may be added now

    // ---------------- publish step t+1's spikes (completion overlaps the push) -----
    if (recurrent && more) {
      uint32_t* out_bits = A.bitmap + nxt * B * total_words;
      for (int64_t w = threadIdx.x; w < tpg * words; w += blockDim.x) {
        const int64_t q = w / words, b = g + q * groups;
        store_agent(out_bits + b * total_words + r * words + (w - q * words), s_bits[w]);
      }
    }
    tick(my_time, last, 1);

    // ---------------- events of step t: inputs, then the preloaded bitmap ----------
    if (A.ff.n_src > 0) {
      const int64_t n_in = io.n_in;
      for (int64_t q = 0; q < tpg; ++q) {
        const int64_t b = g + q * groups, bt = b * T + t;
        const int32_t c = A.in_count[bt];
        const int64_t row_base = (K_rec * tpg + q) * range_n;
        if (c <= kInCap) {
          for (int32_t e = threadIdx.x; e < c; e += blockDim.x) {
            const int32_t j = A.in_idx[bt * kInCap + e];
            const int32_t k = A.ff.pathway[j];
            if (k < 0) continue;
            const int64_t* sp = A.ff.split + (int64_t)j * (R + 1) + r;
            append_event(EL, acc, A.ff, 1, sp[0], sp[1], row_base + k * tpg * range_n, lo,
                         A.in_val[bt * kInCap + e], fscale);
          }
        } else {
          const float* xrow = io.x + bt * n_in;
          for (int64_t j = threadIdx.x; j < n_in; j += blockDim.x) {
            const float xv = xrow[j];
            if (xv == 0.0f) continue;
            const int32_t k = A.ff.pathway[j];
            if (k < 0) continue;
            const int64_t* sp = A.ff.split + j * (R + 1) + r;
            append_event(EL, acc, A.ff, 1, sp[0], sp[1], row_base + k * tpg * range_n, lo,
                         xv, fscale);
          }
        }
      }
    }
    tick(my_time, last, 2);
    if (recurrent) {
      const int64_t n_words = tpg * total_words;
      for (int64_t w = threadIdx.x, u = 0; w < n_words; w += blockDim.x, ++u) {
        uint32_t bits = 0;
#pragma unroll
        for (int v_ = 0; v_ < kPre; ++v_)
          if (u == v_) bits = pre[v_];
        if (u >= kPre)
          bits = load_agent(in_bits + (g + (w / total_words) * groups) * total_words + w % total_words);
        const int64_t q = w / total_words, wl = w % total_words;
        while (bits) {
          const int bit = __builtin_ctz(bits);
          bits &= bits - 1;
          const int64_t j = (wl / words) * range_n + (wl % words) * 32 + bit;
          const int64_t* sp = A.rec.split + j * (R + 1) + r;
          const int64_t e0 = sp[0], e1 = sp[1];
          const int32_t k = A.rec.pathway[j];
          if (k < 0) continue;
          append_event(EL, acc, A.rec, 0, e0, e1, (k * tpg + q) * range_n, lo, 1.0f, fscale);
        }
      }
    }
    __syncthreads();
    {
      const int m = s_nev < EL.cap ? s_nev : EL.cap;
      if (m > 0) {
        const int32_t total = scan_counts(EL, m);
        run_events(EL, m, total, acc, A.rec, A.ff, lo, fscale);
      }
    }
    tick(my_time, last, 4);

    // ---------------- barrier: step t+1's bitmap is complete ----------------
    if (recurrent && more) {
      barrier_arrive(my_barrier);
      if (!barrier_wait(my_barrier, (uint32_t)(++phase * R), A.err, &s_flag)) return;
    } else {
      __syncthreads();
    }
    tick(my_time, last, 3);
  }

  // The activations of the last step enter the conductances that leave the chunk.
#pragma unroll
  for (int i = 0; i < MAXI; ++i) {
    const uint32_t it = opaque(threadIdx.x + (uint32_t)i * blockDim.x);
    if (it >= items32 || T == 0) continue;
    const uint32_t q = it / nr32, ln = it - q * nr32;
    const int64_t n = lo + ln, b = g + (int64_t)q * groups;
    const int64_t ty = (type_pack[i / 4] >> (8 * (i % 4))) & 0xffu;
#pragma unroll
    for (int s = 0; s < S; ++s) {
      gr[i][s] = gr[i][s] * syn.decay_r[s];
      gd[i][s] = gd[i][s] * syn.decay_d[s];
    }
    for (int64_t k = 0; k < K; ++k) {
      long long* cell = acc + (k * tpg + (int64_t)q) * range_n + ln;
      const float a = from_fixed(*cell, inv_fscale);
      if (o_A_saved) o_A_saved[((k * B + b) * T + (T - 1)) * N + n] = a;
      const float sc = s_types[ty * lcols + kTypeCols + k];
#pragma unroll
      for (int s = 0; s < S; ++s) {
        const float mk = tab.made[k * S + s];
        if (mk != 0.0f) {
          gr[i][s] = gr[i][s] + a * (syn.jump_r[s] * sc * mk);
          gd[i][s] = gd[i][s] + a * (syn.jump_d[s] * sc * mk);
        }
      }
    }
    if (o_track_g && (io.track_b < 0 || io.track_b == b)) {
      const int64_t bt = io.track_b < 0 ? b : 0;
      float* out = o_track_g + ((bt * T + (T - 1)) * N + n) * 2 * S;
#pragma unroll
      for (int s = 0; s < S; ++s) {
        out[s] = gr[i][s];
        out[S + s] = gd[i][s];
      }
    }
  }

  // write the state back
#pragma unroll
  for (int i = 0; i < MAXI; ++i) {
    const uint32_t it = threadIdx.x + (uint32_t)i * blockDim.x;
    if (it < items32) {
      const uint32_t q = it / nr32;
      const int64_t n = lo + (it - q * nr32), b = g + (int64_t)q * groups;
      io.v[b * N + n] = v[i];
      if (refractory) io.counter[b * N + n] = counter[i];
#pragma unroll
      for (int s = 0; s < S; ++s) {
        io.g[(b * 2 * S + s) * N + n] = gr[i][s];
        io.g[(b * 2 * S + S + s) * N + n] = gd[i][s];
      }
    }
  }
  if (A.timing && threadIdx.x < kPhases) A.timing[wg * kPhases + threadIdx.x] = s_time[threadIdx.x];
}

template <int S, int MAXI>
inline hipError_t launch_run(RunArgs& a, size_t lds, int block, hipStream_t stream, bool coop) {
  const bool extra = a.io.prob || a.io.v_saved || a.io.A_saved || a.io.track_v || a.io.track_g;
  const void* fn = extra ? reinterpret_cast<const void*>(&cond_run_kernel<S, MAXI, true>)
                         : reinterpret_cast<const void*>(&cond_run_kernel<S, MAXI, false>);
  hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  dim3 grid((unsigned)(a.geo.groups * a.geo.R)), blk((unsigned)block);
  void* params[] = {&a};
  if (coop) return hipLaunchCooperativeKernel(fn, grid, blk, params, (unsigned)lds, stream);
  if (extra)
    hipLaunchKernelGGL((cond_run_kernel<S, MAXI, true>), grid, blk, lds, stream, a);
  else
    hipLaunchKernelGGL((cond_run_kernel<S, MAXI, false>), grid, blk, lds, stream, a);
  return hipGetLastError();
}

template <int S>
struct RunLaunch {  // run() is instantiated in wt_run_s<S>.hip
  static hipError_t run(RunArgs& a, size_t lds, int block, int64_t per_thread,
                        hipStream_t stream, bool coop);
};

template <int S>
hipError_t RunLaunch<S>::run(RunArgs& a, size_t lds, int block, int64_t per_thread,
                             hipStream_t stream, bool coop) {
  {
    switch (per_thread) {
      case 0:
      case 1: return launch_run<S, 1>(a, lds, block, stream, coop);
      case 2: return launch_run<S, 2>(a, lds, block, stream, coop);
      case 3: return launch_run<S, 3>(a, lds, block, stream, coop);
      case 4: return launch_run<S, 4>(a, lds, block, stream, coop);
      case 5: return launch_run<S, 5>(a, lds, block, stream, coop);
      case 6: return launch_run<S, 6>(a, lds, block, stream, coop);
      case 7:
      case 8: return launch_run<S, 8>(a, lds, block, stream, coop);
    }
    return hipErrorInvalidValue;
  }
};

}  // namespace wt
