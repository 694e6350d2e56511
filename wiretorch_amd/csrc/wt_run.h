// wt_run.h — the persistent forward kernel of wt_cond_run (see wt_kernels.hip) and its
// launcher, instantiated per synapse count S in wt_run_s<S>.hip (compiled in parallel).
//
// Registers and LDS, per workgroup of 1024 threads:
//   * each thread owns up to MAXI (trial, neuron) items; their v, conductances and
//     refractory counters stay in VGPRs for the whole launch (an item's trial, target
//     and type row are recomputed from its index each step: see item_at);
//   * LDS holds the int64 activation accumulators [K][tpg][range_n], the workgroup's
//     own fired bits of the next step, the parameter table (one 64-byte row per distinct
//     neuron type) and the step's event list.
// A step: wait for the group's bitmap of this step; preload it into registers; update
// every owned neuron (inject the previous step's activations, spike, membrane,
// refractory) and decide its next spike into the LDS bits; publish them to the group
// and arrive at the group barrier; list this step's input and recurrent events; add
// their synapses onto the workgroup's targets into the accumulators.
#pragma once
#include <hip/hip_runtime.h>
#include <rocprim/block/block_scan.hpp>
#include <stdint.h>

#include <type_traits>

#include "../../include/wiretorch_amd.h"
#include "wt_math.h"
#include "wt_philox.h"

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
  uint32_t* bitmap;     // [3][groups][tpg_max][R * words]: which neurons fired
  const int32_t* in_count;  // [B*T]: nonzero inputs of each (trial, step), or > kInCap
  const int32_t* in_idx;    // [B*T][kInCap]
  const float* in_val;      // [B*T][kInCap]
  uint64_t* timing;     // [wgs][kPhases] wall-clock ticks per phase, or null
  int64_t words;        // bitmap words per workgroup range (range_n / 32)
  int64_t tpg_max;      // trials of the largest group
  int32_t list_cap;     // event list capacity: 1024 or 2048 entries
};

// Phases timed by wt_cond_run_timed (thread 0's view): its own update, the wait for the
// rest of the workgroup's update, publication + event compaction + arrival, the barrier
// wait, range lookups + scan + synapse push.
constexpr int kPhases = 8;
constexpr int kMaxFracBits = 40;  // fractional bits of the exact accumulators at most
constexpr int kInCap = 64;  // inputs listed per (trial, step); denser rows are scanned
constexpr int kMaxLdsTypes = 256;
constexpr int kTypeCols = 6;  // global table: theta, U_reset, E_L, C_m, beta, n_ref; scale[K]
// LDS table row (floats): theta, U_reset, E_L, C_m, n_ref, rate, g_L, -, scale[0..7]
constexpr int kRow = 16;
constexpr int kMaxItemsPerWg = 8 * kRunBlock;        // trials x range per workgroup
constexpr int kMaxOwnWords = kMaxItemsPerWg / 32;    // the workgroup's own fired bits
constexpr int kMaxList = 2 * kRunBlock;  // event list entries at most (two per thread)

// LDS of the event list of `cap` entries and its entry map (cap / 4 buckets of 64
// edges): e0 (8), heads (8 per bucket), count, row, value (4 each), first (2 per bucket),
// side (1).
constexpr int64_t list_bytes(int64_t cap) { return cap * 21 + (cap / 4) * 10; }

using BlockScan = rocprim::block_scan<int32_t, kRunBlock,
                                      rocprim::block_scan_algorithm::using_warp_scan>;

// The kernel's arguments, re-read from the kernarg segment (scalar loads) wherever a
// phase needs them, instead of being held in scalar registers across the whole loop.
typedef const __attribute__((address_space(4))) RunArgs* ArgPtr;
__device__ inline ArgPtr kargs() {
  ArgPtr p = (ArgPtr)__builtin_amdgcn_kernarg_segment_ptr();
  asm volatile("" : "+s"(p));
  return p;
}

// A value the compiler cannot see through: what is derived from an item's index is
// recomputed each step instead of hoisted out of the time loop (which would keep every
// item's addresses live in registers for the whole launch).
__device__ inline uint32_t opaque(uint32_t x) {
  asm volatile("" : "+v"(x));
  return x;
}
// The same for a wave-uniform value (kept in a scalar register).
__device__ inline uint32_t opaque_s(uint32_t x) {
  asm volatile("" : "+s"(x));
  return x;
}

// A load through the global address space. Pointers held in structures reach the
// kernel as generic pointers; generic (flat) loads also count against the LDS wait
// counter, which serialises them with the LDS work around them.
template <class T>
__device__ inline T gload(const T* p) {
  return *(const __attribute__((address_space(1))) T*)p;
}

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

// Exact accumulation of activations. Each product is rounded to a multiple of 2^-f and
// added in float64: the host keeps every accumulator below 2^(53-f) in magnitude, so
// every partial sum is exact, the order of the atomic adds does not matter, and the
// conversion to float32 at the end is the only other rounding.
struct Fixed {
  float scale;  // 2^f
  double inv;   // 2^-f
};
// Fractional bits for activations of magnitude at most `bound`: every per-target sum
// stays below 2^51 / 2^f, so the float64 accumulators stay exact (the host's rule, from a
// bound the host need not read back). ceil(log2 bound) from the exponent: bound = m 2^e
// with m in [0.5, 1) is below 2^e, and exactly 2^(e-1) when m = 0.5.
__device__ inline int frac_bits_of(double bound) {
  if (!(bound > 0.0)) return bound == 0.0 ? kMaxFracBits : 0;  // NaN: the coarsest
  if (isinf(bound)) return 0;
  int e = 0;
  const double m = frexp(bound, &e);
  const int up = m == 0.5 ? e - 1 : e;
  const int f = 51 - up;
  return f < 0 ? 0 : (f > kMaxFracBits ? kMaxFracBits : f);
}

__device__ inline void add_fixed(double* cell, float x, Fixed fx) {
  atomicAdd(cell, (double)rintf(x * fx.scale) * fx.inv);
}

// Serial fallback for an event that did not fit the work list.
__device__ inline void push_edges(double* row, const int32_t* targets, const float* weights,
                                  int64_t e0, int64_t e1, int64_t lo, float value, Fixed fx) {
  for (int64_t e = e0; e < e1; ++e) {
    const float w = gload(weights + e);
    add_fixed(row + (gload(targets + e) - lo), value == 1.0f ? w : value * w, fx);
  }
}

// Phase timer (wt_cond_run_timed): s_time[0 .. kPhases) accumulate wall-clock ticks,
// s_time[kPhases] holds the last reading.
template <bool TIMED>
__device__ inline void tick(uint64_t* s_time, int phase) {
  if (TIMED && threadIdx.x == 0) {
    const uint64_t now = wall_clock64();
    s_time[phase] += now - s_time[kPhases];
    s_time[kPhases] = now;
  }
}

// The workgroup's list of this step's events: a source whose synapses onto the
// workgroup's targets are edges [e0, e0 + count) of side `side` (0 recurrent, 1 input),
// to be added times `value` to the accumulator row at `row` (relative to the range).
struct EventList {
  int64_t* e0;
  int32_t* count;  // becomes the exclusive prefix of the counts
  int32_t* row;
  float* value;
  uint8_t* side;
  int32_t* n;      // entries appended; past the capacity, events pushed at once by
                   // append_event or left for another round
  int16_t* first;  // [nbk] after the scan: the entry holding edge 64 b
  uint64_t* heads; // [nbk] after the scan: bit f % 64 of word f / 64 where an entry starts
  int cap;         // capacity (entries)
  int nbk;         // buckets of the entry map, cap / 4
};

__device__ inline void append_event(const EventList& L, double* acc, const int32_t* targets,
                                    const float* weights, int side_id, int64_t e0, int64_t e1,
                                    int64_t row, int64_t lo, float value, Fixed fx) {
  if (e1 <= e0) return;
  const int pos = atomicAdd(L.n, 1);
  if (pos < L.cap) {
    L.e0[pos] = e0;
    L.count[pos] = (int32_t)(e1 - e0);
    L.row[pos] = (int32_t)(row - lo);
    L.value[pos] = value;
    L.side[pos] = (uint8_t)side_id;
  } else {
    push_edges(acc + row, targets, weights, e0, e1, lo, value, fx);
  }
}

// Entry pos of the event list: a source whose edges [e0, e1) land on `row` (absolute).
__device__ inline void put_event(const EventList& L, int pos, int side_id, int64_t e0,
                                 int64_t e1, int64_t row, int64_t lo, float value) {
  L.e0[pos] = e0;
  L.count[pos] = (int32_t)(e1 - e0);
  L.row[pos] = (int32_t)(row - lo);
  L.value[pos] = value;
  L.side[pos] = (uint8_t)side_id;
}

// Exclusive prefix of n (0 <= n < 2^BITS) over the lanes of the wave below this one, and
// the wave's total, from one ballot per bit. Every lane of the wave takes part.
template <int BITS>
__device__ inline uint32_t wave_prefix(uint32_t n, uint32_t& total) {
  uint32_t below = 0, all = 0;
#pragma unroll
  for (int b = 0; b < BITS; ++b) {
    const uint64_t m = __ballot((n >> b) & 1u);
    below += __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                       __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u)) << b;
    all += (uint32_t)__builtin_popcountll(m) << b;
  }
  total = all;
  return below;
}

template <int M>
__device__ inline bool rest_any(const uint32_t (&bits)[M]) {
  uint32_t any = 0;
#pragma unroll
  for (int u = 0; u < M; ++u) any |= bits[u];
  return any != 0;
}

// The wave's first position of `total` consecutive ones taken from an LDS counter: one
// atomic per wave. Every lane of the wave takes part; all receive the same base.
__device__ inline int wave_reserve(int32_t* counter, uint32_t total) {
  int base = 0;
  if (__lane_id() == 0 && total != 0) base = atomicAdd(counter, (int)total);
  return __builtin_amdgcn_readfirstlane(base);
}

// Every listed synapse, spread evenly over the workgroup (four per thread per round,
// loads issued before the atomics), added to the accumulator. After the scan L.count
// holds the exclusive prefix of the entries' edge counts, L.e0 each entry's first edge
// minus its prefix, and L.first / L.heads the entry map of the first L.nbk buckets.
__device__ inline void run_events(const EventList& L, int m, int32_t total, double* acc,
                                  int64_t lo, Fixed fx) {
  ArgPtr P = kargs();
  const int32_t* const rec_tg = P->rec.targets;
  const int32_t* const ff_tg = P->ff.targets;
  const float* const rec_w = P->rec.weights;
  const float* const ff_w = P->ff.weights;
  const int stride = blockDim.x;
  const int nb = (total + 63) >> 6;
  const uint32_t lane = threadIdx.x & 63u;
  const uint64_t upto = (2ull << lane) - 1ull;  // bucket positions 0 .. lane
  for (int32_t base = threadIdx.x; base < total; base += 4 * stride) {
    // three passes, so that all eight loads are in flight together: locate each edge's
    // entry (LDS), load the edges (HBM), add them (LDS atomics).
    // A wave's 64 edges at u are 64-edge bucket b = (base + u * stride) / 64 (stride is a
    // multiple of 64): lane l's entry is the bucket's first entry plus the entries that
    // start at bucket positions 1 .. l. Past the map, a binary search over the prefixes.
    int a[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int32_t f = base + u * stride, b = f >> 6;
      if (b >= nb) {
        a[u] = 0;  // no edge of the wave here
      } else if (b < L.nbk) {
        a[u] = L.first[b] + __builtin_popcountll(L.heads[b] & upto & ~1ull);
      } else {
        int lo2 = L.first[L.nbk - 1], z = m;
        while (z - lo2 > 1) {
          const int mid = (lo2 + z) >> 1;
          if (L.count[mid] <= f) lo2 = mid; else z = mid;
        }
        a[u] = lo2;
      }
    }
    int64_t e[4];
    int32_t rows[4];
    float val[4];
    bool input[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      e[u] = L.e0[a[u]] + (base + u * stride);  // e0 holds the entry's first edge - prefix
      input[u] = L.side[a[u]] != 0;
      val[u] = L.value[a[u]];
      rows[u] = L.row[a[u]];  // may be negative: rows are relative to the range start
    }
    int32_t tgt[4];
    float w[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (base + u * stride < total) {
        tgt[u] = gload((input[u] ? ff_tg : rec_tg) + e[u]);
        w[u] = gload((input[u] ? ff_w : rec_w) + e[u]);
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (base + u * stride < total)
        add_fixed(acc + rows[u] + tgt[u], val[u] == 1.0f ? w[u] : val[u] * w[u], fx);
  }
}

// The persistent forward. Each thread owns up to MAXI (trial, neuron) items — item
// threadIdx.x + i * blockDim.x of its workgroup — whose state stays in registers for
// the whole launch.
// BIG: the event list holds kMaxList entries, otherwise kRunBlock (static LDS, fixed
// addresses either way; the host takes BIG where the accumulator leaves room).
// ADAPT: the network adapts (tab.adapt set); kernels of their own, so that the others
// carry none of its registers.
template <int S, int MAXI, bool EXTRA, bool REFR, bool BIG, bool TIMED, bool ADAPT>
__global__ __launch_bounds__(kRunBlock) void cond_run_kernel(RunArgs A) {
  static_assert(MAXI <= 8, "the overflow note holds one bit per preloaded word");
  extern __shared__ __align__(16) double acc[];  // [K][tpg][range_n]
  __shared__ __align__(16) float s_types[kMaxLdsTypes * kRow];
  __shared__ uint32_t s_bits[kMaxOwnWords];  // [tpg][words]: the next step's own spikes
  __shared__ uint32_t s_flag;
  __shared__ uint64_t s_time[kPhases + 1];
  __shared__ int32_t s_nev;
  __shared__ int32_t s_nfired;
  __shared__ uint32_t s_fired[kRunBlock];  // this step's fired sources: j | trial << 24
  __shared__ uint8_t s_type_of[kMaxItemsPerWg];  // type row of each target of the range
  __shared__ typename BlockScan::storage_type s_scan;

  // Sizes in 32 bits (the host checks that they fit); offsets into (B, T, N) arrays
  // are formed in 64 bits.
  const int32_t groups = (int32_t)A.geo.groups, R = (int32_t)A.geo.R;
  const int32_t range_n = (int32_t)A.geo.range_n;
  const int32_t N = (int32_t)A.tab.N, K = (int32_t)A.tab.K, B = (int32_t)A.io.B;
  const int32_t T = (int32_t)A.io.T;
  const int32_t wg = blockIdx.x;
  const int32_t g = wg % groups, r = wg / groups;
  const int32_t tpg = g < B ? (B - g + groups - 1) / groups : 0;
  if (tpg == 0) return;  // no trial in this group: it takes part in nothing
  const int32_t lo = r * range_n;
  const int32_t nr = lo < N ? (N - lo < range_n ? N - lo : range_n) : 0;
  const uint32_t items = (uint32_t)(tpg * nr);
  const int32_t words = (int32_t)A.words;
  const int32_t total_words = R * words;        // one trial's bitmap
  const int32_t group_words = tpg * total_words;
  const uint32_t acc_stride = (uint32_t)(tpg * range_n);  // one pathway's accumulators
  const int32_t acc_len = (K > 0 ? K : 1) * (int32_t)acc_stride;
  constexpr bool refractory = REFR;  // the network has refractory periods
  const bool recurrent = A.tab.K_rec > 0 && A.rec.n_src > 0;
  const bool has_ff = A.ff.n_src > 0;
  // spike-frequency adaptation: each item's g_a lives in io.adaptation, read and written
  // by its owning thread each step (no register is held for it across the loop)
  constexpr bool adapting = ADAPT;
  const float dt = *A.tab.dt;
  const int frac = A.geo.bound ? frac_bits_of(*A.geo.bound) : (int)A.geo.frac_bits;
  const Fixed fx{ldexpf(1.0f, frac), ldexp(1.0, -frac)};
  // the event list and its entry map
  constexpr int kList = BIG ? kMaxList : kRunBlock;
  __shared__ int64_t s_e0[kList];
  __shared__ uint64_t s_heads[kList / 4];
  __shared__ int32_t s_count[kList], s_row[kList];
  __shared__ float s_value[kList];
  __shared__ int16_t s_first[kList / 4];
  __shared__ uint8_t s_side[kList];
  constexpr int cap = kList, nbk = kList / 4;
  const EventList EL{s_e0, s_count, s_row, s_value, s_side, &s_nev, s_first, s_heads, cap, nbk};
  Synapses<S> syn;
  load_synapses<S>(A.tab, syn);
  uint64_t made = 0;  // bit k * S + s: pathway k drives synapse type s
  for (int64_t k = 0; k < K; ++k)
#pragma unroll
    for (int s = 0; s < S; ++s)
      if (A.tab.made[k * S + s] != 0.0f) made |= 1ull << (k * S + s);
  if (threadIdx.x < kPhases) s_time[threadIdx.x] = 0;
  if (threadIdx.x == 0) s_time[kPhases] = wall_clock64();

  for (int64_t i = threadIdx.x; i < acc_len; i += blockDim.x) acc[i] = 0.0;
  {
    const int64_t cols = kTypeCols + K;
    // this range's rows: all of them, or its own list (range_rows)
    const int32_t* own = A.tab.range_rows ? A.tab.range_rows + (int64_t)r * kMaxLdsTypes : nullptr;
    for (int64_t ty = threadIdx.x; ty < A.tab.n_types; ty += blockDim.x) {
      const float* src = A.tab.types + (own ? (int64_t)own[ty] : ty) * cols;
      float* dst = s_types + ty * kRow;
      const Leak lk = leak(src[3], src[4], dt);
      dst[0] = src[0];
      dst[1] = src[1];
      dst[2] = src[2];
      dst[3] = src[3];
      dst[4] = src[5];
      dst[5] = lk.rate;
      dst[6] = lk.g_L;
      dst[7] = 0.0f;
      for (int64_t k = 0; k < 8; ++k) dst[8 + k] = k < K ? src[kTypeCols + k] : 0.0f;
    }
  }

  for (int32_t ln = threadIdx.x; ln < nr; ln += blockDim.x)
    s_type_of[ln] = (uint8_t)A.tab.type_of[lo + ln];
  // Item it = threadIdx.x + i * kRunBlock of the workgroup is (trial q, target ln) with
  // it = q * nr + ln: q = floor(it * ceil(2^32 / nr) / 2^32), exact for it, nr < 2^16.
  const uint32_t magic = nr > 0 ? (uint32_t)(0xffffffffull / (uint32_t)nr + 1u) : 0u;
  struct Item {
    bool valid;
    uint32_t q, ln;
  };
  auto item_at = [&](uint32_t it) {
    const bool valid = it < items;
    const uint32_t q = valid ? __umulhi(it, magic) : 0u;
    return Item{valid, q, valid ? it - q * (uint32_t)nr : 0u};
  };

  // Registers: the owned items' state. A thread's item i is item threadIdx.x +
  // i * kRunBlock of the workgroup; past the last item the state is zeros, so every
  // lane may compute (only writes check).
  float v[MAXI], gr[MAXI][S], gd[MAXI][S];
  int32_t counter[MAXI];
#pragma unroll
  for (int i = 0; i < MAXI; ++i) {
    const Item m = item_at(threadIdx.x + (uint32_t)i * kRunBlock);
    v[i] = 0.0f;
    counter[i] = 0;
#pragma unroll
    for (int s = 0; s < S; ++s) gr[i][s] = gd[i][s] = 0.0f;
    if (m.valid) {
      const int64_t n = lo + m.ln, b = g + (int64_t)m.q * groups;
      v[i] = A.io.v[b * N + n];
      counter[i] = refractory ? A.io.counter[b * N + n] : 0;
#pragma unroll
      for (int s = 0; s < S; ++s) {
        gr[i][s] = A.io.g[(b * 2 * S + s) * N + n];
        gd[i][s] = A.io.g[(b * 2 * S + S + s) * N + n];
      }
    }
  }
  uint32_t* const my_barrier = A.barrier + g * 32;
  uint32_t* const group_bits = A.bitmap + g * A.tpg_max * total_words;  // buffer 0
  const int64_t buffer_words = groups * A.tpg_max * total_words;
  uint32_t phase = 0;  // barrier arrivals of this workgroup
  // Per item, as bit masks: the spike s_t of the step about to be integrated, and
  // whether the neuron is held (refractory) during it.
  uint32_t masks = 0;  // bit i: item i spikes at the current step; bit 8 + i: it is held

  // Spikes of step 0, from the entering state.
  for (int64_t w = threadIdx.x; w < tpg * words; w += blockDim.x) s_bits[w] = 0;
  __syncthreads();
#pragma unroll
  for (int i = 0; i < MAXI; ++i) {
    const Item m = item_at(threadIdx.x + (uint32_t)i * kRunBlock);
    if (!m.valid) continue;
    const uint32_t ln = m.ln, q = m.q;
    const float* row = s_types + s_type_of[ln] * kRow;
    const float theta = row[0];
    float r_hold, held;
    const float s0 = spike_step(v[i], theta, counter[i], (int32_t)row[4], refractory,
                                r_hold, held);
    if (s0 != 0.0f) {
      masks |= 1u << i;
      if (recurrent) atomicOr(&s_bits[q * words + (ln >> 5)], 1u << (ln & 31));
    }
    if (held != 0.0f) masks |= 256u << i;
    if (EXTRA && A.io.prob) {
      const int64_t n = lo + ln, b = g + (int64_t)q * groups;
      const float pr = 1.0f / (1.0f + expf(-(*A.tab.surr * (v[i] - theta))));
      A.io.prob[b * T * N + n] = refractory ? pr * (1.0f - held) : pr;
    }
  }
  if (recurrent) {
    __syncthreads();
    for (int64_t w = threadIdx.x; w < tpg * words; w += blockDim.x) {
      const int64_t q = w / words;
      store_agent(group_bits + q * total_words + r * words + (w - q * words), s_bits[w]);
    }
    barrier_arrive(my_barrier);
    ++phase;
  }
  // Every step starts with its own spike bits clear and both lists empty: cleared here
  // for step 0, and after the publication (their last reader) for each next step.
  __syncthreads();
  for (int64_t w = threadIdx.x; w < tpg * words; w += blockDim.x) s_bits[w] = 0;
  if (threadIdx.x == 0) {
    s_nev = 0;
    s_nfired = 0;
  }
  __syncthreads();

  for (int32_t t = 0, buf = 0; t < T; ++t, buf = buf == 2 ? 0 : buf + 1) {
    const bool more = t + 1 < T;
    const uint32_t* in_bits = group_bits + buf * buffer_words;  // step t: buffer t % 3
    // ---- the group's fired bits of step t: complete once every workgroup arrived ----
    if (recurrent) {
      if (!barrier_wait(my_barrier, phase * (uint32_t)R, A.err, &s_flag)) return;
    }
    tick<TIMED>(s_time, 5);
    uint32_t pre[MAXI];
#pragma unroll
    for (int u = 0; u < MAXI; ++u) {
      const int64_t w = threadIdx.x + (int64_t)u * blockDim.x;
      pre[u] = (recurrent && w < group_words) ? load_agent(in_bits + w) : 0u;
    }
    // This step's listed inputs, fetched now and used after the update: thread
    // (q, e) = (tid / kInCap, tid % kInCap) holds input e of trial q's row.
    int32_t in_c = 0, in_j = 0;
    float in_v = 0.0f;
    if (has_ff && threadIdx.x < (uint32_t)(tpg * kInCap)) {
      ArgPtr P = kargs();
      const int64_t bt = (g + (int64_t)(threadIdx.x / kInCap) * groups) * T + t;
      const int64_t slot = bt * kInCap + threadIdx.x % kInCap;
      in_c = gload(P->in_count + bt);
      in_j = gload(P->in_idx + slot);
      in_v = gload(P->in_val + slot);
    }
    tick<TIMED>(s_time, 0);

    // ---------------- events of step t, listed before the update ----------------
    // The fired bits of the preloaded words are compacted into s_fired (source | trial
    // << 24); the bits past its capacity are noted in rest and read again from the
    // bitmap after the update.
    // Then one thread per listed source, and per listed input, issues its range lookups
    // (and pathway) into registers: their latency passes during the update.
    // The list holds 2 x kRunBlock sources: the first kRunBlock in s_fired, the next in
    // the event list's count array (unused until the appends after the update).
    // rest: bit u (u < 8) — every fired bit of preloaded word u is past the list's
    // capacity; bits 8-15 = u + 1 and bits 16-23 = k for the word whose k lowest fired
    // bits were listed and whose others were not (at most one per workgroup).
    constexpr int kListed = 2 * kRunBlock;
    uint32_t* const s_fired2 = reinterpret_cast<uint32_t*>(s_count);
    uint32_t rest = 0u;
#pragma unroll
    for (int u = 0; u < MAXI; ++u) {
      uint32_t bits = pre[u];
      if (__ballot(bits != 0u) == 0) continue;  // uniform over the wave
      const uint32_t n = __builtin_popcount(bits);
      uint32_t total;
      const uint32_t below = wave_prefix<6>(n, total);
      int pos = wave_reserve(&s_nfired, total) + (int)below;
      if (!bits) continue;
      const uint32_t w = threadIdx.x + (uint32_t)u * blockDim.x;
      const uint32_t q = w / (uint32_t)total_words, wl = w - q * (uint32_t)total_words;
      const uint32_t j0 =
          (wl / (uint32_t)words) * (uint32_t)range_n + (wl % (uint32_t)words) * 32;
      if (pos >= kListed) {
        rest |= 1u << u;
        continue;
      }
      if (pos + (int)n > kListed)
        rest |= (uint32_t)(u + 1) << 8 | (uint32_t)(kListed - pos) << 16;
      for (; bits && pos < kListed; ++pos) {
        const uint32_t f = (j0 + __builtin_ctz(bits)) | (q << 24);
        if (pos < kRunBlock)
          s_fired[pos] = f;
        else
          s_fired2[pos - kRunBlock] = f;
        bits &= bits - 1;
      }
    }
    __syncthreads();
    tick<TIMED>(s_time, 1);
    int64_t re0 = 0, re1 = 0, ie0 = 0, ie1 = 0;
    int32_t rk = -1, ik = -1;
    uint32_t rj = 0;
    {
      ArgPtr P = kargs();
      const int n_list = s_nfired < kRunBlock ? s_nfired : kRunBlock;
      if ((int)threadIdx.x < n_list) {
        rj = s_fired[opaque(threadIdx.x)];  // (an address recomputed, not kept live)
        const int64_t* sp = P->rec.split + (int64_t)(rj & 0xffffffu) * (R + 1) + r;
        re0 = gload(sp);
        re1 = gload(sp + 1);
        rk = gload(P->rec.pathway + (rj & 0xffffffu));
      }
      if ((int)(threadIdx.x % kInCap) < in_c && in_c <= kInCap) {
        const int64_t* sp = P->ff.split + (int64_t)in_j * (R + 1) + r;
        ie0 = gload(sp);
        ie1 = gload(sp + 1);
        ik = gload(P->ff.pathway + in_j);
      }
    }

    // ---------------- (A) integrate step t for the owned neurons ----------------
    // (step 0 has no previous activations to inject: its own instance of the loop)
    auto update = [&](auto inject_tag) {
      constexpr bool kInject = decltype(inject_tag)::value;
      float* const spikes = A.io.spikes;
      // element (b, t, n) of a (B, T, N) array: step_base + q * trial_stride + ln
      const int64_t step_base = ((int64_t)g * T + t) * N + lo;
      const uint64_t trial_stride = (uint64_t)groups * T * N;
      uint32_t masks_next = 0;
      const uint32_t wave_base = opaque_s(__builtin_amdgcn_readfirstlane(threadIdx.x) & ~63u);
#pragma unroll
      for (int i = 0; i < MAXI; ++i) {
        // a wave skips item i only when none of its lanes holds one (a uniform branch:
        // the state is then updated in place on every path)
        if (wave_base + (uint32_t)i * kRunBlock >= items) continue;
        const Item m = item_at(opaque(threadIdx.x + (uint32_t)i * kRunBlock));
        const bool valid = m.valid;
        const uint32_t ln = m.ln, q = m.q;
        const float* row = s_types + s_type_of[ln] * kRow;
        const int64_t out = step_base + (int64_t)((uint64_t)q * trial_stride) + ln;
        const int64_t b = EXTRA ? g + (int64_t)q * groups : 0;
        const int64_t n = lo + ln;
        if constexpr (kInject) {
          // g <- g * decay, then each pathway's activation times its kernel, in order
          // (dynamics.py:206-208; kernel = jump * scale * made, dynamics.py:95-100).
#pragma unroll
          for (int s = 0; s < S; ++s) {
            gr[i][s] = gr[i][s] * syn.decay_r[s];
            gd[i][s] = gd[i][s] * syn.decay_d[s];
          }
          // the item's pathways four at a time: their accumulators and scales read
          // together, then cleared, then added in pathway order. The reads and clears
          // take no branch: an index past the last pathway is clamped to it (read again,
          // cleared again after its read: a wave's LDS operations complete in order).
          double* const cell = acc + __umul24(q, (uint32_t)range_n) + ln;
          for (int32_t k0 = 0; k0 < K; k0 += 4) {
            double ad[4];
            float sc[4];
            uint32_t kc[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              kc[j] = (uint32_t)(k0 + j < K ? k0 + j : K - 1);
              ad[j] = cell[kc[j] * acc_stride];
              sc[j] = row[8 + kc[j]];
            }
            if (valid) {
#pragma unroll
              for (int j = 0; j < 4; ++j) cell[kc[j] * acc_stride] = 0.0;
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              if (k0 + j >= K) continue;
              const int64_t k = k0 + j;
              const float a = (float)ad[j];
              if (EXTRA && valid && A.io.A_saved) A.io.A_saved[((k * B + b) * T + (t - 1)) * N + n] = a;
#pragma unroll
              for (int s = 0; s < S; ++s) {
                if ((made >> (k * S + s)) & 1u) {
                  gr[i][s] = gr[i][s] + a * (syn.jump_r[s] * sc[j]);
                  gd[i][s] = gd[i][s] + a * (syn.jump_d[s] * sc[j]);
                }
              }
            }
          }
          if (EXTRA && valid && A.io.track_g && (A.io.track_b < 0 || A.io.track_b == b)) {
            const int64_t bt = A.io.track_b < 0 ? b : 0;
            float* o = A.io.track_g + ((bt * T + (t - 1)) * N + n) * 2 * S;
#pragma unroll
            for (int s = 0; s < S; ++s) {
              o[s] = gr[i][s];
              o[S + s] = gd[i][s];
            }
          }
        }
        const float4 p0 = *reinterpret_cast<const float4*>(row);      // theta U_reset E_L C_m
        const float4 p1 = *reinterpret_cast<const float4*>(row + 4);  // n_ref rate g_L -
        const float s_t = (float)((masks >> i) & 1u);
        const float held_t = (float)((masks >> (8 + i)) & 1u);
        const float r_hold = refractory ? fmaxf(s_t, held_t) : s_t;
        if (valid) spikes[out] = s_t;
        // the adaptation conductance entering step t (dynamics.py:134-137)
        const int64_t sidx = (g + (int64_t)q * groups) * N + n;
        float ga = 0.0f, E_a = 0.0f;
        if (adapting && valid) {
          ga = gload(A.io.adaptation + sidx);
          E_a = gload(A.tab.E_adapt + n);
        }
        float G[S], I[S], I_leak;
        const float v_next = membrane<S>(v[i], r_hold, gr[i], gd[i], syn, p0.z, p0.w, p0.y,
                                         Leak{p1.y, p1.z}, dt, G, I, I_leak, adapting, ga,
                                         E_a);
        if (adapting && valid) {  // it decays, and rises by the neuron's own spike
          const float ga_next = ga * gload(A.tab.adapt_decay + n) + gload(A.tab.adapt + n) * s_t;
          A.io.adaptation[sidx] = ga_next;
          if (EXTRA && A.io.a_saved) A.io.a_saved[out] = ga;
          if (EXTRA && A.io.track_a && (A.io.track_b < 0 || A.io.track_b == b))
            A.io.track_a[((A.io.track_b < 0 ? b : 0) * T + t) * N + n] = ga_next;
        }
        if (EXTRA && valid && A.io.v_saved) {
          A.io.v_saved[out] = v[i];
#pragma unroll
          for (int s = 0; s < S; ++s) A.io.G_saved[out * S + s] = G[s];
          if (refractory && A.io.held) A.io.held[out] = (int8_t)(held_t != 0.0f);
        }
        if (EXTRA && valid && A.io.track_v && (A.io.track_b < 0 || A.io.track_b == b)) {
          const int64_t bt = A.io.track_b < 0 ? b : 0;
          const int64_t trow = (bt * T + t) * N + n;
          A.io.track_v[trow] = v_next;
#pragma unroll
          for (int s = 0; s < S; ++s) A.io.track_I[trow * (S + 1) + s] = I[s];
          A.io.track_I[trow * (S + 1) + S] = I_leak;
        }
        v[i] = v_next;
        if (more) {  // the spike of step t+1 depends on v_{t+1} only: decide it now
          float r_next, held;
          const float s_next = spike_step(v_next, p0.x, counter[i], (int32_t)p1.x, refractory,
                                          r_next, held);
          if (s_next != 0.0f) {
            masks_next |= 1u << i;
            if (recurrent && valid) atomicOr(&s_bits[q * words + (ln >> 5)], 1u << (ln & 31));
          }
          if (held != 0.0f) masks_next |= 256u << i;
          if (EXTRA && valid && A.io.prob) {
            const float pr = 1.0f / (1.0f + expf(-(*A.tab.surr * (v_next - p0.x))));
            A.io.prob[out + N] = refractory ? pr * (1.0f - held) : pr;
          }
        }
        // items one after another: interleaving them only raises register pressure (the
        // workgroup's 16 waves hide the latency)
        __builtin_amdgcn_sched_barrier(0);
      }
      masks = masks_next;
    };
    if (t == 0)
      update(std::false_type{});
    else
      update(std::true_type{});
    // A second listed source per thread (sources kRunBlock .. 2 kRunBlock - 1): its
    // lookups are issued now, its entry read before the barrier below (the appends that
    // follow it write the event list over the entries).
    int64_t re0b = 0, re1b = 0;
    int32_t rkb = -1;
    uint32_t rjb = 0;
    if (s_nfired > kRunBlock) {  // uniform (a burst of firing)
      ArgPtr P = kargs();
      const int n_list2 = (s_nfired < kListed ? s_nfired : kListed) - kRunBlock;
      if ((int)threadIdx.x < n_list2) {
        rjb = s_fired2[threadIdx.x];
        const int64_t* sp = P->rec.split + (int64_t)(rjb & 0xffffffu) * (R + 1) + r;
        re0b = gload(sp);
        re1b = gload(sp + 1);
        rkb = gload(P->rec.pathway + (rjb & 0xffffffu));
      }
    }
    tick<TIMED>(s_time, 2);
    __syncthreads();  // the accumulator is read and cleared; the next bits are complete
    tick<TIMED>(s_time, 3);

    // ---------------- publish step t+1's spikes ----------------
    const bool publish = recurrent && more;
    if (publish) {
      // each word's place recomputed here in 32 bits (hoisted out of the step loop, its
      // first value was spilled to scratch and reloaded before the stores every step)
      uint32_t* out_bits = group_bits + (buf == 2 ? 0 : buf + 1) * buffer_words;
      for (uint32_t w = opaque(threadIdx.x); w < (uint32_t)(tpg * words); w += blockDim.x) {
        const uint32_t q = w / (uint32_t)words;
        store_agent(out_bits + (int64_t)q * total_words + r * words + (w - q * words),
                    s_bits[w]);
      }
    }

    // ---------------- events of step t, after the update ----------------
    // (1) Fired sources in bitmap words beyond the preload, and inputs of rows with more
    // than kInCap of them, are appended by the thread that finds them (an event past the
    // list's capacity is pushed at once: the update has already read the accumulator).
    // Step t's bitmap stays readable after the arrival at the barrier: the others write
    // step t+1's bits into the next of three buffers, and step t+2's only once this
    // workgroup has arrived again.
    {
      ArgPtr P = kargs();
      const int64_t* rec_split = P->rec.split;
      const int32_t* rec_path = P->rec.pathway;
      if (recurrent) {
        for (int64_t w = threadIdx.x + (int64_t)MAXI * blockDim.x; w < group_words;
             w += blockDim.x) {
          uint32_t bits = load_agent(in_bits + w);
          const uint32_t q = (uint32_t)w / (uint32_t)total_words;
          const uint32_t wl = (uint32_t)w - q * (uint32_t)total_words;
          const uint32_t j0 =
              (wl / (uint32_t)words) * (uint32_t)range_n + (wl % (uint32_t)words) * 32;
          while (bits) {
            const uint32_t j = j0 + __builtin_ctz(bits);
            bits &= bits - 1;
            const int32_t k = gload(rec_path + j);
            const int64_t* sp = rec_split + (int64_t)j * (R + 1) + r;
            if (k >= 0)
              append_event(EL, acc, P->rec.targets, P->rec.weights, 0, gload(sp),
                           gload(sp + 1), k * acc_stride + (int64_t)q * range_n, lo, 1.0f, fx);
          }
        }
      }
      if (has_ff) {
        const int64_t n_in = P->io.n_in, K_rec = P->tab.K_rec;
        for (int64_t q = 0; q < tpg; ++q) {
          const int64_t bt = (g + q * groups) * T + t;
          if (gload(P->in_count + bt) <= kInCap) continue;  // uniform
          const float* xrow = P->io.x + bt * n_in;  // (null with Poisson input)
          const bool drawn = P->io.x == nullptr;
          const uint32_t pb = (uint32_t)(g + q * groups), pt = (uint32_t)(P->io.in_t0 + t);
          const int64_t row_base = (K_rec * tpg + q) * range_n;
          for (int64_t j = threadIdx.x; j < n_in; j += blockDim.x) {
            const float xv = drawn ? (poisson_fires(P->io.in_seed, pb, pt, (uint32_t)j,
                                                    gload(P->io.in_prob + j)) ? 1.0f : 0.0f)
                                   : gload(xrow + j);
            if (xv == 0.0f) continue;
            const int32_t k = gload(P->ff.pathway + j);
            if (k < 0) continue;
            const int64_t* sp = P->ff.split + j * (R + 1) + r;
            append_event(EL, acc, P->ff.targets, P->ff.weights, 1, gload(sp), gload(sp + 1),
                         row_base + k * acc_stride, lo, xv, fx);
          }
        }
      }
    }
    if (publish) {
      barrier_arrive(my_barrier);
      ++phase;
    } else {
      __syncthreads();
    }
    tick<TIMED>(s_time, 4);
    // the next step's own bits and fired list start empty (their readers are done)
    for (int64_t w = threadIdx.x; w < tpg * words; w += blockDim.x) s_bits[w] = 0;
    if (threadIdx.x == 0) s_nfired = 0;
    // (2) The listed sources and inputs (their lookups issued before the update), then
    // the fired sources the list could not hold (rest), in rounds of at most cap
    // events: each round appends what fits, scans and pushes it. A round that could not
    // take every event leaves the list's count past its capacity — read by every thread
    // after the round's barrier — and the events not taken for the next round. (Sparse
    // firing takes one round.)
    {
      ArgPtr P = kargs();
      bool rec_pending = rk >= 0 && re1 > re0, in_pending = ik >= 0 && ie1 > ie0;
      bool rec2_pending = rkb >= 0 && re1b > re0b;
      uint32_t rest_bits[MAXI];
#pragma unroll
      for (int u = 0; u < MAXI; ++u) rest_bits[u] = 0u;
      if (rest) {  // every word read at once (an index past the group's words is clamped)
#pragma unroll
        for (int u = 0; u < MAXI; ++u) {  // (32-bit indexes, recomputed: not kept live)
          const uint32_t w = opaque(threadIdx.x) + (uint32_t)u * blockDim.x;
          const uint32_t last = (uint32_t)group_words - 1u;
          rest_bits[u] = load_agent(in_bits + (w < last ? w : last));
        }
#pragma unroll
        for (int u = 0; u < MAXI; ++u) {
          const bool whole = (rest >> u) & 1u;
          const bool split = ((rest >> 8) & 0xffu) == (uint32_t)(u + 1);
          if (!whole && !split) rest_bits[u] = 0u;
          if (split)
            for (uint32_t k = (rest >> 16) & 0xffu; k > 0; --k) rest_bits[u] &= rest_bits[u] - 1;
        }
      }
      for (;;) {
        // the listed source and input of each thread: one reservation per wave
        {
          uint32_t total;
          const uint32_t below =
              wave_prefix<2>((uint32_t)rec_pending + rec2_pending + in_pending, total);
          int pos = wave_reserve(EL.n, total) + (int)below;
          if (rec_pending) {
            if (pos < cap) {
              put_event(EL, pos, 0, re0, re1, rk * acc_stride + (int64_t)(rj >> 24) * range_n,
                        lo, 1.0f);
              rec_pending = false;
            }
            ++pos;
          }
          if (rec2_pending) {
            if (pos < cap) {
              put_event(EL, pos, 0, re0b, re1b,
                        rkb * acc_stride + (int64_t)(rjb >> 24) * range_n, lo, 1.0f);
              rec2_pending = false;
            }
            ++pos;
          }
          if (in_pending && pos < cap) {
            put_event(EL, pos, 1, ie0, ie1,
                      (P->tab.K_rec * tpg + (int64_t)(threadIdx.x / kInCap)) * range_n +
                          ik * acc_stride,
                      lo, in_v);
            in_pending = false;
          }
        }
        // the unlisted fired sources, up to kTake per thread at a time with their lookups
        // in flight together, while the wave has any and the list has room
        // (a list already full takes nothing more this round: its count, which only
        // grows, then calls for another)
        while (__ballot(rest_any(rest_bits)) != 0 &&
               __builtin_amdgcn_readfirstlane(*EL.n) < cap) {
          constexpr int kTake = 4;
          uint32_t src[kTake], trial[kTake];
          bool has[kTake];
          {
            uint32_t left[MAXI];
#pragma unroll
            for (int u = 0; u < MAXI; ++u) left[u] = rest_bits[u];
#pragma unroll
            for (int c = 0; c < kTake; ++c) {
              has[c] = false;
              src[c] = 0;
              trial[c] = 0;
#pragma unroll
              for (int u = 0; u < MAXI; ++u) {
                if (has[c] || !left[u]) continue;
                const uint32_t w = threadIdx.x + (uint32_t)u * blockDim.x;
                const uint32_t q = w / (uint32_t)total_words, wl = w - q * (uint32_t)total_words;
                src[c] = (wl / (uint32_t)words) * (uint32_t)range_n +
                         (wl % (uint32_t)words) * 32 + __builtin_ctz(left[u]);
                trial[c] = q;
                left[u] &= left[u] - 1;
                has[c] = true;
              }
            }
          }
          int32_t kk[kTake];
          int64_t f0[kTake], f1[kTake];
#pragma unroll
          for (int c = 0; c < kTake; ++c) {
            kk[c] = -1;
            f0[c] = f1[c] = 0;
            if (has[c]) {
              const int64_t* sp = P->rec.split + (int64_t)src[c] * (R + 1) + r;
              kk[c] = gload(P->rec.pathway + src[c]);
              f0[c] = gload(sp);
              f1[c] = gload(sp + 1);
            }
          }
          uint32_t n = 0;
#pragma unroll
          for (int c = 0; c < kTake; ++c) n += (has[c] && kk[c] >= 0 && f1[c] > f0[c]) ? 1u : 0u;
          uint32_t total;
          const uint32_t below = wave_prefix<3>(n, total);
          const int base = wave_reserve(EL.n, total);
          int pos = base + (int)below;
          // taken sources are consumed in order up to the first event without room
          int consumed = 0;
          bool stop = false;
#pragma unroll
          for (int c = 0; c < kTake; ++c) {
            if (!has[c] || stop) continue;
            if (kk[c] >= 0 && f1[c] > f0[c]) {
              if (pos >= cap) {
                stop = true;
                continue;
              }
              put_event(EL, pos, 0, f0[c], f1[c],
                        kk[c] * acc_stride + (int64_t)trial[c] * range_n, lo, 1.0f);
              ++pos;
            }
            ++consumed;
          }
#pragma unroll
          for (int c = 0; c < kTake; ++c) {
            if (c >= consumed) continue;
            bool done = false;
#pragma unroll
            for (int u = 0; u < MAXI; ++u) {
              if (done || !rest_bits[u]) continue;
              rest_bits[u] &= rest_bits[u] - 1;
              done = true;
            }
          }
          if (base + (int)total >= cap) break;  // uniform: the list is full
        }
        // the entry map is cleared for this round's scan (its last reader, the previous
        // round's push, is behind a barrier; its next writer after the one below)
        for (int w = threadIdx.x; w < nbk; w += blockDim.x) s_heads[w] = 0;
        __syncthreads();
        tick<TIMED>(s_time, 6);
        const int n_ev = s_nev;
        const int m = n_ev < cap ? n_ev : cap;
        if (m > 0) {  // m is uniform: every thread takes part in the scan
          const int tid = threadIdx.x;
          // thread tid scans entries tid * per .. + per - 1
          constexpr int per = cap / kRunBlock;
          const int a0 = tid * per;
          int32_t cnt[kMaxList / kRunBlock], sum = 0, c, total;
#pragma unroll
          for (int j = 0; j < kMaxList / kRunBlock; ++j) {
            cnt[j] = (j < per && a0 + j < m) ? s_count[a0 + j] : 0;
            sum += cnt[j];
          }
          BlockScan().exclusive_scan(sum, c, 0, total, s_scan);
#pragma unroll
          for (int j = 0; j < kMaxList / kRunBlock; ++j) {
            if (j >= per || a0 + j >= m) continue;
            const int a = a0 + j;  // entry a holds edges [c, c + cnt) of the round, cnt > 0
            s_count[a] = c;
            s_e0[a] -= c;
            for (int32_t b = (c + 63) >> 6; b < nbk && (b << 6) < c + cnt[j]; ++b)
              s_first[b] = (int16_t)a;
            if (c < nbk * 64)
              atomicOr((unsigned long long*)&s_heads[c >> 6], 1ull << (c & 63));
            c += cnt[j];
          }
          __syncthreads();
          run_events(EL, m, total, acc, lo, fx);
        }
        if (n_ev < cap) break;  // uniform: every event of the step was taken
        // (a full list may leave events: n_ev == cap takes one more, possibly empty,
        // round)
        __syncthreads();  // the list is consumed
        if (threadIdx.x == 0) s_nev = 0;
        __syncthreads();
      }
    }
    __syncthreads();  // the accumulator is complete for the next update
    if (threadIdx.x == 0) s_nev = 0;  // every thread has read it; its next use is behind barriers
    tick<TIMED>(s_time, 7);
  }

  // The activations of the last step enter the conductances that leave the chunk.
#pragma unroll
  for (int i = 0; i < MAXI; ++i) {
    const Item m = item_at(threadIdx.x + (uint32_t)i * kRunBlock);
    if (!m.valid || T == 0) continue;
    const uint32_t ln = m.ln, q = m.q;
    const float* row = s_types + s_type_of[ln] * kRow;
    const int64_t n = lo + ln, b = g + (int64_t)q * groups;
#pragma unroll
    for (int s = 0; s < S; ++s) {
      gr[i][s] = gr[i][s] * syn.decay_r[s];
      gd[i][s] = gd[i][s] * syn.decay_d[s];
    }
    const double* cell = acc + q * range_n + ln;
    for (int64_t k = 0; k < K; ++k, cell += acc_stride) {
      const float a = (float)*cell;
      if (EXTRA && A.io.A_saved) A.io.A_saved[((k * B + b) * T + (T - 1)) * N + n] = a;
      const float sc = row[8 + k];
#pragma unroll
      for (int s = 0; s < S; ++s) {
        if ((made >> (k * S + s)) & 1u) {
          gr[i][s] = gr[i][s] + a * (syn.jump_r[s] * sc);
          gd[i][s] = gd[i][s] + a * (syn.jump_d[s] * sc);
        }
      }
    }
    if (EXTRA && A.io.track_g && (A.io.track_b < 0 || A.io.track_b == b)) {
      const int64_t bt = A.io.track_b < 0 ? b : 0;
      float* o = A.io.track_g + ((bt * T + (T - 1)) * N + n) * 2 * S;
#pragma unroll
      for (int s = 0; s < S; ++s) {
        o[s] = gr[i][s];
        o[S + s] = gd[i][s];
      }
    }
  }

  // write the state back
#pragma unroll
  for (int i = 0; i < MAXI; ++i) {
    const Item m = item_at(threadIdx.x + (uint32_t)i * kRunBlock);
    if (!m.valid) continue;
    const int64_t n = lo + m.ln, b = g + (int64_t)m.q * groups;
    A.io.v[b * N + n] = v[i];
    if (refractory) A.io.counter[b * N + n] = counter[i];
#pragma unroll
    for (int s = 0; s < S; ++s) {
      A.io.g[(b * 2 * S + s) * N + n] = gr[i][s];
      A.io.g[(b * 2 * S + S + s) * N + n] = gd[i][s];
    }
  }
  if (TIMED && threadIdx.x < kPhases) A.timing[wg * kPhases + threadIdx.x] = s_time[threadIdx.x];
}

template <int S, int MAXI, bool EXTRA, bool REFR, bool BIG, bool TIMED = false,
          bool ADAPT = false>
inline hipError_t launch_one(RunArgs& a, size_t lds, hipStream_t stream, bool coop) {
  const void* fn =
      reinterpret_cast<const void*>(&cond_run_kernel<S, MAXI, EXTRA, REFR, BIG, TIMED, ADAPT>);
  hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  dim3 grid((unsigned)(a.geo.groups * a.geo.R)), blk((unsigned)kRunBlock);
  void* params[] = {&a};
  if (coop) return hipLaunchCooperativeKernel(fn, grid, blk, params, (unsigned)lds, stream);
  hipLaunchKernelGGL((cond_run_kernel<S, MAXI, EXTRA, REFR, BIG, TIMED, ADAPT>), grid, blk, lds,
                     stream, a);
  return hipGetLastError();
}

template <int S, int MAXI, bool BIG>
inline hipError_t launch_flags(RunArgs& a, size_t lds, hipStream_t stream, bool coop) {
  const bool extra = a.io.prob || a.io.v_saved || a.io.A_saved || a.io.track_v || a.io.track_g;
  const bool refr = a.tab.n_ref != nullptr;
  if (a.tab.adapt) {  // adapting networks: the saving kernels with the 1024-entry list
    if constexpr (BIG) {
      return hipErrorInvalidValue;
    } else {
      if (a.timing) return hipErrorInvalidValue;
      return refr ? launch_one<S, MAXI, true, true, false, false, true>(a, lds, stream, coop)
                  : launch_one<S, MAXI, true, false, false, false, true>(a, lds, stream, coop);
    }
  }
  if (a.timing) {  // timed kernels: lean outputs and the 1024-entry list only
    if (extra || BIG) return hipErrorInvalidValue;
    return refr ? launch_one<S, MAXI, false, true, false, true>(a, lds, stream, coop)
                : launch_one<S, MAXI, false, false, false, true>(a, lds, stream, coop);
  }
  if (extra)
    return refr ? launch_one<S, MAXI, true, true, BIG>(a, lds, stream, coop)
                : launch_one<S, MAXI, true, false, BIG>(a, lds, stream, coop);
  return refr ? launch_one<S, MAXI, false, true, BIG>(a, lds, stream, coop)
              : launch_one<S, MAXI, false, false, BIG>(a, lds, stream, coop);
}

// The large-list kernels exist for up to kBigMaxi items per thread (workgroups whose
// accumulator leaves room for the list); the host asks for them only there.
constexpr int kBigMaxi = 4;

template <int S, int MAXI>
inline hipError_t launch_run(RunArgs& a, size_t lds, hipStream_t stream, bool coop) {
  if (a.list_cap > kRunBlock) {
    if constexpr (MAXI <= kBigMaxi) return launch_flags<S, MAXI, true>(a, lds, stream, coop);
    return hipErrorInvalidValue;
  }
  return launch_flags<S, MAXI, false>(a, lds, stream, coop);
}

template <int S>
struct RunLaunch {  // run() is instantiated in wt_run_s<S>.hip
  static hipError_t run(RunArgs& a, size_t lds, int64_t per_thread, hipStream_t stream,
                        bool coop);
};

template <int S>
hipError_t RunLaunch<S>::run(RunArgs& a, size_t lds, int64_t per_thread, hipStream_t stream,
                             bool coop) {
  switch (per_thread) {
    case 0:
    case 1: return launch_run<S, 1>(a, lds, stream, coop);
    case 2: return launch_run<S, 2>(a, lds, stream, coop);
    case 3: return launch_run<S, 3>(a, lds, stream, coop);
    case 4: return launch_run<S, 4>(a, lds, stream, coop);
    case 5: return launch_run<S, 5>(a, lds, stream, coop);
    case 6: return launch_run<S, 6>(a, lds, stream, coop);
    case 7:
    case 8: return launch_run<S, 8>(a, lds, stream, coop);
  }
  return hipErrorInvalidValue;
}

}  // namespace wt
