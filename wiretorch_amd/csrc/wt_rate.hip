// wt_rate.hip — rate networks on gfx950: the step of rate/dynamics.py as one fused launch
// per step (an MFMA matrix product of the rates with the weights, whose epilogue filters
// the currents, integrates the voltages and outputs the next rates), and its reverse.
//
// Every matrix operand is zero-padded to whole tiles by the host, so the tile loads need
// no bounds checks:
//   * the forward product's K dimension holds every pathway's rows as a segment of whole
//     k-blocks (recurrent pathways first: their rows are neurons, read from the rate
//     buffer `rin`; then the feedforward pathways: their rows are input columns, read
//     from the padded input X of the step); W is (K_pad x N_pad);
//   * a segment's partial product is the pathway's activation a_k; at the end of the
//     segment it enters the synaptic targets, target[s] += a_k * scale_k * made_k[s], in
//     pathway order as the reference sums them.
// Tiles: 64 x 64 outputs per workgroup of four waves, each wave a 32 x 32 MFMA block;
// k-blocks of 32 staged in LDS. MFMA: v_mfma_f32_32x32x2_f32 (float32 storage) or
// v_mfma_f32_32x32x16_bf16 (bfloat16 storage), accumulating in float32.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/wiretorch_amd.h"

namespace wt {
namespace rate {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kTile = 64;     // outputs per workgroup, per side
constexpr int kThreads = 256;
constexpr int kMaxS = 8;
constexpr int kMaxSeg = 16;

// The reference's nonlinearities (rate/dynamics.py:63-69, torch's definitions) and
// their derivatives. Codes follow wiretorch_amd.rate.NONLINEARITIES.
__device__ inline float nonlin(int code, float x) {
  switch (code) {
    case 0: return x > 0.0f ? x : 0.0f;                        // relu
    case 1: return x > 20.0f ? x : log1pf(expf(x));            // softplus (beta 1, threshold 20)
    case 2: return 1.0f / (1.0f + expf(-x));                   // sigmoid
    default: return tanhf(x);                                  // tanh
  }
}
__device__ inline float nonlin_grad(int code, float x) {
  switch (code) {
    case 0: return x > 0.0f ? 1.0f : 0.0f;
    case 1: {
      if (x > 20.0f) return 1.0f;
      const float z = expf(x);
      return z / (z + 1.0f);
    }
    case 2: {
      const float s = 1.0f / (1.0f + expf(-x));
      return s * (1.0f - s);
    }
    default: {
      const float t = tanhf(x);
      return 1.0f - t * t;
    }
  }
}

// Output element v of a lane's 32 x 32 block: row 8(v/4) + 4(l/32) + v%4, column l%32.
__device__ inline int out_row(int v, int lane) { return 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3); }

// ---------------------------------------------------------------------------------
// The tile product C[64 x 64] += A[64 x k] Bt[64 x k]^T with both operands k-contiguous
// (row-major, k along the row: the rates or inputs by trial, the weights transposed by
// target), in stages of 128 bytes of k (64 bfloat16 or 32 float32).
//
// A stage is 8 KB per operand: thread t fetches the 16-byte chunk t % 8 of rows t / 8 and
// 32 + t / 8, so eight consecutive threads read one row's 128 bytes. Stages are fetched
// kDepth ahead into a ring of registers and stored to one of two LDS buffers; one
// barrier per stage. In LDS, chunk c of row r sits in slot c ^ (r % 8) of its row: the
// MFMA operand reads (one 16-byte chunk per lane, rows r..r+7 at one chunk) then fall in
// eight different slots — no bank conflicts.
// ---------------------------------------------------------------------------------

constexpr int kStageBytes = 128;
constexpr int kDepth = 4;

struct StageRegs {
  u32x4 a[2], b[2];
};

__device__ inline u32x4 gload16(const char* p) {
  return *(const __attribute__((address_space(1))) u32x4*)p;
}

// One stage's operands: rows [0, 64) of A at byte offset `a` (row pitch lda bytes), of
// Bt at `b` (pitch ldb).
__device__ inline void stage_load(StageRegs& r, const char* a, int64_t lda, const char* b,
                                  int64_t ldb) {
  const int t = threadIdx.x, row = t >> 3, off = (t & 7) * 16;
  r.a[0] = gload16(a + row * lda + off);
  r.a[1] = gload16(a + (row + 32) * lda + off);
  r.b[0] = gload16(b + row * ldb + off);
  r.b[1] = gload16(b + (row + 32) * ldb + off);
}

// LDS: [buffer][operand][row * 8 + slot] in 16-byte units.
typedef u32x4 StageLds[2][2][512];

__device__ inline void stage_store(StageLds& lds, int buf, const StageRegs& r) {
  const int t = threadIdx.x, row = t >> 3, slot = (t & 7) ^ (row & 7);
  lds[buf][0][row * 8 + slot] = r.a[0];
  lds[buf][0][(row + 32) * 8 + slot] = r.a[1];
  lds[buf][1][row * 8 + slot] = r.b[0];
  lds[buf][1][(row + 32) * 8 + slot] = r.b[1];
}

template <typename T>
struct Mma;
// bfloat16, v_mfma_f32_32x32x16_bf16: C += A[32 x 16] B[16 x 32], lane l supplying
// A[l % 32][8 (l / 32) + e] and B[8 (l / 32) + e][l % 32], e < 8 — one 16-byte chunk of
// each operand row. A stage is four of them.
template <>
struct Mma<__bf16> {
  __device__ static void stage(f32x16& c, const u32x4* sa, const u32x4* sb, int lane) {
    const int r = lane & 31, h = lane >> 5;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int slot = (2 * q + h) ^ (r & 7);
      const u32x4 x = sa[r * 8 + slot], y = sb[r * 8 + slot];
      c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(*reinterpret_cast<const bf16x8*>(&x),
                                                  *reinterpret_cast<const bf16x8*>(&y), c, 0,
                                                  0, 0);
    }
  }
};
// float32, v_mfma_f32_32x32x2_f32: C += A[32 x 2] B[2 x 32], lane l supplying one element
// of k-slot l / 32. The 32 k of a stage are dealt as: MFMA step q takes element q % 4 of
// chunk 2 (q / 4) + l / 32 — A and B lanes agree on it, so each k enters exactly once.
template <>
struct Mma<float> {
  __device__ static void stage(f32x16& c, const u32x4* sa, const u32x4* sb, int lane) {
    const int r = lane & 31, h = lane >> 5;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int slot = (2 * p + h) ^ (r & 7);
      const u32x4 x = sa[r * 8 + slot], y = sb[r * 8 + slot];
      const float xa[4] = {__uint_as_float(x.x), __uint_as_float(x.y), __uint_as_float(x.z),
                           __uint_as_float(x.w)};
      const float yb[4] = {__uint_as_float(y.x), __uint_as_float(y.y), __uint_as_float(y.z),
                           __uint_as_float(y.w)};
#pragma unroll
      for (int e = 0; e < 4; ++e) c = __builtin_amdgcn_mfma_f32_32x32x2f32(xa[e], yb[e], c, 0, 0, 0);
    }
  }
};

// Runs stages [0, n) of a tile: src(s, a, lda, b, ldb) names stage s's operands;
// after stage s, done(s, c) sees the accumulator (and may reset it). Every iteration
// fetches a stage — past the end, the last one again — so that the loads in flight are
// the same on every path and the wait before each LDS store lets kDepth - 1 stages stay
// in flight.
template <typename T, class Src, class Done>
__device__ inline void tile_product(StageLds& lds, f32x16& c, int n, Src src, Done done) {
  if (n <= 0) return;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int wi = wave >> 1, wj = wave & 1;
  StageRegs ring[kDepth];
  auto fetch = [&](int s, StageRegs& r) {
    const char *a, *b;
    int64_t lda, ldb;
    src(s < n ? s : n - 1, a, lda, b, ldb);
    stage_load(r, a, lda, b, ldb);
  };
#pragma unroll
  for (int j = 0; j < kDepth; ++j) fetch(j, ring[j]);
  stage_store(lds, 0, ring[0]);
  fetch(kDepth, ring[0]);
  __syncthreads();
  for (int s0 = 0; s0 < n; s0 += kDepth) {
#pragma unroll
    for (int j = 0; j < kDepth; ++j) {
      const int s = s0 + j;
      if (s >= n) return;  // (not break: the next trip's waits assume a whole trip)
      Mma<T>::stage(c, &lds[s & 1][0][wi * 32 * 8], &lds[s & 1][1][wj * 32 * 8], lane);
      done(s, c);
      const int next = (j + 1) % kDepth;  // static once the loop is unrolled
      stage_store(lds, (s + 1) & 1, ring[next]);
      fetch(s + 1 + kDepth, ring[next]);
      __syncthreads();
    }
  }
}

// Everything a launch reads, by value.
struct RateArgs {
  wt_rate_tables tab;
  wt_rate_operand op;
  wt_rate_io io;
  int32_t t;
};

template <typename T>
__device__ inline T to_storage(float x) { return (T)x; }

// Rates of the state entering step 0 (and what the backward saves of it).
template <typename T>
__global__ __launch_bounds__(kThreads) void rate_init_kernel(RateArgs a) {
  const wt_rate_tables& tb = a.tab;
  const wt_rate_io& io = a.io;
  const int64_t N = tb.N, S = tb.S, T_ = io.T;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= io.B * N) return;
  const int64_t b = idx / N, n = idx - b * N;
  const float v = io.v[idx];
  const float r = tb.gain[n] * nonlin(tb.nonlinearity[n], v - tb.theta[n]);
  io.out[(b * T_) * N + n] = r;
  const int32_t pos = a.op.rpos ? a.op.rpos[n] : -1;
  if (pos >= 0) static_cast<T*>(a.op.rin)[b * a.op.K_rec_pad + pos] = to_storage<T>(r);
  if (io.v_saved) io.v_saved[(b * T_) * N + n] = v;
  if (io.I_saved)
    for (int64_t s = 0; s < S; ++s) io.I_saved[((b * T_) * N + n) * S + s] = io.I[(b * S + s) * N + n];
}

// Step t: a = [rin | X_t] W by segments, then the currents, voltages and next rates.
// S (synapse types) is a template parameter: each lane keeps 16 x S targets.
template <typename T, int S>
__global__ __launch_bounds__(kThreads) void rate_step_kernel(RateArgs a) {
  __shared__ StageLds lds;
  const wt_rate_tables& tb = a.tab;
  const wt_rate_operand& op = a.op;
  const wt_rate_io& io = a.io;
  const int64_t N = tb.N, B = io.B, T_ = io.T, t = a.t;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int wi = wave >> 1, wj = wave & 1;
  const int64_t n0 = (int64_t)blockIdx.x * kTile, b0 = (int64_t)blockIdx.y * kTile;
  const int64_t n = n0 + wj * 32 + (lane & 31);
  constexpr int kStageK = kStageBytes / (int)sizeof(T);
  const int64_t Kp = op.K_rec_pad + op.K_ff_pad;
  const int rec_stages = (int)(op.K_rec_pad / kStageK);
  const char* rin_b = reinterpret_cast<const char*>(
      static_cast<const T*>(op.rin) + ((t & 1) * op.B_pad + b0) * op.K_rec_pad);
  const char* X_b = reinterpret_cast<const char*>(
      static_cast<const T*>(op.X) + (t * op.B_pad + b0) * op.K_ff_pad);
  const char* Wt_n = reinterpret_cast<const char*>(static_cast<const T*>(op.Wt) + n0 * Kp);
  const int64_t ldr = op.K_rec_pad * (int64_t)sizeof(T), ldx = op.K_ff_pad * (int64_t)sizeof(T);
  const int64_t ldw = Kp * (int64_t)sizeof(T);

  float target[16][S];
#pragma unroll
  for (int v = 0; v < 16; ++v)
#pragma unroll
    for (int s = 0; s < S; ++s) target[v][s] = 0.0f;

  // k runs over the recurrent rows (the rates of the step), then the input rows (the
  // step's input); at the end of each pathway's segment its activation a_k enters the
  // targets, in pathway order.
  int g = 0;
  auto src = [&](int s, const char*& pa, int64_t& lda, const char*& pb, int64_t& ldb) {
    if (s < rec_stages) {
      pa = rin_b + (int64_t)s * kStageBytes;
      lda = ldr;
    } else {
      pa = X_b + (int64_t)(s - rec_stages) * kStageBytes;
      lda = ldx;
    }
    pb = Wt_n + (int64_t)s * kStageBytes;
    ldb = ldw;
  };
  // every segment's kernel scale for this tile's 64 targets, staged in LDS before the
  // product (the fold at a segment's end then issues no global load)
  __shared__ float s_jump[kMaxSeg][S][kTile];
  for (int i = threadIdx.x; i < op.n_seg * S * kTile; i += kThreads) {
    const int seg = i / (S * kTile), s = (i / kTile) % S, col = i % kTile;
    const int64_t tn = n0 + col;
    s_jump[seg][s][col] = tn < N ? tb.jump[((int64_t)op.seg[seg][2] * N + tn) * S + s] : 0.0f;
  }
  const int col = wj * 32 + (lane & 31);
  auto done = [&](int s, f32x16& c) {
    if ((int64_t)(s + 1) * kStageK != op.seg[g][1]) return;
    const int64_t path = op.seg[g][2];
    float jump[S];
#pragma unroll
    for (int q = 0; q < S; ++q) jump[q] = s_jump[g][q][col];
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int64_t b = b0 + wi * 32 + out_row(v, lane);
      if (io.A_saved && n < N && b < B) io.A_saved[((path * B + b) * T_ + t) * N + n] = c[v];
#pragma unroll
      for (int q = 0; q < S; ++q) target[v][q] = target[v][q] + c[v] * jump[q];
    }
    c = f32x16{};
    ++g;
  };
  f32x16 c = {};
  tile_product<T>(lds, c, (int)(Kp / kStageK), src, done);
  if (n >= N) return;
  const float beta = tb.beta[n], theta = tb.theta[n], gain = tb.gain[n];
  const int code = tb.nonlinearity[n];
  const int32_t pos = op.rpos ? op.rpos[n] : -1;
  T* rin_next = static_cast<T*>(op.rin) + ((t + 1) & 1) * op.B_pad * op.K_rec_pad;
  const bool last = t + 1 == T_;
  // With the voltages saved, the voltage entering this step is the saved one (written by
  // the previous step, or the first rates' launch), and the state v is written only
  // after the last step. A current whose decay is 0 is its target: its state is neither
  // read nor, before the last step, written.
  float decay[S], sign[S];
#pragma unroll
  for (int s = 0; s < S; ++s) {
    decay[s] = tb.decay[s];
    sign[s] = tb.sign[s];
  }
  // every load of the state first (16 trials), then the update and the stores
  float v_in[16], I_prev[16][S];
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int64_t b = b0 + wi * 32 + out_row(v, lane);
    const bool ok = b < B;
    const int64_t el = (b * T_ + t) * N + n;
    v_in[v] = !ok ? 0.0f : io.v_saved ? io.v_saved[el] : io.v[b * N + n];
#pragma unroll
    for (int s = 0; s < S; ++s)
      I_prev[v][s] = ok && decay[s] != 0.0f ? io.I[(b * S + s) * N + n] : 0.0f;
  }
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int64_t b = b0 + wi * 32 + out_row(v, lane);
    if (b >= B) continue;
    const int64_t el = (b * T_ + t) * N + n;
    float I[S];
    float I_syn = 0.0f;
#pragma unroll
    for (int s = 0; s < S; ++s) {
      if (io.target_saved) io.target_saved[el * S + s] = target[v][s];
      const float d = decay[s];
      I[s] = d * I_prev[v][s] + (1.0f - d) * target[v][s];
      if (d != 0.0f || last) io.I[(b * S + s) * N + n] = I[s];
      I_syn = I_syn + I[s] * sign[s];
    }
    const float vv = beta * v_in[v] + (1.0f - beta) * I_syn;
    if (!io.v_saved || last) io.v[b * N + n] = vv;
    if (io.track_v && (io.track_b < 0 || io.track_b == b)) {
      const int64_t row = ((io.track_b < 0 ? b : 0) * T_ + t) * N + n;
      io.track_v[row] = vv;
#pragma unroll
      for (int s = 0; s < S; ++s) io.track_I[row * S + s] = I[s];
    }
    if (!last) {
      const float r = gain * nonlin(code, vv - theta);
      io.out[el + N] = r;
      if (pos >= 0) rin_next[b * op.K_rec_pad + pos] = to_storage<T>(r);
      if (io.v_saved) io.v_saved[el + N] = vv;
      if (io.I_saved)
#pragma unroll
        for (int s = 0; s < S; ++s) io.I_saved[(el + N) * S + s] = I[s];
    }
  }
}

// Reverse, elementwise over (trial, neuron): (C) of step t+1 — the rate's gradient
// reaches the voltage entering step t+1 — then (A) of step t — the voltage's and
// currents' gradients reach this step's targets, hence dL/da_k of step t.
struct RateBackArgs {
  wt_rate_tables tab;
  wt_rate_operand op;
  wt_rate_back_io io;
  int32_t t;       // step of (A), or -1 for none
  int32_t t_rate;  // step of (C), or -1 for none
};

template <typename T>
__global__ __launch_bounds__(kThreads) void rate_back_elem_kernel(RateBackArgs a) {
  const wt_rate_tables& tb = a.tab;
  const wt_rate_back_io& io = a.io;
  const int64_t N = tb.N, S = tb.S, K = tb.K, B = io.B, T_ = io.T;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= B * N) return;
  const int64_t b = idx / N, n = idx - b * N;
  float lv = io.lam_v[idx];
  if (a.t_rate >= 0) {  // (C): v_u enters r_u; lv holds beta dL/dv_{u+1} already
    const int64_t u = a.t_rate;
    const int64_t el = (b * T_ + u) * N + n;
    const float dr = io.grad_out[el] + (io.d_rate ? io.d_rate[b * tb.N + n] : 0.0f);
    const float x = io.v_saved[el] - tb.theta[n];
    const int code = tb.nonlinearity[n];
    const float gf = dr * tb.gain[n];
    const float fp = nonlin_grad(code, x);
    lv = lv + gf * fp;
    if (io.acc_theta) io.acc_theta[idx] -= gf * fp;
    if (io.acc_gain) io.acc_gain[idx] += dr * nonlin(code, x);
  }
  if (a.t >= 0) {  // (A) of step t: v_{t+1} = beta v_t + (1 - beta) sum_s sign_s I_{t+1,s}
    const int64_t t = a.t;
    const int64_t el = (b * T_ + t) * N + n;
    const float beta = tb.beta[n];
    float dtarget[kMaxS];
    float I_next_syn = 0.0f;
#pragma unroll
    for (int s = 0; s < kMaxS; ++s) {
      if (s >= S) break;
      if (io.acc_beta) {
        const float I_next =
            t + 1 < T_ ? io.I_saved[(el + N) * S + s] : io.I_final[(b * S + s) * N + n];
        I_next_syn = I_next_syn + I_next * tb.sign[s];
      }
      const float dI = io.lam_I[(b * S + s) * N + n] + lv * (1.0f - beta) * tb.sign[s];
      const float d = tb.decay[s];
      dtarget[s] = dI * (1.0f - d);
      io.lam_I[(b * S + s) * N + n] = dI * d;
      if (io.acc_decay)
        io.acc_decay[(b * S + s) * N + n] += dI * (io.I_saved[el * S + s] - io.target_saved[el * S + s]);
    }
    if (io.acc_beta) io.acc_beta[idx] += lv * (io.v_saved[el] - I_next_syn);
    for (int64_t k = 0; k < K; ++k) {
      float g = 0.0f;
      for (int64_t s = 0; s < S; ++s) g = g + dtarget[s] * tb.jump[(k * N + n) * S + s];
      io.grad_A[((k * B + b) * T_ + t) * N + n] = g;
      if (k < tb.K_rec)
        static_cast<T*>(io.gA_op)[(k * a.op.B_pad + b) * a.op.N_pad + n] = to_storage<T>(g);
      if (io.acc_scale) {
        float m = 0.0f;
        for (int64_t s = 0; s < S; ++s) m = m + dtarget[s] * tb.made[k * S + s];
        io.acc_scale[(k * B + b) * N + n] += m * io.A_saved[((k * B + b) * T_ + t) * N + n];
      }
    }
    lv = lv * beta;  // dL/dv_t before its rate's term
  }
  io.lam_v[idx] = lv;
}

// Reverse product of step t: d_rate[b, neuron of row j] = sum_n dL/da_k[b, n] W[j, n] for
// the recurrent rows j of pathway k (the rates' gradient through the recurrence). W's
// rows are k-contiguous along n: the tile product's second operand as it is.
template <typename T>
__global__ __launch_bounds__(kThreads) void rate_back_gemm_kernel(RateBackArgs a) {
  __shared__ StageLds lds;
  const wt_rate_operand& op = a.op;
  const wt_rate_back_io& io = a.io;
  const int64_t N = a.tab.N, B = io.B;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t j0 = (int64_t)blockIdx.x * kTile, b0 = (int64_t)blockIdx.y * kTile;
  // the recurrent segment holding rows [j0, j0 + 64): segments are whole tiles
  int64_t path = -1;
  for (int g = 0; g < op.n_seg; ++g)
    if (!op.seg[g][3] && j0 >= op.seg[g][0] && j0 < op.seg[g][1]) path = op.seg[g][2];
  if (path < 0) return;
  constexpr int kStageK = kStageBytes / (int)sizeof(T);
  const char* gA = reinterpret_cast<const char*>(static_cast<const T*>(io.gA_op) +
                                                 (path * op.B_pad + b0) * op.N_pad);
  const char* Wj = reinterpret_cast<const char*>(static_cast<const T*>(op.W) + j0 * op.N_pad);
  const int64_t ld = op.N_pad * (int64_t)sizeof(T);
  f32x16 c = {};
  tile_product<T>(
      lds, c, (int)(op.N_pad / kStageK),
      [&](int s, const char*& pa, int64_t& lda, const char*& pb, int64_t& ldb) {
        pa = gA + (int64_t)s * kStageBytes;
        pb = Wj + (int64_t)s * kStageBytes;
        lda = ldb = ld;
      },
      [](int, f32x16&) {});
  const int wi = wave >> 1, wj = wave & 1;
  const int64_t j = j0 + wj * 32 + (lane & 31);
  const int32_t neuron = op.src_of[j];
  if (neuron < 0) return;
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int64_t b = b0 + wi * 32 + out_row(v, lane);
    if (b < B) io.d_rate[b * N + neuron] = c[v];
  }
}

template <typename T>
static hipError_t forward_impl(const RateArgs& base, hipStream_t stream) {
  RateArgs a = base;
  const int64_t BN = a.io.B * a.tab.N;
  a.t = 0;
  hipLaunchKernelGGL(rate_init_kernel<T>, dim3((unsigned)((BN + kThreads - 1) / kThreads)),
                     dim3(kThreads), 0, stream, a);
  const dim3 grid((unsigned)(a.op.N_pad / kTile), (unsigned)(a.op.B_pad / kTile));
  void (*step)(RateArgs) = nullptr;
  switch (a.tab.S) {
    case 1: step = rate_step_kernel<T, 1>; break;
    case 2: step = rate_step_kernel<T, 2>; break;
    case 3: step = rate_step_kernel<T, 3>; break;
    case 4: step = rate_step_kernel<T, 4>; break;
    case 5: step = rate_step_kernel<T, 5>; break;
    case 6: step = rate_step_kernel<T, 6>; break;
    case 7: step = rate_step_kernel<T, 7>; break;
    case 8: step = rate_step_kernel<T, 8>; break;
    default: return hipErrorInvalidValue;
  }
  for (int64_t t = 0; t < a.io.T; ++t) {
    a.t = (int32_t)t;
    hipLaunchKernelGGL(step, grid, dim3(kThreads), 0, stream, a);
  }
  return hipGetLastError();
}

template <typename T>
static hipError_t backward_impl(const RateBackArgs& base, hipStream_t stream) {
  RateBackArgs a = base;
  const int64_t BN = a.io.B * a.tab.N;
  const dim3 egrid((unsigned)((BN + kThreads - 1) / kThreads));
  const dim3 ggrid((unsigned)(a.op.K_rec_pad / kTile), (unsigned)(a.op.B_pad / kTile));
  const bool rec = a.tab.K_rec > 0 && a.op.K_rec_pad > 0;
  for (int64_t t = a.io.T - 1; t >= -1; --t) {
    a.t = (int32_t)t;
    a.t_rate = t + 1 < a.io.T ? (int32_t)(t + 1) : -1;
    hipLaunchKernelGGL(rate_back_elem_kernel<T>, egrid, dim3(kThreads), 0, stream, a);
    if (t >= 0 && rec)
      hipLaunchKernelGGL(rate_back_gemm_kernel<T>, ggrid, dim3(kThreads), 0, stream, a);
  }
  return hipGetLastError();
}

static bool operand_ok(const wt_rate_tables* tb, const wt_rate_operand* op, int64_t B) {
  if (op->dtype != 0 && op->dtype != 1) return false;
  if (op->B_pad < B || op->B_pad % kTile || op->N_pad < tb->N || op->N_pad % kTile) return false;
  if (op->K_rec_pad % kTile || op->K_ff_pad % kTile || op->n_seg < 0 || op->n_seg > kMaxSeg)
    return false;
  int64_t end = 0;  // segments tile [0, K_rec_pad + K_ff_pad) in order
  for (int64_t g = 0; g < op->n_seg; ++g) {
    const int32_t* s = op->seg[g];
    if (s[0] != end) return false;
    end = s[1];
    const int64_t lo = s[3] ? op->K_rec_pad : 0, hi = s[3] ? op->K_rec_pad + op->K_ff_pad : op->K_rec_pad;
    if (s[0] < lo || s[1] > hi || s[0] >= s[1] || s[0] % kTile || s[1] % kTile) return false;
    if (s[2] < 0 || s[2] >= tb->K || (!s[3] && s[2] >= tb->K_rec)) return false;
  }
  if (end != op->K_rec_pad + op->K_ff_pad) return false;
  return op->W && op->Wt && (op->K_rec_pad == 0 || (op->rin && op->rpos));
}

}  // namespace rate
}  // namespace wt

using namespace wt::rate;

extern "C" int wt_rate_forward(const wt_rate_tables* tab, const wt_rate_operand* op,
                               const wt_rate_io* io, wt_stream_t stream) {
  if (!tab || !op || !io || !io->v || !io->I || !io->out) return hipErrorInvalidValue;
  if (tab->S < 1 || tab->S > kMaxS || tab->K < 0 || tab->K_rec < 0 || tab->K_rec > tab->K)
    return hipErrorInvalidValue;
  if (!operand_ok(tab, op, io->B)) return hipErrorInvalidValue;
  if (op->K_ff_pad > 0 && !op->X) return hipErrorInvalidValue;
  if ((io->track_v != nullptr) != (io->track_I != nullptr)) return hipErrorInvalidValue;
  if (io->B * tab->N == 0 || io->T == 0) return hipSuccess;
  RateArgs a = {};
  a.tab = *tab;
  a.op = *op;
  a.io = *io;
  return op->dtype == 1 ? forward_impl<__bf16>(a, (hipStream_t)stream)
                        : forward_impl<float>(a, (hipStream_t)stream);
}

extern "C" int wt_rate_backward(const wt_rate_tables* tab, const wt_rate_operand* op,
                                const wt_rate_back_io* io, wt_stream_t stream) {
  if (!tab || !op || !io || !io->grad_out || !io->v_saved || !io->lam_v || !io->lam_I ||
      !io->grad_A || !io->I_final)
    return hipErrorInvalidValue;
  if (tab->S < 1 || tab->S > kMaxS || tab->K < 0 || tab->K_rec < 0 || tab->K_rec > tab->K)
    return hipErrorInvalidValue;
  if (!operand_ok(tab, op, io->B)) return hipErrorInvalidValue;
  if (tab->K_rec > 0 && (!io->gA_op || !io->d_rate || !op->src_of)) return hipErrorInvalidValue;
  if ((io->acc_decay || io->acc_scale) && (!io->I_saved || !io->target_saved))
    return hipErrorInvalidValue;
  if (io->acc_scale && !io->A_saved) return hipErrorInvalidValue;
  if (io->acc_beta && io->T > 1 && !io->I_saved) return hipErrorInvalidValue;
  if (io->B * tab->N == 0 || io->T == 0) return hipSuccess;
  RateBackArgs a = {};
  a.tab = *tab;
  a.op = *op;
  a.io = *io;
  return op->dtype == 1 ? backward_impl<__bf16>(a, (hipStream_t)stream)
                        : backward_impl<float>(a, (hipStream_t)stream);
}
