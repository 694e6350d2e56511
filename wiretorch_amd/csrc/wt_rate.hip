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

constexpr int kTile = 64;     // outputs per workgroup, per side
constexpr int kKB = 32;       // k per LDS stage
constexpr int kPad = 8;       // LDS row padding (elements)
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

template <typename T>
struct Mma;
template <>
struct Mma<float> {  // C[32x32] += A[32x2] B[2x32]: lane l holds A[l%32][l/32], B[l/32][l%32]
  static constexpr int kStep = 2;
  __device__ static void run(f32x16& c, const float* a_row, const float* b_col, int lane) {
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(a_row[lane >> 5], b_col[lane >> 5], c, 0, 0, 0);
  }
};
template <>
struct Mma<__bf16> {  // C += A[32x16] B[16x32]: lane l holds A[l%32][8(l/32)+e], B[8(l/32)+e][l%32]
  static constexpr int kStep = 16;
  __device__ static void run(f32x16& c, const __bf16* a_row, const __bf16* b_col, int lane) {
    const bf16x8 a = *reinterpret_cast<const bf16x8*>(a_row + 8 * (lane >> 5));
    const bf16x8 b = *reinterpret_cast<const bf16x8*>(b_col + 8 * (lane >> 5));
    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};

// Output element v of a lane's 32 x 32 block: row 8(v/4) + 4(l/32) + v%4, column l%32.
__device__ inline int out_row(int v, int lane) { return 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3); }

// One k-block of a 64 x 64 tile: A rows [0, 64) x k [kA, kA + 32) (row-major, lda), and
// B either as [k][j] (row-major, ldb; B_ROWS_ARE_K) or as [j][k], from k = kB. Staged in
// LDS as sA[i][k] and sB[j][k], then each wave multiplies its 32 x 32 block.
template <typename T, bool B_ROWS_ARE_K>
__device__ inline void kblock(f32x16& c, T (*sA)[kKB + kPad], T (*sB)[kKB + kPad], const T* A,
                              int64_t lda, int64_t kA, const T* Bm, int64_t ldb, int64_t kB,
                              int wave, int lane) {
  const int tid = threadIdx.x;
  for (int e = tid; e < kTile * kKB; e += kThreads) {
    const int i = e / kKB, kk = e % kKB;
    sA[i][kk] = A[(int64_t)i * lda + kA + kk];
  }
  if (B_ROWS_ARE_K) {
    for (int e = tid; e < kTile * kKB; e += kThreads) {
      const int kk = e / kTile, j = e % kTile;
      sB[j][kk] = Bm[(kB + kk) * ldb + j];
    }
  } else {
    for (int e = tid; e < kTile * kKB; e += kThreads) {
      const int j = e / kKB, kk = e % kKB;
      sB[j][kk] = Bm[(int64_t)j * ldb + kB + kk];
    }
  }
  __syncthreads();
  const int wi = wave >> 1, wj = wave & 1;
  const T* a_row = &sA[wi * 32 + (lane & 31)][0];
  const T* b_col = &sB[wj * 32 + (lane & 31)][0];
#pragma unroll
  for (int ks = 0; ks < kKB; ks += Mma<T>::kStep) Mma<T>::run(c, a_row + ks, b_col + ks, lane);
  __syncthreads();
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
  __shared__ __align__(16) T sA[kTile][kKB + kPad];
  __shared__ __align__(16) T sB[kTile][kKB + kPad];
  const wt_rate_tables& tb = a.tab;
  const wt_rate_operand& op = a.op;
  const wt_rate_io& io = a.io;
  const int64_t N = tb.N, B = io.B, T_ = io.T, t = a.t;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t n0 = (int64_t)blockIdx.x * kTile, b0 = (int64_t)blockIdx.y * kTile;
  const T* rin = static_cast<const T*>(op.rin) + (t & 1) * op.B_pad * op.K_rec_pad;
  const T* X = static_cast<const T*>(op.X) + t * op.B_pad * op.K_ff_pad;
  const T* W = static_cast<const T*>(op.W);

  float target[16][S];
#pragma unroll
  for (int v = 0; v < 16; ++v)
#pragma unroll
    for (int s = 0; s < S; ++s) target[v][s] = 0.0f;
  const int wi = wave >> 1, wj = wave & 1;
  const int64_t n = n0 + wj * 32 + (lane & 31);

  for (int g = 0; g < op.n_seg; ++g) {
    const int64_t k0 = op.seg[g][0], k1 = op.seg[g][1], path = op.seg[g][2];
    const bool input = op.seg[g][3] != 0;
    f32x16 c = {};
    for (int64_t k = k0; k < k1; k += kKB) {  // W rows are absolute; the operands' k is not
      if (input)
        kblock<T, true>(c, sA, sB, X + b0 * op.K_ff_pad, op.K_ff_pad, k - op.K_rec_pad,
                        W + n0, op.N_pad, k, wave, lane);
      else
        kblock<T, true>(c, sA, sB, rin + b0 * op.K_rec_pad, op.K_rec_pad, k, W + n0, op.N_pad, k,
                        wave, lane);
    }
    if (n < N) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t b = b0 + wi * 32 + out_row(v, lane);
        if (b >= B) continue;
        if (io.A_saved) io.A_saved[((path * B + b) * T_ + t) * N + n] = c[v];
#pragma unroll
        for (int s = 0; s < S; ++s)
          target[v][s] = target[v][s] + c[v] * tb.jump[(path * N + n) * S + s];
      }
    }
  }
  if (n >= N) return;
  const float beta = tb.beta[n], theta = tb.theta[n], gain = tb.gain[n];
  const int code = tb.nonlinearity[n];
  const int32_t pos = op.rpos ? op.rpos[n] : -1;
  T* rin_next = static_cast<T*>(op.rin) + ((t + 1) & 1) * op.B_pad * op.K_rec_pad;
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
      const float d = tb.decay[s];
      I[s] = d * io.I[(b * S + s) * N + n] + (1.0f - d) * target[v][s];
      io.I[(b * S + s) * N + n] = I[s];
      I_syn = I_syn + I[s] * tb.sign[s];
    }
    const float vv = beta * io.v[b * N + n] + (1.0f - beta) * I_syn;
    io.v[b * N + n] = vv;
    if (io.track_v && (io.track_b < 0 || io.track_b == b)) {
      const int64_t row = ((io.track_b < 0 ? b : 0) * T_ + t) * N + n;
      io.track_v[row] = vv;
#pragma unroll
      for (int s = 0; s < S; ++s) io.track_I[row * S + s] = I[s];
    }
    if (t + 1 < T_) {
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
// the recurrent rows j of pathway k (the rates' gradient through the recurrence).
template <typename T>
__global__ __launch_bounds__(kThreads) void rate_back_gemm_kernel(RateBackArgs a) {
  __shared__ __align__(16) T sA[kTile][kKB + kPad];
  __shared__ __align__(16) T sB[kTile][kKB + kPad];
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
  const T* gA = static_cast<const T*>(io.gA_op) + (path * op.B_pad + b0) * op.N_pad;
  const T* W = static_cast<const T*>(op.W) + j0 * op.N_pad;
  f32x16 c = {};
  for (int64_t k = 0; k < op.N_pad; k += kKB)
    kblock<T, false>(c, sA, sB, gA, op.N_pad, k, W, op.N_pad, k, wave, lane);
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
  for (int64_t g = 0; g < op->n_seg; ++g) {
    const int32_t* s = op->seg[g];
    const int64_t lo = s[3] ? op->K_rec_pad : 0, hi = s[3] ? op->K_rec_pad + op->K_ff_pad : op->K_rec_pad;
    if (s[0] < lo || s[1] > hi || s[0] >= s[1] || s[0] % kTile || s[1] % kTile) return false;
    if (s[2] < 0 || s[2] >= tb->K || (!s[3] && s[2] >= tb->K_rec)) return false;
  }
  return op->W && (op->K_rec_pad == 0 || (op->rin && op->rpos));
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
