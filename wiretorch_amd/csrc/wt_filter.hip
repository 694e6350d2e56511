// Causal double-exponential filter of spike trains along time, and its reverse.
//
// Forward (training_utils/filtering.py:103-123), per (trial b, neuron n) column:
//   r[t] = a_r * r[t-1] + x[t],  s[t] = a_d * s[t-1] + r[t],
// with r[-1], s[-1] the carried state, entering undecayed at t = 0: r[0] = r_c + x[0],
// s[0] = s_c + r[0]. Backward (filtering.py:125-135), in reverse time:
//   gs = g[t] + a_d * gs,  gr = gs + a_r * gr,  dL/dx[t] = gr.
// Every multiply and add is rounded separately (this file is built with
// -ffp-contract=off), so the result is reproducible bit for bit by a float32 recursion.
//
// Layout: x, rise, smooth, grad are (B, T, N) float32, contiguous; carried states (B, N).
// One lane per column, consecutive lanes on consecutive neurons, so each step's loads
// and stores of a wavefront are 256 contiguous bytes. The recursion is serial in t, so
// each lane loads a chunk of CH steps ahead of the arithmetic: CH independent loads in
// flight per lane hide HBM latency. The kernel is HBM-bound: 12 B per element forward
// (x read, rise and smooth written), 8 B backward.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/wiretorch_amd.h"

namespace wt {
namespace filter {

constexpr int BLOCK = 256;
constexpr int CH = 8;

__global__ __launch_bounds__(BLOCK) void forward_kernel(
    const float* __restrict__ x, const float* __restrict__ carried_rise,
    const float* __restrict__ carried_smooth, float* __restrict__ rise,
    float* __restrict__ smooth, float a_r, float a_d, uint32_t B, uint32_t T, uint32_t N) {
  const uint64_t col = (uint64_t)blockIdx.x * BLOCK + threadIdx.x;
  if (col >= (uint64_t)B * N) return;
  const uint32_t b = (uint32_t)(col / N), n = (uint32_t)(col - (uint64_t)b * N);
  const uint64_t base = (uint64_t)b * T * N + n;
  float r = carried_rise ? carried_rise[col] : 0.0f;
  float s = carried_smooth ? carried_smooth[col] : 0.0f;
  float ar = 1.0f, ad = 1.0f;  // t = 0: the carried state enters undecayed
  uint32_t t = 0;
  for (; t + CH <= T; t += CH) {
    float xs[CH];
#pragma unroll
    for (int k = 0; k < CH; ++k) xs[k] = x[base + (uint64_t)(t + k) * N];
#pragma unroll
    for (int k = 0; k < CH; ++k) {
      r = ar * r + xs[k];
      s = ad * s + r;
      ar = a_r;
      ad = a_d;
      const uint64_t at = base + (uint64_t)(t + k) * N;
      rise[at] = r;
      smooth[at] = s;
    }
  }
  for (; t < T; ++t) {
    const uint64_t at = base + (uint64_t)t * N;
    r = ar * r + x[at];
    s = ad * s + r;
    ar = a_r;
    ad = a_d;
    rise[at] = r;
    smooth[at] = s;
  }
}

__global__ __launch_bounds__(BLOCK) void backward_kernel(
    const float* __restrict__ grad_smooth, float* __restrict__ grad_x, float a_r, float a_d,
    uint32_t B, uint32_t T, uint32_t N) {
  const uint64_t col = (uint64_t)blockIdx.x * BLOCK + threadIdx.x;
  if (col >= (uint64_t)B * N) return;
  const uint32_t b = (uint32_t)(col / N), n = (uint32_t)(col - (uint64_t)b * N);
  const uint64_t base = (uint64_t)b * T * N + n;
  float gs = 0.0f, gr = 0.0f;
  uint32_t left = T;  // steps not yet done: T-1 .. 0 in order
  for (; left >= CH; left -= CH) {
    float gv[CH];
#pragma unroll
    for (int k = 0; k < CH; ++k) gv[k] = grad_smooth[base + (uint64_t)(left - 1 - k) * N];
#pragma unroll
    for (int k = 0; k < CH; ++k) {
      gs = gv[k] + a_d * gs;
      gr = gs + a_r * gr;
      grad_x[base + (uint64_t)(left - 1 - k) * N] = gr;
    }
  }
  for (; left > 0; --left) {
    const uint64_t at = base + (uint64_t)(left - 1) * N;
    gs = grad_smooth[at] + a_d * gs;
    gr = gs + a_r * gr;
    grad_x[at] = gr;
  }
}

static bool sizes_ok(int64_t B, int64_t T, int64_t N) {
  // 32-bit B, T, N; the flat element index stays in 64 bits
  return B >= 0 && T >= 0 && N >= 0 && B <= UINT32_MAX && T <= UINT32_MAX && N <= UINT32_MAX &&
         B * N <= (int64_t)UINT32_MAX * BLOCK;
}

}  // namespace filter
}  // namespace wt

extern "C" int wt_filter_forward(const float* x, const float* carried_rise,
                                 const float* carried_smooth, float* rise, float* smooth,
                                 float a_rise, float a_decay, int64_t B, int64_t T, int64_t N,
                                 wt_stream_t stream) {
  if (!wt::filter::sizes_ok(B, T, N)) return hipErrorInvalidValue;
  if (B * T * N == 0) return hipSuccess;
  if (!x || !rise || !smooth) return hipErrorInvalidValue;
  const int64_t cols = B * N;
  hipLaunchKernelGGL(wt::filter::forward_kernel,
                     dim3((unsigned)((cols + wt::filter::BLOCK - 1) / wt::filter::BLOCK)),
                     dim3(wt::filter::BLOCK), 0, (hipStream_t)stream, x, carried_rise,
                     carried_smooth, rise, smooth, a_rise, a_decay, (uint32_t)B, (uint32_t)T,
                     (uint32_t)N);
  return hipGetLastError();
}

extern "C" int wt_filter_backward(const float* grad_smooth, float* grad_x, float a_rise,
                                  float a_decay, int64_t B, int64_t T, int64_t N,
                                  wt_stream_t stream) {
  if (!wt::filter::sizes_ok(B, T, N)) return hipErrorInvalidValue;
  if (B * T * N == 0) return hipSuccess;
  if (!grad_smooth || !grad_x) return hipErrorInvalidValue;
  const int64_t cols = B * N;
  hipLaunchKernelGGL(wt::filter::backward_kernel,
                     dim3((unsigned)((cols + wt::filter::BLOCK - 1) / wt::filter::BLOCK)),
                     dim3(wt::filter::BLOCK), 0, (hipStream_t)stream, grad_smooth, grad_x,
                     a_rise, a_decay, (uint32_t)B, (uint32_t)T, (uint32_t)N);
  return hipGetLastError();
}
