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
// One lane per column (or per 4 consecutive columns), consecutive lanes on consecutive
// neurons, so each step's loads and stores of a wavefront are contiguous. The recursion
// is serial in t, so each lane loads a chunk of CH steps ahead of the arithmetic: CH
// independent loads in flight per lane hide HBM latency. The kernel is HBM-bound: 12 B per element forward
// (x read, rise and smooth written), 8 B backward.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <initializer_list>

#include "../../include/wiretorch_amd.h"

namespace wt {
namespace filter {

constexpr int BLOCK = 256;
constexpr int CH = 8;

// V consecutive neurons per lane (V = 4 when N is a multiple of 4 and the arrays are
// 16-byte aligned: 16-byte accesses, and a quarter of the lanes, so that config 3's
// 640k columns fit the chip's resident waves in one pass instead of 1.2).
template <int V> struct Lanes;
template <> struct Lanes<1> { using T = float; };
template <> struct Lanes<4> { using T = float4; };

template <int V>
__device__ inline float& at(typename Lanes<V>::T& v, int i) {
  return reinterpret_cast<float*>(&v)[i];
}

template <int V>
__global__ __launch_bounds__(BLOCK) void forward_kernel(
    const float* __restrict__ x, const float* __restrict__ carried_rise,
    const float* __restrict__ carried_smooth, float* __restrict__ rise,
    float* __restrict__ smooth, float a_r, float a_d, uint32_t B, uint32_t T, uint32_t N) {
  using L = typename Lanes<V>::T;
  const uint32_t NV = N / V;  // lanes per trial
  const uint64_t col = (uint64_t)blockIdx.x * BLOCK + threadIdx.x;
  if (col >= (uint64_t)B * NV) return;
  const uint32_t b = (uint32_t)(col / NV), n = (uint32_t)(col - (uint64_t)b * NV);
  const uint64_t base = (uint64_t)b * T * NV + n;  // in units of L
  const L* xv = reinterpret_cast<const L*>(x);
  L* rv = reinterpret_cast<L*>(rise);
  L* sv = reinterpret_cast<L*>(smooth);
  L r, s;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    at<V>(r, i) = carried_rise ? carried_rise[col * V + i] : 0.0f;
    at<V>(s, i) = carried_smooth ? carried_smooth[col * V + i] : 0.0f;
  }
  float ar = 1.0f, ad = 1.0f;  // t = 0: the carried state enters undecayed
  uint32_t t = 0;
  for (; t + CH <= T; t += CH) {
    L xs[CH];
#pragma unroll
    for (int k = 0; k < CH; ++k) xs[k] = xv[base + (uint64_t)(t + k) * NV];
#pragma unroll
    for (int k = 0; k < CH; ++k) {
#pragma unroll
      for (int i = 0; i < V; ++i) {
        at<V>(r, i) = ar * at<V>(r, i) + at<V>(xs[k], i);
        at<V>(s, i) = ad * at<V>(s, i) + at<V>(r, i);
      }
      ar = a_r;
      ad = a_d;
      const uint64_t o = base + (uint64_t)(t + k) * NV;
      rv[o] = r;
      sv[o] = s;
    }
  }
  for (; t < T; ++t) {
    const uint64_t o = base + (uint64_t)t * NV;
    L xt = xv[o];
#pragma unroll
    for (int i = 0; i < V; ++i) {
      at<V>(r, i) = ar * at<V>(r, i) + at<V>(xt, i);
      at<V>(s, i) = ad * at<V>(s, i) + at<V>(r, i);
    }
    ar = a_r;
    ad = a_d;
    rv[o] = r;
    sv[o] = s;
  }
}

template <int V>
__global__ __launch_bounds__(BLOCK) void backward_kernel(
    const float* __restrict__ grad_smooth, float* __restrict__ grad_x, float a_r, float a_d,
    uint32_t B, uint32_t T, uint32_t N) {
  using L = typename Lanes<V>::T;
  const uint32_t NV = N / V;
  const uint64_t col = (uint64_t)blockIdx.x * BLOCK + threadIdx.x;
  if (col >= (uint64_t)B * NV) return;
  const uint32_t b = (uint32_t)(col / NV), n = (uint32_t)(col - (uint64_t)b * NV);
  const uint64_t base = (uint64_t)b * T * NV + n;
  const L* gv = reinterpret_cast<const L*>(grad_smooth);
  L* ov = reinterpret_cast<L*>(grad_x);
  L gs, gr;
#pragma unroll
  for (int i = 0; i < V; ++i) at<V>(gs, i) = at<V>(gr, i) = 0.0f;
  uint32_t left = T;  // steps not yet done: T-1 .. 0 in order
  for (; left >= CH; left -= CH) {
    L g[CH];
#pragma unroll
    for (int k = 0; k < CH; ++k) g[k] = gv[base + (uint64_t)(left - 1 - k) * NV];
#pragma unroll
    for (int k = 0; k < CH; ++k) {
#pragma unroll
      for (int i = 0; i < V; ++i) {
        at<V>(gs, i) = at<V>(g[k], i) + a_d * at<V>(gs, i);
        at<V>(gr, i) = at<V>(gs, i) + a_r * at<V>(gr, i);
      }
      ov[base + (uint64_t)(left - 1 - k) * NV] = gr;
    }
  }
  for (; left > 0; --left) {
    const uint64_t o = base + (uint64_t)(left - 1) * NV;
    L g = gv[o];
#pragma unroll
    for (int i = 0; i < V; ++i) {
      at<V>(gs, i) = at<V>(g, i) + a_d * at<V>(gs, i);
      at<V>(gr, i) = at<V>(gs, i) + a_r * at<V>(gr, i);
    }
    ov[o] = gr;
  }
}

static bool wide(int64_t N, std::initializer_list<const void*> ptrs) {
  if (N % 4) return false;
  for (const void* p : ptrs)
    if ((uintptr_t)p & 15) return false;
  return true;
}

static bool sizes_ok(int64_t B, int64_t T, int64_t N) {
  // 32-bit B, T, N; the flat element index stays in 64 bits. The forward's chunked loop
  // tests t + CH <= T in 32 bits, so T stays CH below the 32-bit limit (no wrap-around).
  return B >= 0 && T >= 0 && N >= 0 && B <= UINT32_MAX && T <= (int64_t)UINT32_MAX - CH &&
         N <= UINT32_MAX && B * N <= (int64_t)UINT32_MAX * BLOCK;
}

}  // namespace filter
}  // namespace wt

extern "C" int wt_filter_forward(const float* x, const float* carried_rise,
                                 const float* carried_smooth, float* rise, float* smooth,
                                 float a_rise, float a_decay, int64_t B, int64_t T, int64_t N,
                                 wt_stream_t stream) {
  if (!wt::filter::sizes_ok(B, T, N)) return hipErrorInvalidValue;
  if (B == 0 || T == 0 || N == 0) return hipSuccess;
  if (!x || !rise || !smooth) return hipErrorInvalidValue;
  const bool v4 = wt::filter::wide(N, {x, rise, smooth, carried_rise, carried_smooth});
  const int64_t cols = B * N / (v4 ? 4 : 1);
  const dim3 grid((unsigned)((cols + wt::filter::BLOCK - 1) / wt::filter::BLOCK));
  if (v4)
    hipLaunchKernelGGL(wt::filter::forward_kernel<4>, grid, dim3(wt::filter::BLOCK), 0,
                       (hipStream_t)stream, x, carried_rise, carried_smooth, rise, smooth,
                       a_rise, a_decay, (uint32_t)B, (uint32_t)T, (uint32_t)N);
  else
    hipLaunchKernelGGL(wt::filter::forward_kernel<1>, grid, dim3(wt::filter::BLOCK), 0,
                       (hipStream_t)stream, x, carried_rise, carried_smooth, rise, smooth,
                       a_rise, a_decay, (uint32_t)B, (uint32_t)T, (uint32_t)N);
  return hipGetLastError();
}

extern "C" int wt_filter_backward(const float* grad_smooth, float* grad_x, float a_rise,
                                  float a_decay, int64_t B, int64_t T, int64_t N,
                                  wt_stream_t stream) {
  if (!wt::filter::sizes_ok(B, T, N)) return hipErrorInvalidValue;
  if (B == 0 || T == 0 || N == 0) return hipSuccess;
  if (!grad_smooth || !grad_x) return hipErrorInvalidValue;
  const bool v4 = wt::filter::wide(N, {grad_smooth, grad_x});
  const int64_t cols = B * N / (v4 ? 4 : 1);
  const dim3 grid((unsigned)((cols + wt::filter::BLOCK - 1) / wt::filter::BLOCK));
  if (v4)
    hipLaunchKernelGGL(wt::filter::backward_kernel<4>, grid, dim3(wt::filter::BLOCK), 0,
                       (hipStream_t)stream, grad_smooth, grad_x, a_rise, a_decay,
                       (uint32_t)B, (uint32_t)T, (uint32_t)N);
  else
    hipLaunchKernelGGL(wt::filter::backward_kernel<1>, grid, dim3(wt::filter::BLOCK), 0,
                       (hipStream_t)stream, grad_smooth, grad_x, a_rise, a_decay,
                       (uint32_t)B, (uint32_t)T, (uint32_t)N);
  return hipGetLastError();
}
