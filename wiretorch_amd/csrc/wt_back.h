// wt_back.h — the surrogate-gradient backward of the conductance-LIF scan: the reverse
// step shared by two drivers, instantiated per synapse count S in wt_run_s<S>.hip.
//
//  * BackLaunch<S>::run (wt_cond_scan_backward): one thread per (trial, neuron) runs all
//    T steps in reverse with its adjoint state in registers. The recurrent activations
//    are treated as inputs (gradients do not flow back through the recurrent spikes).
//  * BackLaunch<S>::recurrent (wt_cond_recurrent_backward): gradients also flow through
//    the recurrent spikes (the reference's recurrent_gradients=True). Every step couples
//    all neurons: dL/ds_j(t) gains R_j = sum over j's synapses e of w_e dL/da(t)[target e].
//    Each step is then two launches, with the adjoint state in global memory between
//    them: (1) every neuron's adjoint through the membrane and the conductances, which
//    gives dL/da(t); (2) per source, R gathered along its synapses (CSR by source, a
//    fixed order: deterministic) and the surrogate spike term.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/wiretorch_amd.h"
#include "wt_math.h"

namespace wt {

struct BackArgs {
  wt_tables tab;
  wt_backward_io io;
  wt_side rec;      // recurrent side (recurrent path only)
  float* state;     // adjoint state, [back_fields<S>()][B * N] (recurrent path only)
  float* grad_now;  // dL/da of the current step, [K_rec][N][B] (recurrent path only)
  float* R;         // the recurrent term of the current step, [N][B] (recurrent path only)
};

// The adjoint state of one (trial, neuron) between reverse steps.
template <int S>
struct BackState {
  float dv;                          // dL/dv entering the step after
  float lr[S], ld[S];                // dL/dg (rise, decay) entering the step after
  float Hr[S], Hd[S];                // decay-gradient recursions
  float accE[S], accDr[S], accDd[S], accJr[S], accJd[S];
  float acc_scale[WT_MAX_K];
  float acc_theta, acc_reset, acc_EL, acc_Cm, acc_beta;
  float la;                          // dL/dg_a (adaptation) entering the step after
  float acc_adapt, acc_adecay, acc_Ea;
};
template <int S>
constexpr int back_fields() { return 1 + 9 * S + WT_MAX_K + 5 + 4; }

// Global layout of the recurrent path's state: field f of item idx at f * BN + idx. A
// field that feeds no wanted gradient is neither read (it reads as zero) nor written:
// the decay recursions and partials only with grad_decay, and so on; the adaptation's
// only with AD (the network adapts).
template <int S, bool AD>
__device__ inline void state_io(BackState<S>& st, float* base, int64_t BN, int64_t idx,
                                bool store, const wt_backward_io& io, int64_t K) {
  float* p = base + idx;
  auto y = [&](bool want, float& v) {
    if (want) {
      if (store) *p = v; else v = *p;
    } else if (!store) {
      v = 0.0f;
    }
    p += BN;
  };
  const bool decay = io.grad_decay != nullptr, jump = io.grad_jump != nullptr;
  const bool esyn = io.grad_E_syn != nullptr, scale = io.grad_scale != nullptr;
  y(true, st.dv);
#pragma unroll
  for (int s = 0; s < S; ++s) {
    y(true, st.lr[s]); y(true, st.ld[s]); y(decay, st.Hr[s]); y(decay, st.Hd[s]);
    y(esyn, st.accE[s]); y(decay, st.accDr[s]); y(decay, st.accDd[s]);
    y(jump, st.accJr[s]); y(jump, st.accJd[s]);
  }
#pragma unroll
  for (int k = 0; k < WT_MAX_K; ++k) y(scale && k < K, st.acc_scale[k]);
  y(io.grad_theta != nullptr, st.acc_theta); y(io.grad_reset != nullptr, st.acc_reset);
  y(io.grad_E_L != nullptr, st.acc_EL); y(io.grad_C_m != nullptr, st.acc_Cm);
  y(io.grad_beta != nullptr, st.acc_beta);
  // the adaptation's adjoint feeds only the gradients of its rise and decay
  y(AD && (io.grad_adapt != nullptr || io.grad_adapt_decay != nullptr), st.la);
  y(AD && io.grad_adapt != nullptr, st.acc_adapt);
  y(AD && io.grad_adapt_decay != nullptr, st.acc_adecay);
  y(AD && io.grad_E_adapt != nullptr, st.acc_Ea);
}

template <int S>
__device__ inline void state_zero(BackState<S>& st) {
  st.dv = 0.0f;
#pragma unroll
  for (int s = 0; s < S; ++s)
    st.lr[s] = st.ld[s] = st.Hr[s] = st.Hd[s] = st.accE[s] = st.accDr[s] = st.accDd[s] =
        st.accJr[s] = st.accJd[s] = 0.0f;
#pragma unroll
  for (int k = 0; k < WT_MAX_K; ++k) st.acc_scale[k] = 0.0f;
  st.acc_theta = st.acc_reset = st.acc_EL = st.acc_Cm = st.acc_beta = 0.0f;
  st.la = st.acc_adapt = st.acc_adecay = st.acc_Ea = 0.0f;
}

// One neuron's constants of the backward.
struct BackNeuron {
  float theta, E_L, C_m, beta, dt, k_surr;
  Leak lk;
  float a_decay, E_a;  // adaptation (0 without)
  // bit k * S + s: pathway k makes synapse type s (tab.made), read once here: loads of
  // the table between the reverse steps' stores would each wait for all of the thread's
  // outstanding memory operations (the compiler cannot rule out that a store aliases it)
  uint64_t made;
};

// tab.made[k * S + s] (0 or 1) from the mask.
__device__ inline float made_at(uint64_t made, int bit) {
  return ((made >> bit) & 1ull) ? 1.0f : 0.0f;
}

// AD: the network adapts (tab.adapt set). The backward kernels are compiled with and
// without it, so that a network without adaptation carries none of its registers.
template <bool AD>
__device__ inline BackNeuron back_neuron(const wt_tables& tab, int64_t n) {
  BackNeuron c;
  c.theta = tab.theta[n];
  c.E_L = tab.E_L[n];
  c.C_m = tab.C_m[n];
  c.beta = tab.beta[n];
  c.dt = *tab.dt;
  c.k_surr = *tab.surr;
  c.lk = leak(c.C_m, c.beta, c.dt);
  c.a_decay = AD ? tab.adapt_decay[n] : 0.0f;
  c.E_a = AD ? tab.E_adapt[n] : 0.0f;
  c.made = 0;
  for (int64_t i = 0; i < tab.K * tab.S; ++i)
    if (tab.made[i] != 0.0f) c.made |= 1ull << i;
  return c;
}

// One reverse step's inputs at (b, t, n): what the forward saved of step t and the
// spike's gradient. The reverse loop loads them a step ahead, so that their latency
// passes during the step before.
constexpr int kPreK = 4;  // pathways whose activations are loaded ahead (the rest in step)
constexpr int kBackBlock = 256;  // threads (items) of a scan backward workgroup

template <int S>
struct StepIn {
  float v, spike, held, grad_spike, grad_prob;
  float ga;  // the adaptation conductance entering the step (0 without)
  float G[S];
  float A[kPreK];  // the injected activations (when their partials are wanted)
};

template <int S, bool AD>
__device__ inline void load_step(StepIn<S>& in, const BackArgs& P, int64_t b, int64_t n,
                                 int64_t t) {
  const wt_tables& tab = P.tab;
  const wt_backward_io& io = P.io;
  const int64_t N = tab.N, K = tab.K, B = io.B, T = io.T;
  const int64_t out = (b * T + t) * N + n;
  in.v = io.v_saved[out];
  in.spike = io.spikes[out];
  in.held = io.held ? (float)io.held[out] : 0.0f;
  in.grad_spike = io.grad_spikes[out];
  in.grad_prob = io.grad_prob ? io.grad_prob[out] : 0.0f;
  in.ga = AD ? io.a_saved[out] : 0.0f;
#pragma unroll
  for (int s = 0; s < S; ++s) in.G[s] = io.G_saved[out * S + s];
  const bool want_A = io.grad_decay || io.grad_jump || io.grad_scale;
#pragma unroll
  for (int k = 0; k < kPreK; ++k)
    in.A[k] = want_A && k < K ? io.A[((k * B + b) * T + t) * N + n] : 0.0f;
}

// Activation k of the step at (b, t, n): loaded ahead for the first kPreK pathways.
template <int S>
__device__ inline float step_A(const StepIn<S>& in, const BackArgs& P, int k, int64_t b,
                               int64_t n, int64_t t) {
  if (k < kPreK) return in.A[k];
  return P.io.A[((k * P.io.B + b) * P.io.T + t) * P.tab.N + n];
}

// Reverse step t, all but the spike of step t: the injections of step t (dL/da_k, the
// jump and decay partials), the membrane update, and the conductances decaying into
// step t+1. Leaves st.dv = dL/dv_t without the spike's term. When ga_rec is given,
// dL/da_k of the recurrent pathways (k < K_rec) is also left there.
template <int S, bool AD>
__device__ inline void back_membrane_step(BackState<S>& st, const BackArgs& P,
                                          const Synapses<S>& syn, const BackNeuron& c,
                                          int64_t b, int64_t n, int64_t t,
                                          const StepIn<S>& in, const float (&scale)[WT_MAX_K],
                                          float* ga_rec = nullptr, float* ga_stage = nullptr,
                                          int stage_stride = 0) {
  const wt_tables& tab = P.tab;
  const wt_backward_io& io = P.io;
  const int64_t N = tab.N, K = tab.K, B = io.B, T = io.T;
  const bool refractory = io.held != nullptr;
  const bool want_A = io.grad_A != nullptr, want_scale = io.grad_scale != nullptr;
  const bool want_decay = io.grad_decay != nullptr, want_jump = io.grad_jump != nullptr;
  const float v = in.v;
  const float s_sp = in.spike;
  const float held = in.held;
  const float r = refractory ? fmaxf(s_sp, held) : s_sp;
  float G[S];
#pragma unroll
  for (int s = 0; s < S; ++s) G[s] = in.G[s];

  // Injections of step t: per unit jump, sum_k a_k scale_k made_k (jump, decay).
  if (want_decay || want_jump) {
    float base[S];
#pragma unroll
    for (int s = 0; s < S; ++s) base[s] = 0.0f;
#pragma unroll
    for (int k = 0; k < WT_MAX_K; ++k) {
      if (k >= K) break;
      const float as = step_A<S>(in, P, k, b, n, t) * scale[k];
#pragma unroll
      for (int s = 0; s < S; ++s) base[s] += as * made_at(c.made, k * S + s);
    }
#pragma unroll
    for (int s = 0; s < S; ++s) {
      if (want_jump) {
        st.accJr[s] += st.lr[s] * base[s];
        st.accJd[s] += st.ld[s] * base[s];
      }
      if (want_decay) {
        st.accDr[s] += syn.jump_r[s] * base[s] * st.Hr[s];
        st.accDd[s] += syn.jump_d[s] * base[s] * st.Hd[s];
        st.Hr[s] = st.lr[s] + syn.decay_r[s] * st.Hr[s];
        st.Hd[s] = st.ld[s] + syn.decay_d[s] * st.Hd[s];
      }
    }
  }
  // dL/da_k of step t: the adjoint of the conductances it was injected into.
#pragma unroll
  for (int k = 0; k < WT_MAX_K; ++k) {
    if (k >= K) break;
    float qk = 0.0f;
#pragma unroll
    for (int s = 0; s < S; ++s)
      qk += (syn.jump_r[s] * st.lr[s] + syn.jump_d[s] * st.ld[s]) * made_at(c.made, k * S + s);
    const int64_t ka = ((k * B + b) * T + t) * N + n;
    const float ga = qk * scale[k];
    if (want_A) io.grad_A[ka] = ga;
    if (ga_rec && k < tab.K_rec) ga_rec[k] = ga;
    if (ga_stage) ga_stage[k * stage_stride] = ga;
    if (want_scale) st.acc_scale[k] += qk * step_A<S>(in, P, k, b, n, t);
  }
  // The adaptation after step t, g_a(t) adapt_decay + adapt s_t: st.la is its adjoint
  // (conductance/kernels.py:498-504).
  constexpr bool adapting = AD;
  if (adapting) {
    if (io.grad_adapt) st.acc_adapt += st.la * s_sp;
    if (io.grad_adapt_decay) st.acc_adecay += st.la * in.ga;
  }
  // Membrane.
  const float gx = st.dv * (1.0f - r);
  float dG[S], Gc[S];
  const MembraneAdjoint m = membrane_adjoint<S>(gx, v, G, syn, c.E_L, c.C_m, c.lk, c.dt, dG,
                                                Gc, adapting, in.ga, c.E_a);
  if (adapting) {
    if (io.grad_E_adapt) st.acc_Ea += gx * m.phi * in.ga;
    st.la = st.la * c.a_decay + m.d_ga;
  }
  st.acc_reset += st.dv * r;
  st.acc_EL += gx * m.phi * c.lk.g_L;
  if (io.grad_C_m || io.grad_beta) {
    const float g_v = v - c.E_L;
    if (io.grad_C_m) {  // g_L = C rate and a both depend on C
      const float inv_C = 1.0f / c.C_m;
      const float dphi =
          -(m.a * c.dt * m.Gt * inv_C * inv_C + m.phi * c.lk.g_L * inv_C) * m.inv_g;
      st.acc_Cm -= gx * (dphi * m.J + m.phi * g_v * c.lk.g_L * inv_C);
    }
    if (io.grad_beta) {  // rate = -log(beta) / dt
      const float dg_L = -c.C_m / (c.beta * c.dt);
      const float dphi = -(m.a / c.beta + m.phi * dg_L) * m.inv_g;
      st.acc_beta -= gx * (dphi * m.J + m.phi * g_v * dg_L);
    }
  }
  if (io.grad_E_syn) {
#pragma unroll
    for (int s = 0; s < S; ++s) st.accE[s] += gx * m.phi * Gc[s];
  }
  st.dv = m.dv;
  // Conductances decay into step t+1 and feed the currents of step t.
#pragma unroll
  for (int s = 0; s < S; ++s) {
    st.lr[s] = st.lr[s] * syn.decay_r[s] + dG[s];
    st.ld[s] = st.ld[s] * syn.decay_d[s] + dG[s];
  }
}

// The spike (and probability) of step t, both functions of v - theta; `carried` is
// dL/ds_t through the recurrent synapses (0 when gradients do not flow there).
template <int S>
__device__ inline void back_spike_step(BackState<S>& st, const BackArgs& P,
                                       const BackNeuron& c, float carried,
                                       const StepIn<S>& in) {
  const wt_backward_io& io = P.io;
  const float x = in.v - c.theta;
  float g_x = surrogate(x, in.grad_spike + carried, c.k_surr);
  if (io.grad_prob) {
    const float p = 1.0f / (1.0f + expf(-(c.k_surr * x)));
    g_x += in.grad_prob * c.k_surr * p * (1.0f - p);
  }
  if (io.held) g_x *= 1.0f - in.held;
  st.dv += g_x;
  st.acc_theta -= g_x;
}

// The accumulated partials of one (trial, neuron), written once after step 0.
template <int S>
__device__ inline void back_finish(const BackState<S>& st, const BackArgs& P, int64_t b,
                                   int64_t n) {
  const wt_tables& tab = P.tab;
  const wt_backward_io& io = P.io;
  const int64_t N = tab.N, K = tab.K, B = io.B;
  const int64_t idx = b * N + n;
  if (io.grad_scale) {
#pragma unroll
    for (int k = 0; k < WT_MAX_K; ++k)
      if (k < K) io.grad_scale[k * B * N + idx] = st.acc_scale[k];
  }
  if (io.grad_theta) io.grad_theta[idx] = st.acc_theta;
  if (io.grad_reset) io.grad_reset[idx] = st.acc_reset;
  if (io.grad_E_L) io.grad_E_L[idx] = st.acc_EL;
  if (io.grad_C_m) io.grad_C_m[idx] = st.acc_Cm;
  if (io.grad_beta) io.grad_beta[idx] = st.acc_beta;
  if (io.grad_adapt) io.grad_adapt[idx] = st.acc_adapt;
  if (io.grad_adapt_decay) io.grad_adapt_decay[idx] = st.acc_adecay;
  if (io.grad_E_adapt) io.grad_E_adapt[idx] = st.acc_Ea;
#pragma unroll
  for (int s = 0; s < S; ++s) {
    if (io.grad_E_syn) io.grad_E_syn[(b * S + s) * N + n] = st.accE[s];
    if (io.grad_jump) {
      io.grad_jump[(b * 2 * S + s) * N + n] = st.accJr[s];
      io.grad_jump[(b * 2 * S + S + s) * N + n] = st.accJd[s];
    }
    if (io.grad_decay) {  // the conductances entering the chunk
      const float gr0 = io.g_init[(b * 2 * S + s) * N + n];
      const float gd0 = io.g_init[(b * 2 * S + S + s) * N + n];
      io.grad_decay[(b * 2 * S + s) * N + n] = st.accDr[s] + gr0 * st.Hr[s];
      io.grad_decay[(b * 2 * S + S + s) * N + n] = st.accDd[s] + gd0 * st.Hd[s];
    }
  }
}

// The scan backward with dL/da written as rows (see cond_backward_kernel). Each wave
// stages its own 64 items ([16 steps][K][64 lanes] of the workgroup's LDS) and writes
// them out itself: no workgroup barrier, so the waves stay apart in time (a wave's LDS
// accesses are executed in its program order). A lane past the last item runs item 0's
// steps and writes nothing.
template <int S, bool AD>
__device__ inline void rows_backward(const BackArgs& P, float* stage) {
  const int64_t N = P.tab.N, B = P.io.B, T = P.io.T, Tp = P.io.T_pad;
  const int K = (int)P.tab.K;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t first = (int64_t)blockIdx.x * kBackBlock + wave * 64;  // the wave's items
  stage += wave * 16 * K * 64;
  const int64_t idx = first + lane;
  const bool valid = idx < B * N;
  const int64_t item = valid ? idx : 0;
  const int64_t b = item / N, n = item - b * N;
  Synapses<S> syn;
  load_synapses<S>(P.tab, syn);
  const BackNeuron c = back_neuron<AD>(P.tab, n);
  float scale[WT_MAX_K];
#pragma unroll
  for (int k = 0; k < WT_MAX_K; ++k) scale[k] = k < K ? P.tab.scale[k * N + n] : 0.0f;
  BackState<S> st;
  state_zero(st);
  StepIn<S> cur, next;
  load_step<S, AD>(cur, P, b, n, T - 1);
  for (int64_t t = T - 1; t >= 0; --t) {
    if (t > 0) load_step<S, AD>(next, P, b, n, t - 1);  // a step ahead
    back_membrane_step<S, AD>(st, P, syn, c, b, n, t, cur, scale, nullptr,
                              stage + (int)(t & 15) * K * 64 + lane, 64);
    back_spike_step<S>(st, P, c, 0.0f, cur);
    cur = next;
    if ((t & 15) == 0) {  // steps t .. t + 15 are staged: 64 bytes per (pathway, item)
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      __builtin_amdgcn_wave_barrier();
      const int64_t pitch = B * Tp;
      for (int w = lane; w < K * 64 * 4; w += 64) {
        const int k = w >> 8, i = (w >> 2) & 63, q = w & 3;
        const int64_t it = first + i;
        if (it >= B * N) continue;
        const int64_t bi = it / N, ni = it - bi * N;
        float4 v;
        v.x = stage[((4 * q + 0) * K + k) * 64 + i];
        v.y = stage[((4 * q + 1) * K + k) * 64 + i];
        v.z = stage[((4 * q + 2) * K + k) * 64 + i];
        v.w = stage[((4 * q + 3) * K + k) * 64 + i];
        *reinterpret_cast<float4*>(P.io.grad_A_rows + ((int64_t)k * N + ni) * pitch +
                                   bi * Tp + t + 4 * q) = v;
      }
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      __builtin_amdgcn_wave_barrier();  // the stage is written again from the next step on
    }
  }
  if (valid) back_finish<S>(st, P, b, n);
}

// Recurrent activations as inputs: one thread per (trial, neuron), all steps. Held to
// three waves per SIMD (at most 168 VGPRs; a few values spill): with two, too few reverse
// steps are in flight to cover the loads a step ahead (config 3: 3.39 ms against 3.89).
// ROWS: dL/da goes to io.grad_A_rows as (pathway, target) rows of pitch B*T_pad: each
// step's K values per item are staged in LDS ([16 steps][K][256 items], dynamic) and
// every 16 steps (t a multiple of 16) the workgroup writes each item's 16 consecutive
// steps of each pathway as 64 aligned bytes.
template <int S, bool AD, bool ROWS>
__global__ __launch_bounds__(kBackBlock) __attribute__((amdgpu_waves_per_eu(3))) void
cond_backward_kernel(BackArgs P) {
  extern __shared__ float stage[];
  const int64_t N = P.tab.N, B = P.io.B, T = P.io.T;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (!ROWS && idx >= B * N) return;
  if (ROWS) {  // the whole workgroup takes part in the staging; items past the end idle
    rows_backward<S, AD>(P, stage);
    return;
  }
  const int64_t b = idx / N, n = idx - b * N;
  Synapses<S> syn;
  load_synapses<S>(P.tab, syn);
  const BackNeuron c = back_neuron<AD>(P.tab, n);
  float scale[WT_MAX_K];
#pragma unroll
  for (int k = 0; k < WT_MAX_K; ++k) scale[k] = k < P.tab.K ? P.tab.scale[k * N + n] : 0.0f;
  BackState<S> st;
  state_zero(st);
  StepIn<S> cur, next;
  if (T > 0) load_step<S, AD>(cur, P, b, n, T - 1);
  for (int64_t t = T - 1; t >= 0; --t) {
    if (t > 0) load_step<S, AD>(next, P, b, n, t - 1);  // a step ahead
    back_membrane_step<S, AD>(st, P, syn, c, b, n, t, cur, scale);
    back_spike_step<S>(st, P, c, 0.0f, cur);
    cur = next;
  }
  back_finish<S>(st, P, b, n);
}

// Recurrent path. Per reverse step t: (1) the membrane kernel: for every item (b, n) the
// spike part of step t + 1 (which needs R of step t + 1) and the membrane part of step t,
// with the adjoint state in global memory between the steps, writing dL/da of step t;
// (2) a gather kernel: R[j][b] = sum over source j's synapses e of w_e dL/da(t)[target e]
// [b]. After step 0, the finish kernel: the spike part of step 0 and the partials.

// The spike part of item (b, n) at step t, given R: only dv and the threshold partial.
template <int S>
__device__ inline void rg_spike_at(BackState<S>& st, const BackArgs& P, const BackNeuron& c,
                                   int64_t b, int64_t n, int64_t t, float R) {
  const wt_backward_io& io = P.io;
  const int64_t out = (b * io.T + t) * P.tab.N + n;
  StepIn<S> in;
  in.v = io.v_saved[out];
  in.grad_spike = io.grad_spikes[out];
  in.grad_prob = io.grad_prob ? io.grad_prob[out] : 0.0f;
  in.held = io.held ? (float)io.held[out] : 0.0f;
  back_spike_step<S>(st, P, c, R, in);
}

// Workgroup i runs on XCD i % 8. The logical index that gives each XCD one contiguous run
// of the n workgroups (XCDs below r = n % 8 take q + 1 of them, the others q = n / 8).
__device__ inline unsigned xcd_contiguous(unsigned i, unsigned n) {
  const unsigned x = i & 7u, slot = i >> 3, q = n >> 3, r = n & 7u;
  return x < r ? x * (q + 1) + slot : r * (q + 1) + (x - r) * q + slot;
}

// The membrane kernel's workgroup: a tile of 32 neurons x 8 trials, neurons fastest, so
// the per-item rows (v, G, spikes, state: neuron fastest) are read in 128-byte runs; R
// ([n][b]) comes in and dL/da ([k][n][b]) leaves through LDS in rows of 8 trials. The
// tiles of one neuron range are consecutive (and on one XCD), so each 128-byte line of
// dL/da is completed in one L2.
constexpr int kRgTileN = 32, kRgTileB = 8;

template <int S, bool AD>
__global__ __launch_bounds__(256) void rg_membrane_kernel(BackArgs P, int64_t t) {
  __shared__ float ga_tile[WT_MAX_K][kRgTileN][kRgTileB + 1];
  __shared__ float r_tile[kRgTileN][kRgTileB + 1];
  const int64_t N = P.tab.N, B = P.io.B;
  const int64_t tiles_b = (B + kRgTileB - 1) / kRgTileB;
  const int64_t tile = xcd_contiguous(blockIdx.x, gridDim.x);
  const int64_t tn = tile / tiles_b, tb = tile - tn * tiles_b;
  const int nn = threadIdx.x % kRgTileN, bb = threadIdx.x / kRgTileN;
  const int64_t n = tn * kRgTileN + nn, b = tb * kRgTileB + bb;
  // the transposed position: trials fastest
  const int wb = threadIdx.x % kRgTileB, wn = threadIdx.x / kRgTileB;
  const int64_t n2 = tn * kRgTileN + wn, b2 = tb * kRgTileB + wb;
  const int K_rec = (int)P.tab.K_rec;
  const bool carry = t < P.io.T - 1;  // the spike part of step t + 1 is done here
  if (carry) {
    r_tile[wn][wb] = n2 < N && b2 < B ? P.R[n2 * B + b2] : 0.0f;
    __syncthreads();
  }
  float ga[WT_MAX_K];
#pragma unroll
  for (int k = 0; k < WT_MAX_K; ++k) ga[k] = 0.0f;
  if (n < N && b < B) {
    const int64_t idx = b * N + n;
    Synapses<S> syn;
    load_synapses<S>(P.tab, syn);
    const BackNeuron c = back_neuron<AD>(P.tab, n);
    float scale[WT_MAX_K];
#pragma unroll
    for (int k = 0; k < WT_MAX_K; ++k) scale[k] = k < P.tab.K ? P.tab.scale[k * N + n] : 0.0f;
    BackState<S> st;
    if (!carry) {
      state_zero(st);
    } else {
      state_io<S, AD>(st, P.state, B * N, idx, false, P.io, P.tab.K);
      rg_spike_at<S>(st, P, c, b, n, t + 1, r_tile[nn][bb]);
    }
    StepIn<S> in;
    load_step<S, AD>(in, P, b, n, t);
    back_membrane_step<S, AD>(st, P, syn, c, b, n, t, in, scale, ga);
    state_io<S, AD>(st, P.state, B * N, idx, true, P.io, P.tab.K);
  }
#pragma unroll
  for (int k = 0; k < WT_MAX_K; ++k)
    if (k < K_rec) ga_tile[k][nn][bb] = ga[k];
  __syncthreads();
  if (n2 < N && b2 < B) {
#pragma unroll
    for (int k = 0; k < WT_MAX_K; ++k)
      if (k < K_rec) P.grad_now[((int64_t)k * N + n2) * B + b2] = ga_tile[k][wn][wb];
  }
}

// The gather, any B: per (source j, trial b), threads b fastest. j's synapses sixteen at
// a time: their targets and weights, then the sixteen dL/da values, all in flight
// together; the products added one by one in synapse order.
template <int S>
__global__ __launch_bounds__(256) void rg_gather_kernel(BackArgs P) {
  const int64_t N = P.tab.N, B = P.io.B;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= B * N) return;
  const int64_t j = idx / B, b = idx - j * B;
  float R = 0.0f;
  const int32_t k = P.rec.pathway[j];
  if (k >= 0 && k < P.tab.K_rec) {
    const float* g = P.grad_now + (int64_t)k * N * B + b;
    const int32_t* tg = P.rec.targets;
    const float* w = P.rec.weights;
    int64_t e = P.rec.indptr[j];
    const int64_t e1 = P.rec.indptr[j + 1];
    constexpr int kU = 16;
    for (; e + kU <= e1; e += kU) {
      int32_t t8[kU];
      float w8[kU], g8[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        t8[u] = tg[e + u];
        w8[u] = w[e + u];
      }
#pragma unroll
      for (int u = 0; u < kU; ++u) g8[u] = g[(int64_t)t8[u] * B];
#pragma unroll
      for (int u = 0; u < kU; ++u) R += w8[u] * g8[u];
    }
    for (; e < e1; ++e) R += w[e] * g[(int64_t)tg[e] * B];
  }
  P.R[j * B + b] = R;
}

// The gather with B a multiple of 64: each wave holds one source j (wave-uniform) and 64
// consecutive trials, whose dL/da row of a target is 256 contiguous bytes. j's synapses
// come in 32 at a time, one per lane (lanes 32-63 repeat 0-31); lane (q, g), q = lane %
// 16, g = lane / 16, takes synapse 4i + g's target and weight from its lane (ds_bpermute)
// and loads trials 4q .. 4q + 3 of its row, so one 16-byte-per-lane load brings four
// synapses' rows and eight such loads are in flight. Lane group g sums every fourth
// synapse in order; the four groups' sums are added at the end. The next 32 targets and
// weights are requested before the current rows.
constexpr int kRgChunk = 32;

template <int S>
__global__ __launch_bounds__(256) void rg_gather_wave_kernel(BackArgs P) {
  const int64_t N = P.tab.N, B = P.io.B;
  const int64_t per_j = B >> 6;  // waves per source
  const unsigned wg = xcd_contiguous(blockIdx.x, gridDim.x);
  const int64_t wave = (int64_t)wg * 4 + (threadIdx.x >> 6);
  const int64_t j = __builtin_amdgcn_readfirstlane((int)(wave / per_j));
  if (j >= N) return;
  const int lane = threadIdx.x & 63, q = lane & 15, g = lane >> 4;
  const int64_t b0 = (wave - j * per_j) * 64;
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  const int32_t k = P.rec.pathway[j];
  if (k >= 0 && k < P.tab.K_rec) {
    const int64_t e0 = P.rec.indptr[j], e1 = P.rec.indptr[j + 1];
    if (e1 > e0) {
      const int32_t* __restrict__ tg = P.rec.targets;
      const float* __restrict__ w = P.rec.weights;
      // dL/da of pathway k, [N][B]: target row * B * 4 bytes, then the lane's trials
      const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<float*>(P.grad_now + (int64_t)k * N * B), (short)0,
          (int)(N * B * 4), 0x00020000);
      const int voff = (int)(b0 * 4 + q * 16);
      const int row = (int)(B * 4);
      const int mine = lane & (kRgChunk - 1);
      // the lane's synapse of the chunk at c; past j's last synapse, that one's target
      // (a row in range) with weight 0, which adds exact zeros
      auto load = [&](int64_t c, int32_t& tt, float& ww) {
        const bool in = c + mine < e1;
        const int64_t i = in ? c + mine : e1 - 1;
        tt = tg[i];
        ww = in ? w[i] : 0.0f;
      };
      int32_t tc;
      float wc;
      load(e0, tc, wc);
      for (int64_t e = e0; e < e1; e += kRgChunk) {
        int32_t tn;
        float wn;
        load(e + kRgChunk, tn, wn);
        float4 gv[kRgChunk / 4];
        float wv[kRgChunk / 4];
#pragma unroll
        for (int i = 0; i < kRgChunk / 4; ++i) {
          const int from = (4 * i + g) * 4;  // byte address of the source lane
          const int ti = __builtin_amdgcn_ds_bpermute(from, tc);
          wv[i] = __builtin_bit_cast(
              float, __builtin_amdgcn_ds_bpermute(from, __builtin_bit_cast(int, wc)));
          gv[i] = __builtin_bit_cast(
              float4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, voff + ti * row, 0, 0));
        }
#pragma unroll
        for (int i = 0; i < kRgChunk / 4; ++i) {  // synapse order within the lane group
          acc[0] += wv[i] * gv[i].x;
          acc[1] += wv[i] * gv[i].y;
          acc[2] += wv[i] * gv[i].z;
          acc[3] += wv[i] * gv[i].w;
        }
        tc = tn;
        wc = wn;
      }
    }
  }
  // (g0 + g1) + (g2 + g3), the same in every lane group
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    acc[c] += __shfl_xor(acc[c], 16);
    acc[c] += __shfl_xor(acc[c], 32);
  }
  const float r = (g & 2) ? ((g & 1) ? acc[3] : acc[2]) : ((g & 1) ? acc[1] : acc[0]);
  P.R[j * B + b0 + 4 * q + g] = r;
}

// After step 0: the spike part of step 0, then the partials from the global state.
template <int S>
__global__ __launch_bounds__(256) void rg_finish_kernel(BackArgs P) {
  const int64_t N = P.tab.N, B = P.io.B;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= B * N) return;
  const int64_t b = idx / N, n = idx - b * N;
  BackState<S> st;
  state_io<S, true>(st, P.state, B * N, idx, false, P.io, P.tab.K);  // (null grads: no read)
  BackNeuron c;
  c.theta = P.tab.theta[n];
  c.k_surr = *P.tab.surr;
  rg_spike_at<S>(st, P, c, b, n, 0, P.R[n * B + b]);
  back_finish<S>(st, P, b, n);
}

template <int S>
struct BackLaunch {
  static hipError_t run(BackArgs& a, hipStream_t stream);
  static hipError_t recurrent(BackArgs& a, hipStream_t stream);
};

template <int S>
hipError_t BackLaunch<S>::run(BackArgs& a, hipStream_t stream) {
  const int64_t total = a.io.B * a.tab.N;
  const int block = kBackBlock;
  const dim3 grid((unsigned)((total + block - 1) / block));
  if (a.io.grad_A_rows) {  // dL/da as rows: the stage of 16 steps in dynamic LDS
    const size_t lds = (size_t)16 * a.tab.K * kBackBlock * sizeof(float);
    const void* fn = a.tab.adapt ? (const void*)cond_backward_kernel<S, true, true>
                                 : (const void*)cond_backward_kernel<S, false, true>;
    const hipError_t e =
        hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    if (a.tab.adapt)
      hipLaunchKernelGGL((cond_backward_kernel<S, true, true>), grid, dim3(block), lds, stream, a);
    else
      hipLaunchKernelGGL((cond_backward_kernel<S, false, true>), grid, dim3(block), lds, stream, a);
    return hipGetLastError();
  }
  if (a.tab.adapt)
    hipLaunchKernelGGL((cond_backward_kernel<S, true, false>), grid, dim3(block), 0, stream, a);
  else
    hipLaunchKernelGGL((cond_backward_kernel<S, false, false>), grid, dim3(block), 0, stream, a);
  return hipGetLastError();
}

template <int S>
hipError_t BackLaunch<S>::recurrent(BackArgs& a, hipStream_t stream) {
  const int64_t B = a.io.B, N = a.tab.N, total = B * N;
  const int block = 256;
  const dim3 grid((unsigned)((total + block - 1) / block));
  const dim3 tiles((unsigned)(((N + kRgTileN - 1) / kRgTileN) * ((B + kRgTileB - 1) / kRgTileB)));
  // one wave per (source, 64 trials) when the trials fill whole waves (and the dL/da
  // rows of a pathway stay within the 32-bit offsets of a buffer load)
  const bool by_wave = B % 64 == 0 && N * B * 4 < INT32_MAX;
  const dim3 wave_grid((unsigned)((total / 64 + 3) / 4));
  for (int64_t t = a.io.T - 1; t >= 0; --t) {
    if (a.tab.adapt)
      hipLaunchKernelGGL((rg_membrane_kernel<S, true>), tiles, dim3(block), 0, stream, a, t);
    else
      hipLaunchKernelGGL((rg_membrane_kernel<S, false>), tiles, dim3(block), 0, stream, a, t);
    if (by_wave)
      hipLaunchKernelGGL(rg_gather_wave_kernel<S>, wave_grid, dim3(block), 0, stream, a);
    else
      hipLaunchKernelGGL(rg_gather_kernel<S>, grid, dim3(block), 0, stream, a);
  }
  hipLaunchKernelGGL(rg_finish_kernel<S>, grid, dim3(block), 0, stream, a);
  return hipGetLastError();
}

}  // namespace wt
