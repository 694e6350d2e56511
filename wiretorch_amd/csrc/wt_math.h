// wt_math.h — per-neuron conductance-LIF arithmetic for gfx950, in the reference's
// operation order.
//
// The reference step is conductance/dynamics.py:103-143 (+ network.py:294-318): the
// forward functions below evaluate it in float32 with the same association as torch's
// CPU kernels (no fused multiply-add: this file is compiled with -ffp-contract=off),
// so that spike decisions agree with the reference bit for bit unless a voltage lies
// within rounding of threshold. The adjoint follows from differentiating those
// equations (the autograd graph of dynamics.py, whose values the reference's
// conductance/kernels.py:315-379 also reproduces).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/wiretorch_amd.h"

namespace wt {

// A short row summed the way torch's CPU reduction associates it (checked against
// torch for rows of up to five): four interleaved partial sums, then combined in order.
template <int S>
__host__ __device__ inline float row_sum(const float (&a)[S]) {
  constexpr int L = S < 4 ? S : 4;
  float acc[L];
#pragma unroll
  for (int i = 0; i < L; ++i) acc[i] = a[i];
#pragma unroll
  for (int i = L; i < S; ++i) acc[i % 4] = acc[i % 4] + a[i];
  float out = acc[0];
#pragma unroll
  for (int i = 1; i < L; ++i) out = out + acc[i];
  return out;
}

struct Leak {
  float rate;  // 1 / tau_mem, from beta precisely (log1p: beta is close to 1)
  float g_L;   // C_m * rate
};

__host__ __device__ inline Leak leak(float C_m, float beta, float dt) {
  float rate = -log1pf(beta - 1.0f) / dt;
  return {rate, C_m * rate};
}

// Synapse tables of one call, held by every thread (S entries each). With `mg`, each
// type's conductance is scaled by its Mg block B(v) = sigmoid(mg_a v - mg_lc), mg_lc =
// log(mg / mg_k) (-inf for a type without one: B = 1 exactly).
template <int S>
struct Synapses {
  float E[S], clip[S], decay_r[S], decay_d[S], jump_r[S], jump_d[S];
  float mg_a[S], mg_lc[S];
  bool mg;
};

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
  syn.mg = tab.mg_a != nullptr;
#pragma unroll
  for (int s = 0; s < S; ++s) {
    syn.mg_a[s] = syn.mg ? tab.mg_a[s] : 0.0f;
    syn.mg_lc[s] = syn.mg ? tab.mg_lc[s] : 0.0f;
  }
}

// The Mg block at v (conductance/dynamics.py:110-113): 1 / (1 + exp(-(mg_a v - mg_lc))),
// the product and the difference rounded as torch rounds them.
__host__ __device__ inline float mg_block(float v, float mg_a, float mg_lc) {
  const float z = mg_a * v - mg_lc;
  return 1.0f / (1.0f + expf(-z));
}

// Spike and refractory part of a step (dynamics.py:103-107, network.py:294-318):
// returns the spike; r is what holds the voltage at reset, held the refractory mask.
__host__ __device__ inline float spike_step(float v, float theta, int32_t& counter,
                                            int32_t n_ref, bool refractory, float& r,
                                            float& held) {
  float s = (v - theta) > 0.0f ? 1.0f : 0.0f;
  if (refractory) {
    held = counter > 0 ? 1.0f : 0.0f;
    s = s * (1.0f - held);
    r = fmaxf(s, held);
    counter = s > 0.0f ? n_ref : (counter - 1 > 0 ? counter - 1 : 0);
  } else {
    held = 0.0f;
    r = s;
  }
  return s;
}

// The exponential-Euler membrane step (dynamics.py:127-142). G (summed rise + decay
// per synapse type, before clipping) and the currents are returned for saving and
// tracking. With `adapting`, the adaptation conductance ga (by E_a) is one more term of
// the total conductance and of the current, added after the synapses' sums.
template <int S>
__host__ __device__ inline float membrane(float v, float r, const float (&gr)[S],
                                          const float (&gd)[S], const Synapses<S>& syn,
                                          float E_L, float C_m, float U_reset, Leak lk,
                                          float dt, float (&G)[S], float (&I)[S],
                                          float& I_leak, bool adapting = false,
                                          float ga = 0.0f, float E_a = 0.0f) {
  float Gc[S];
#pragma unroll
  for (int s = 0; s < S; ++s) {
    G[s] = gr[s] + gd[s];
    Gc[s] = fminf(fmaxf(G[s], 0.0f), syn.clip[s]);
    if (syn.mg) Gc[s] = Gc[s] * mg_block(v, syn.mg_a[s], syn.mg_lc[s]);
    I[s] = Gc[s] * (v - syn.E[s]);
  }
  I_leak = lk.g_L * (v - E_L);
  float Gt = row_sum<S>(Gc);
  float J = row_sum<S>(I) + I_leak;
  if (adapting) {
    Gt = Gt + ga;
    J = J + ga * (v - E_a);
  }
  float x = dt * lk.rate + dt * Gt / C_m;
  float step = -expm1f(-x) / (lk.g_L + Gt);
  return (v - step * J) * (1.0f - r) + U_reset * r;
}

// One step of the adjoint through the membrane update, given gx = dL/dv_next * (1 - r):
// returns dL/dv (membrane part) and writes dL/dG_s (through the clip) to dG.
// Differentiating v_next = v - phi(Gt) J(v, Gc) with phi = (1 - a) / (g_L + Gt),
// a = exp(-x), x = dt (rate + Gt / C_m):
//   d v_next / d v   = a                      (J' = g_L + Gt, 1 - phi (g_L + Gt) = a)
//   d v_next / d Gc_s = -(phi_G J + phi (v - E_s)),  phi_G = (a dt / C_m - phi) / (g_L + Gt)
// and the physiology terms below. With the Mg block Gc_s = C_s B_s(v) (C_s the clipped
// conductance): dL/dC_s = dL/dGc_s B_s, and v gains dL/dGc_s C_s mg_a_s B_s (1 - B_s).
// The adaptation conductance ga (by E_a) enters as a synapse type would, unclipped:
// dL/dga = -(phi_G J + phi (v - E_a)) gx, and dL/dE_a = gx phi ga; d v_next / d v stays
// a (J' = g_L + Gt with ga in Gt).
struct MembraneAdjoint {
  float dv;      // dL/dv entering the step (membrane part)
  float phi, a, inv_g, J, Gt;
  float d_ga;    // dL/dga (0 without adaptation)
};

template <int S>
__host__ __device__ inline MembraneAdjoint membrane_adjoint(
    float gx, float v, const float (&G)[S], const Synapses<S>& syn, float E_L, float C_m,
    Leak lk, float dt, float (&dG)[S], float (&Gc_out)[S], bool adapting = false,
    float ga = 0.0f, float E_a = 0.0f) {
  float Gc[S], I[S], C[S], Bm[S];
#pragma unroll
  for (int s = 0; s < S; ++s) {
    C[s] = fminf(fmaxf(G[s], 0.0f), syn.clip[s]);
    Bm[s] = syn.mg ? mg_block(v, syn.mg_a[s], syn.mg_lc[s]) : 1.0f;
    Gc[s] = syn.mg ? C[s] * Bm[s] : C[s];
    I[s] = Gc[s] * (v - syn.E[s]);
    Gc_out[s] = Gc[s];
  }
  float Gt = row_sum<S>(Gc);
  float J = row_sum<S>(I) + lk.g_L * (v - E_L);
  if (adapting) {
    Gt = Gt + ga;
    J = J + ga * (v - E_a);
  }
  float x = dt * lk.rate + dt * Gt / C_m;
  float em = expm1f(-x);
  float a = 1.0f + em;
  float inv_g = 1.0f / (lk.g_L + Gt);
  float phi = -em * inv_g;
  float phi_G = (a * dt / C_m - phi) * inv_g;
  float k0 = -gx * (phi_G * J + phi * v);
  float k1 = gx * phi;
  float dv = gx * a;
#pragma unroll
  for (int s = 0; s < S; ++s) {
    float d = k0 + k1 * syn.E[s];  // dL/dGc_s
    if (syn.mg) {  // through B_s(v), then on to the clipped conductance
      dv = dv + d * C[s] * (Bm[s] * (1.0f - Bm[s])) * syn.mg_a[s];
      d = d * Bm[s];
    }
    // torch: clamp(min=0) passes the gradient where G >= 0; minimum(., clip) splits it
    // evenly where G == clip.
    float pass = G[s] < syn.clip[s] ? 1.0f : (G[s] == syn.clip[s] ? 0.5f : 0.0f);
    dG[s] = G[s] >= 0.0f ? d * pass : 0.0f;
  }
  const float d_ga = adapting ? k0 + k1 * E_a : 0.0f;
  return {dv, phi, a, inv_g, J, Gt, d_ga};
}

// Surrogate gradient of the spike at x = v - theta (surrogate_gradients.py:30-33).
__host__ __device__ inline float surrogate(float x, float grad, float k) {
  float d = k * fabsf(x) + 1.0f;
  return grad / (d * d);
}

}  // namespace wt
