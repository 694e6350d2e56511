// wt_philox.h — the counter-based generator of on-device Poisson input.
//
// Philox4x32-10 (Salmon, Moraes, Dror and Shaw, "Parallel random numbers: as easy as 1, 2,
// 3", SC 2011): a 128-bit counter and a 64-bit key pass 10 rounds of two 32x32->64-bit
// multiplications (multipliers 0xD2511F53 and 0xCD9E8D57) with the key bumped by the
// Weyl constants 0x9E3779B9, 0xBB67AE85 between rounds. Every draw is a pure function of
// (key, counter), so the host replays any element of the stream exactly
// (wiretorch_amd/inputs.py) and a draw needs no state.
//
// Input spikes: channel j of trial b at absolute step t fires when u < p_j, u the top 24
// bits of the first output word of counter (j, t, b, 0) under key (seed low, seed high),
// scaled by 2^-24 (a float32 in [0, 1), exactly) — the comparison the reference's
// Poisson dataset makes with torch.rand (dataloaders/unsupervised.py:85-90).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wt {

__host__ __device__ inline void philox4x32_10(uint32_t (&c)[4], uint32_t k0, uint32_t k1) {
  constexpr uint32_t M0 = 0xD2511F53u, M1 = 0xCD9E8D57u;
  constexpr uint32_t W0 = 0x9E3779B9u, W1 = 0xBB67AE85u;
#pragma unroll
  for (int round = 0; round < 10; ++round) {
    const uint64_t p0 = (uint64_t)M0 * c[0], p1 = (uint64_t)M1 * c[2];
    const uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
    const uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
    const uint32_t n0 = hi1 ^ c[1] ^ k0, n2 = hi0 ^ c[3] ^ k1;
    c[0] = n0;
    c[1] = lo1;
    c[2] = n2;
    c[3] = lo0;
    k0 += W0;
    k1 += W1;
  }
}

// Whether input channel j of trial b fires at absolute step t (probability p).
__host__ __device__ inline bool poisson_fires(uint64_t seed, uint32_t b, uint32_t t, uint32_t j,
                                              float p) {
  uint32_t c[4] = {j, t, b, 0u};
  philox4x32_10(c, (uint32_t)seed, (uint32_t)(seed >> 32));
  const float u = (float)(c[0] >> 8) * 0x1p-24f;
  return u < p;
}

}  // namespace wt
