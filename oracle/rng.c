/*
 * ORACLE ONLY (test infrastructure): CPU restatement of the sampler's uniform
 * stream, Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers:
 * as easy as 1, 2, 3", SC 2011), pinned by the paper's published known-answer
 * vectors (tests/test_oracle_rng.py).
 *
 * Stream convention (shared with the kernel): draw event c (a 64-bit counter
 * the sampler advances by one per draw) with key (seed_lo, seed_hi) gives
 *   u(c, i) = (philox({c_lo, c_hi, i / 4, 0}, key)[i % 4] >> 8) * 2^-24,
 * uniform on [0, 1) with 24 random bits. The reference draws from MLX's
 * generator (engine/speculative.py:79-81, engine/sampler.py:57-58), which is
 * not importable here; only the law U(0, 1) is shared.
 */
#include <stdint.h>

#include "oracle.h"

static inline void mulhilo(uint32_t a, uint32_t b, uint32_t* hi, uint32_t* lo) {
  const uint64_t p = (uint64_t)a * (uint64_t)b;
  *hi = (uint32_t)(p >> 32);
  *lo = (uint32_t)p;
}

void orc_philox4x32_10(const uint32_t ctr_in[4], const uint32_t key_in[2], uint32_t out[4]) {
  uint32_t c0 = ctr_in[0], c1 = ctr_in[1], c2 = ctr_in[2], c3 = ctr_in[3];
  uint32_t k0 = key_in[0], k1 = key_in[1];
  for (int r = 0; r < 10; ++r) {
    if (r > 0) {
      k0 += 0x9E3779B9u;
      k1 += 0xBB67AE85u;
    }
    uint32_t hi0, lo0, hi1, lo1;
    mulhilo(0xD2511F53u, c0, &hi0, &lo0);
    mulhilo(0xCD9E8D57u, c2, &hi1, &lo1);
    const uint32_t n0 = hi1 ^ c1 ^ k0, n1 = lo1, n2 = hi0 ^ c3 ^ k1, n3 = lo0;
    c0 = n0;
    c1 = n1;
    c2 = n2;
    c3 = n3;
  }
  out[0] = c0;
  out[1] = c1;
  out[2] = c2;
  out[3] = c3;
}

void orc_philox_uniforms(uint64_t seed, uint64_t event, int n, float* out) {
  const uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
  for (int i = 0; i < n; ++i) {
    const uint32_t ctr[4] = {(uint32_t)event, (uint32_t)(event >> 32), (uint32_t)(i >> 2), 0u};
    uint32_t r[4];
    orc_philox4x32_10(ctr, key, r);
    out[i] = (float)(r[i & 3] >> 8) * 0x1p-24f;
  }
}
