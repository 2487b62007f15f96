/* Counter-based Beta(2,2) action stream for synthetic rollouts (oracle side).
 *
 * TEST INFRASTRUCTURE: used only by tests, smoke() and bench.py's cpu_baseline.
 *
 * Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy
 * as 1, 2, 3", SC 2011): 10 rounds of two 32x32->64 multiplies with the
 * published multipliers and Weyl key increments. Key = 64-bit seed, counter =
 * (env, step, slot, 0). Outputs x0..x2 become uniforms u = ((x >> 8) + 0.5) / 2^24
 * (exact in float32, strictly inside (0,1)); the median of three U(0,1) is
 * Beta(2,2) distributed. Continuous slot i gets 2x - 1, discrete slot d gets
 * (x > 0.5). The reference trainer draws its Beta samples with cuRAND
 * (complete_port/patches/pufferlib_core.diff:2547-2601); this stream is an
 * independent, published construction chosen so CPU and GPU agree bit for bit.
 */
#ifndef SBO_PHILOX_H
#define SBO_PHILOX_H
#include <stdint.h>

static inline void sbo_philox4x32_10(uint32_t c[4], uint32_t k0, uint32_t k1) {
    const uint32_t M0 = 0xD2511F53u, M1 = 0xCD9E8D57u;
    const uint32_t W0 = 0x9E3779B9u, W1 = 0xBB67AE85u;
    for (int r = 0; r < 10; r++) {
        uint64_t p0 = (uint64_t)M0 * c[0];
        uint64_t p1 = (uint64_t)M1 * c[2];
        uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
        uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
        uint32_t n0 = hi1 ^ c[1] ^ k0;
        uint32_t n2 = hi0 ^ c[3] ^ k1;
        c[0] = n0; c[1] = lo1; c[2] = n2; c[3] = lo0;
        k0 += W0; k1 += W1;
    }
}

static inline float sbo_u24(uint32_t x) {
    return ((float)(x >> 8) + 0.5f) * (1.0f / 16777216.0f);
}

/* Beta(2,2) draw in (0,1) for (seed, env, step, slot). */
static inline float sbo_beta22(uint64_t seed, uint32_t env, uint32_t step, uint32_t slot) {
    uint32_t c[4] = {env, step, slot, 0u};
    sbo_philox4x32_10(c, (uint32_t)seed, (uint32_t)(seed >> 32));
    float a = sbo_u24(c[0]), b = sbo_u24(c[1]), d = sbo_u24(c[2]);
    float lo = a < b ? a : b, hi = a < b ? b : a;
    return d < lo ? lo : (d > hi ? hi : d);
}

/* Fills one trainer action row (SB_CONT continuous then SB_DISC discrete). */
static inline void sbo_action_row_philox(uint64_t seed, uint32_t env, uint32_t step,
                                  int n_cont, int n_disc, float* row,
                                  int sb_cont, int sb_disc) {
    for (int i = 0; i < sb_cont; i++)
        row[i] = (i < n_cont) ? 2.0f * sbo_beta22(seed, env, step, (uint32_t)i) - 1.0f : 0.0f;
    for (int d = 0; d < sb_disc; d++)
        row[sb_cont + d] = (d < n_disc)
            ? (sbo_beta22(seed, env, step, (uint32_t)(sb_cont + d)) > 0.5f ? 1.0f : 0.0f) : 0.0f;
}
#endif
