// Beta policy head math for the rollout buffer of the shared-policy loop: the
// log-density of a draw, the entropy, and their derivatives with respect to the
// head's raw outputs (u, v), for shapes a = softplus(u) + f, b = softplus(v) + f
// with the policy's shape floor f (1 by default; below 1 the shapes may be
// below 1) (complete_port/patches/pufferlib_core.diff:944-1000,
// beta_continuous_head; :1008-1014 beta_kl).
//
//   log p(x)  = (a - 1) log x + (b - 1) log(1 - x) - ln B(a, b)
//   H         = ln B(a, b) - (a - 1) psi(a) - (b - 1) psi(b) + (a + b - 2) psi(a + b)
//   d log p / da = log x - psi(a) + psi(a + b)
//   d H / da     = -(a - 1) psi'(a) + (a + b - 2) psi'(a + b)
//   d a / du     = softplus'(u) = sigmoid(u)
//
// ln B from the device libm's lgamma; psi and psi' by upward recurrence to
// x >= 10 and the asymptotic series of Abramowitz & Stegun 6.3.18 / 6.4.12
// (truncation below 1e-15 relative there); shapes are positive.
//
//   KL(Beta(a1, b1) || Beta(a2, b2)) = ln B(a2, b2) - ln B(a1, b1) + (a1 - a2) psi(a1)
//                                      + (b1 - b2) psi(b1) + (a2 - a1 + b2 - b1) psi(a1 + b1)
// (the difference of the cross-entropy E_1[-log p_2] and the entropy of p_1,
// with E_1[log x] = psi(a1) - psi(a1 + b1) and E_1[log(1 - x)] = psi(b1) - psi(a1 + b1)).
#pragma once
#include <hip/hip_runtime.h>

namespace sbk {

// psi(x), x > 0: psi(x) = psi(x + 1) - 1/x, then the series at x >= 10.
__device__ __forceinline__ double beta_digamma(double x) {
    double r = 0.0;
    while (x < 10.0) {
        r -= 1.0 / x;
        x += 1.0;
    }
    const double i2 = 1.0 / (x * x);
    // ln x - 1/(2x) - sum B_2k / (2k x^2k), k = 1..6
    const double s = i2 * (1.0 / 12 - i2 * (1.0 / 120 - i2 * (1.0 / 252 - i2 * (1.0 / 240 - i2 * (1.0 / 132
                                                                                        - i2 * (691.0 / 32760))))));
    return r + log(x) - 0.5 / x - s;
}

// psi'(x), x > 0: psi'(x) = psi'(x + 1) + 1/x^2, then the series at x >= 10.
__device__ __forceinline__ double beta_trigamma(double x) {
    double r = 0.0;
    while (x < 10.0) {
        r += 1.0 / (x * x);
        x += 1.0;
    }
    const double i1 = 1.0 / x, i2 = i1 * i1;
    // 1/x + 1/(2x^2) + sum B_2k / x^(2k+1), k = 1..6
    const double s = i2 * i1 * (1.0 / 6 - i2 * (1.0 / 30 - i2 * (1.0 / 42 - i2 * (1.0 / 30 - i2 * (5.0 / 66
                                                                                        - i2 * (691.0 / 2730))))));
    return r + i1 + 0.5 * i2 + s;
}

// The sampler's shape map (float, as the draws use it) and its derivative.
__device__ __forceinline__ float beta_shape(float raw, float floor) {
    return (raw > 20.0f ? raw : log1pf(expf(raw))) + floor;
}
__device__ __forceinline__ double beta_shape_grad(float raw) {
    return raw > 20.0f ? 1.0 : 1.0 / (1.0 + exp(-(double)raw));
}

// Draws are floats in (0, 1); a ratio of gamma draws can round to 0 or 1, so
// the density is evaluated at x clamped to [2^-24, 1 - 2^-24].
__device__ __forceinline__ double beta_clamp_x(float x) {
    const double lo = 5.9604644775390625e-8;
    return x < lo ? lo : (x > 1.0 - lo ? 1.0 - lo : (double)x);
}

struct BetaHead {
    double logp, entropy;
    double g[4];   // d logp / du, d logp / dv, d H / du, d H / dv
};

__device__ __forceinline__ BetaHead beta_head(float u, float v, float x, float floor) {
    const double a = beta_shape(u, floor), b = beta_shape(v, floor), s = a + b;
    const double xc = beta_clamp_x(x);
    const double lx = log(xc), l1 = log1p(-xc);
    const double lnb = lgamma(a) + lgamma(b) - lgamma(s);
    const double pa = beta_digamma(a), pb = beta_digamma(b), ps = beta_digamma(s);
    BetaHead h;
    h.logp = (a - 1.0) * lx + (b - 1.0) * l1 - lnb;
    h.entropy = lnb - (a - 1.0) * pa - (b - 1.0) * pb + (s - 2.0) * ps;
    const double ta = beta_trigamma(a), tb = beta_trigamma(b), ts = beta_trigamma(s);
    const double su = beta_shape_grad(u), sv = beta_shape_grad(v);
    h.g[0] = (lx - pa + ps) * su;
    h.g[1] = (l1 - pb + ps) * sv;
    h.g[2] = (-(a - 1.0) * ta + (s - 2.0) * ts) * su;
    h.g[3] = (-(b - 1.0) * tb + (s - 2.0) * ts) * sv;
    return h;
}

__device__ __forceinline__ double beta_lnb(double a, double b) { return lgamma(a) + lgamma(b) - lgamma(a + b); }

__device__ __forceinline__ double beta_kl(double a1, double b1, double a2, double b2) {
    const double s1 = a1 + b1;
    return beta_lnb(a2, b2) - beta_lnb(a1, b1) + (a1 - a2) * beta_digamma(a1) + (b1 - b2) * beta_digamma(b1)
           + (a2 - a1 + b2 - b1) * beta_digamma(s1);
}

}  // namespace sbk
