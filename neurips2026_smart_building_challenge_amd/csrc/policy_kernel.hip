// Shared-policy MLP forward + Beta action sampling for MI355X (gfx950), the
// rollout-loop workload of BASELINE config 5: every env's observation row goes
// through the same fp32 MLP
//
//   h1 = tanh(obs W1 + b1)   [n x 1024] x [1024 x 128]
//   h2 = tanh(h1 W2 + b2)    [n x 128]  x [128 x 128]
//   y  = h2 W3 + b3          [n x 128]  x [128 x 2 SB_ACT] = (u[SB_CONT], v[SB_CONT], ud[16], vd[16])
//
// and each action head j draws x ~ Beta(softplus(u_j) + f, softplus(v_j) + f)
// (f the policy's shape floor, 1 by default);
// continuous heads write 2x - 1, discrete heads x > 0.5 into the action row the
// next env step decodes.
//
// The three products run on fp32 MFMA (v_mfma_f32_16x16x4_f32). The two
// hidden layers take one workgroup per 16 x 16 output tile, its K range split
// over up to four wavefronts whose partial tiles are summed in LDS in a fixed
// order, then bias and activation; the third layer is fused with the Beta
// draws, one workgroup per (16 envs, 16 heads).
// Within a 16-wide K block, lane group g (lanes 16g .. 16g + 15) feeds the
// k values 4g .. 4g + 3 over the four MFMA steps, so each lane reads its A
// operand as one contiguous float4 (the product over a block is the same sum).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include "sb_betamath.h"
#include "sb_philox.h"
#include "sbenv.h"

namespace sbk {

typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kPolicyHidden = 128;
constexpr int kPolicyHeads = 2 * SB_ACT;   // u, v of the continuous and the discrete heads
constexpr int kObsWidth = 1024;
constexpr int kActWidth = SB_ACT;
static_assert(SB_CONT % 16 == 0 && SB_DISC == 16, "head groups of 16: the continuous block, then one discrete group");
// y column of head h's u (which 0) or v (which 1): continuous heads h < SB_CONT
// at h and SB_CONT + h, discrete head d = h - SB_CONT at 2 SB_CONT + d and
// 2 SB_CONT + SB_DISC + d
__device__ __forceinline__ int head_col(int h, int which) {
    return h < SB_CONT ? h + SB_CONT * which : 2 * SB_CONT + SB_DISC * which + (h - SB_CONT);
}

// C[M x N] = act(A[M x K] B[K x N] + bias) with K = KW * (blockDim.x / 64):
// wavefront w takes K range [w KW, (w + 1) KW) and issues every load of that
// range before its first MFMA (one memory latency per tile). Columns of A at
// kmax and beyond are zero (an observation row's tail), so a wavefront skips
// its 16-wide K blocks that start there: their products add exactly nothing,
// and the fixed K partition keeps every result independent of kmax. lda / ldc
// in floats; N a multiple of 16. ACT: 0 identity, 1 tanh.
template <int ACT, int KW>
__global__ __launch_bounds__(512) void mlp_layer_kernel(const float* __restrict__ A, int lda,
                                                        const float* __restrict__ B,
                                                        const float* __restrict__ bias, float* __restrict__ C,
                                                        int ldc, int M, int N, int kmax) {
    static_assert(KW % 16 == 0, "K per wavefront is a multiple of 16");
    constexpr int NB = KW / 16;
    __shared__ v4f part[8][64];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, ksplit = blockDim.x >> 6;
    const int m0 = blockIdx.x * 16, n0 = blockIdx.y * 16;
    const int g = lane >> 4, i = lane & 15;
    const int m = m0 + i;
    const int mc = m < M ? m : M - 1;   // rows past M read row M - 1; their outputs are dropped
    const int nb = min(NB, max(0, (kmax - w * KW + 15) / 16));   // wave-uniform
    const float* a_row = A + (size_t)mc * lda + w * KW + 4 * g;
    const float* b_col = B + (size_t)(w * KW + 4 * g) * N + n0 + i;
    float4 a[NB];
    float b[NB][4];
#pragma unroll
    for (int j = 0; j < NB; j++) {
        if (j < nb) {
            a[j] = *reinterpret_cast<const float4*>(a_row + 16 * j);
            const float* bp = b_col + (size_t)(16 * j) * N;
#pragma unroll
            for (int s = 0; s < 4; s++) b[j][s] = bp[s * N];
        }
    }
    // the empty asm "uses" every loaded register here, so the compiler keeps
    // all loads ahead of the first MFMA instead of sinking each to its use
#pragma unroll
    for (int j = 0; j < NB; j++) {
        if (j < nb) {
            asm volatile("" : "+v"(a[j].x), "+v"(a[j].y), "+v"(a[j].z), "+v"(a[j].w));
            asm volatile("" : "+v"(b[j][0]), "+v"(b[j][1]), "+v"(b[j][2]), "+v"(b[j][3]));
        }
    }
    v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < NB; j++) {
        if (j < nb) {
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j].x, b[j][0], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j].y, b[j][1], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j].z, b[j][2], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j].w, b[j][3], acc, 0, 0, 0);
        }
    }
    if (ksplit > 1) {
        part[w][lane] = acc;
        __syncthreads();
        if (w != 0) return;
        for (int s = 1; s < ksplit; s++) acc += part[s][lane];
    }
    // lane holds C[4g + r][i] of the tile
    const float bv = bias[n0 + i];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int row = m0 + 4 * g + r;
        float v = acc[r] + bv;
        if (ACT == 1) v = tanhf(v);
        if (row < M) C[(size_t)row * ldc + n0 + i] = v;
    }
}

// Gamma(a), a > 0 (Marsaglia and Tsang, "A simple method for generating gamma
// variables", ACM TOMS 26(3), 2000): for k = a (a >= 1) or k = a + 1 (a < 1),
// d = k - 1/3, c = 1/sqrt(9d); draw z ~ N(0, 1) (Box-Muller) and u ~ U(0, 1),
// t = (1 + cz)^3, accept d t when cz > -1 and u < 1 - 0.0331 z^4 or
// log u < z^2/2 + d (1 - t + log t). With w = cz the last term is written
// 1 - t = -w (3 + 3w + w^2) and log t = 3 log1p(w), which keeps its precision
// when d is large and t is close to 1 (where 1 - t + log t cancels). For
// a < 1 the draw is boosted, G(a) = G(a + 1) U^(1/a) (the paper's section 6),
// with U from Philox block (env, step, stream, 0xffffffff). Attempt t uses
// Philox block (env, step, stream, 1 + t); after 32 rejected attempts
// (probability below 1e-40) the mean a is returned. The sampler is statistical,
// so it uses the hardware log2 / cos / sqrt for the proposal.
__device__ __forceinline__ float gamma_mt(float a, uint32_t env, uint32_t step, uint32_t stream, uint32_t k0,
                                          uint32_t k1) {
    const bool boost = a < 1.0f;
    const float k = boost ? a + 1.0f : a;
    const float d = k - (1.0f / 3.0f);
    const float c = __frsqrt_rn(9.0f * d);
    for (uint32_t t = 0; t < 32; t++) {
        const Ctr4 r = philox4x32_10(Ctr4{env, step, stream, 1u + t}, k0, k1);
        const float u1 = u24(r.x), u2 = u24(r.y), u = u24(r.z);
        const float z = __fsqrt_rn(-2.0f * __logf(u1)) * __cosf(6.283185307f * u2);
        const float w = c * z;
        if (w <= -1.0f) continue;
        const float v = 1.0f + w;
        const float cube = v * v * v;
        const float z2 = z * z;
        bool ok = u < 1.0f - 0.0331f * z2 * z2;
        if (!ok) {
            const float one_minus_t = -w * (3.0f + w * (3.0f + w));
            ok = __logf(u) < 0.5f * z2 + d * (one_minus_t + 3.0f * log1pf(w));
        }
        if (ok) {
            float g = d * cube;
            if (boost) {
                const Ctr4 rb = philox4x32_10(Ctr4{env, step, stream, 0xffffffffu}, k0, k1);
                g *= powf(u24(rb.x), 1.0f / a);
            }
            return g;
        }
    }
    return a;
}

// Third layer fused with the Beta draws: one workgroup per (16-env tile, group
// of 16 heads). Waves 0 and 1 compute the group's u and v column tiles of
// y = h2 W3 + b3 (K = 128, every load ahead of the first MFMA), the tile is
// kept in LDS (and written to y for sbx_policy_heads), and the 256 threads then
// take the group's 16 x 16 x 2 gamma draws, two each: lanes 2t and 2t + 1
// draw Ga and Gb of one head and the even lane writes x = Ga / (Ga + Gb)
// (continuous 2x - 1, discrete x > 0.5; 0 past the env's head counts). With
// `draws` set, the even lane also stores x and the head's log-density at x and
// entropy (hlp, hent; 0 past the head counts) for the rollout buffer.
constexpr int kHeadGroups = kActWidth / 16;   // 16 continuous groups, 1 discrete

__global__ __launch_bounds__(256) void heads_layer_kernel(const float* __restrict__ h2, const float* __restrict__ w3,
                                                          const float* __restrict__ b3, float* __restrict__ y,
                                                          float* __restrict__ actions, const int* __restrict__ n_cont,
                                                          const int* __restrict__ n_disc, int n, uint64_t seed,
                                                          uint32_t step, float* __restrict__ draws,
                                                          float* __restrict__ hlp, float* __restrict__ hent,
                                                          float floor) {
    constexpr int H = kPolicyHidden;
    __shared__ float ys[16][32 + 1];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int g = lane >> 4, i = lane & 15;
    const int m0 = blockIdx.x * 16, q = blockIdx.y;
    if (w < 2) {
        const int which = w;
        const int n0 = head_col(16 * q, which);
        const int mc = m0 + i < n ? m0 + i : n - 1;
        const float* a_row = h2 + (size_t)mc * H + 4 * g;
        const float* b_col = w3 + (size_t)(4 * g) * kPolicyHeads + n0 + i;
        float4 a[H / 16];
        float b[H / 16][4];
#pragma unroll
        for (int j = 0; j < H / 16; j++) {
            a[j] = *reinterpret_cast<const float4*>(a_row + 16 * j);
#pragma unroll
            for (int s = 0; s < 4; s++) b[j][s] = b_col[(size_t)(16 * j + s) * kPolicyHeads];
        }
#pragma unroll
        for (int j = 0; j < H / 16; j++) {
            asm volatile("" : "+v"(a[j].x), "+v"(a[j].y), "+v"(a[j].z), "+v"(a[j].w));
            asm volatile("" : "+v"(b[j][0]), "+v"(b[j][1]), "+v"(b[j][2]), "+v"(b[j][3]));
        }
        v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < H / 16; j++) {
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j].x, b[j][0], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j].y, b[j][1], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j].z, b[j][2], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j].w, b[j][3], acc, 0, 0, 0);
        }
        const float bv = b3[n0 + i];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int row = 4 * g + r;
            const float v = acc[r] + bv;
            ys[row][16 * which + i] = v;
            if (m0 + row < n) y[(size_t)(m0 + row) * kPolicyHeads + n0 + i] = v;
        }
    }
    __syncthreads();
    // draw d = 2 (row * 16 + k) + which of this group: 512 draws, two per thread
#pragma unroll
    for (int d0 = 0; d0 < 16 * 16 * 2; d0 += 256) {
        const int d = d0 + (int)threadIdx.x;
        const int which = d & 1, p = d >> 1;
        const int row = p >> 4, k = p & 15;
        const int e = m0 + row;
        const int h = 16 * q + k;
        const bool live = e < n;
        const int ec = live ? e : n - 1;
        const bool used = live && (h < SB_CONT ? h < n_cont[ec] : h - SB_CONT < n_disc[ec]);
        float gm = 1.0f;
        if (used) {
            const float a = beta_shape(ys[row][16 * which + k], floor);
            gm = gamma_mt(a, (uint32_t)e, step, 2u * (uint32_t)h + (uint32_t)which, (uint32_t)seed,
                          (uint32_t)(seed >> 32));
        }
        const float other = __shfl_xor(gm, 1, 64);
        if (live && which == 0) {
            float v = 0.0f, x = 0.0f;
            if (used) {
                x = gm / (gm + other);
                v = h < SB_CONT ? 2.0f * x - 1.0f : (x > 0.5f ? 1.0f : 0.0f);
            }
            actions[(size_t)e * kActWidth + h] = v;
            if (draws) {
                const size_t o = (size_t)e * kActWidth + h;
                draws[o] = x;
                float lp = 0.0f, en = 0.0f;
                if (used) {
                    const BetaHead bh = beta_head(ys[row][k], ys[row][16 + k], x, floor);
                    lp = (float)bh.logp;
                    en = (float)bh.entropy;
                }
                hlp[o] = lp;
                hent[o] = en;
            }
        }
    }
}

// Rollout-buffer evaluation of given draws (complete_port/patches/
// pufferlib_core.diff:944-1000): thread (e, h) takes head h of env e, u and v
// from y (head_col) and its draw x; writes the head's log-density,
// entropy and grad[e][k][h] (k: d logp/du, d logp/dv, d H/du, d H/dv), zeros
// past the env's head counts.
__global__ void beta_eval_kernel(const float* __restrict__ y, const float* __restrict__ draws,
                                 const int* __restrict__ n_cont, const int* __restrict__ n_disc, int n,
                                 float* __restrict__ hlp, float* __restrict__ hent, float* __restrict__ grad,
                                 float floor) {
    const int e = blockIdx.x, h = threadIdx.x;
    if (e >= n || h >= kActWidth) return;
    const bool used = h < SB_CONT ? h < n_cont[e] : h - SB_CONT < n_disc[e];
    const size_t o = (size_t)e * kActWidth + h;
    float lp = 0.0f, en = 0.0f, g[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (used) {
        const float* ye = y + (size_t)e * kPolicyHeads;
        const float u = ye[head_col(h, 0)];
        const float v = ye[head_col(h, 1)];
        const BetaHead bh = beta_head(u, v, draws[o], floor);
        lp = (float)bh.logp;
        en = (float)bh.entropy;
#pragma unroll
        for (int k = 0; k < 4; k++) g[k] = (float)bh.g[k];
    }
    hlp[o] = lp;
    hent[o] = en;
    if (grad) {
#pragma unroll
        for (int k = 0; k < 4; k++) grad[((size_t)e * 4 + k) * kActWidth + h] = g[k];
    }
}

// Per-env sums of the heads' log-densities and entropies, one wavefront per env
// in a fixed order (lane-strided partial sums, then a butterfly), so a sum does
// not depend on the batch it is in.
__global__ void beta_sum_kernel(const float* __restrict__ hlp, const float* __restrict__ hent, int n,
                                float* __restrict__ logp, float* __restrict__ entropy) {
    const int e = blockIdx.x, lane = threadIdx.x;
    if (e >= n) return;
    float a = 0.0f, b = 0.0f;
    for (int h = lane; h < kActWidth; h += 64) {
        a += hlp[(size_t)e * kActWidth + h];
        b += hent[(size_t)e * kActWidth + h];
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        a += __shfl_xor(a, m, 64);
        b += __shfl_xor(b, m, 64);
    }
    if (lane == 0) {
        logp[e] = a;
        entropy[e] = b;
    }
}

// Draws out[i] ~ Beta(alpha[i], beta[i]) with the heads' sampler (env = i, step 0, head 0).
__global__ void beta_sample_kernel(const float* alpha, const float* beta, float* out, int n, uint64_t seed) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
    const float ga = gamma_mt(alpha[i], (uint32_t)i, 0u, 0u, k0, k1);
    const float gb = gamma_mt(beta[i], (uint32_t)i, 0u, 1u, k0, k1);
    out[i] = ga / (ga + gb);
}

constexpr int kPpoThreads = (kActWidth + 63) / 64 * 64;   // one thread per head
static_assert(kPpoThreads <= 512, "the PPO reduction sums 512 slots");

// The PPO side of the Beta heads for one minibatch row per env
// (complete_port/patches/pufferlib_core.diff:1205-1252 ppo loss and its
// ratio_per_dim, :539-543, :1008-1014 beta_kl): one workgroup per env, thread h takes
// head h. Over the env's used heads (D of them), in f64 and a fixed summation
// order: logp = sum log p_new(x), H = sum entropies under the new heads,
// KL = sum KL(old head || new head). Then
//   r = exp(clamp(lr, -20, 20)), lr = (logp - logp_old) / (D if per_dim else 1)
//   pg = s * max(-A r, -A clamp(r, 1 - eps, 1 + eps)),  s = D if per_dim else 1
// (a non-finite lr counts as 0), and the gradient of pg - ent_coef * H in each
// head's raw outputs: d pg / d logp = g_r r with g_r = -A, or 0 where the
// clipped term is the larger and r lies outside the clip range; the per-dim
// scale s cancels the 1/D of the ratio. out[e][0..5] = logp, H, KL, r, pg, lr;
// grad[e][0][h] = d / du, grad[e][1][h] = d / dv (0 for unused heads).
__global__ __launch_bounds__(kPpoThreads) void ppo_beta_kernel(const float* __restrict__ y_new, const float* __restrict__ y_old,
                                                       const float* __restrict__ draws,
                                                       const float* __restrict__ logp_old, const float* __restrict__ adv,
                                                       const int* __restrict__ n_cont, const int* __restrict__ n_disc,
                                                       int n, float floor, float clip, float ent_coef, int per_dim,
                                                       float* __restrict__ out, float* __restrict__ grad) {
    __shared__ double red[3][512];
    __shared__ float dlp;
    const int e = blockIdx.x, t = (int)threadIdx.x;
    if (e >= n) return;
    const int nc = n_cont[e], nd = n_disc[e];
    const int h = t;
    const bool used = h < kActWidth && (h < SB_CONT ? h < nc : h - SB_CONT < nd);
    double lp = 0.0, en = 0.0, kl = 0.0;
    double g[4] = {0.0, 0.0, 0.0, 0.0};
    if (used) {
        const float* yn = y_new + (size_t)e * kPolicyHeads;
        const float* yo = y_old + (size_t)e * kPolicyHeads;
        const int cu = head_col(h, 0), cv = head_col(h, 1);
        const BetaHead bh = beta_head(yn[cu], yn[cv], draws[(size_t)e * kActWidth + h], floor);
        lp = bh.logp;
        en = bh.entropy;
#pragma unroll
        for (int k = 0; k < 4; k++) g[k] = bh.g[k];
        kl = beta_kl(beta_shape(yo[cu], floor), beta_shape(yo[cv], floor), beta_shape(yn[cu], floor),
                     beta_shape(yn[cv], floor));
    }
    for (int i = t; i < 512; i += (int)blockDim.x) {
        const bool mine = i == t;
        red[0][i] = mine ? lp : 0.0;
        red[1][i] = mine ? en : 0.0;
        red[2][i] = mine ? kl : 0.0;
    }
    __syncthreads();
    for (int w = 256; w > 0; w >>= 1) {
        for (int i = t; i < w; i += (int)blockDim.x)
            for (int q = 0; q < 3; q++) red[q][i] += red[q][i + w];
        __syncthreads();
    }
    if (t == 0) {
        const double lps = red[0][0], ens = red[1][0], kls = red[2][0];
        const int D = nc + nd;
        double lr = lps - (double)logp_old[e];
        if (per_dim) lr /= (double)(D > 0 ? D : 1);
        if (!isfinite(lr)) lr = 0.0;
        lr = fmin(20.0, fmax(-20.0, lr));
        const double r = exp(lr);
        const double A = (double)adv[e];
        const double lo = 1.0 - (double)clip, hi = 1.0 + (double)clip;
        const double l1 = -A * r, l2 = -A * fmin(hi, fmax(lo, r));
        double gr = -A;
        if (l2 > l1 && (r < lo || r > hi)) gr = 0.0;
        const double s = per_dim ? (double)(D > 0 ? D : 1) : 1.0;
        float* o = out + (size_t)e * 6;
        o[0] = (float)lps;
        o[1] = (float)ens;
        o[2] = (float)kls;
        o[3] = (float)r;
        o[4] = (float)(s * fmax(l1, l2));
        o[5] = (float)lr;
        dlp = (float)(gr * r);
    }
    __syncthreads();
    if (grad && h < kActWidth) {
        const double d = (double)dlp;
        grad[((size_t)e * 2 + 0) * kActWidth + h] = used ? (float)(d * g[0] - (double)ent_coef * g[2]) : 0.0f;
        grad[((size_t)e * 2 + 1) * kActWidth + h] = used ? (float)(d * g[1] - (double)ent_coef * g[3]) : 0.0f;
    }
}

}  // namespace sbk

// ---------------------------------------------------------------- launchers
// obs [n x 1024] -> h1, h2 [n x 128] -> y [n x 2 SB_ACT] -> actions [n x SB_ACT], on stream s.
// obs_cols: every observation row is zero from this column on (the longest
// observation prefix of the vec's envs).
// With draws set, also the rollout buffer's draws, per-head log-densities and
// entropies (hlp, hent [n x SB_ACT]) and their per-env sums (logp, entropy [n]).
extern "C" int sbk_launch_policy(const float* obs, const float* w1, const float* b1, const float* w2,
                                 const float* b2, const float* w3, const float* b3, float* h1, float* h2, float* y,
                                 float* actions, const int* n_cont, const int* n_disc, int n, uint64_t seed,
                                 uint32_t step, float* draws, float* hlp, float* hent, float* logp, float* entropy,
                                 float floor, int obs_cols, hipStream_t s) {
    using namespace sbk;
    if (n <= 0) return (int)hipErrorInvalidValue;
    if (obs_cols < 1 || obs_cols > kObsWidth) return (int)hipErrorInvalidValue;
    const int mt = (n + 15) / 16;
    // K split over 8 wavefronts (layer 1, K = 1024; the observation's zero
    // tail past obs_cols skipped) or 4 (K = 128)
    hipLaunchKernelGGL((mlp_layer_kernel<1, kObsWidth / 8>), dim3(mt, kPolicyHidden / 16), dim3(512), 0, s, obs,
                       kObsWidth, w1, b1, h1, kPolicyHidden, n, kPolicyHidden, obs_cols);
    hipLaunchKernelGGL((mlp_layer_kernel<1, kPolicyHidden / 4>), dim3(mt, kPolicyHidden / 16), dim3(256), 0, s, h1,
                       kPolicyHidden, w2, b2, h2, kPolicyHidden, n, kPolicyHidden, kPolicyHidden);
    // third layer and the Beta draws in one launch per (env tile, head group)
    hipLaunchKernelGGL(heads_layer_kernel, dim3(mt, kHeadGroups), dim3(256), 0, s, h2, w3, b3, y, actions, n_cont,
                       n_disc, n, seed, step, draws, hlp, hent, floor);
    if (draws) hipLaunchKernelGGL(beta_sum_kernel, dim3(n), dim3(64), 0, s, hlp, hent, n, logp, entropy);
    return (int)hipGetLastError();
}

// Log-densities, entropies and their gradients of given draws under heads y.
extern "C" int sbk_launch_beta_eval(const float* y, const float* draws, const int* n_cont, const int* n_disc, int n,
                                    float* hlp, float* hent, float* grad, float* logp, float* entropy, float floor,
                                    hipStream_t s) {
    using namespace sbk;
    if (n <= 0) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(beta_eval_kernel, dim3(n), dim3(kActWidth + 16), 0, s, y, draws, n_cont, n_disc, n, hlp,
                       hent, grad, floor);
    hipLaunchKernelGGL(beta_sum_kernel, dim3(n), dim3(64), 0, s, hlp, hent, n, logp, entropy);
    return (int)hipGetLastError();
}

extern "C" int sbk_launch_ppo_beta(const float* y_new, const float* y_old, const float* draws, const float* logp_old,
                                   const float* adv, const int* n_cont, const int* n_disc, int n, float floor,
                                   float clip, float ent_coef, int per_dim, float* out, float* grad, hipStream_t s) {
    if (n <= 0) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(sbk::ppo_beta_kernel, dim3(n), dim3(sbk::kPpoThreads), 0, s, y_new, y_old, draws, logp_old, adv, n_cont,
                       n_disc, n, floor, clip, ent_coef, per_dim, out, grad);
    return (int)hipGetLastError();
}

extern "C" int sbk_launch_beta_sample(const float* alpha, const float* beta, float* out, int n, uint64_t seed,
                                      hipStream_t s) {
    if (n <= 0) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(sbk::beta_sample_kernel, dim3((n + 255) / 256), dim3(256), 0, s, alpha, beta, out, n, seed);
    return (int)hipGetLastError();
}

// ------------------------------------------------- allocation-free policy step
// Activations of sbk_launch_policy_noalloc (h1 [n][128], h2 [n][128] and
// y [n][2 SB_ACT], at most kNoAllocEnvs envs: 12.5 MiB, 14.5 MiB with SB_CONT_BIG) in a file-scope device
// array. Each GPU the library runs on holds its own copy until the process
// ends. Every call on a GPU uses that GPU's copy: calls that overlap on one GPU
// race. Nothing in it needs clearing between calls: each layer writes every
// element of its output rows before the next layer reads them.
namespace {
constexpr int kNoAllocEnvs = 4096;
constexpr size_t kNoAllocFloats = (size_t)kNoAllocEnvs * (2 * sbk::kPolicyHidden + sbk::kPolicyHeads);
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch[kMaxDevices] = {};
}  // namespace

static __device__ __align__(256) float scratch[kNoAllocFloats];

// The device address of this GPU's scratch, looked up once per device with
// that device current (the array's name is only a host-side stand-in).
static int scratch_of_device(float** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    if (dev < 0 || dev >= kMaxDevices) return (int)hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return (int)e;
        g_scratch[dev] = static_cast<float*>(p);
    }
    *out = g_scratch[dev];
    return 0;
}

extern "C" int sbk_noalloc_max_envs(void) { return kNoAllocEnvs; }

// sbk_launch_policy without the rollout-buffer outputs, its activations in the
// scratch array: launches only, no allocation.
extern "C" int sbk_launch_policy_noalloc(const float* obs, const float* w1, const float* b1, const float* w2,
                                         const float* b2, const float* w3, const float* b3, float* actions,
                                         const int* n_cont, const int* n_disc, int n, uint64_t seed, uint32_t step,
                                         float floor, int obs_cols, hipStream_t s) {
    if (n <= 0 || n > kNoAllocEnvs) return (int)hipErrorInvalidValue;
    float* base = nullptr;
    const int rc = scratch_of_device(&base);
    if (rc != 0) return rc;
    float* h1 = base;
    float* h2 = h1 + (size_t)kNoAllocEnvs * sbk::kPolicyHidden;
    float* y = h2 + (size_t)kNoAllocEnvs * sbk::kPolicyHidden;
    return sbk_launch_policy(obs, w1, b1, w2, b2, w3, b3, h1, h2, y, actions, n_cont, n_disc, n, seed, step,
                             nullptr, nullptr, nullptr, nullptr, nullptr, floor, obs_cols, s);
}
