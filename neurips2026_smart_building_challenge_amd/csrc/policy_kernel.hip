// Shared-policy MLP forward + Beta action sampling for MI355X (gfx950), the
// rollout-loop workload of BASELINE config 5: every env's observation row goes
// through the same fp32 MLP
//
//   h1 = tanh(obs W1 + b1)   [n x 1024] x [1024 x 128]
//   h2 = tanh(h1 W2 + b2)    [n x 128]  x [128 x 128]
//   y  = h2 W3 + b3          [n x 128]  x [128 x 544] = (u[256], v[256], ud[16], vd[16])
//
// and each action head j draws x ~ Beta(softplus(u_j) + 1, softplus(v_j) + 1);
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

namespace sbk {

typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kPolicyHidden = 128;
constexpr int kPolicyHeads = 2 * 256 + 2 * 16;   // u, v of the continuous and the discrete heads
constexpr int kObsWidth = 1024;
constexpr int kActWidth = 272;

// C[M x N] = act(A[M x K] B[K x N] + bias) with K = KW * (blockDim.x / 64):
// wavefront w takes K range [w KW, (w + 1) KW) and issues every load of that
// range before its first MFMA (one memory latency per tile). lda / ldc in
// floats; N a multiple of 16. ACT: 0 identity, 1 tanh.
template <int ACT, int KW>
__global__ __launch_bounds__(256) void mlp_layer_kernel(const float* __restrict__ A, int lda,
                                                        const float* __restrict__ B,
                                                        const float* __restrict__ bias, float* __restrict__ C,
                                                        int ldc, int M, int N) {
    static_assert(KW % 16 == 0, "K per wavefront is a multiple of 16");
    constexpr int NB = KW / 16;
    __shared__ v4f part[4][64];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, ksplit = blockDim.x >> 6;
    const int m0 = blockIdx.x * 16, n0 = blockIdx.y * 16;
    const int g = lane >> 4, i = lane & 15;
    const int m = m0 + i;
    const int mc = m < M ? m : M - 1;   // rows past M read row M - 1; their outputs are dropped
    const float* a_row = A + (size_t)mc * lda + w * KW + 4 * g;
    const float* b_col = B + (size_t)(w * KW + 4 * g) * N + n0 + i;
    float4 a[NB];
    float b[NB][4];
#pragma unroll
    for (int j = 0; j < NB; j++) {
        a[j] = *reinterpret_cast<const float4*>(a_row + 16 * j);
        const float* bp = b_col + (size_t)(16 * j) * N;
#pragma unroll
        for (int s = 0; s < 4; s++) b[j][s] = bp[s * N];
    }
    // the empty asm "uses" every loaded register here, so the compiler keeps
    // all loads ahead of the first MFMA instead of sinking each to its use
#pragma unroll
    for (int j = 0; j < NB; j++) {
        asm volatile("" : "+v"(a[j].x), "+v"(a[j].y), "+v"(a[j].z), "+v"(a[j].w));
        asm volatile("" : "+v"(b[j][0]), "+v"(b[j][1]), "+v"(b[j][2]), "+v"(b[j][3]));
    }
    v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < NB; j++) {
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j].x, b[j][0], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j].y, b[j][1], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j].z, b[j][2], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j].w, b[j][3], acc, 0, 0, 0);
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

__device__ __forceinline__ float softplus(float x) { return x > 20.0f ? x : log1pf(expf(x)); }

// Gamma(a) for a >= 1 (Marsaglia and Tsang, "A simple method for generating
// gamma variables", ACM TOMS 26(3), 2000): d = a - 1/3, c = 1/sqrt(9d); draw
// z ~ N(0, 1) (Box-Muller) and u ~ U(0, 1), v = (1 + cz)^3, accept d v when
// v > 0 and u < 1 - 0.0331 z^4 or log u < z^2/2 + d (1 - v + log v). Attempt t
// uses Philox block (env, step, stream, 1 + t); after 32 rejected attempts
// (probability below 1e-40 for a >= 1) the mean a is returned. The sampler is
// statistical, so it uses the hardware log2 / cos / sqrt.
__device__ __forceinline__ float gamma_mt(float a, uint32_t env, uint32_t step, uint32_t stream, uint32_t k0,
                                          uint32_t k1) {
    const float d = a - (1.0f / 3.0f);
    const float c = __frsqrt_rn(9.0f * d);
    for (uint32_t t = 0; t < 32; t++) {
        const Ctr4 r = philox4x32_10(Ctr4{env, step, stream, 1u + t}, k0, k1);
        const float u1 = u24(r.x), u2 = u24(r.y), u = u24(r.z);
        const float z = __fsqrt_rn(-2.0f * __logf(u1)) * __cosf(6.283185307f * u2);
        float v = 1.0f + c * z;
        if (v <= 0.0f) continue;
        v = v * v * v;
        const float z2 = z * z;
        if (u < 1.0f - 0.0331f * z2 * z2) return d * v;
        if (__logf(u) < 0.5f * z2 + d * (1.0f - v + __logf(v))) return d * v;
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
                                                          float* __restrict__ hlp, float* __restrict__ hent) {
    constexpr int H = kPolicyHidden;
    __shared__ float ys[16][32 + 1];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int g = lane >> 4, i = lane & 15;
    const int m0 = blockIdx.x * 16, q = blockIdx.y;
    if (w < 2) {
        const int which = w;
        const int n0 = q < 16 ? 16 * q + 256 * which : 512 + 16 * which;
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
        const bool used = live && (h < 256 ? h < n_cont[ec] : h - 256 < n_disc[ec]);
        float gm = 1.0f;
        if (used) {
            const float a = softplus(ys[row][16 * which + k]) + 1.0f;
            gm = gamma_mt(a, (uint32_t)e, step, 2u * (uint32_t)h + (uint32_t)which, (uint32_t)seed,
                          (uint32_t)(seed >> 32));
        }
        const float other = __shfl_xor(gm, 1, 64);
        if (live && which == 0) {
            float v = 0.0f, x = 0.0f;
            if (used) {
                x = gm / (gm + other);
                v = h < 256 ? 2.0f * x - 1.0f : (x > 0.5f ? 1.0f : 0.0f);
            }
            actions[(size_t)e * kActWidth + h] = v;
            if (draws) {
                const size_t o = (size_t)e * kActWidth + h;
                draws[o] = x;
                float lp = 0.0f, en = 0.0f;
                if (used) {
                    const BetaHead bh = beta_head(ys[row][k], ys[row][16 + k], x);
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
// from y (continuous head h: columns h and 256 + h; discrete head d = h - 256:
// columns 512 + d and 528 + d) and its draw x; writes the head's log-density,
// entropy and grad[e][k][h] (k: d logp/du, d logp/dv, d H/du, d H/dv), zeros
// past the env's head counts.
__global__ void beta_eval_kernel(const float* __restrict__ y, const float* __restrict__ draws,
                                 const int* __restrict__ n_cont, const int* __restrict__ n_disc, int n,
                                 float* __restrict__ hlp, float* __restrict__ hent, float* __restrict__ grad) {
    const int e = blockIdx.x, h = threadIdx.x;
    if (e >= n || h >= kActWidth) return;
    const bool used = h < 256 ? h < n_cont[e] : h - 256 < n_disc[e];
    const size_t o = (size_t)e * kActWidth + h;
    float lp = 0.0f, en = 0.0f, g[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (used) {
        const float* ye = y + (size_t)e * kPolicyHeads;
        const float u = h < 256 ? ye[h] : ye[512 + (h - 256)];
        const float v = h < 256 ? ye[256 + h] : ye[528 + (h - 256)];
        const BetaHead bh = beta_head(u, v, draws[o]);
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

}  // namespace sbk

// ---------------------------------------------------------------- launchers
// obs [n x 1024] -> h1, h2 [n x 128] -> y [n x 544] -> actions [n x 272], on stream s.
// With draws set, also the rollout buffer's draws, per-head log-densities and
// entropies (hlp, hent [n x 272]) and their per-env sums (logp, entropy [n]).
extern "C" int sbk_launch_policy(const float* obs, const float* w1, const float* b1, const float* w2,
                                 const float* b2, const float* w3, const float* b3, float* h1, float* h2, float* y,
                                 float* actions, const int* n_cont, const int* n_disc, int n, uint64_t seed,
                                 uint32_t step, float* draws, float* hlp, float* hent, float* logp, float* entropy,
                                 hipStream_t s) {
    using namespace sbk;
    if (n <= 0) return (int)hipErrorInvalidValue;
    const int mt = (n + 15) / 16;
    // K split over 4 wavefronts (layer 1, K = 1024) or 2 (K = 128)
    hipLaunchKernelGGL((mlp_layer_kernel<1, kObsWidth / 4>), dim3(mt, kPolicyHidden / 16), dim3(256), 0, s, obs,
                       kObsWidth, w1, b1, h1, kPolicyHidden, n, kPolicyHidden);
    hipLaunchKernelGGL((mlp_layer_kernel<1, kPolicyHidden / 2>), dim3(mt, kPolicyHidden / 16), dim3(128), 0, s, h1,
                       kPolicyHidden, w2, b2, h2, kPolicyHidden, n, kPolicyHidden);
    // third layer and the Beta draws in one launch per (env tile, head group)
    hipLaunchKernelGGL(heads_layer_kernel, dim3(mt, kHeadGroups), dim3(256), 0, s, h2, w3, b3, y, actions, n_cont,
                       n_disc, n, seed, step, draws, hlp, hent);
    if (draws) hipLaunchKernelGGL(beta_sum_kernel, dim3(n), dim3(64), 0, s, hlp, hent, n, logp, entropy);
    return (int)hipGetLastError();
}

// Log-densities, entropies and their gradients of given draws under heads y.
extern "C" int sbk_launch_beta_eval(const float* y, const float* draws, const int* n_cont, const int* n_disc, int n,
                                    float* hlp, float* hent, float* grad, float* logp, float* entropy,
                                    hipStream_t s) {
    using namespace sbk;
    if (n <= 0) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(beta_eval_kernel, dim3(n), dim3(kActWidth + 16), 0, s, y, draws, n_cont, n_disc, n, hlp,
                       hent, grad);
    hipLaunchKernelGGL(beta_sum_kernel, dim3(n), dim3(64), 0, s, hlp, hent, n, logp, entropy);
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
// y [n][544], at most kNoAllocEnvs envs: 12.5 MiB) in a file-scope device
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
                                         hipStream_t s) {
    if (n <= 0 || n > kNoAllocEnvs) return (int)hipErrorInvalidValue;
    float* base = nullptr;
    const int rc = scratch_of_device(&base);
    if (rc != 0) return rc;
    float* h1 = base;
    float* h2 = h1 + (size_t)kNoAllocEnvs * sbk::kPolicyHidden;
    float* y = h2 + (size_t)kNoAllocEnvs * sbk::kPolicyHidden;
    return sbk_launch_policy(obs, w1, b1, w2, b2, w3, b3, h1, h2, y, actions, n_cont, n_disc, n, seed, step,
                             nullptr, nullptr, nullptr, nullptr, nullptr, s);
}
