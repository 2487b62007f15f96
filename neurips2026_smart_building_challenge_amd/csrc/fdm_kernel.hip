// Building-scale field step on the device: the reference core's FDM step
// (complete_port/csim/sb_fdm.c:142-188, batched as sb_fdm_step_batch,
// :190-270) for a group of envs that share one baked factorization.
//
// Per step: forcing into the permuted vector (sb_fdm.c:147-151 with the
// permutation of sb_lu.c:41), the unit-lower and upper sweeps (sb_lu.c:42-61)
// as level-ordered row solves, the air-side correction (sb_fdm.c:153-182:
// sensed dots, the dense k x k solve, the applied scatter, a second solve),
// then the interior mass and the field (sb_fdm.c:183-187).
//
// Row form of the reference's column sweeps: the reference subtracts column
// j's product from every later row as it reaches j, so row i receives its
// products in ascending j (L) or descending j (U), each from a final value.
// Summing a row's terms in that order, with products rounded before the
// subtraction (this file is built with FP contraction off) and IEEE division,
// gives the reference's value bit for bit.
//
// Parallel form: one workgroup per block of envs runs every level of a factor
// (the envs of the block are lanes: a row's terms are read once and applied
// to Gl envs; 64 / Gl rows per wavefront), with a workgroup barrier between
// levels; blocks run independently. Every loop is bounded by the tables.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "fdm.h"

namespace {

constexpr int kSolveThreads = 1024;
constexpr int kEltThreads = 256;

__device__ __forceinline__ size_t gtid() { return (size_t)blockIdx.x * blockDim.x + threadIdx.x; }
__device__ __forceinline__ size_t gstride() { return (size_t)gridDim.x * blockDim.x; }

// Levels of one factor over the envs of block blockIdx.x, in place on W. A
// block with bact[b] == 0 (no env with an air side: a zero right-hand side
// whose solution is not used) returns at once. GL lanes per row (the block's
// envs), 64 / GL rows per wavefront.
template <bool UPPER, int GL>
__global__ __launch_bounds__(kSolveThreads) void solve_kernel(sbf::Tri tri, int n, double* W, const int* bact) {
    constexpr int R = 64 / GL;
    constexpr int STEP = (kSolveThreads / 64) * R;
    const int b = blockIdx.x;
    if (bact && !bact[b]) return;
    double* Wb = W + (size_t)b * n * GL;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int gl = lane % GL, rs = lane / GL;
    for (int l = 0; l < tri.nlev; l++) {
        const int lo = tri.lev[l], hi = tri.lev[l + 1];
        for (int q = lo + wave * R + rs; q < hi; q += STEP) {
            const int i = tri.rows[q];
            double acc = Wb[(size_t)i * GL + gl];
            const int e1 = tri.ptr[q + 1];
#pragma unroll 4
            for (int e = tri.ptr[q]; e < e1; e++) acc = acc - tri.val[e] * Wb[(size_t)tri.col[e] * GL + gl];
            if (UPPER) acc = acc / tri.diag[q];
            Wb[(size_t)i * GL + gl] = acc;
        }
        __syncthreads();
    }
}

// sum_p x[p] * W[row w[p]] over [p0, p1) in order, 8 terms per round trip
__device__ __forceinline__ double sensed_dot(const int* wrow, const double* x, int p0, int p1, const double* Wb,
                                             int Gl, int l) {
    constexpr int CH = 8;
    double acc = 0.0;
    for (int p = p0; p < p1; p += CH) {
        int c[CH];
        double v[CH], w[CH];
#pragma unroll
        for (int j = 0; j < CH; j++) {
            const bool ok = p + j < p1;
            c[j] = ok ? wrow[p + j] : 0;
            v[j] = ok ? x[p + j] : 0.0;
        }
#pragma unroll
        for (int j = 0; j < CH; j++) w[j] = Wb[(size_t)c[j] * Gl + l];
#pragma unroll
        for (int j = 0; j < CH; j++)
            if (p + j < p1) acc += v[j] * w[j];
    }
    return acc;
}

// Forcing (sb_fdm.c:147-151, exposure :126-140) written to the permuted row
// i = the row of solved cell ir[i]; clears the blocks' air-side flags.
__global__ void forcing_kernel(sbf::Tables t, sbf::Group g, sbf::StepIn in) {
    const int n = t.n, Gl = g.Gl, G = g.G;
    const size_t total = (size_t)g.nblk * n * Gl;
    for (size_t x = gtid(); x < total; x += gstride()) {
        const int l = (int)(x % Gl);
        const size_t bi = x / Gl;
        const int i = (int)(bi % n), b = (int)(bi / n);
        const int env = b * Gl + l;
        double w = 0.0;
        if (env < G) {
            const int tt = t.ir[i];
            const int p = t.solved[tt];
            const double h = in.h[env];
            double e = 0.0;
            const double a0 = t.a0[tt];
            if (a0 > 0.0) e += h * a0 / (1.0 + h * 0.5 * t.hz[tt] / t.cd[tt]);
            const double a1 = t.a1[tt];
            if (a1 > 0.0) e += h * a1 / (1.0 + h * 0.5 * t.vt[tt] / t.cd[tt]);
            w = t.cap[tt] * g.T[((size_t)b * t.n_cvs + p) * Gl + l] + in.q[(size_t)p * G + env]
                + in.amb[env] * (t.dir[tt] + e) + t.mcoup[tt] * g.M[((size_t)b * n + tt) * Gl + l];
        }
        g.W1[x] = w;
    }
    if (gtid() < (size_t)g.nblk) g.bact[gtid()] = 0;
}

// Per env and sensed row: the sensed temperature of the solution and the
// air-side power g (T_air - sensed) (sb_fdm.c:157-162).
__global__ void sensed_kernel(sbf::Tables t, sbf::Group g, sbf::StepIn in) {
    const int k = t.k, Gl = g.Gl;
    const size_t total = (size_t)g.G * k;
    for (size_t x = gtid(); x < total; x += gstride()) {
        const int env = (int)(x / k), i = (int)(x % k);
        const int b = env / Gl, l = env % Gl;
        const double acc = sensed_dot(t.sn_w, t.sn_x, t.sn_p[i], t.sn_p[i + 1], g.W1 + (size_t)b * t.n * Gl, Gl, l);
        g.pw[x] = in.g[x] * (in.airT[x] - acc);
    }
}

// Per env (one wavefront): whether its air side is on (sb_fdm.c:153-155), then
// M = I + diag(g) S and the partial-pivot solve of sb_fdm.c:9-38 in place on
// its power row: lanes own rows for the eliminations, lane 0 picks pivots and
// back-substitutes.
__global__ __launch_bounds__(64) void dense_kernel(sbf::Tables t, sbf::Group g, sbf::StepIn in) {
    __shared__ int s_piv, s_sing;
    const int env = blockIdx.x, k = t.k, lane = threadIdx.x;
    const double* gv = in.g + (size_t)env * k;
    int any = 0;
    for (int i = lane; i < k; i += 64) any |= gv[i] != 0.0;
    any = __any(any);
    if (lane == 0) {
        g.eact[env] = any;
        if (any) atomicOr(&g.bact[env / g.Gl], 1);
    }
    if (!any) return;
    double* M = g.mat + (size_t)env * k * k;
    double* bv = g.pw + (size_t)env * k;
    for (int x = lane; x < k * k; x += 64) {
        const int i = x / k, j = x % k;
        M[x] = (i == j ? 1.0 : 0.0) + gv[i] * t.S[x];
    }
    __syncthreads();
    for (int c = 0; c < k; c++) {
        if (lane == 0) {
            int piv = c;
            double best = fabs(M[(size_t)c * k + c]);
            for (int r = c + 1; r < k; r++) {
                const double v = fabs(M[(size_t)r * k + c]);
                if (v > best) {
                    best = v;
                    piv = r;
                }
            }
            s_piv = piv;
            s_sing = best == 0.0;
        }
        __syncthreads();
        if (s_sing) return;   // the reference returns here, leaving the partly reduced row
        const int piv = s_piv;
        if (piv != c) {
            for (int j = c + lane; j < k; j += 64) {
                const double tmp = M[(size_t)c * k + j];
                M[(size_t)c * k + j] = M[(size_t)piv * k + j];
                M[(size_t)piv * k + j] = tmp;
            }
            if (lane == 0) {
                const double tmp = bv[c];
                bv[c] = bv[piv];
                bv[piv] = tmp;
            }
            __syncthreads();
        }
        const double d = M[(size_t)c * k + c];
        for (int r = c + 1 + lane; r < k; r += 64) {
            const double f = M[(size_t)r * k + c] / d;
            if (f == 0.0) continue;
            for (int j = c; j < k; j++) M[(size_t)r * k + j] -= f * M[(size_t)c * k + j];
            bv[r] -= f * bv[c];
        }
        __syncthreads();
    }
    if (lane == 0) {
        for (int r = k - 1; r >= 0; r--) {
            double s = bv[r];
            for (int j = r + 1; j < k; j++) s -= M[(size_t)r * k + j] * bv[j];
            bv[r] = s / M[(size_t)r * k + r];
        }
    }
}

// The applied heat of the solved powers (sb_fdm.c:171-177), permuted into the
// correction's right-hand side; zero for envs without an air side.
__global__ void applied_kernel(sbf::Tables t, sbf::Group g) {
    const int n = t.n, Gl = g.Gl, G = g.G, k = t.k;
    const size_t total = (size_t)g.nblk * n * Gl;
    for (size_t x = gtid(); x < total; x += gstride()) {
        const int l = (int)(x % Gl);
        const size_t bi = x / Gl;
        const int i = (int)(bi % n), b = (int)(bi / n);
        const int env = b * Gl + l;
        double acc = 0.0;
        if (env < G && g.eact[env]) {
            const double* qv = g.pw + (size_t)env * k;
            for (int e = t.at_p[i]; e < t.at_p[i + 1]; e++) {
                const double qj = qv[t.at_j[e]];
                if (qj == 0.0) continue;
                acc += t.at_x[e] * qj;
            }
        }
        g.W2[x] = acc;
    }
}

// y = the forcing solve (+ the correction where the air side is on), the
// interior mass and the field (sb_fdm.c:178, 183-187).
__global__ void update_kernel(sbf::Tables t, sbf::Group g, sbf::StepIn in) {
    const int n = t.n, Gl = g.Gl, G = g.G;
    const size_t total = (size_t)g.nblk * n * Gl;
    for (size_t x = gtid(); x < total; x += gstride()) {
        const int l = (int)(x % Gl);
        const size_t bt = x / Gl;
        const int tt = (int)(bt % n), b = (int)(bt / n);
        const int env = b * Gl + l;
        if (env >= G) continue;
        const size_t wi = ((size_t)b * n + t.pc[tt]) * Gl + l;
        double y = g.W1[wi];
        if (g.eact[env]) y += g.W2[wi];
        g.M[x] = g.M[x] * t.mret[tt] + t.mgain[tt] * y;
        g.T[((size_t)b * t.n_cvs + t.solved[tt]) * Gl + l] = y;
    }
    const size_t tu = (size_t)g.nblk * t.n_unsolved * Gl;
    for (size_t x = gtid(); x < tu; x += gstride()) {
        const int l = (int)(x % Gl);
        const size_t bu = x / Gl;
        const int u = (int)(bu % t.n_unsolved), b = (int)(bu / t.n_unsolved);
        const int env = b * Gl + l;
        if (env >= G) continue;
        g.T[((size_t)b * t.n_cvs + t.unsolved[u]) * Gl + l] = in.amb[env];
    }
}

// Every env's fields from the blob's initial fields.
__global__ void init_kernel(sbf::Tables t, sbf::Group g, const double* temp_init, const double* mass_init) {
    const int Gl = g.Gl;
    const size_t tc = (size_t)g.nblk * t.n_cvs * Gl;
    for (size_t x = gtid(); x < tc; x += gstride()) g.T[x] = temp_init[(x / Gl) % t.n_cvs];
    const size_t tm = (size_t)g.nblk * t.n * Gl;
    for (size_t x = gtid(); x < tm; x += gstride()) g.M[x] = mass_init[(x / Gl) % t.n];
}

// Right-hand sides b [G][n] (solved order) into the permuted vector, or the
// unit columns of the applied matrix (column j = env; sb_fdm.c:106-107 assigns
// them) when b is null.
__global__ void rhs_kernel(sbf::Tables t, sbf::Group g, const double* b_in) {
    const int n = t.n, Gl = g.Gl, G = g.G;
    const size_t total = (size_t)g.nblk * n * Gl;
    for (size_t x = gtid(); x < total; x += gstride()) {
        const int l = (int)(x % Gl);
        const size_t bi = x / Gl;
        const int i = (int)(bi % n), b = (int)(bi / n);
        const int env = b * Gl + l;
        double w = 0.0;
        if (env < G) {
            if (b_in) {
                w = b_in[(size_t)env * n + t.ir[i]];
            } else {
                for (int e = t.at_p[i]; e < t.at_p[i + 1]; e++)
                    if (t.at_j[e] == env) w = t.at_x[e];
            }
        }
        g.W1[x] = w;
    }
}

// x [G][n] (solved order) from the permuted solution.
__global__ void sol_kernel(sbf::Tables t, sbf::Group g, double* x_out) {
    const int n = t.n, Gl = g.Gl;
    const size_t total = (size_t)g.G * n;
    for (size_t x = gtid(); x < total; x += gstride()) {
        const int env = (int)(x / n), tt = (int)(x % n);
        const int b = env / Gl, l = env % Gl;
        x_out[x] = g.W1[((size_t)b * n + t.pc[tt]) * Gl + l];
    }
}

// S[i][j] = sensed row i of the solution of applied column j (sb_fdm.c:104-116).
__global__ void sresp_kernel(sbf::Tables t, sbf::Group g, double* S) {
    const int k = t.k, Gl = g.Gl;
    const size_t total = (size_t)k * k;
    for (size_t x = gtid(); x < total; x += gstride()) {
        const int i = (int)(x / k), j = (int)(x % k);
        const int b = j / Gl, l = j % Gl;
        S[x] = sensed_dot(t.sn_w, t.sn_x, t.sn_p[i], t.sn_p[i + 1], g.W1 + (size_t)b * t.n * Gl, Gl, l);
    }
}

int elt_grid(size_t total) {
    const size_t b = (total + kEltThreads - 1) / kEltThreads;
    return (int)(b < 1 ? 1 : (b > 16384 ? 16384 : b));
}

template <int GL>
void solve_gl(const sbf::Tables& t, const sbf::Group& g, double* W, const int* bact, hipStream_t s) {
    hipLaunchKernelGGL((solve_kernel<false, GL>), dim3(g.nblk), dim3(kSolveThreads), 0, s, t.L, t.n, W, bact);
    hipLaunchKernelGGL((solve_kernel<true, GL>), dim3(g.nblk), dim3(kSolveThreads), 0, s, t.U, t.n, W, bact);
}

int solve(const sbf::Tables& t, const sbf::Group& g, double* W, const int* bact, hipStream_t s) {
    switch (g.Gl) {
    case 1: solve_gl<1>(t, g, W, bact, s); break;
    case 2: solve_gl<2>(t, g, W, bact, s); break;
    case 4: solve_gl<4>(t, g, W, bact, s); break;
    case 8: solve_gl<8>(t, g, W, bact, s); break;
    case 16: solve_gl<16>(t, g, W, bact, s); break;
    case 32: solve_gl<32>(t, g, W, bact, s); break;
    case 64: solve_gl<64>(t, g, W, bact, s); break;
    default: return (int)hipErrorInvalidValue;
    }
    return (int)hipGetLastError();
}

}  // namespace

// One batched step of a group (all launches on stream s).
extern "C" int sbf_launch_step(const sbf::Tables* t, const sbf::Group* g, const sbf::StepIn* in, hipStream_t s) {
    const size_t rows = (size_t)g->nblk * t->n * g->Gl;
    hipLaunchKernelGGL(forcing_kernel, dim3(elt_grid(rows)), dim3(kEltThreads), 0, s, *t, *g, *in);
    if (int e = solve(*t, *g, g->W1, nullptr, s)) return e;
    if (t->k > 0) {
        hipLaunchKernelGGL(sensed_kernel, dim3(elt_grid((size_t)g->G * t->k)), dim3(kEltThreads), 0, s, *t, *g, *in);
        hipLaunchKernelGGL(dense_kernel, dim3(g->G), dim3(64), 0, s, *t, *g, *in);
        hipLaunchKernelGGL(applied_kernel, dim3(elt_grid(rows)), dim3(kEltThreads), 0, s, *t, *g);
        if (int e = solve(*t, *g, g->W2, g->bact, s)) return e;
    }
    hipLaunchKernelGGL(update_kernel, dim3(elt_grid(rows)), dim3(kEltThreads), 0, s, *t, *g, *in);
    return (int)hipGetLastError();
}

extern "C" int sbf_launch_init(const sbf::Tables* t, const sbf::Group* g, const double* temp_init,
                               const double* mass_init, hipStream_t s) {
    hipLaunchKernelGGL(init_kernel, dim3(elt_grid((size_t)g->nblk * t->n_cvs * g->Gl)), dim3(kEltThreads), 0, s, *t,
                       *g, temp_init, mass_init);
    return (int)hipGetLastError();
}

// x = A^-1 b for the G columns of b [G][n] (b null: the applied columns, then
// S [k][k] is written from the solutions).
extern "C" int sbf_launch_solve_cols(const sbf::Tables* t, const sbf::Group* g, const double* b, double* x,
                                     double* S, hipStream_t s) {
    const size_t rows = (size_t)g->nblk * t->n * g->Gl;
    hipLaunchKernelGGL(rhs_kernel, dim3(elt_grid(rows)), dim3(kEltThreads), 0, s, *t, *g, b);
    if (int e = solve(*t, *g, g->W1, nullptr, s)) return e;
    if (x) hipLaunchKernelGGL(sol_kernel, dim3(elt_grid((size_t)g->G * t->n)), dim3(kEltThreads), 0, s, *t, *g, x);
    if (S) hipLaunchKernelGGL(sresp_kernel, dim3(elt_grid((size_t)t->k * t->k)), dim3(kEltThreads), 0, s, *t, *g, S);
    return (int)hipGetLastError();
}
