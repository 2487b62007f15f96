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

#include <algorithm>

#include "fdm.h"

namespace {

constexpr int kSolveThreads = 1024;
// the chunked runs: a level's chain (chunk sums, LDS barrier, row finishes,
// barrier) is shorter with 8 wavefronts than with 16 (16.4 ms with 4, 15.2
// with 8, 17.9 with 16 per step at 256 envs of the 205K-cell plan)
constexpr int kRunThreads = 512;
constexpr int kEltThreads = 256;

__device__ __forceinline__ size_t gtid() { return (size_t)blockIdx.x * blockDim.x + threadIdx.x; }
__device__ __forceinline__ size_t gstride() { return (size_t)gridDim.x * blockDim.x; }

// Levels of one factor over the envs of block blockIdx.x, in place on W. A
// block with bact[b] == 0 (no env with an air side: a zero right-hand side
// whose solution is not used) returns at once. GL lanes per row (the block's
// envs), 64 / GL rows per wavefront.
template <bool UPPER, int GL>
__global__ __launch_bounds__(kSolveThreads) void solve_kernel(sbf::Tri tri, int lev_begin, int lev_end, int n,
                                                              double* W, const int* bact) {
    constexpr int R = 64 / GL;
    constexpr int STEP = (kSolveThreads / 64) * R;
    const int b = blockIdx.x;
    if (bact && !bact[b]) return;
    double* Wb = W + (size_t)b * n * GL;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int gl = lane % GL, rs = lane / GL;
    for (int l = lev_begin; l < lev_end; l++) {
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

template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ double dpp_d(double v) {
    const unsigned long long x = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_update_dpp(0, (int)(unsigned)x, CTRL, ROWS, 0xF, false);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(unsigned)(x >> 32), CTRL, ROWS, 0xF, false);
    return __longlong_as_double((long long)(((unsigned long long)(unsigned)hi << 32) | (unsigned)lo));
}

// Sum over a wavefront's lanes that share an env (lanes l, l + GL, ...), in a
// fixed order; every lane gets the total. One env per wavefront (GL = 1): DPP
// lane moves (quad permutes, row mirrors, row broadcasts; no LDS traffic),
// the total read from lane 63; otherwise a butterfly over the env's lanes.
template <int GL>
__device__ __forceinline__ double lane_sum(double v) {
    if constexpr (GL == 1) {
        v += dpp_d<0xB1>(v);          // quad_perm [1,0,3,2]
        v += dpp_d<0x4E>(v);          // quad_perm [2,3,0,1]
        v += dpp_d<0x141>(v);         // row_half_mirror
        v += dpp_d<0x140>(v);         // row_mirror
        v += dpp_d<0x142, 0xA>(v);    // row_bcast:15
        v += dpp_d<0x143, 0xC>(v);    // row_bcast:31
        const unsigned long long x = __double_as_longlong(v);
        const unsigned lo = __builtin_amdgcn_readlane((int)(unsigned)x, 63);
        const unsigned hi = __builtin_amdgcn_readlane((int)(unsigned)(x >> 32), 63);
        return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
    } else {
#pragma unroll
        for (int off = GL; off < 64; off <<= 1) v += __shfl_xor(v, off, 64);
        return v;
    }
}

// Head terms of the tail rows (columns finished before the tail's first
// level): W[row] -= their sum, one wavefront per (group of kHeadBlocks blocks,
// tail row), block groups outermost (each block's vector stays in the caches
// from row to row), the terms spread over the lanes of each env. A term's
// value and column are loaded once for the group's blocks, so the factor's
// head terms are read once per kHeadBlocks blocks; every env's sum has the
// same terms per lane, order and lane tree as with one block per wavefront.
constexpr int kHeadBlocks = 8;
template <int GL>
__global__ __launch_bounds__(256) void head_kernel(sbf::Tail tl, int n, int nblk, double* W, const int* bact) {
    constexpr int S = 64 / GL, E = kHeadBlocks;
    const int lane = threadIdx.x & 63;
    const int gl = lane % GL, s = lane / GL;
    const int nbg = (nblk + E - 1) / E;
    const size_t nw = (size_t)gridDim.x * (blockDim.x >> 6);
    for (size_t x = (size_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6); x < (size_t)nbg * tl.m; x += nw) {
        const int bg = (int)(x / tl.m), r = (int)(x % tl.m);
        bool on[E];
        double* Wb[E];
        double acc[E];
        bool any = false;
#pragma unroll
        for (int k = 0; k < E; k++) {
            const int b = bg * E + k;
            on[k] = b < nblk && (!bact || bact[b]);   // wavefront-uniform
            any |= on[k];
            Wb[k] = W + (size_t)(b < nblk ? b : 0) * n * GL;
            acc[k] = 0.0;
        }
        if (!any) continue;
        const int e1 = tl.hptr[r + 1];
        for (int e = tl.hptr[r] + s; e < e1; e += S) {
            const double v = tl.hval[e];
            const size_t c = (size_t)tl.hcol[e] * GL + gl;
#pragma unroll
            for (int k = 0; k < E; k++)
                if (on[k]) acc[k] += v * Wb[k][c];
        }
        const size_t row = (size_t)tl.rows[r] * GL + gl;
#pragma unroll
        for (int k = 0; k < E; k++) {
            if (!on[k]) continue;
            const double t = lane_sum<GL>(acc[k]);
            if (s == 0) Wb[k][row] -= t;
        }
    }
}

// Workgroup barrier ordering LDS accesses only: global loads in flight (the
// next level's chunks) stay in flight across it.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// The levels of one run (sbf::Tail) of one block (one workgroup), in order:
//   tmode 0 (no row has more than one chunk): each lane takes a row, forms its
//     chunk's sum and finishes it;
//   tmode 1 and 2: each lane forms the partial sum of one chunk of kChunk
//     terms into LDS, then, after an LDS barrier, rows are finished from their
//     chunks' partials, one lane per row (tmode 1, wide levels) or one
//     wavefront per row (tmode 2, a few long rows);
//   tmode 3 (a few rows, each with no more chunks than a wavefront has lanes
//     per env): each wavefront takes a row, its lanes sum the row's chunks and
//     the wavefront adds the lanes' sums.
// Each level starts by loading the first chunk each lane uses in the next
// level and, in HBM runs, the value of the first row it will finish there.
// LDSW: the run's row values live in LDS (loaded at the start, stored at the
// end), chunk positions index the run and levels are separated by LDS
// barriers; otherwise values are read from and written to HBM, positions are
// row ids and levels are separated by full workgroup barriers.
typedef const __attribute__((address_space(4))) int* cint_ptr;

template <bool UPPER, int GL, bool LDSW>
__global__ __launch_bounds__(kRunThreads) void run_kernel(sbf::Tail tl, int n, double* W, const int* bact) {
    extern __shared__ double lds[];
    // level metadata is uniform: read through the scalar (constant) path, so
    // these reads do not queue behind the vector loads of the prefetch
    const cint_ptr trow = (cint_ptr)tl.trow;
    const cint_ptr tchunk = (cint_ptr)tl.tchunk;
    const cint_ptr tmode = (cint_ptr)tl.tmode;
    constexpr int NS = kRunThreads / GL;   // lane slots of the workgroup per env
    constexpr int NW = kRunThreads / 64;
    constexpr int S = 64 / GL;
    constexpr int K = sbf::kChunk;
    const int b = blockIdx.x;
    if (bact && !bact[b]) return;
    double* Wb = W + (size_t)b * n * GL;
    double* Wt = lds;
    double* P = LDSW ? lds + (size_t)tl.m * GL : lds;
    // the wavefront index through readfirstlane: a row taken by a whole
    // wavefront is then known to be wave-uniform, so its chunk bounds and
    // metadata are read with scalar loads
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int gl = tid % GL, slot = tid / GL;
    const int s = lane / GL;
    if (LDSW)
        for (int x = tid; x < tl.m * GL; x += kRunThreads) Wt[x] = Wb[(size_t)tl.rows[x / GL] * GL + x % GL];
    struct Chunk {
        int4 a0, a1;
        double v[K];
    };
    auto fetch = [&](int c, Chunk& ch) {
        const int4* cp = reinterpret_cast<const int4*>(tl.cpos + (size_t)K * c);
        const double2* cv = reinterpret_cast<const double2*>(tl.cval + (size_t)K * c);
        ch.a0 = cp[0];
        ch.a1 = cp[1];
#pragma unroll
        for (int j = 0; j < K / 2; j++) {
            const double2 d = cv[j];
            ch.v[2 * j] = d.x;
            ch.v[2 * j + 1] = d.y;
        }
    };
    auto val = [&](int pos) -> double { return LDSW ? Wt[pos * GL + gl] : Wb[(size_t)pos * GL + gl]; };
    auto part = [&](const Chunk& ch) {
        const int pos[K] = {ch.a0.x, ch.a0.y, ch.a0.z, ch.a0.w, ch.a1.x, ch.a1.y, ch.a1.z, ch.a1.w};
        double w[K];
#pragma unroll
        for (int j = 0; j < K; j++) w[j] = val(pos[j]);
        double acc = ch.v[0] * w[0];
#pragma unroll
        for (int j = 1; j < K; j++) acc += ch.v[j] * w[j];
        return acc;
    };
    auto own_ref = [&](int r) -> double* { return LDSW ? &Wt[r * GL + gl] : &Wb[(size_t)tl.rows[r] * GL + gl]; };

    // the first row this lane finishes in level t (-1: none) and the chunk it
    // starts the level with (-1: none)
    auto first_row = [&](int t) -> int {
        const int mode = tmode[t];
        const bool by_wave = mode >= 2;
        const int r = trow[t] + (by_wave ? wave : slot);
        return (r < trow[t + 1] && (!by_wave || s == 0)) ? r : -1;
    };
    auto first_chunk = [&](int t) -> int {
        const int mode = tmode[t];
        if (mode == 1 || mode == 2) {
            const int c = tchunk[t] + slot;
            return c < tchunk[t + 1] ? c : -1;
        }
        const int r = trow[t] + (mode == 3 ? wave : slot);
        if (r >= trow[t + 1]) return -1;
        const int c = tl.rchunk[r] + (mode == 3 ? s : 0);
        return c < tl.rchunk[r + 1] ? c : -1;
    };
    // this level's first chunk, row value (HBM runs) and diagonal (U) of the
    // first row this lane finishes (cur*), the next level's (nxt*)
    Chunk cur, nxt;
    int curc = -1, curr = -1, nxtc = -1, nxtr = -1;
    double curo = 0.0, nxto = 0.0, curd = 1.0, nxtd = 1.0;
    // loads issued whether or not the lane uses them (index 0 when not), so
    // the compiler can wait for exactly the ones a use needs
    auto load_first = [&](int t, Chunk& ch, int& c, int& r, double& o, double& d) {
        c = first_chunk(t);
        fetch(c >= 0 ? c : 0, ch);
        if (!LDSW || UPPER) r = first_row(t);
        if (!LDSW) o = Wb[(size_t)tl.rows[r >= 0 ? r : 0] * GL + gl];
        if (UPPER) d = tl.diag[r >= 0 ? r : 0];
    };
    // row r's value from its own value less the sum of its terms (divided by
    // U's diagonal), with the prefetched own value and diagonal where r is
    // the lane's first row of the level
    auto finish_row = [&](int r, double acc) {
        double own, dg = 1.0;
        if (r == curr) {
            own = LDSW ? *own_ref(r) : curo;
            dg = curd;
            curr = -1;
        } else {
            own = *own_ref(r);
            if (UPPER) dg = tl.diag[r];
        }
        double w = own - acc;
        if (UPPER) w = w / dg;
        *own_ref(r) = w;
    };
    auto chunk_of = [&](int c, Chunk& tmp) -> const Chunk& {
        if (c == curc) return cur;
        fetch(c, tmp);
        return tmp;
    };
    if (tl.nlev > 0) load_first(0, cur, curc, curr, curo, curd);
    __syncthreads();
    for (int t = 0; t < tl.nlev; t++) {
        if (t + 1 < tl.nlev) load_first(t + 1, nxt, nxtc, nxtr, nxto, nxtd);
        const int clo = tchunk[t], chi = tchunk[t + 1];
        const int mode = tmode[t];
        Chunk tmp;
        if (mode == 0) {
            for (int r = trow[t] + slot; r < trow[t + 1]; r += NS) {
                double acc = 0.0;
                if (tl.rchunk[r] < tl.rchunk[r + 1]) acc = part(chunk_of(tl.rchunk[r], tmp));
                finish_row(r, acc);
            }
        } else if (mode == 1 || mode == 2) {
            for (int c = clo + slot; c < chi; c += NS) P[(size_t)(c - clo) * GL + gl] = part(chunk_of(c, tmp));
            lds_barrier();
            if (mode == 1) {
                for (int r = trow[t] + slot; r < trow[t + 1]; r += NS) {
                    // the row's partials four reads at a time, summed in order
                    const int c0 = tl.rchunk[r] - clo, c1 = tl.rchunk[r + 1] - clo;
                    double acc = 0.0;
                    for (int c = c0; c < c1; c += 4) {
                        double pv[4];
#pragma unroll
                        for (int j = 0; j < 4; j++) pv[j] = P[(size_t)(c + j < c1 ? c + j : c1 - 1) * GL + gl];
#pragma unroll
                        for (int j = 0; j < 4; j++) acc += c + j < c1 ? pv[j] : 0.0;
                    }
                    finish_row(r, acc);
                }
            } else {
                for (int r = trow[t] + wave; r < trow[t + 1]; r += NW) {
                    const int c1 = tl.rchunk[r + 1] - clo;
                    double acc = 0.0;
                    for (int c = tl.rchunk[r] - clo + s; c < c1; c += S) acc += P[(size_t)c * GL + gl];
                    acc = lane_sum<GL>(acc);
                    if (s == 0) finish_row(r, acc);
                }
            }
        } else {
            for (int r = trow[t] + wave; r < trow[t + 1]; r += NW) {
                double acc = 0.0;
                for (int c = tl.rchunk[r] + s; c < tl.rchunk[r + 1]; c += S) acc += part(chunk_of(c, tmp));
                acc = lane_sum<GL>(acc);
                if (s == 0) finish_row(r, acc);
            }
        }
        cur = nxt;
        curc = nxtc;
        curr = nxtr;
        curo = nxto;
        curd = nxtd;
        if (LDSW) lds_barrier();
        else __syncthreads();
    }
    if (LDSW)
        for (int x = tid; x < tl.m * GL; x += kRunThreads) Wb[(size_t)tl.rows[x / GL] * GL + x % GL] = Wt[x];
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

// Forcing (sb_fdm.c:147-151, exposure :126-140) of every solved cell t, in
// the cells' order (the field, the heat input and the mass read in order),
// written to its row ipr[t] of the permuted vector; one thread per (group of
// kForceBlocks blocks, cell, lane), so the cell's tables are read once for the
// group's envs; clears the blocks' air-side flags.
constexpr int kForceBlocks = 8;
__global__ void forcing_kernel(sbf::Tables t, sbf::Group g, sbf::StepIn in) {
    const int n = t.n, Gl = g.Gl, G = g.G;
    const int nbg = (g.nblk + kForceBlocks - 1) / kForceBlocks;
    const size_t total = (size_t)nbg * n * Gl;
    for (size_t x = gtid(); x < total; x += gstride()) {
        const int l = (int)(x % Gl);
        const size_t bt = x / Gl;
        const int tt = (int)(bt % n), bg = (int)(bt / n);
        const int p = t.solved[tt];
        const double a0 = t.a0[tt], a1 = t.a1[tt], hz = t.hz[tt], vt = t.vt[tt], cd = t.cd[tt];
        const double cap = t.cap[tt], dir = t.dir[tt], mcoup = t.mcoup[tt];
        const int z = in.q ? -1 : t.czone[tt];
        const int row = t.ipr[tt];
#pragma unroll
        for (int k = 0; k < kForceBlocks; k++) {
            const int b = bg * kForceBlocks + k;
            if (b >= g.nblk) break;
            const int env = b * Gl + l;
            double w = 0.0;
            if (env < G) {
                const double h = in.h[env];
                double e = 0.0;
                if (a0 > 0.0) e += h * a0 / (1.0 + h * 0.5 * hz / cd);
                if (a1 > 0.0) e += h * a1 / (1.0 + h * 0.5 * vt / cd);
                double q;
                if (in.q) q = in.q[(size_t)env * t.n_cvs + p];
                else q = z >= 0 ? in.qz[(size_t)env * t.nz + z] : 0.0;
                w = cap * g.T[((size_t)b * t.n_cvs + p) * Gl + l] + q + in.amb[env] * (dir + e)
                    + mcoup * g.M[((size_t)b * n + tt) * Gl + l];
            }
            g.W1[((size_t)b * n + row) * Gl + l] = w;
        }
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

// The same with each dot spread over a wavefront's 64 lanes (one wavefront per
// env and row; the sum in another, fixed, order).
__global__ __launch_bounds__(256) void sensed_wide_kernel(sbf::Tables t, sbf::Group g, sbf::StepIn in) {
    const int k = t.k, Gl = g.Gl, lane = threadIdx.x & 63;
    const size_t nw = (size_t)gridDim.x * (blockDim.x >> 6);
    for (size_t x = (size_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6); x < (size_t)g.G * k; x += nw) {
        const int env = (int)(x / k), i = (int)(x % k);
        const int b = env / Gl, l = env % Gl;
        const double* Wb = g.W1 + (size_t)b * t.n * Gl;
        double acc = 0.0;
        for (int p = t.sn_p[i] + lane; p < t.sn_p[i + 1]; p += 64) acc += t.sn_x[p] * Wb[(size_t)t.sn_w[p] * Gl + l];
        acc = lane_sum<1>(acc);
        if (lane == 0) g.pw[x] = in.g[x] * (in.airT[x] - acc);
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

// The same solve per env with M, the power row and the step's row factors in
// LDS, one workgroup of kDenseThreads per env (k <= kDenseLdsK). Every value
// sees the operations of sb_fdm.c:9-38 in their order: the pivot is the first
// row reaching the largest |M[r][c]| over r >= c (NaNs never win; row c stays
// when |M[c][c]| is NaN), as the sequential strictly-greater scan picks it;
// the rows' factors f = M[r][c] / d are taken before the step's updates;
// M[r][j] -= f M[c][j] for j >= c (the product rounded: this file is built
// without contraction) and b[r] -= f b[c], rows with f == 0 skipped; then
// lane 0 back-substitutes row by row, each row's terms in ascending column.
constexpr int kDenseThreads = 256, kDenseLdsK = 89;
__global__ __launch_bounds__(kDenseThreads) void dense_lds_kernel(sbf::Tables t, sbf::Group g, sbf::StepIn in) {
    extern __shared__ __align__(16) double dl[];
    __shared__ int s_piv, s_sing;
    const int env = blockIdx.x, k = t.k, tid = threadIdx.x;
    const double* gv = in.g + (size_t)env * k;
    int any = 0;
    for (int i = tid; i < k; i += kDenseThreads) any |= gv[i] != 0.0;
    any = __syncthreads_or(any);
    if (tid == 0) {
        g.eact[env] = any;
        if (any) atomicOr(&g.bact[env / g.Gl], 1);
    }
    if (!any) return;   // workgroup-uniform
    double* M = dl;             // [k][k]
    double* bv = dl + k * k;    // [k]
    double* fr = bv + k;        // [k]: the step's row factors
    double* pw = g.pw + (size_t)env * k;
    for (int x = tid; x < k * k; x += kDenseThreads) {
        const int i = x / k, j = x % k;
        M[x] = (i == j ? 1.0 : 0.0) + gv[i] * t.S[x];
    }
    for (int i = tid; i < k; i += kDenseThreads) bv[i] = pw[i];
    __syncthreads();
    for (int c = 0; c < k; c++) {
        if (tid < 64) {
            double m = -1.0;
            for (int r = c + tid; r < k; r += 64) {
                const double v = fabs(M[r * k + c]);
                if (v > m) m = v;
            }
            for (int o = 32; o > 0; o >>= 1) m = fmax(m, __shfl_xor(m, o));
            int first = k;
            for (int r = c + tid; r < k; r += 64)
                if (fabs(M[r * k + c]) == m) {
                    first = r;
                    break;
                }
            for (int o = 32; o > 0; o >>= 1) first = min(first, __shfl_xor(first, o));
            if (tid == 0) {
                const double vc = fabs(M[c * k + c]);
                const bool nan_c = vc != vc;
                s_piv = nan_c ? c : first;
                s_sing = !nan_c && m == 0.0;
            }
        }
        __syncthreads();
        if (s_sing) {
            // the reference returns here, leaving the partly reduced row
            for (int i = tid; i < k; i += kDenseThreads) pw[i] = bv[i];
            return;
        }
        const int piv = s_piv;
        if (piv != c) {
            for (int j = c + tid; j < k; j += kDenseThreads) {
                const double x = M[c * k + j];
                M[c * k + j] = M[piv * k + j];
                M[piv * k + j] = x;
            }
            if (tid == 0) {
                const double x = bv[c];
                bv[c] = bv[piv];
                bv[piv] = x;
            }
            __syncthreads();
        }
        const double d = M[c * k + c];
        for (int r = c + 1 + tid; r < k; r += kDenseThreads) fr[r] = M[r * k + c] / d;
        __syncthreads();
        const int nc = k - c, nx = (k - c - 1) * nc;
        for (int x = tid; x < nx; x += kDenseThreads) {
            const int r = c + 1 + x / nc, j = c + x % nc;
            const double f = fr[r];
            if (f != 0.0) M[r * k + j] -= f * M[c * k + j];
        }
        for (int r = c + 1 + tid; r < k; r += kDenseThreads) {
            const double f = fr[r];
            if (f != 0.0) bv[r] -= f * bv[c];
        }
        __syncthreads();
    }
    if (tid == 0) {
        for (int r = k - 1; r >= 0; r--) {
            double s = bv[r];
            for (int j = r + 1; j < k; j++) s -= M[r * k + j] * bv[j];
            bv[r] = s / M[r * k + r];
        }
    }
    __syncthreads();
    for (int i = tid; i < k; i += kDenseThreads) pw[i] = bv[i];
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

// Default mode with the air side: y = the forcing solve + R^T q, R's rows the
// solutions of the applied columns (solved once at open), q the dense solve's
// result per env; the same y as sb_fdm.c:171-178's second solve of the
// applied heat up to rounding (the correction is linear in q). Then the
// interior mass and the field (sb_fdm.c:183-187). A block is 64 solved cells
// (a lane each) by 4 wavefronts of kREnvs envs; each R value loaded is used
// for kREnvs envs, and an env's q row is wave-uniform (scalar loads). The
// correction of an env sums j = 0 .. k-1 in order.
constexpr int kREnvs = 16;

__global__ __launch_bounds__(256) void update_r_kernel(sbf::Tables t, sbf::Group g, sbf::StepIn in) {
    const int n = t.n, k = t.k, Gl = g.Gl, G = g.G;
    // the wavefront index through readfirstlane: the compiler then knows the
    // envs (and their q rows) are wave-uniform and reads q with scalar loads
    const int lane = (int)(threadIdx.x & 63), wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int egs = (G + 4 * kREnvs - 1) / (4 * kREnvs);
    const int tile = (int)blockIdx.x / egs, eg = (int)blockIdx.x % egs;
    const int e0 = (eg * 4 + wv) * kREnvs;
    const int tt = tile * 64 + lane;
    if (e0 < G && tile * 64 < n) {
        const bool ok = tt < n;
        const int tc = ok ? tt : n - 1;
        double acc[kREnvs];
#pragma unroll
        for (int e = 0; e < kREnvs; e++) acc[e] = 0.0;
        // columns eight at a time, then one at a time (j0 and k are wave-uniform)
        int j0 = 0;
        for (; j0 + 8 <= k; j0 += 8) {
            double r[8];
#pragma unroll
            for (int jj = 0; jj < 8; jj++) r[jj] = t.R[(size_t)(j0 + jj) * n + tc];
#pragma unroll
            for (int e = 0; e < kREnvs; e++) {
                const int env = e0 + e < G ? e0 + e : G - 1;
                const double* qv = g.pw + (size_t)env * k + j0;
#pragma unroll
                for (int jj = 0; jj < 8; jj++) acc[e] = fma(r[jj], qv[jj], acc[e]);
            }
        }
        for (; j0 < k; j0++) {
            const double r = t.R[(size_t)j0 * n + tc];
#pragma unroll
            for (int e = 0; e < kREnvs; e++) {
                const int env = e0 + e < G ? e0 + e : G - 1;
                acc[e] = fma(r, g.pw[(size_t)env * k + j0], acc[e]);
            }
        }
        if (ok) {
            const int pcv = t.pc[tc], cell = t.solved[tc];
            const double mr = t.mret[tc], mg = t.mgain[tc];
#pragma unroll
            for (int e = 0; e < kREnvs; e++) {
                const int env = e0 + e;
                if (env >= G) break;
                const int b = env / Gl, l = env % Gl;
                double y = g.W1[((size_t)b * n + pcv) * Gl + l];
                if (g.eact[env]) y += acc[e];
                const size_t mi = ((size_t)b * n + tc) * Gl + l;
                g.M[mi] = g.M[mi] * mr + mg * y;
                g.T[((size_t)b * t.n_cvs + cell) * Gl + l] = y;
            }
        }
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

template <bool UPPER, int GL>
void sweep(const sbf::Tri& tri, const sbf::Sweep* sw, const sbf::Group& g, int n, double* W, const int* bact,
           hipStream_t s) {
    auto plain = [&](int l0, int l1) {
        if (l1 > l0)
            hipLaunchKernelGGL((solve_kernel<UPPER, GL>), dim3(g.nblk), dim3(kSolveThreads), 0, s, tri, l0, l1, n, W,
                               bact);
    };
    if (!sw) {
        plain(0, tri.nlev);
        return;
    }
    // levels before the LDS run; the run's head terms and the run; the levels after it
    if (sw->pre_chunked) {
        const size_t lds = (size_t)sw->pre.max_chunks * GL * sizeof(double);
        hipLaunchKernelGGL((run_kernel<UPPER, GL, false>), dim3(g.nblk), dim3(kRunThreads), lds, s, sw->pre, n, W,
                           bact);
    } else {
        plain(0, sw->pre_end);
    }
    const sbf::Tail& mid = sw->mid;
    if (mid.nlev > 0) {
        if (mid.lev0 > 0) {
            const size_t waves = (size_t)((g.nblk + kHeadBlocks - 1) / kHeadBlocks) * mid.m;
            const int grid = (int)std::min<size_t>((waves + 3) / 4, 8192);
            hipLaunchKernelGGL((head_kernel<GL>), dim3(grid), dim3(256), 0, s, mid, n, g.nblk, W, bact);
        }
        const size_t lds = (size_t)(mid.m + mid.max_chunks) * GL * sizeof(double);
        hipLaunchKernelGGL((run_kernel<UPPER, GL, true>), dim3(g.nblk), dim3(kRunThreads), lds, s, mid, n, W, bact);
    }
    if (sw->post_chunked) {
        const size_t lds = (size_t)sw->post.max_chunks * GL * sizeof(double);
        hipLaunchKernelGGL((run_kernel<UPPER, GL, false>), dim3(g.nblk), dim3(kRunThreads), lds, s, sw->post, n, W,
                           bact);
    } else {
        plain(sw->post_begin, tri.nlev);
    }
}

template <int GL>
void solve_gl(const sbf::Tables& t, const sbf::Group& g, double* W, const int* bact, bool exact, hipStream_t s) {
    const bool fast = t.fast && !exact;
    sweep<false, GL>(t.L, fast ? &t.SL : nullptr, g, t.n, W, bact, s);
    sweep<true, GL>(t.U, fast ? &t.SU : nullptr, g, t.n, W, bact, s);
}

// The L then U sweep of every block's columns of W; exact: every level in the
// reference's order (the tails are laid out for the step's group only).
int solve(const sbf::Tables& t, const sbf::Group& g, double* W, const int* bact, bool exact, hipStream_t s) {
    switch (g.Gl) {
    case 1: solve_gl<1>(t, g, W, bact, exact, s); break;
    case 2: solve_gl<2>(t, g, W, bact, exact, s); break;
    case 4: solve_gl<4>(t, g, W, bact, exact, s); break;
    case 8: solve_gl<8>(t, g, W, bact, exact, s); break;
    case 16: solve_gl<16>(t, g, W, bact, exact, s); break;
    case 32: solve_gl<32>(t, g, W, bact, exact, s); break;
    case 64: solve_gl<64>(t, g, W, bact, exact, s); break;
    default: return (int)hipErrorInvalidValue;
    }
    return (int)hipGetLastError();
}

template <int GL>
hipError_t run_limit(int bytes) {
    const void* fns[4] = {(const void*)run_kernel<false, GL, true>, (const void*)run_kernel<true, GL, true>,
                          (const void*)run_kernel<false, GL, false>, (const void*)run_kernel<true, GL, false>};
    for (const void* f : fns) {
        const hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace

// One batched step of a group (all launches on stream s).
extern "C" int sbf_launch_step(const sbf::Tables* t, const sbf::Group* g, const sbf::StepIn* in, hipStream_t s) {
    const size_t rows = (size_t)g->nblk * t->n * g->Gl;
    const size_t fitems = (size_t)((g->nblk + kForceBlocks - 1) / kForceBlocks) * t->n * g->Gl;
    hipLaunchKernelGGL(forcing_kernel, dim3(elt_grid(fitems)), dim3(kEltThreads), 0, s, *t, *g, *in);
    if (int e = solve(*t, *g, g->W1, nullptr, false, s)) return e;
    if (t->k > 0) {
        if (t->fast)
            hipLaunchKernelGGL(sensed_wide_kernel, dim3((int)std::min<size_t>(((size_t)g->G * t->k + 3) / 4, 16384)),
                               dim3(256), 0, s, *t, *g, *in);
        else
            hipLaunchKernelGGL(sensed_kernel, dim3(elt_grid((size_t)g->G * t->k)), dim3(kEltThreads), 0, s, *t, *g,
                               *in);
        if (t->k <= kDenseLdsK)
            hipLaunchKernelGGL(dense_lds_kernel, dim3(g->G), dim3(kDenseThreads),
                               sizeof(double) * ((size_t)t->k * t->k + 2 * (size_t)t->k), s, *t, *g, *in);
        else
            hipLaunchKernelGGL(dense_kernel, dim3(g->G), dim3(64), 0, s, *t, *g, *in);
        if (t->R) {
            // the correction as R^T q, fused with the mass and field update
            const size_t tiles = ((size_t)t->n + 63) / 64, egs = ((size_t)g->G + 4 * kREnvs - 1) / (4 * kREnvs);
            hipLaunchKernelGGL(update_r_kernel, dim3((unsigned)(tiles * egs)), dim3(256), 0, s, *t, *g, *in);
            return (int)hipGetLastError();
        }
        hipLaunchKernelGGL(applied_kernel, dim3(elt_grid(rows)), dim3(kEltThreads), 0, s, *t, *g);
        if (int e = solve(*t, *g, g->W2, g->bact, false, s)) return e;
    }
    hipLaunchKernelGGL(update_kernel, dim3(elt_grid(rows)), dim3(kEltThreads), 0, s, *t, *g, *in);
    return (int)hipGetLastError();
}

// Lets the run kernels use `bytes` of dynamic LDS.
extern "C" int sbf_run_lds_limit(int bytes) {
    for (hipError_t e : {run_limit<1>(bytes), run_limit<2>(bytes), run_limit<4>(bytes), run_limit<8>(bytes),
                         run_limit<16>(bytes), run_limit<32>(bytes), run_limit<64>(bytes)})
        if (e != hipSuccess) return (int)e;
    return 0;
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
    if (int e = solve(*t, *g, g->W1, nullptr, true, s)) return e;
    if (x) hipLaunchKernelGGL(sol_kernel, dim3(elt_grid((size_t)g->G * t->n)), dim3(kEltThreads), 0, s, *t, *g, x);
    if (S) hipLaunchKernelGGL(sresp_kernel, dim3(elt_grid((size_t)t->k * t->k)), dim3(kEltThreads), 0, s, *t, *g, S);
    return (int)hipGetLastError();
}
