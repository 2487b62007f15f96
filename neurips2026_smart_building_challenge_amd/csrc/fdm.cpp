// Host side of the building-scale field step (sbx_fdm_*): reads a blob's
// field sections (the ones complete_port/csim/sb_fdm.c:40-118 reads), checks
// them, turns the baked CSC factors into level-ordered row solves, uploads
// every table once and owns the group's device buffers.
#include <hip/hip_runtime_api.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <string>
#include <vector>

#include "fdm.h"
#include "fdm_host.h"
#include "sbb_reader.h"
#include "sbenv.h"

extern "C" int sbf_run_lds_limit(int bytes);
extern "C" int sbf_launch_solve_cols(const sbf::Tables* t, const sbf::Group* g, const double* b, double* x,
                                     double* S, hipStream_t s);

void sbx_set_error(const std::string& msg);


namespace {

struct Arena {
    std::vector<unsigned char> host;
    size_t add(const void* p, size_t bytes) {
        size_t off = (host.size() + 255) & ~(size_t)255;
        host.resize(off + bytes + 8, 0);
        if (p && bytes) memcpy(host.data() + off, p, bytes);
        return off;
    }
    template <class T>
    size_t vec(const std::vector<T>& v) { return add(v.data(), v.size() * sizeof(T)); }
};

bool fail(const std::string& msg) {
    sbx_set_error(msg);
    return false;
}

// Level-ordered rows of one factor: terms[i] holds row i's off-diagonal terms
// in application order; a lower factor's levels count from the first row up,
// an upper one's from the last row down (a row's level is one more than the
// highest level among the rows its terms read).
struct TriHost {
    int nlev = 0;
    std::vector<int> lev, rows, ptr, col;
    std::vector<double> val, diag;
    long long nnz = 0;
};

void level_order(const std::vector<std::vector<std::pair<int, double>>>& terms, const std::vector<double>* diag,
                 bool upper, TriHost* out) {
    const int n = (int)terms.size();
    // a row of the unit lower factor without terms keeps its value: it is
    // left out of the schedule (level -1)
    auto skip = [&](int i) { return !upper && terms[i].empty(); };
    std::vector<int> lvl(n, 0);
    int nlev = 0;
    for (int s = 0; s < n; s++) {
        const int i = upper ? n - 1 - s : s;
        int l = skip(i) ? -1 : 0;
        for (const auto& e : terms[i]) l = std::max(l, lvl[e.first] + 1);
        lvl[i] = l;
        nlev = std::max(nlev, l + 1);
    }
    std::vector<int> cnt(nlev + 1, 0);
    for (int i = 0; i < n; i++)
        if (lvl[i] >= 0) cnt[lvl[i] + 1]++;
    for (int l = 0; l < nlev; l++) cnt[l + 1] += cnt[l];
    const int nr = cnt[nlev];
    out->nlev = nlev;
    out->lev = cnt;
    out->rows.assign(std::max(nr, 1), 0);
    std::vector<int> fill(cnt.begin(), cnt.end() - 1);
    for (int i = 0; i < n; i++)
        if (lvl[i] >= 0) out->rows[fill[lvl[i]]++] = i;   // ascending i within a level
    out->rows.resize(nr);
    out->ptr.assign(nr + 1, 0);
    out->col.clear();
    out->val.clear();
    out->diag.clear();
    for (int q = 0; q < nr; q++) {
        const int i = out->rows[q];
        for (const auto& e : terms[i]) {
            out->col.push_back(e.first);
            out->val.push_back(e.second);
        }
        out->ptr[q + 1] = (int)out->col.size();
        if (diag) out->diag.push_back((*diag)[i]);
    }
    out->nnz = (long long)out->col.size();
    if (out->col.empty()) {   // keep the device arrays non-empty
        out->col.push_back(0);
        out->val.push_back(0.0);
    }
    if (out->diag.empty()) out->diag.push_back(1.0);
}

// Runs of the default mode (see sbf::Tail and sbf::Sweep). The LDS run is the
// longest run of consecutive levels with at most kTailRows rows each, cut from
// its side that borders wider levels until its row values and one level's
// chunk partials fit in kRunLds bytes for Gl envs.
constexpr int kTailRows = 64;
constexpr size_t kRunLds = 152 * 1024;
constexpr int kWaveFinishRows = 16;   // levels with more rows (some long) finish one row per lane

struct RunHost {
    int lds = 0, lev0 = 0, m = 0, nlev = 0, max_chunks = 0;
    std::vector<int> rows, hptr, hcol, trow, tchunk, tmode, rchunk, cpos;
    std::vector<double> diag, hval, cval;
    size_t need(int Gl) const { return (size_t)((lds ? m : 0) + max_chunks) * Gl * 8; }
};

struct LevelOf {
    // level of a row (-1: not scheduled, final from the start), its position in level order
    std::vector<int> lvl, q_of;
    LevelOf(const TriHost& T, int n) : lvl(n, -1), q_of(n, -1) {
        for (int l = 0; l < T.nlev; l++)
            for (int q = T.lev[l]; q < T.lev[l + 1]; q++) lvl[T.rows[q]] = l;
        for (size_t q = 0; q < T.rows.size(); q++) q_of[T.rows[q]] = (int)q;
    }
};

void lay_run(const TriHost& T, const LevelOf& V, int lev0, int lev1, bool lds, int Gl, RunHost* out) {
    const int nr = (int)T.rows.size();
    const int q0 = T.lev[lev0];
    RunHost& o = *out;
    o = RunHost();
    o.lds = lds;
    o.lev0 = lev0;
    o.m = T.lev[lev1] - q0;
    o.nlev = lev1 - lev0;
    o.hptr.push_back(0);
    o.rchunk.push_back(0);
    for (int t = 0; t < o.nlev; t++) {
        o.trow.push_back(T.lev[lev0 + t] - q0);
        o.tchunk.push_back((int)o.cpos.size() / sbf::kChunk);
        int most = 0;
        for (int q = T.lev[lev0 + t]; q < T.lev[lev0 + t + 1]; q++) {
            o.rows.push_back(T.rows[q]);
            if ((int)T.diag.size() == nr) o.diag.push_back(T.diag[q]);
            int cnt = 0;
            for (int e = T.ptr[q]; e < T.ptr[q + 1]; e++) {
                const int j = T.col[e];
                if (!lds) {
                    o.cpos.push_back(j);
                } else if (V.lvl[j] >= lev0) {   // a row reads earlier levels only: lvl[j] < lev0 + t
                    o.cpos.push_back(V.q_of[j] - q0);
                } else {
                    o.hcol.push_back(j);
                    o.hval.push_back(T.val[e]);
                    continue;
                }
                o.cval.push_back(T.val[e]);
                cnt++;
            }
            while (cnt % sbf::kChunk) {
                o.cpos.push_back(0);
                o.cval.push_back(0.0);
                cnt++;
            }
            o.hptr.push_back((int)o.hcol.size());
            o.rchunk.push_back((int)o.cpos.size() / sbf::kChunk);
            most = std::max(most, cnt / sbf::kChunk);
        }
        const int nrows = T.lev[lev0 + t + 1] - T.lev[lev0 + t];
        const int mode = most <= 1 ? 0 : nrows > kWaveFinishRows ? 1 : most > 64 / Gl ? 2 : 3;
        o.tmode.push_back(mode);
        if (mode == 1 || mode == 2)
            o.max_chunks = std::max(o.max_chunks, (int)o.cpos.size() / sbf::kChunk - o.tchunk.back());
    }
    o.trow.push_back(o.m);
    o.tchunk.push_back((int)o.cpos.size() / sbf::kChunk);
    for (auto* v : {&o.rows, &o.hcol, &o.cpos, &o.tmode})
        if (v->empty()) v->push_back(0);
    for (auto* v : {&o.diag, &o.hval, &o.cval})
        if (v->empty()) v->push_back(1.0);
}

struct SweepHost {
    int pre_end = 0, post_begin = 0, pre_chunked = 0, post_chunked = 0;
    RunHost pre, mid, post;
};

void plan_sweep(const TriHost& T, int n, int Gl, SweepHost* out) {
    const LevelOf V(T, n);
    auto narrow = [&](int l) { return T.lev[l + 1] - T.lev[l] <= kTailRows; };
    int a = 0, b = 0;   // the longest run [a, b) of narrow levels
    for (int l = 0; l < T.nlev;) {
        if (!narrow(l)) { l++; continue; }
        int e = l;
        while (e < T.nlev && narrow(e)) e++;
        if (e - l > b - a) { a = l; b = e; }
        l = e;
    }
    RunHost& mid = out->mid;
    auto need = [&](int lo, int hi) {
        lay_run(T, V, lo, hi, true, Gl, &mid);
        return mid.need(Gl);
    };
    if (b > a && need(a, b) > kRunLds) {
        // cut the side that borders wider levels (for the L sweep the run ends
        // the schedule, for the U sweep it starts it); fewer levels need less
        // LDS, so bisect for the longest run that fits
        const bool keep_end = b == T.nlev;
        int lo = 0, hi = b - a;   // levels kept
        while (lo < hi) {
            const int mid_n = lo + (hi - lo + 1) / 2;
            if (need(keep_end ? b - mid_n : a, keep_end ? b : a + mid_n) <= kRunLds) lo = mid_n;
            else hi = mid_n - 1;
        }
        if (keep_end) a = b - lo;
        else b = a + lo;
    }
    lay_run(T, V, a, b, true, Gl, &mid);
    out->pre_end = a;
    out->post_begin = b;
    lay_run(T, V, 0, a, false, Gl, &out->pre);
    out->pre_chunked = out->pre.nlev > 0 && out->pre.need(Gl) <= kRunLds;
    lay_run(T, V, b, T.nlev, false, Gl, &out->post);
    out->post_chunked = out->post.nlev > 0 && out->post.need(Gl) <= kRunLds;
}

bool csc_ok(const sbh::Blob& b, const char* name, int n_rows, int n_cols, const int32_t** p, const int32_t** ix,
            const double** x, uint64_t* nnz) {
    uint64_t np = 0, ni = 0, nx = 0;
    const std::string s(name);
    *p = b.i32(s + "_indptr", &np);
    *ix = b.i32(s + "_indices", &ni);
    *x = b.f64(s + "_data", &nx);
    if (!*p || !*ix || !*x) return fail(s + ": sections missing");
    if ((int64_t)np != (int64_t)n_cols + 1 || ni != nx) return fail(s + ": inconsistent sizes");
    if ((*p)[0] != 0 || (uint64_t)(*p)[n_cols] != ni) return fail(s + ": bad pointers");
    for (int j = 0; j < n_cols; j++)
        if ((*p)[j + 1] < (*p)[j]) return fail(s + ": pointers decrease");
    for (uint64_t e = 0; e < ni; e++)
        if ((*ix)[e] < 0 || (*ix)[e] >= n_rows) return fail(s + ": index out of range");
    *nnz = ni;
    return true;
}

bool perm_ok(const int32_t* p, uint64_t count, int n) {
    if (!p || (int64_t)count != n) return false;
    std::vector<char> seen(n, 0);
    for (int i = 0; i < n; i++) {
        if (p[i] < 0 || p[i] >= n || seen[p[i]]) return false;
        seen[p[i]] = 1;
    }
    return true;
}

int next_pow2(int x) {
    int p = 1;
    while (p < x) p *= 2;
    return p;
}

void* dalloc(SbxFdm* f, size_t bytes) {
    void* p = nullptr;
    if (hipMalloc(&p, std::max<size_t>(bytes, 8)) != hipSuccess) return nullptr;
    f->owned.push_back(p);
    return p;
}

// Device buffers of a group of G envs in blocks of Gl lanes.
bool make_group(SbxFdm* f, int G, int Gl, bool fields, sbf::Group* g) {
    const sbf::Tables& t = f->tab;
    g->G = G;
    g->Gl = Gl;
    g->nblk = (G + Gl - 1) / Gl;
    const size_t lanes = (size_t)g->nblk * Gl;
    g->W1 = (double*)dalloc(f, sizeof(double) * lanes * t.n);
    const bool w2 = fields && !t.R;   // the second solve's vector (exact mode)
    g->W2 = w2 ? (double*)dalloc(f, sizeof(double) * lanes * t.n) : nullptr;
    g->T = fields ? (double*)dalloc(f, sizeof(double) * lanes * t.n_cvs) : nullptr;
    g->M = fields ? (double*)dalloc(f, sizeof(double) * lanes * t.n) : nullptr;
    const size_t k = std::max(t.k, 1);
    g->pw = (double*)dalloc(f, sizeof(double) * G * k);
    g->mat = fields ? (double*)dalloc(f, sizeof(double) * G * k * k) : nullptr;
    g->eact = (int*)dalloc(f, sizeof(int) * G);
    g->bact = (int*)dalloc(f, sizeof(int) * g->nblk);
    if (!g->W1 || !g->pw || !g->eact || !g->bact || (w2 && !g->W2) || (fields && (!g->T || !g->M || !g->mat)))
        return fail("hipMalloc failed for the field buffers");
    return true;
}

bool hip_check(hipError_t e, const char* what) {
    if (e == hipSuccess) return true;
    return fail(std::string(what) + ": " + hipGetErrorString(e));
}

bool build(SbxFdm* f, const char* path, int G, int epb, int flags) {
    sbh::Blob b;
    std::string err;
    if (!b.open(path, &err)) return fail(err);
    uint64_t cnt = 0;
    const int64_t* grid = b.i64("grid", &cnt);
    if (!grid || cnt != 2 || grid[0] < 1 || grid[1] < 1) return fail("grid section missing or malformed");
    const long long ncvs_ll = grid[0] * grid[1];
    if (ncvs_ll > (1ll << 30)) return fail("grid too large");
    const int n_cvs = (int)ncvs_ll;
    const int64_t* solved = b.i64("solved", &cnt);
    if (!solved || cnt < 1 || (long long)cnt > ncvs_ll) return fail("solved section missing or malformed");
    const int n = (int)cnt;
    for (int t = 0; t < n; t++)
        if (solved[t] < 0 || solved[t] >= n_cvs || (t && solved[t] <= solved[t - 1]))
            return fail("solved cells must be ascending cell ids inside the grid");
    const int64_t* sshape = b.i64("sensed_shape", &cnt);
    const int k = sshape && cnt == 2 ? (int)sshape[0] : -1;
    if (k < 0 || sshape[1] != n) return fail("sensed_shape missing or not (k, n_solved)");
    const int64_t* ashape = b.i64("applied_shape", &cnt);
    if (!ashape || cnt != 2 || ashape[0] != n || ashape[1] != k) return fail("applied_shape is not (n_solved, k)");
    auto per_t = [&](const char* name, const double** out) {
        uint64_t c = 0;
        *out = b.f64(name, &c);
        return *out && (int64_t)c == n;
    };
    auto per_p = [&](const char* name, const double** out) {
        uint64_t c = 0;
        *out = b.f64(name, &c);
        return *out && (int64_t)c == n_cvs;
    };
    const double *cap, *dir, *mc, *mret, *mgain, *minit, *tinit, *hz, *vt, *cd, *f0, *f1;
    if (!per_t("capacitance_rate", &cap) || !per_t("dirichlet_conductance", &dir) || !per_t("mass_coupling", &mc)
        || !per_t("mass_retained", &mret) || !per_t("mass_gained", &mgain) || !per_t("mass_temp_init", &minit))
        return fail("per-solved-cell field sections missing or of the wrong size");
    if (!per_p("temp_init", &tinit) || !per_p("horizontal", &hz) || !per_p("vertical", &vt)
        || !per_p("solver_conductivity", &cd) || !per_p("ambient_face_areas_0", &f0)
        || !per_p("ambient_face_areas_1", &f1))
        return fail("per-cell field sections missing or of the wrong size");
    const int32_t *Lp, *Li, *Up, *Ui, *ap, *ai, *sp, *si;
    const double *Lx, *Ux, *ax, *sx;
    uint64_t nnzL, nnzU, nnzA, nnzS;
    if (!csc_ok(b, "lu_L", n, n, &Lp, &Li, &Lx, &nnzL) || !csc_ok(b, "lu_U", n, n, &Up, &Ui, &Ux, &nnzU)
        || !csc_ok(b, "applied", n, k, &ap, &ai, &ax, &nnzA) || !csc_ok(b, "sensed", n, k, &sp, &si, &sx, &nnzS))
        return false;   // sensed is CSR (k rows over n columns): the same checks apply
    uint64_t npr = 0, npc = 0;
    const int32_t* pr = b.i32("lu_perm_r", &npr);
    const int32_t* pcol = b.i32("lu_perm_c", &npc);
    if (!perm_ok(pr, npr, n) || !perm_ok(pcol, npc, n)) return fail("lu_perm_r / lu_perm_c are not permutations");

    // factors as rows (sb_lu.c:42-61 applies L's column j to its rows in
    // ascending j and U's in descending j; the first diagonal entry of each
    // column is the pivot, sb_lu.c:18-24)
    std::vector<std::vector<std::pair<int, double>>> lt(n), ut(n);
    std::vector<double> udiag(n, 0.0);
    for (int j = 0; j < n; j++) {
        bool dl = false;
        for (int e = Lp[j]; e < Lp[j + 1]; e++) {
            const int i = Li[e];
            if (i == j && !dl) { dl = true; continue; }
            if (i <= j) return fail("lu_L is not unit lower triangular with one diagonal entry per column");
            lt[i].push_back({j, Lx[e]});
        }
        if (!dl) return fail("lu_L column without its diagonal entry");
    }
    for (int j = n - 1; j >= 0; j--) {
        bool du = false;
        for (int e = Up[j]; e < Up[j + 1]; e++) {
            const int i = Ui[e];
            if (i == j && !du) { du = true; udiag[j] = Ux[e]; continue; }
            if (i >= j) return fail("lu_U is not upper triangular with one diagonal entry per column");
            ut[i].push_back({j, Ux[e]});
        }
        if (!du) return fail("lu_U column without its diagonal entry");
    }
    TriHost L, U;
    level_order(lt, nullptr, false, &L);
    level_order(ut, &udiag, true, &U);
    lt.clear();
    ut.clear();

    std::vector<int> ir(n), pcv(pcol, pcol + n), sol(n);
    for (int i = 0; i < n; i++) ir[pr[i]] = i;
    for (int t = 0; t < n; t++) sol[t] = (int)solved[t];
    std::vector<int> unsolved;
    {
        std::vector<char> is(n_cvs, 0);
        for (int t = 0; t < n; t++) is[solved[t]] = 1;
        for (int p = 0; p < n_cvs; p++)
            if (!is[p]) unsolved.push_back(p);
        if (unsolved.empty()) unsolved.push_back(0);   // non-empty array; count below stays exact
    }
    const int n_unsolved = n_cvs - n;
    std::vector<double> a0(n), a1(n), hzt(n), vtt(n), cdt(n);
    for (int t = 0; t < n; t++) {
        const int64_t p = solved[t];
        a0[t] = f0[p];
        a1[t] = f1[p];
        hzt[t] = hz[p];
        vtt[t] = vt[p];
        cdt[t] = cd[p];
    }
    // zones (env scenarios): the zone whose heat each solved cell carries
    std::vector<int> czone;
    int nz = 0;
    {
        uint64_t nzc = 0, nro = 0, nrc = 0;
        const double* za = b.f64("zone_area", &nzc);
        const int32_t* phys = b.i32("phys_room_idx");
        const int32_t* ro = b.i32("room_offsets", &nro);
        const int32_t* rc = b.i32("room_cells", &nrc);
        if (za && phys && ro && rc && nro >= 1) {
            nz = (int)nzc;
            std::vector<int> tof(n_cvs, -1);
            for (int t = 0; t < n; t++) tof[solved[t]] = t;
            czone.assign(n, -1);
            const int nrooms = (int)nro - 1;
            for (int z = 0; z < nz; z++) {
                const int rm = phys[z];
                if (rm < 0 || rm >= nrooms || ro[rm] < 0 || ro[rm + 1] < ro[rm] || 2 * (uint64_t)ro[rm + 1] > nrc)
                    return fail("zone rooms out of range");
                for (int q = ro[rm]; q < ro[rm + 1]; q++) {
                    const long long cell = (long long)rc[2 * q] * grid[1] + rc[2 * q + 1];
                    if (rc[2 * q] < 0 || rc[2 * q] >= grid[0] || rc[2 * q + 1] < 0 || rc[2 * q + 1] >= grid[1]
                        || tof[cell] < 0)
                        return fail("room cell outside the solved field");
                    czone[tof[cell]] = z;
                }
            }
        }
    }
    // sensed rows over the permuted solution; applied columns transposed per
    // permuted row, ascending column (sb_fdm.c:173-176 scatters them in that order)
    std::vector<int> snw(std::max<uint64_t>(nnzS, 1), 0);
    for (uint64_t e = 0; e < nnzS; e++) snw[e] = pcv[si[e]];
    std::vector<std::vector<std::pair<int, double>>> by_t(n);
    for (int j = 0; j < k; j++)
        for (int e = ap[j]; e < ap[j + 1]; e++) by_t[ai[e]].push_back({j, ax[e]});
    std::vector<int> atp(n + 1, 0), atj;
    std::vector<double> atx;
    for (int i = 0; i < n; i++) {
        for (const auto& e : by_t[ir[i]]) {
            atj.push_back(e.first);
            atx.push_back(e.second);
        }
        atp[i + 1] = (int)atj.size();
    }
    if (atj.empty()) {
        atj.push_back(0);
        atx.push_back(0.0);
    }

    Arena A;
    std::vector<std::pair<const void**, size_t>> fix;
    sbf::Tables& T = f->tab;
    T.n = n;
    T.n_cvs = n_cvs;
    T.k = k;
    T.n_unsolved = n_unsolved;
    auto put = [&](const void** dst, size_t off) { fix.push_back({dst, off}); };
    put((const void**)&T.ir, A.vec(ir));
    {
        std::vector<int> ipr(n);
        for (int i = 0; i < n; i++) ipr[ir[i]] = i;
        put((const void**)&T.ipr, A.vec(ipr));
    }
    put((const void**)&T.pc, A.vec(pcv));
    put((const void**)&T.solved, A.vec(sol));
    put((const void**)&T.unsolved, A.vec(unsolved));
    put((const void**)&T.cap, A.add(cap, 8 * (size_t)n));
    put((const void**)&T.dir, A.add(dir, 8 * (size_t)n));
    put((const void**)&T.mcoup, A.add(mc, 8 * (size_t)n));
    put((const void**)&T.mret, A.add(mret, 8 * (size_t)n));
    put((const void**)&T.mgain, A.add(mgain, 8 * (size_t)n));
    put((const void**)&T.a0, A.vec(a0));
    put((const void**)&T.a1, A.vec(a1));
    put((const void**)&T.hz, A.vec(hzt));
    put((const void**)&T.vt, A.vec(vtt));
    put((const void**)&T.cd, A.vec(cdt));
    T.nz = nz;
    T.czone = nullptr;
    if (nz > 0) put((const void**)&T.czone, A.vec(czone));
    auto put_tri = [&](sbf::Tri* d, const TriHost& h) {
        d->nlev = h.nlev;
        put((const void**)&d->lev, A.vec(h.lev));
        put((const void**)&d->rows, A.vec(h.rows));
        put((const void**)&d->ptr, A.vec(h.ptr));
        put((const void**)&d->col, A.vec(h.col));
        put((const void**)&d->val, A.vec(h.val));
        put((const void**)&d->diag, A.vec(h.diag));
    };
    put_tri(&T.L, L);
    put_tri(&T.U, U);
    // envs per block: as asked; by default one (the default mode keeps a run's
    // rows in LDS per env), two once the group has more than 256 envs, the
    // MI355X's compute-unit count (a block's level chain then serves two envs:
    // 512 envs of a 205K-cell plan 18.6 -> 17.5 ms per step, 1,024 envs
    // 28.2 ms; four were slower), or, in exact mode, up to 64. The threshold
    // is a constant, not the device's count: the default mode's sums are
    // reassociated by the block width, so an env's rounding depends on the
    // group size only (both widths are held to the reference within 1e-9)
    const bool exact = (flags & SBX_FDM_EXACT) != 0;
    constexpr int kTwoPerBlockAbove = 256;
    const int dflt = exact ? 64 : (G > kTwoPerBlockAbove ? 2 : 1);
    const int gl = std::min(64, next_pow2(std::min(G, epb > 0 ? epb : dflt)));
    T.fast = exact ? 0 : 1;
    SweepHost sl, su;
    if (T.fast) {
        plan_sweep(L, n, gl, &sl);
        plan_sweep(U, n, gl, &su);
    }
    auto put_run = [&](sbf::Tail* d, const RunHost& h) {
        d->lds = h.lds;
        d->lev0 = h.lev0;
        d->m = h.m;
        d->nlev = h.nlev;
        d->max_chunks = h.max_chunks;
        put((const void**)&d->rows, A.vec(h.rows));
        put((const void**)&d->diag, A.vec(h.diag));
        put((const void**)&d->hptr, A.vec(h.hptr));
        put((const void**)&d->hcol, A.vec(h.hcol));
        put((const void**)&d->hval, A.vec(h.hval));
        put((const void**)&d->trow, A.vec(h.trow));
        put((const void**)&d->tchunk, A.vec(h.tchunk));
        put((const void**)&d->tmode, A.vec(h.tmode));
        put((const void**)&d->rchunk, A.vec(h.rchunk));
        put((const void**)&d->cpos, A.vec(h.cpos));
        put((const void**)&d->cval, A.vec(h.cval));
    };
    auto put_sweep = [&](sbf::Sweep* d, const SweepHost& h) {
        d->pre_end = h.pre_end;
        d->post_begin = h.post_begin;
        d->pre_chunked = h.pre_chunked;
        d->post_chunked = h.post_chunked;
        put_run(&d->mid, h.mid);
        if (h.pre_chunked) put_run(&d->pre, h.pre);
        if (h.post_chunked) put_run(&d->post, h.post);
    };
    if (T.fast) {
        put_sweep(&T.SL, sl);
        put_sweep(&T.SU, su);
    }
    put((const void**)&T.sn_p, A.add(sp, 4 * (size_t)(k + 1)));
    put((const void**)&T.sn_w, A.vec(snw));
    put((const void**)&T.sn_x, A.add(sx, 8 * (size_t)std::max<uint64_t>(nnzS, 1)));
    put((const void**)&T.at_p, A.vec(atp));
    put((const void**)&T.at_j, A.vec(atj));
    put((const void**)&T.at_x, A.vec(atx));
    const size_t s_off = A.add(nullptr, 8 * (size_t)std::max(k * k, 1));
    put((const void**)&T.S, s_off);
    if (!hip_check(hipMalloc(&f->d_tables, A.host.size()), "hipMalloc(field tables)")) return false;
    if (!hip_check(hipMemcpy(f->d_tables, A.host.data(), A.host.size(), hipMemcpyHostToDevice), "upload field tables"))
        return false;
    for (auto& e : fix) *e.first = f->d_tables + e.second;
    if (T.fast && !hip_check((hipError_t)sbf_run_lds_limit((int)kRunLds), "run LDS limit")) return false;
    if (!hip_check(hipMalloc(&f->d_temp_init, 8 * (size_t)n_cvs), "hipMalloc(temp_init)")) return false;
    if (!hip_check(hipMalloc(&f->d_mass_init, 8 * (size_t)n), "hipMalloc(mass_temp_init)")) return false;
    if (!hip_check(hipMemcpy(f->d_temp_init, tinit, 8 * (size_t)n_cvs, hipMemcpyHostToDevice), "upload temp_init")
        || !hip_check(hipMemcpy(f->d_mass_init, minit, 8 * (size_t)n, hipMemcpyHostToDevice), "upload mass_temp_init"))
        return false;

    // S = sensed A^-1 applied (sb_fdm.c:104-116), on the device: the applied
    // columns solved as a group of k envs (in exact mode, as the reference
    // solves them); the default mode keeps the solutions themselves (R) for
    // its air-side corrections
    T.R = nullptr;
    if (k > 0) {
        sbf::Group sg{};
        if (!make_group(f, k, std::min(64, next_pow2(k)), false, &sg)) return false;
        double* R = nullptr;
        if (T.fast) {
            R = (double*)dalloc(f, sizeof(double) * (size_t)k * n);
            if (!R) return fail("hipMalloc failed for the air-side responses");
        }
        if (!hip_check((hipError_t)sbf_launch_solve_cols(&T, &sg, nullptr, R, (double*)T.S, nullptr),
                       "sensed response")
            || !hip_check(hipDeviceSynchronize(), "sensed response"))
            return false;
        T.R = R;
        for (void* p : {(void*)sg.W1, (void*)sg.pw, (void*)sg.eact, (void*)sg.bact}) {
            (void)hipFree(p);
            f->owned.erase(std::find(f->owned.begin(), f->owned.end(), p));
        }
    }
    if (!make_group(f, G, gl, true, &f->grp)) return false;
    if (!hip_check((hipError_t)sbf_launch_init(&T, &f->grp, f->d_temp_init, f->d_mass_init, nullptr), "field init")
        || !hip_check(hipDeviceSynchronize(), "field init"))
        return false;

    SbxFdmInfo& I = f->info;
    I.n_cvs = n_cvs;
    I.n_solved = n;
    I.k = k;
    I.n_envs = G;
    I.envs_per_block = gl;
    I.n_blocks = f->grp.nblk;
    I.levels_l = L.nlev;
    I.levels_u = U.nlev;
    I.nnz_l = L.nnz;
    I.nnz_u = U.nnz;
    I.tail_rows_l = T.fast ? sl.mid.m : 0;
    I.tail_rows_u = T.fast ? su.mid.m : 0;
    I.tail_levels_l = T.fast ? sl.mid.nlev : 0;
    I.tail_levels_u = T.fast ? su.mid.nlev : 0;
    I.chunked_levels_l = T.fast && sl.post_chunked ? sl.post.nlev : 0;
    I.chunked_levels_u = T.fast && su.post_chunked ? su.post.nlev : 0;
    // algorithmic HBM bytes of one batched step: both factors read once per
    // solve for the whole group (value + column per term, U's diagonal, row
    // ids and row pointers: shared by every env, however the blocks re-read
    // them); per env the heat input, the field read (solved cells) and
    // written (all cells), the mass read and written, and each solve's vector
    // read and written once per sweep
    // (two solves in exact mode; in the default mode one, plus R read once and
    // its k-term combination per env and solved cell)
    const double solves = T.R ? 1.0 : 2.0;
    const double per_solve = 12.0 * (double)(L.nnz + U.nnz) + 8.0 * n + 2.0 * 8.0 * n;
    const double per_env = 8.0 * ((double)n_cvs + n + n_cvs + 2.0 * n) + solves * (2.0 * 2.0 * 8.0 * n);
    const double r_bytes = T.R ? 8.0 * (double)k * n : 0.0;
    I.bytes_per_step = solves * per_solve + r_bytes + (double)G * per_env;
    I.flops_per_step = (double)G * (solves * 2.0 * (double)(L.nnz + U.nnz) + (T.R ? 2.0 * (double)k * n : 0.0));
    return true;
}

}  // namespace

extern "C" {

SbxFdm* sbx_fdm_open(const char* blob_path, int n_envs, int envs_per_block, int flags) {
    if (!blob_path || n_envs < 1 || envs_per_block < 0 || (flags & ~SBX_FDM_EXACT)) {
        sbx_set_error("sbx_fdm_open: blob path, n_envs >= 1, envs_per_block >= 0 and known flags required");
        return nullptr;
    }
    SbxFdm* f = new SbxFdm();
    if (!build(f, blob_path, n_envs, envs_per_block, flags)) {
        sbx_fdm_close(f);
        return nullptr;
    }
    return f;
}

void sbx_fdm_close(SbxFdm* f) {
    if (!f) return;
    (void)hipDeviceSynchronize();
    for (void* p : f->owned) (void)hipFree(p);
    if (f->d_tables) (void)hipFree(f->d_tables);
    if (f->d_temp_init) (void)hipFree(f->d_temp_init);
    if (f->d_mass_init) (void)hipFree(f->d_mass_init);
    delete f;
}

int sbx_fdm_info(const SbxFdm* f, SbxFdmInfo* out) {
    if (!f || !out) return -1;
    *out = f->info;
    return 0;
}

int sbx_fdm_step(SbxFdm* f, const double* input_q, const double* ambient, const double* h, const double* air_g,
                 const double* air_T, void* stream) {
    if (!f || !input_q || !ambient || !h || (f->tab.k > 0 && (!air_g || !air_T))) {
        sbx_set_error("sbx_fdm_step: null argument");
        return -1;
    }
    sbf::StepIn in{input_q, ambient, h, air_g, air_T, nullptr};
    const int e = sbf_launch_step(&f->tab, &f->grp, &in, (hipStream_t)stream);
    if (e) {
        sbx_set_error(std::string("sbx_fdm_step: ") + hipGetErrorString((hipError_t)e));
        return -1;
    }
    return 0;
}

int sbx_fdm_reset(SbxFdm* f, void* stream) {
    if (!f) return -1;
    return sbf_launch_init(&f->tab, &f->grp, f->d_temp_init, f->d_mass_init, (hipStream_t)stream) ? -1 : 0;
}

int sbx_fdm_get_state(SbxFdm* f, double* temp, double* mass_temp) {
    if (!f || !temp || !mass_temp) return -1;
    const sbf::Group& g = f->grp;
    const sbf::Tables& t = f->tab;
    std::vector<double> buf((size_t)g.nblk * g.Gl * std::max(t.n_cvs, t.n));
    if (!hip_check(hipDeviceSynchronize(), "sbx_fdm_get_state")) return -1;
    if (!hip_check(hipMemcpy(buf.data(), g.T, 8 * (size_t)g.nblk * g.Gl * t.n_cvs, hipMemcpyDeviceToHost), "copy T"))
        return -1;
    for (int e = 0; e < g.G; e++) {
        const size_t b = e / g.Gl, l = e % g.Gl;
        for (int p = 0; p < t.n_cvs; p++) temp[(size_t)e * t.n_cvs + p] = buf[(b * t.n_cvs + p) * g.Gl + l];
    }
    if (!hip_check(hipMemcpy(buf.data(), g.M, 8 * (size_t)g.nblk * g.Gl * t.n, hipMemcpyDeviceToHost), "copy M"))
        return -1;
    for (int e = 0; e < g.G; e++) {
        const size_t b = e / g.Gl, l = e % g.Gl;
        for (int q = 0; q < t.n; q++) mass_temp[(size_t)e * t.n + q] = buf[(b * t.n + q) * g.Gl + l];
    }
    return 0;
}

int sbx_fdm_set_state(SbxFdm* f, const double* temp, const double* mass_temp) {
    if (!f || !temp || !mass_temp) return -1;
    const sbf::Group& g = f->grp;
    const sbf::Tables& t = f->tab;
    std::vector<double> buf((size_t)g.nblk * g.Gl * t.n_cvs, 0.0);
    for (int e = 0; e < g.G; e++) {
        const size_t b = e / g.Gl, l = e % g.Gl;
        for (int p = 0; p < t.n_cvs; p++) buf[(b * t.n_cvs + p) * g.Gl + l] = temp[(size_t)e * t.n_cvs + p];
    }
    if (!hip_check(hipDeviceSynchronize(), "sbx_fdm_set_state")
        || !hip_check(hipMemcpy(g.T, buf.data(), 8 * buf.size(), hipMemcpyHostToDevice), "upload T"))
        return -1;
    buf.assign((size_t)g.nblk * g.Gl * t.n, 0.0);
    for (int e = 0; e < g.G; e++) {
        const size_t b = e / g.Gl, l = e % g.Gl;
        for (int q = 0; q < t.n; q++) buf[(b * t.n + q) * g.Gl + l] = mass_temp[(size_t)e * t.n + q];
    }
    return hip_check(hipMemcpy(g.M, buf.data(), 8 * buf.size(), hipMemcpyHostToDevice), "upload M") ? 0 : -1;
}

int sbx_fdm_sensed_response(SbxFdm* f, double* out) {
    if (!f || !out) return -1;
    const int k = f->tab.k;
    if (k == 0) return 0;
    return hip_check(hipMemcpy(out, f->tab.S, 8 * (size_t)k * k, hipMemcpyDeviceToHost), "copy S") ? 0 : -1;
}

int sbx_fdm_air_responses(SbxFdm* f, double* out) {
    if (!f || !out) return -1;
    const sbf::Tables& t = f->tab;
    if (!t.R || t.k == 0) return 1;
    return hip_check(hipMemcpy(out, t.R, 8 * (size_t)t.k * t.n, hipMemcpyDeviceToHost), "copy R") ? 0 : -1;
}

int sbx_fdm_lu_solve(SbxFdm* f, const double* b, double* x, int n_rhs) {
    if (!f || !b || !x || n_rhs < 1) return -1;
    const int n = f->tab.n;
    sbf::Group g{};
    const size_t before = f->owned.size();
    double *db = nullptr, *dx = nullptr;
    bool ok = make_group(f, n_rhs, std::min(64, next_pow2(n_rhs)), false, &g)
              && hip_check(hipMalloc(&db, 8 * (size_t)n_rhs * n), "hipMalloc(b)")
              && hip_check(hipMalloc(&dx, 8 * (size_t)n_rhs * n), "hipMalloc(x)")
              && hip_check(hipMemcpy(db, b, 8 * (size_t)n_rhs * n, hipMemcpyHostToDevice), "upload b")
              && hip_check((hipError_t)sbf_launch_solve_cols(&f->tab, &g, db, dx, nullptr, nullptr), "solve")
              && hip_check(hipMemcpy(x, dx, 8 * (size_t)n_rhs * n, hipMemcpyDeviceToHost), "copy x");
    (void)hipFree(db);
    (void)hipFree(dx);
    for (size_t i = before; i < f->owned.size(); i++) (void)hipFree(f->owned[i]);
    f->owned.resize(before);
    return ok ? 0 : -1;
}

}  // extern "C"
