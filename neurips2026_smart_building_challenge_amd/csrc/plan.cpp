// Solve planner.
//
// The reference csim replays baked factors of A (complete_port/csim/sb_lu.c)
// and folds the air side in with a dense k x k solve (sb_fdm.c:153-181). The
// device instead refactorizes S = P (A + P_a G S_a) P^T every step in the
// baked permutation P, whose fill pattern equals the baked one because G only
// touches diagonal entries. Each entry of L and U is one "task" (Crout form):
//
//   U[i][j] = S[i][j] - sum_{k<i} L[i][k] U[k][j]             (i <= j)
//   L[i][j] = (S[i][j] - sum_{k<j} L[i][k] U[k][j]) * r_j      (i >  j)
//   r_j     = 1 / U[j][j]   (written by the task of U[j][j])
//
// and the solves reuse the same machinery on a vector of slots:
//
//   y_i = w_i - sum_{k<i} L[i][k] y_k                          (forward)
//   x_i = (y_i - sum_{j>i} U[i][j] x_j) * r_i                  (backward, in place)
//
// With compact terms (systems of at most 255 unknowns and 4,096 slots) L is
// kept unscaled, L'[i][j] = L[i][j] * U[j][j], and every product that reads it
// takes the reciprocal as a third factor:
//
//   U[i][j]  = S[i][j] - sum_{k<i} L'[i][k] r_k U[k][j]
//   L'[i][j] = S[i][j] - sum_{k<j} L'[i][k] r_k U[k][j]
//   y_i      = w_i - sum_{k<i} L'[i][k] r_k y_k
//
// so an L entry no longer waits for its column's pivot: a column costs one
// level of the dependency chain instead of two (81 zones: 140 levels -> 94).
// L'[i][k] * r_k rounds to the value the scaled form stores for L[i][k].
//
// Every task multiplies its result by a slot (the pivot reciprocal, or the
// constant 1.0), so a pass runs without divergent branches; a pass holding a
// diagonal task also computes the reciprocal of every lane's result and
// stores it to the lane's reciprocal slot (the sink for other tasks).
//
// A task's level is one more than the levels of everything it reads; tasks of
// one level are independent. A task runs on a segment of S lanes (S a power of
// two up to kPlanSegMax, aligned, so the segment lies in one 16-lane row):
// lane j of the segment takes the task's terms j, j + S, j + 2S, ..., the
// segment's first lane (its leader) starts from the target's value and the
// others from 0, and a butterfly over the segment (partners lane ^ 1, ^ 2,
// ^ 4, ^ 8) leaves the sum in every lane; the leader stores it. A level's
// tasks, sorted by term count (descending), fill passes of `width` lanes with
// the narrowest segments that keep every lane at kPlanKmax terms or fewer;
// lanes a pass leaves free then widen the segment of its longest lane load,
// one doubling at a time, as long as that shortens the pass. A pass stores one
// 64-bit header for each of the `width` lanes (idle lanes included) and its
// terms lane by lane: lane l's terms sit at word_off + l * stride + m, stride =
// maxcnt rounded up to 4 (a lane's terms past its count are the (0, 0) term,
// which reads the zero slot), so a lane reads its pass with four 16-byte loads
// whose addresses need nothing but the pass record, and no loaded value is
// inspected before the pass runs. The pass count is padded with empty passes
// to a multiple of kPlanDepth, the kernel's prefetch depth.
// Dot products longer than kPlanKmax * kPlanSegMax terms become a chain of
// tasks on the same slot; only the last one divides.
//
// build_relax prepares the alternative used for strongly diagonally dominant
// systems: Jacobi sweeps with a certified contraction bound (see plan.h).
#include "plan.h"

#include <algorithm>
#include <cmath>
#include <unordered_map>

namespace sbh {

namespace {

// One product of a task's sum: slot[a] * slot[r] * slot[b] (r = kSlotOne when
// the product has two factors).
struct Term {
    int a, b, r;
};

struct Task {
    int target;
    int mul;          // slot multiplying the result (reciprocal or kSlotOne)
    int inv_target;   // slot receiving 1/result (kSlotSink unless a pivot)
    int level;
    std::vector<Term> terms;
};

// a | b << 16 (16-bit terms, r always kSlotOne), or a | b << 12 | v << 24
// (compact terms), v = r - scale_base: 0 reads the scale base's 1.0, k + 1 the
// reciprocal of pivot k
uint32_t term_word(const SolvePlan& P, const Term& t) {
    if (P.term_bits == 16) return (uint32_t)t.a | ((uint32_t)t.b << 16);
    const int v = t.r == kSlotOne ? 0 : t.r - P.scale_base;
    return (uint32_t)t.a | ((uint32_t)t.b << 12) | ((uint32_t)v << 24);
}

bool fail(std::string* err, const std::string& msg) {
    *err = msg;
    return false;
}

}  // namespace

bool build_plan(const Blob& b, int width, SolvePlan* out, std::string* err) {
    SolvePlan& P = *out;
    P = SolvePlan();
    P.width = width;
    uint64_t ns = 0, cnt = 0;
    const int64_t* solved = b.i64("solved", &ns);
    const int64_t* grid = b.i64("grid");
    if (!solved || !grid) return fail(err, "blob lacks grid/solved");
    const int n = (int)ns;
    if ((int64_t)n != grid[0] * grid[1]) return fail(err, "only blobs with every cell solved are supported");
    for (int t = 0; t < n; t++)
        if (solved[t] != t) return fail(err, "solved cells must be 0..n-1 in order");
    P.n = n;

    const int32_t* Ap = b.i32("A_system_indptr", &cnt);
    if (!Ap || (int)cnt != n + 1) return fail(err, "blob lacks A_system (CSC n x n)");
    const int32_t* Ai = b.i32("A_system_indices");
    const double* Ax = b.f64("A_system_data");
    const int32_t* pr = b.i32("lu_perm_r", &cnt);
    const int32_t* pc = b.i32("lu_perm_c");
    if (!pr || !pc || (int)cnt != n) return fail(err, "blob lacks lu_perm_r/lu_perm_c");
    P.pos.assign(pc, pc + n);
    std::vector<int> q(n, -1);
    for (int t = 0; t < n; t++) {
        if (pr[t] != pc[t]) return fail(err, "row and column permutations differ (pivoting is not supported)");
        if (pc[t] < 0 || pc[t] >= n || q[pc[t]] >= 0) return fail(err, "lu_perm_c is not a permutation");
        q[pc[t]] = t;
    }
    const int32_t* Lp = b.i32("lu_L_indptr", &cnt);
    if (!Lp || (int)cnt != n + 1) return fail(err, "blob lacks lu_L");
    const int32_t* Li = b.i32("lu_L_indices");
    const int32_t* Up = b.i32("lu_U_indptr", &cnt);
    if (!Up || (int)cnt != n + 1) return fail(err, "blob lacks lu_U");
    const int32_t* Ui = b.i32("lu_U_indices");

    // structural pattern in permuted coordinates
    std::vector<std::vector<int>> Lcol(n), Lrow(n), Ucol(n), Urow(n);   // strict parts
    for (int j = 0; j < n; j++) {
        bool diagL = false, diagU = false;
        for (int p = Lp[j]; p < Lp[j + 1]; p++) {
            int i = Li[p];
            if (i == j) diagL = true;
            else if (i > j && i < n) { Lcol[j].push_back(i); Lrow[i].push_back(j); }
            else return fail(err, "lu_L has an entry above the diagonal");
        }
        for (int p = Up[j]; p < Up[j + 1]; p++) {
            int i = Ui[p];
            if (i == j) diagU = true;
            else if (i < j && i >= 0) { Ucol[j].push_back(i); Urow[i].push_back(j); }
            else return fail(err, "lu_U has an entry below the diagonal");
        }
        if (!diagL || !diagU) return fail(err, "lu_L/lu_U lack a diagonal entry");
    }
    for (int i = 0; i < n; i++) {
        std::sort(Lcol[i].begin(), Lcol[i].end());
        std::sort(Lrow[i].begin(), Lrow[i].end());
        std::sort(Ucol[i].begin(), Ucol[i].end());
        std::sort(Urow[i].begin(), Urow[i].end());
    }

    // slots: 0 zero, 1 sink, 2 one, then per k: U row k (diagonal first),
    // L column k; then a second 1.0 (the scale base), the n pivot reciprocals,
    // the vector
    std::unordered_map<long long, int> slot;
    slot.reserve(8 * n);
    auto key = [n](int i, int j) { return (long long)i * n + j; };
    int ns_ = 3;
    for (int k = 0; k < n; k++) {
        slot[key(k, k)] = ns_++;
        for (int j : Urow[k]) slot[key(k, j)] = ns_++;
        for (int i : Lcol[k]) slot[key(i, k)] = ns_++;
    }
    P.scale_base = ns_;
    P.inv_base = ns_ + 1;
    P.vec_base = P.inv_base + n;
    P.n_slots = P.vec_base + n;
    if (P.n_slots > 65535) return fail(err, "system too large for 16-bit slots");
    // compact terms (12-bit slots and the 8-bit scale index) where they fit:
    // L then stays unscaled and each product reading it takes the column's
    // reciprocal as its third factor
    P.term_bits = (P.n_slots <= (1 << 12) && n <= 255) ? 12 : 16;
    const bool defer = P.term_bits == 12;

    // fill closure: every update target must be structural
    for (int k = 0; k < n; k++)
        for (int i : Lcol[k])
            for (int j : Urow[k])
                if (!slot.count(key(i, j))) return fail(err, "baked LU pattern is not closed under elimination");

    // initial values: permuted A
    P.slot_init.assign(P.n_slots, 0.0);
    P.slot_init[kSlotOne] = 1.0;
    P.slot_init[P.scale_base] = 1.0;
    for (int c = 0; c < n; c++)
        for (int p = Ap[c]; p < Ap[c + 1]; p++) {
            int r = Ai[p];
            auto it = slot.find(key(P.pos[r], P.pos[c]));
            if (it == slot.end()) return fail(err, "A_system entry outside the LU pattern");
            P.slot_init[it->second] = Ax[p];
        }

    // air side: one unit entry per applied column and sensed row, same node
    const int64_t* sshape = b.i64("sensed_shape");
    const int k = sshape ? (int)sshape[0] : 0;
    P.k = k;
    const int32_t* ap = b.i32("applied_indptr");
    const int32_t* ai = b.i32("applied_indices");
    const double* ax = b.f64("applied_data");
    const int32_t* sp = b.i32("sensed_indptr");
    const int32_t* si = b.i32("sensed_indices");
    const double* sx = b.f64("sensed_data");
    if (k > 0 && (!ap || !ai || !ax || !sp || !si || !sx)) return fail(err, "blob lacks applied/sensed");
    std::vector<char> seen(n, 0);
    for (int c = 0; c < k; c++) {
        if (ap[c + 1] - ap[c] != 1 || sp[c + 1] - sp[c] != 1)
            return fail(err, "air side must have one applied and one sensed entry per column");
        int t = ai[ap[c]];
        if (si[sp[c]] != t || ax[ap[c]] != 1.0 || sx[sp[c]] != 1.0 || t < 0 || t >= n || seen[t])
            return fail(err, "air side must couple each column to its own node with unit weight");
        seen[t] = 1;
        P.air_node.push_back(t);
        P.air_slot.push_back(slot[key(P.pos[t], P.pos[t])]);
    }

    // tasks
    std::vector<int> slot_level(P.n_slots, 0);
    std::vector<Task> tasks;
    auto intersect = [](const std::vector<int>& a, const std::vector<int>& b, int lim,
                        std::vector<int>& o) {
        o.clear();
        size_t x = 0, y = 0;
        while (x < a.size() && y < b.size()) {
            if (a[x] >= lim || b[y] >= lim) break;
            if (a[x] < b[y]) x++;
            else if (a[x] > b[y]) y++;
            else { o.push_back(a[x]); x++; y++; }
        }
    };
    std::vector<int> ks;
    // target, multiplier slot (reciprocal to depend on, or kSlotOne), reciprocal
    // slot to produce (or kSlotSink), terms, extra dependency level
    auto add_task = [&](int target, int mul, int inv_target, std::vector<Term>&& terms,
                        int extra_level) {
        // split into chains of at most kTaskTerms terms; the last piece
        // scales and produces the reciprocal
        constexpr size_t kTaskTerms = (size_t)kPlanKmax * kPlanSegMax;
        size_t nt = terms.size();
        size_t pieces = nt == 0 ? 1 : (nt + kTaskTerms - 1) / kTaskTerms;
        int prev = extra_level;
        for (size_t pc = 0; pc < pieces; pc++) {
            size_t lo = pc * kTaskTerms, hi = std::min(nt, lo + kTaskTerms);
            std::vector<Term> part(terms.begin() + lo, terms.begin() + hi);
            int lv = prev;
            for (auto& t : part)
                lv = std::max(lv, std::max(slot_level[t.a], std::max(slot_level[t.b], slot_level[t.r])));
            const bool last = pc + 1 == pieces;
            if (last) lv = std::max(lv, slot_level[mul]);
            lv += 1;
            slot_level[target] = lv;
            if (last && inv_target != kSlotSink) slot_level[inv_target] = lv;
            prev = lv;
            tasks.push_back(Task{target, last ? mul : kSlotOne, last ? inv_target : kSlotSink, lv,
                                 std::move(part)});
        }
    };
    const int vb = P.vec_base, ib = P.inv_base;
    for (int r = 0; r < n; r++) {
        // U row r (j >= r): terms over k < r; the diagonal task always runs
        // (it produces the reciprocal even without terms)
        std::vector<int> ucols;
        ucols.push_back(r);
        ucols.insert(ucols.end(), Urow[r].begin(), Urow[r].end());
        for (int j : ucols) {
            intersect(Lrow[r], Ucol[j], r, ks);
            const bool diag = j == r;
            if (ks.empty() && !diag) continue;   // slot already holds its value
            std::vector<Term> terms;
            for (int m : ks) terms.push_back({slot[key(r, m)], slot[key(m, j)], defer ? ib + m : kSlotOne});
            add_task(slot[key(r, j)], kSlotOne, diag ? ib + r : kSlotSink, std::move(terms), 0);
        }
        // L column r (i > r): terms over k < r, scaled by 1/U[r][r] (compact
        // terms: left unscaled, L[i][r] * U[r][r], so the task does not wait
        // for the pivot; its readers multiply by the reciprocal)
        for (int i : Lcol[r]) {
            intersect(Lrow[i], Ucol[r], r, ks);
            std::vector<Term> terms;
            for (int m : ks) terms.push_back({slot[key(i, m)], slot[key(m, r)], defer ? ib + m : kSlotOne});
            add_task(slot[key(i, r)], defer ? kSlotOne : ib + r, kSlotSink, std::move(terms), 0);
        }
    }
    // forward solve
    std::vector<int> y_read_max(n, 0);
    for (int i = 0; i < n; i++) {
        if (Lrow[i].empty()) continue;
        std::vector<Term> terms;
        for (int m : Lrow[i]) terms.push_back({slot[key(i, m)], vb + m, defer ? ib + m : kSlotOne});
        add_task(vb + i, kSlotOne, kSlotSink, std::move(terms), 0);
        for (int m : Lrow[i]) y_read_max[m] = std::max(y_read_max[m], slot_level[vb + i]);
    }
    // backward solve, in place over y; a slot is overwritten only after its
    // last forward reader
    for (int i = n - 1; i >= 0; i--) {
        std::vector<Term> terms;
        for (int j : Urow[i]) terms.push_back({slot[key(i, j)], vb + j, kSlotOne});
        int lv0 = std::max(slot_level[vb + i], y_read_max[i]);
        add_task(vb + i, ib + i, kSlotSink, std::move(terms), lv0);
    }

    // levels -> passes of lane segments
    int maxlv = 0;
    for (auto& t : tasks) maxlv = std::max(maxlv, t.level);
    P.n_levels = maxlv;
    P.n_tasks = (int)tasks.size();
    std::vector<std::vector<int>> by_level(maxlv + 1);
    for (int t = 0; t < (int)tasks.size(); t++) by_level[tasks[t].level].push_back(t);
    long long npairs = 0, ndiv = 0;
    auto load = [&](int id, int seg) { return ((int)tasks[id].terms.size() + seg - 1) / seg; };
    for (int lv = 1; lv <= maxlv; lv++) {
        auto& ids = by_level[lv];
        std::stable_sort(ids.begin(), ids.end(), [&](int a, int c) {
            if (tasks[a].terms.size() != tasks[c].terms.size()) return tasks[a].terms.size() > tasks[c].terms.size();
            return tasks[a].target < tasks[c].target;
        });
        size_t s = 0;
        while (s < ids.size()) {
            // the pass's tasks at their narrowest segments
            std::vector<int> pid, seg;
            int used = 0;
            while (s < ids.size()) {
                int sg = 1;
                while (load(ids[s], sg) > kPlanKmax) sg *= 2;
                if (used + sg > width) break;
                pid.push_back(ids[s]);
                seg.push_back(sg);
                used += sg;
                s++;
            }
            // widen the longest lane load while lanes are free
            for (;;) {
                int best = -1;
                for (size_t q = 0; q < pid.size(); q++)
                    if (best < 0 || load(pid[q], seg[q]) > load(pid[best], seg[best])) best = (int)q;
                if (best < 0 || load(pid[best], seg[best]) <= 1 || seg[best] >= kPlanSegMax
                    || used + seg[best] > width)
                    break;
                used += seg[best];
                seg[best] *= 2;
            }
            // place segments widest first (power-of-two sizes in descending
            // order land on aligned offsets)
            std::vector<int> ord(pid.size());
            for (size_t q = 0; q < ord.size(); q++) ord[q] = (int)q;
            std::stable_sort(ord.begin(), ord.end(), [&](int a, int c) { return seg[a] > seg[c]; });
            struct Lane {
                int task, j, seg;
            };
            std::vector<Lane> lanes;
            for (int q : ord)
                for (int j = 0; j < seg[q]; j++) lanes.push_back(Lane{pid[q], j, seg[q]});
            const int nact = (int)lanes.size();
            int maxcnt = 0, piv = 0;
            PassInfo pi{};
            pi.hdr_off = (int)P.hdr.size();
            pi.word_off = (int)P.words.size();
            for (const Lane& l : lanes) {
                const Task& t = tasks[l.task];
                const int cnt = ((int)t.terms.size() - l.j + l.seg - 1) / l.seg;
                maxcnt = std::max(maxcnt, cnt);
                int lg = 0;
                while ((1 << lg) < l.seg) lg++;
                const bool lead = l.j == 0;
                const uint64_t flags = (uint64_t)lg | ((uint64_t)(lead ? 1 : 0) << 3) | ((uint64_t)cnt << 4);
                const int tgt = lead ? t.target : kSlotZero;
                const int mul = lead ? t.mul : kSlotOne;
                const int inv = lead ? t.inv_target : kSlotSink;
                P.hdr.push_back((uint64_t)(uint32_t)tgt | ((uint64_t)(uint32_t)mul << 16)
                                | ((uint64_t)(uint32_t)inv << 32) | (flags << 48));
                if (lead) {
                    npairs += (long long)t.terms.size();
                    ndiv += t.inv_target != kSlotSink ? 1 : 0;
                    if (t.inv_target != kSlotSink) piv = 1;
                }
            }
            for (int l = nact; l < width; l++) P.hdr.push_back(kIdleHeader);
            // butterfly steps the pass needs: log2 of its widest segment
            int lgmax = 0;
            for (const Lane& l : lanes)
                while ((1 << lgmax) < l.seg) lgmax++;
            pi.packed = nact | (maxcnt << 8) | (piv << 16) | (lgmax << 17);
            const int stride = (maxcnt + 3) & ~3;
            for (const Lane& l : lanes) {
                const Task& t = tasks[l.task];
                for (int m = 0; m < stride; m++) {
                    const size_t q = (size_t)l.j + (size_t)m * l.seg;
                    P.words.push_back(q < t.terms.size() ? term_word(P, t.terms[q]) : 0u);
                }
            }
            P.passes.push_back(pi);
        }
    }
    // empty passes up to a multiple of the prefetch depth: no lane leads, no pivot
    while (P.passes.size() % kPlanDepth) {
        PassInfo pi{};
        pi.hdr_off = (int)P.hdr.size();
        pi.word_off = (int)P.words.size();
        for (int l = 0; l < width; l++) P.hdr.push_back(kIdleHeader);
        P.passes.push_back(pi);
    }
    P.words.resize(P.words.size() + kWordTail, 0u);
    P.n_pairs = npairs;
    P.n_divs = ndiv;
    return true;
}

void build_relax(const Blob& b, const SolvePlan& lu, RelaxPlan* out) {
    RelaxPlan& R = *out;
    R = RelaxPlan();
    const int n = lu.n;
    R.n = n;
    auto no = [&](const std::string& why) { R.ok = false; R.why = why; };
    if (n > kRelaxRows) return no("more than " + std::to_string(kRelaxRows) + " solved cells");
    uint64_t cnt = 0;
    const int32_t* Ap = b.i32("A_system_indptr", &cnt);
    const int32_t* Ai = b.i32("A_system_indices");
    const double* Ax = b.f64("A_system_data");
    if (!Ap || !Ai || !Ax || (int)cnt != n + 1) return no("blob lacks A_system");
    // CSC -> rows (duplicates summed, explicit zeros dropped)
    std::vector<std::vector<std::pair<int, double>>> rows(n);
    std::vector<double> diag(n, 0.0);
    for (int c = 0; c < n; c++)
        for (int p = Ap[c]; p < Ap[c + 1]; p++) {
            const int r = Ai[p];
            if (r < 0 || r >= n) return no("A_system row index out of range");
            if (r == c) { diag[r] += Ax[p]; continue; }
            bool merged = false;
            for (auto& e : rows[r])
                if (e.first == c) { e.second += Ax[p]; merged = true; }
            if (!merged) rows[r].push_back({c, Ax[p]});
        }
    double rho = 0.0;
    int terms = 0;
    for (int i = 0; i < n; i++) {
        auto& row = rows[i];
        row.erase(std::remove_if(row.begin(), row.end(), [](const std::pair<int, double>& e) { return e.second == 0.0; }),
                  row.end());
        std::sort(row.begin(), row.end());
        if (!(diag[i] > 0.0)) return no("a diagonal entry of A is not positive");
        double off = 0.0;
        for (auto& e : row) off += std::fabs(e.second);
        rho = std::max(rho, off / diag[i]);
        terms = std::max(terms, (int)row.size());
    }
    R.rho = rho;
    R.terms = terms;
    if (terms > kRelaxTerms) return no("a row of A has more than " + std::to_string(kRelaxTerms) + " off-diagonal entries");
    if (!(rho <= kRelaxRhoMax)) return no("A is not diagonally dominant enough (rho " + std::to_string(rho) + ")");
    R.diag.assign(kRelaxRows, 1.0);
    R.air_col.assign(kRelaxRows, -1);
    R.val.assign((size_t)kRelaxTerms * kRelaxRows, 0.0);
    R.col.assign((size_t)kRelaxTerms * kRelaxRows, 0);
    for (int i = 0; i < n; i++) {
        R.diag[i] = diag[i];
        for (size_t m = 0; m < rows[i].size(); m++) {
            R.val[m * kRelaxRows + i] = rows[i][m].second;
            R.col[m * kRelaxRows + i] = rows[i][m].first;
        }
    }
    for (int c = 0; c < lu.k; c++) R.air_col[lu.air_node[c]] = c;
    R.ok = true;
}

namespace {

// Inverse of a small dense matrix (row-major, m x m) by Gauss-Jordan with
// partial pivoting; false if singular.
bool invert_small(std::vector<double> a, int m, std::vector<double>* inv) {
    std::vector<double>& r = *inv;
    r.assign((size_t)m * m, 0.0);
    for (int i = 0; i < m; i++) r[(size_t)i * m + i] = 1.0;
    for (int c = 0; c < m; c++) {
        int p = c;
        for (int i = c + 1; i < m; i++)
            if (std::fabs(a[(size_t)i * m + c]) > std::fabs(a[(size_t)p * m + c])) p = i;
        if (a[(size_t)p * m + c] == 0.0) return false;
        for (int j = 0; j < m; j++) {
            std::swap(a[(size_t)c * m + j], a[(size_t)p * m + j]);
            std::swap(r[(size_t)c * m + j], r[(size_t)p * m + j]);
        }
        const double d = a[(size_t)c * m + c];
        for (int j = 0; j < m; j++) {
            a[(size_t)c * m + j] /= d;
            r[(size_t)c * m + j] /= d;
        }
        for (int i = 0; i < m; i++) {
            if (i == c) continue;
            const double f = a[(size_t)i * m + c];
            if (f == 0.0) continue;
            for (int j = 0; j < m; j++) {
                a[(size_t)i * m + j] -= f * a[(size_t)c * m + j];
                r[(size_t)i * m + j] -= f * r[(size_t)c * m + j];
            }
        }
    }
    return true;
}

}  // namespace

void build_block(const Blob& b, const SolvePlan& lu, BlockPlan* out) {
    BlockPlan& B = *out;
    B = BlockPlan();
    const int n = lu.n;
    auto no = [&](const std::string& why) { B.ok = false; B.why = why; };
    if (n > 64 * kBlockSlots * kBlockRows)
        return no("more than " + std::to_string(64 * kBlockSlots * kBlockRows) + " solved cells");
    uint64_t cnt = 0;
    const int32_t* Ap = b.i32("A_system_indptr", &cnt);
    const int32_t* Ai = b.i32("A_system_indices");
    const double* Ax = b.f64("A_system_data");
    if (!Ap || !Ai || !Ax || (int)cnt != n + 1) return no("blob lacks A_system");
    std::vector<double> A((size_t)n * n, 0.0);
    for (int c = 0; c < n; c++)
        for (int p = Ap[c]; p < Ap[c + 1]; p++) {
            if (Ai[p] < 0 || Ai[p] >= n) return no("A_system row index out of range");
            A[(size_t)Ai[p] * n + c] += Ax[p];
        }
    auto a = [&](int i, int j) { return A[(size_t)i * n + j]; };
    for (int i = 0; i < n; i++) {
        if (!(a(i, i) > 0.0)) return no("a diagonal entry of A is not positive");
        for (int j = 0; j < n; j++)
            if (j != i && a(i, j) > 0.0) return no("A has a positive off-diagonal entry (not an M-matrix)");
    }
    // greedy partition: strongest couplings first, blocks of at most kBlockRows
    struct Edge {
        double s;
        int i, j;
    };
    std::vector<Edge> edges;
    for (int i = 0; i < n; i++)
        for (int j = i + 1; j < n; j++) {
            const double s = std::max(std::fabs(a(i, j)), std::fabs(a(j, i)));
            if (s > 0.0) edges.push_back({s / std::min(a(i, i), a(j, j)), i, j});
        }
    std::stable_sort(edges.begin(), edges.end(), [](const Edge& x, const Edge& y) { return x.s > y.s; });
    std::vector<int> parent(n), size(n, 1);
    for (int i = 0; i < n; i++) parent[i] = i;
    auto find = [&](int x) {
        while (parent[x] != x) x = parent[x] = parent[parent[x]];
        return x;
    };
    for (const Edge& e : edges) {
        int x = find(e.i), y = find(e.j);
        if (x == y || size[x] + size[y] > kBlockRows) continue;
        if (y < x) std::swap(x, y);
        parent[y] = x;
        size[x] += size[y];
    }
    std::vector<int> bid(n, -1);
    for (int i = 0; i < n; i++) {
        const int r = find(i);
        if (bid[r] < 0) {
            bid[r] = (int)B.blocks.size();
            B.blocks.push_back({});
        }
        B.blocks[bid[r]].push_back(i);
        bid[i] = bid[r];
    }
    B.n_blocks = (int)B.blocks.size();
    if (B.n_blocks > 64 * kBlockSlots) return no("more than " + std::to_string(64 * kBlockSlots) + " blocks");
    // per-row bound and off-block terms
    double rho = 0.0;
    int terms = 0;
    std::vector<std::vector<double>> binv(B.n_blocks);
    for (int k = 0; k < B.n_blocks; k++) {
        const auto& blk = B.blocks[k];
        const int m = (int)blk.size();
        std::vector<double> M((size_t)m * m);
        for (int x = 0; x < m; x++)
            for (int y = 0; y < m; y++) M[(size_t)x * m + y] = a(blk[x], blk[y]);
        if (!invert_small(M, m, &binv[k])) return no("a diagonal block of A is singular");
        double mx = 0.0;
        for (double v : binv[k]) mx = std::max(mx, std::fabs(v));
        for (double v : binv[k])
            if (v < -1e-14 * mx) return no("a diagonal block of A has a negative inverse entry");
        int t = 0;
        for (int x = 0; x < m; x++) {
            double s = 0.0;
            for (int j = 0; j < n; j++) {
                if (bid[j] == k) continue;
                double col_sum = 0.0;
                for (int y = 0; y < m; y++) col_sum += std::fabs(binv[k][(size_t)x * m + y]) * std::fabs(a(blk[y], j));
                s += col_sum;
                if (a(blk[x], j) != 0.0) t++;
            }
            rho = std::max(rho, s);
        }
        terms = std::max(terms, t);
    }
    B.rho = rho;
    B.terms = terms;
    if (terms > kBlockTerms) return no("a block has more than " + std::to_string(kBlockTerms) + " off-block entries");
    if (!(rho <= kRelaxRhoMax)) return no("block bound too large (rho " + std::to_string(rho) + ")");
    // tables
    const int R = kBlockRows, T = kBlockTerms, Q = kBlockSlots;
    B.row.assign((size_t)Q * R * 64, -1);
    B.diag.assign((size_t)Q * R * 64, 1.0);
    B.air.assign((size_t)Q * R * 64, -1);
    B.in.assign((size_t)Q * R * R * 64, 0.0);
    B.val.assign((size_t)Q * T * 64, 0.0);
    B.col.assign((size_t)Q * T * 64, 0);
    B.trow.assign((size_t)Q * T * 64, 0);
    std::vector<int> air_of(n, -1);
    for (int c = 0; c < lu.k; c++) air_of[lu.air_node[c]] = c;
    for (int k = 0; k < B.n_blocks; k++) {
        const auto& blk = B.blocks[k];
        const int lane = k % 64, q = k / 64;
        int t = 0;
        for (int p = 0; p < (int)blk.size(); p++) {
            const int i = blk[p];
            const size_t at = (size_t)(q * R + p) * 64 + lane;
            B.row[at] = i;
            B.diag[at] = a(i, i);
            B.air[at] = air_of[i];
            for (int p2 = 0; p2 < (int)blk.size(); p2++)
                if (p2 != p) B.in[((size_t)(q * R + p) * R + p2) * 64 + lane] = a(i, blk[p2]);
            for (int j = 0; j < n; j++)
                if (bid[j] != k && a(i, j) != 0.0) {
                    const size_t e = (size_t)(q * T + t) * 64 + lane;
                    B.val[e] = a(i, j);
                    B.col[e] = j;
                    B.trow[e] = p;
                    t++;
                }
        }
    }
    B.ok = true;
}

}  // namespace sbh
