// Building-scale field step (FDM plans with 10^5-10^6 cells): the shared
// device tables and per-group buffers the host (fdm.cpp) builds and the
// kernels (fdm_kernel.hip) read. Not part of the public ABI.
//
// Layouts. A group of G envs shares one factorization; its envs are split
// into nblk blocks of Gl lanes (the last block may hold fewer envs), and every
// per-env field array is block-major, env-minor: element (cell or row x, env
// b * Gl + l) of array A sits at A[(b * rows + x) * Gl + l], so the envs of a
// block read one row as Gl adjacent doubles. The solve works on the permuted
// vector of the baked factorization (SuperLU convention, complete_port/csim/
// sb_lu.c:38-63): w[i] = b[ir[i]], L w' = w, U z = w', x[t] = z[pc[t]].
#pragma once
#include <stddef.h>
#include <stdint.h>

namespace sbf {

// One triangular factor as level-ordered rows: rows[q] is the q-th row in
// level order (level l spans q in [lev[l], lev[l + 1])); its off-diagonal
// terms are (col[e], val[e]) for e in [ptr[q], ptr[q + 1]), in the order the
// reference's column sweep applies them (L: ascending column, U: descending);
// diag[q] is U's diagonal (unused for the unit L).
struct Tri {
    int nlev;
    const int* lev;
    const int* rows;
    const int* ptr;
    const int* col;
    const double* val;
    const double* diag;
};

// A run of consecutive levels lev0 .. lev0 + nlev - 1 of a factor's Tri,
// solved level by level by one workgroup per block with each row's terms cut
// into chunks of kChunk spread over the lanes (partial sums in LDS, then one
// wavefront per row, or one lane per row where no row of the level has more
// than one chunk, adds them and finishes the row). Two kinds:
//   lds = 1: the run's own row values live in LDS for its duration (the narrow
//     levels at the top of the elimination tree: the last levels of the L
//     sweep, the first of the U sweep); terms on earlier levels ("head" terms,
//     final before the run starts) per row in [hptr[r], hptr[r + 1]) of
//     (hcol, hval) are applied first, and chunk positions index the run;
//   lds = 0: values stay in HBM and chunk positions are row ids.
// Rows in level order r = 0 .. m-1 (rows[r]); level t spans chunks
// [tchunk[t], tchunk[t + 1]) and rows [trow[t], trow[t + 1]); row r's chunks
// are [rchunk[r], rchunk[r + 1]). tmode[t]: 0 no row of the level has more
// than one chunk (each lane finishes its rows directly, no partials); 1 and 2
// chunks spread over all lanes, partials in LDS, rows finished one lane each
// (1, wide levels) or one wavefront each (2, a few rows longer than a
// wavefront's lanes); 3 one wavefront per row, no partials. Padding terms are
// (0, 0.0).
constexpr int kChunk = 8;

struct Tail {
    int lds;
    int lev0, m, nlev, max_chunks;
    const int* rows;
    const double* diag;     // [m] U's diagonal (unused for L)
    const int* hptr;
    const int* hcol;
    const double* hval;
    const int* trow;
    const int* tchunk;
    const int* tmode;
    const int* rchunk;
    const int* cpos;        // [chunks * kChunk]
    const double* cval;     // [chunks * kChunk]
};

// How one factor's sweep runs in the default (non-exact) mode: the levels
// before the LDS run, the LDS run, the levels after it; the levels before and
// after run chunked from HBM when one level's partials fit in LDS, else as
// plain row solves.
struct Sweep {
    int pre_end;            // levels [0, pre_end) before the LDS run
    int post_begin;         // levels [post_begin, nlev) after it
    int pre_chunked, post_chunked;
    Tail pre, mid, post;    // (mid.nlev may be 0)
};

struct Tables {
    int n, n_cvs, k, n_unsolved;
    const int* ir;          // [n] row of the permuted vector -> solved index t of its right-hand side
    const int* ipr;         // [n] solved index t -> that row (the inverse of ir)
    const int* pc;          // [n] solved index t -> row of the permuted solution
    const int* solved;      // [n] t -> cell p
    const int* unsolved;    // [n_unsolved] cells held at the ambient temperature
    const double *cap, *dir, *mcoup, *mret, *mgain;   // [n] by t
    const double *a0, *a1, *hz, *vt, *cd;             // [n] by t: exterior face areas, half widths, conductivity
    Tri L, U;
    int fast;               // chunked runs (reassociated sums) instead of every level in order
    Sweep SL, SU;
    // sensed rows (k): entries p in [sn_p[i], sn_p[i + 1]) weigh row sn_w[p] of the solution
    const int* sn_p;
    const int* sn_w;
    const double* sn_x;
    // applied columns, transposed per permuted row i: (column at_j[e], value at_x[e]) for
    // e in [at_p[i], at_p[i + 1]), ascending column
    const int* at_p;
    const int* at_j;
    const double* at_x;
    const double* S;        // [k][k] sensed A^-1 applied
    // default mode: R [k][n], row j the solution A^-1 applied_j of applied
    // column j by solved index t (exact-mode solves at open), so a step's
    // air-side correction A^-1 (applied q) is the combination R^T q instead of
    // a second solve; null in exact mode
    const double* R;
    // blobs with zones (full env scenarios): the zone whose heat each solved
    // cell t carries, or -1 (a zone's heat goes to its room's cells; a cell of
    // two zones' rooms takes the later zone's, as csim assigns input_q)
    const int* czone;       // [n] or null
    int nz;
};

struct Group {
    int G, Gl, nblk;
    double* T;              // [nblk][n_cvs][Gl]
    double* M;              // [nblk][n][Gl]
    double* W1;             // [nblk][n][Gl] the forcing solve
    double* W2;             // [nblk][n][Gl] the air-side correction (exact mode; null with Tables::R)
    double* pw;             // [G][k] air-side power, then the dense solve's result
    double* mat;            // [G][k][k] I + diag(g) S
    int* eact;              // [G] env has a nonzero air-side conductance this step
    int* bact;              // [nblk] some env of the block has
};

// One batched step's inputs (device): input_q [G][n_cvs], ambient / h [G],
// air_g / air_T [G][k]. With q null, each cell's input_q is its zone's heat
// per cell qz [G][nz] (Tables::czone; 0 outside the rooms).
struct StepIn {
    const double* q;
    const double* amb;
    const double* h;
    const double* g;
    const double* airT;
    const double* qz;
};

// The host (g++) and the device (hipcc) compile these structs separately and
// exchange them byte for byte: both builds check the same sizes and offsets.
static_assert(sizeof(Tri) == 56 && sizeof(Tail) == 112 && sizeof(Sweep) == 352, "Tri / Tail / Sweep layout");
static_assert(sizeof(Tables) == 1040 && offsetof(Tables, S) == 1008 && offsetof(Tables, R) == 1016
              && offsetof(Tables, nz) == 1032, "Tables layout");
static_assert(sizeof(Group) == 80 && sizeof(StepIn) == 48, "Group / StepIn layout");

}  // namespace sbf
