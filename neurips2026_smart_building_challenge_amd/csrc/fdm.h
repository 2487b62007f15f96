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

struct Tables {
    int n, n_cvs, k, n_unsolved;
    const int* ir;          // [n] row of the permuted vector -> solved index t
    const int* pc;          // [n] solved index t -> row of the permuted vector
    const int* solved;      // [n] t -> cell p
    const int* unsolved;    // [n_unsolved] cells held at the ambient temperature
    const double *cap, *dir, *mcoup, *mret, *mgain;   // [n] by t
    const double *a0, *a1, *hz, *vt, *cd;             // [n] by t: exterior face areas, half widths, conductivity
    Tri L, U;
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
};

struct Group {
    int G, Gl, nblk;
    double* T;              // [nblk][n_cvs][Gl]
    double* M;              // [nblk][n][Gl]
    double* W1;             // [nblk][n][Gl] the forcing solve
    double* W2;             // [nblk][n][Gl] the air-side correction
    double* pw;             // [G][k] air-side power, then the dense solve's result
    double* mat;            // [G][k][k] I + diag(g) S
    int* eact;              // [G] env has a nonzero air-side conductance this step
    int* bact;              // [nblk] some env of the block has
};

// One batched step's inputs (device): input_q [n_cvs][G] (the G envs' heat of
// one cell adjacent), ambient / h [G], air_g / air_T [G][k].
struct StepIn {
    const double* q;
    const double* amb;
    const double* h;
    const double* g;
    const double* airT;
};

}  // namespace sbf
