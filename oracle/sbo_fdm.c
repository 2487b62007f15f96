/* Building-scale field step of the CPU oracle (TEST INFRASTRUCTURE: only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * liboracle.so).
 *
 * A restatement of the reference core's FDM field model over a blob's field
 * sections alone, for blobs that carry no env sections (the FDM-scale plans of
 * scenario/fdm.py):
 *   sbo_fdm_open          sb_fdm_init   (complete_port/csim/sb_fdm.c:40-118)
 *                         sb_lu_build   (complete_port/csim/sb_lu.c:6-30)
 *   sbo_fdm_lu_solve      sb_lu_solve   (sb_lu.c:38-63)
 *   sbo_fdm_exposure      sb_fdm_exposure (sb_fdm.c:126-140)
 *   sbo_fdm_step          sb_fdm_step   (sb_fdm.c:142-188)
 *   sbo_fdm_step_batch    sb_fdm_step_batch (sb_fdm.c:190-270): per env the
 *                         operations of sb_fdm_step in the same order, which
 *                         the reference documents as bit-identical to it
 * Every loop keeps the reference's operation order; with FP contraction off
 * the results are bit-identical to the reference compiled the same way
 * (checked against oracle/_ref in tests/test_fdm_oracle.py). */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "sbo.h"

struct SboFdm {
    SboBlob blob;
    int nr, nc, n_cvs, n, k;
    const int64_t* solved;
    const double *cap, *dir, *mcoup, *mret, *mgain;
    const double *horiz, *vert, *cond, *face0, *face1;
    const double *temp_init, *mass_init;
    const int32_t *Lp, *Li, *Up, *Ui;
    const double *Lx, *Ux;
    int *Ldiag, *Udiag, *ir, *pc;
    const int32_t *ap_p, *ap_i, *sn_p, *sn_i;
    const double *ap_x, *sn_x;
    double* S;          /* k x k: sensed A^-1 applied */
    double* work;       /* n */
};

void sbo_fdm_lu_solve(const SboFdm* f, const double* b, double* x) {
    const int n = f->n;
    double* w = f->work;
    for (int i = 0; i < n; i++) w[i] = b[f->ir[i]];
    for (int j = 0; j < n; j++) {
        double v = w[j];
        for (int p = f->Lp[j]; p < f->Lp[j + 1]; p++)
            if (p != f->Ldiag[j]) w[f->Li[p]] -= f->Lx[p] * v;
    }
    for (int j = n - 1; j >= 0; j--) {
        double v = w[j] / f->Ux[f->Udiag[j]];
        w[j] = v;
        for (int p = f->Up[j]; p < f->Up[j + 1]; p++)
            if (p != f->Udiag[j]) w[f->Ui[p]] -= f->Ux[p] * v;
    }
    for (int i = 0; i < n; i++) x[i] = w[f->pc[i]];
}

void sbo_fdm_close(SboFdm* f) {
    if (!f) return;
    free(f->Ldiag); free(f->Udiag); free(f->ir); free(f->pc); free(f->S); free(f->work);
    sbo_blob_free(&f->blob);
    free(f);
}

SboFdm* sbo_fdm_open(const char* path) {
    SboFdm* f = (SboFdm*)calloc(1, sizeof(SboFdm));
    if (!f) return NULL;
    if (sbo_blob_load(&f->blob, path) != 0) { free(f); return NULL; }
    const SboBlob* b = &f->blob;
    const int64_t* grid = sbo_i64(b, "grid");
    const SboSec* sv = sbo_sec(b, "solved");
    const int64_t* shp = sbo_i64(b, "sensed_shape");
    if (!grid || !sv || !shp) { fprintf(stderr, "sbo_fdm_open: field sections missing\n"); sbo_fdm_close(f); return NULL; }
    f->nr = (int)grid[0];
    f->nc = (int)grid[1];
    f->n_cvs = f->nr * f->nc;
    f->n = (int)sv->count;
    f->k = (int)shp[0];
    f->solved = sbo_i64(b, "solved");
    f->cap = sbo_f64(b, "capacitance_rate");
    f->dir = sbo_f64(b, "dirichlet_conductance");
    f->mcoup = sbo_f64(b, "mass_coupling");
    f->mret = sbo_f64(b, "mass_retained");
    f->mgain = sbo_f64(b, "mass_gained");
    f->horiz = sbo_f64(b, "horizontal");
    f->vert = sbo_f64(b, "vertical");
    f->cond = sbo_f64(b, "solver_conductivity");
    f->face0 = sbo_f64(b, "ambient_face_areas_0");
    f->face1 = sbo_f64(b, "ambient_face_areas_1");
    f->temp_init = sbo_f64(b, "temp_init");
    f->mass_init = sbo_f64(b, "mass_temp_init");
    f->Lp = sbo_i32(b, "lu_L_indptr"); f->Li = sbo_i32(b, "lu_L_indices"); f->Lx = sbo_f64(b, "lu_L_data");
    f->Up = sbo_i32(b, "lu_U_indptr"); f->Ui = sbo_i32(b, "lu_U_indices"); f->Ux = sbo_f64(b, "lu_U_data");
    f->ap_p = sbo_i32(b, "applied_indptr"); f->ap_i = sbo_i32(b, "applied_indices"); f->ap_x = sbo_f64(b, "applied_data");
    f->sn_p = sbo_i32(b, "sensed_indptr"); f->sn_i = sbo_i32(b, "sensed_indices"); f->sn_x = sbo_f64(b, "sensed_data");
    const int32_t* prr = sbo_i32(b, "lu_perm_r");
    const int32_t* pcc = sbo_i32(b, "lu_perm_c");
    if (!f->cap || !f->dir || !f->mcoup || !f->mret || !f->mgain || !f->horiz || !f->vert || !f->cond || !f->face0
        || !f->face1 || !f->temp_init || !f->mass_init || !f->Lp || !f->Li || !f->Lx || !f->Up || !f->Ui || !f->Ux
        || !f->ap_p || !f->ap_i || !f->ap_x || !f->sn_p || !f->sn_i || !f->sn_x || !prr || !pcc) {
        fprintf(stderr, "sbo_fdm_open: field sections missing\n");
        sbo_fdm_close(f);
        return NULL;
    }
    const int n = f->n, k = f->k;
    f->Ldiag = (int*)malloc(sizeof(int) * n);
    f->Udiag = (int*)malloc(sizeof(int) * n);
    f->ir = (int*)malloc(sizeof(int) * n);
    f->pc = (int*)malloc(sizeof(int) * n);
    f->S = (double*)malloc(sizeof(double) * (k ? k * k : 1));
    f->work = (double*)malloc(sizeof(double) * n);
    if (!f->Ldiag || !f->Udiag || !f->ir || !f->pc || !f->S || !f->work) { sbo_fdm_close(f); return NULL; }
    for (int j = 0; j < n; j++) {
        f->Ldiag[j] = f->Udiag[j] = -1;
        for (int p = f->Lp[j]; p < f->Lp[j + 1]; p++) if (f->Li[p] == j) { f->Ldiag[j] = p; break; }
        for (int p = f->Up[j]; p < f->Up[j + 1]; p++) if (f->Ui[p] == j) { f->Udiag[j] = p; break; }
        if (f->Ldiag[j] < 0 || f->Udiag[j] < 0) {
            fprintf(stderr, "sbo_fdm_open: factor column %d has no diagonal\n", j);
            sbo_fdm_close(f);
            return NULL;
        }
    }
    for (int i = 0; i < n; i++) f->ir[prr[i]] = i;
    for (int j = 0; j < n; j++) f->pc[j] = pcc[j];
    /* S = sensed A^-1 applied, one column per solve */
    double* r = (double*)malloc(sizeof(double) * n);
    double* yr = (double*)malloc(sizeof(double) * n);
    if (!r || !yr) { free(r); free(yr); sbo_fdm_close(f); return NULL; }
    for (int j = 0; j < k; j++) {
        for (int t = 0; t < n; t++) r[t] = 0.0;
        for (int p = f->ap_p[j]; p < f->ap_p[j + 1]; p++) r[f->ap_i[p]] = f->ap_x[p];
        sbo_fdm_lu_solve(f, r, yr);
        for (int i = 0; i < k; i++) {
            double acc = 0.0;
            for (int p = f->sn_p[i]; p < f->sn_p[i + 1]; p++) acc += f->sn_x[p] * yr[f->sn_i[p]];
            f->S[i * k + j] = acc;
        }
    }
    free(r);
    free(yr);
    return f;
}

void sbo_fdm_dims(const SboFdm* f, int* out) {
    out[0] = f->n_cvs;
    out[1] = f->n;
    out[2] = f->k;
    out[3] = f->nr;
    out[4] = f->nc;
}

const double* sbo_fdm_sensed_response(const SboFdm* f) { return f->S; }

void sbo_fdm_init_state(const SboFdm* f, double* T, double* M) {
    memcpy(T, f->temp_init, sizeof(double) * f->n_cvs);
    memcpy(M, f->mass_init, sizeof(double) * f->n);
}

void sbo_fdm_exposure(const SboFdm* f, double h, double* out) {
    for (int t = 0; t < f->n; t++) {
        int64_t p = f->solved[t];
        double e = 0.0;
        double a0 = f->face0[p];
        if (a0 > 0.0) e += h * a0 / (1.0 + h * 0.5 * f->horiz[p] / f->cond[p]);
        double a1 = f->face1[p];
        if (a1 > 0.0) e += h * a1 / (1.0 + h * 0.5 * f->vert[p] / f->cond[p]);
        out[t] = e;
    }
}

/* One env: T [n_cvs], M [n] updated in place; air_g / air_T [k] or NULL. */
int sbo_fdm_step(const SboFdm* f, double* T, double* M, const double* input_q, double ambient, double h,
                 const double* air_g, const double* air_T) {
    const int n = f->n, k = f->k;
    double* ex = (double*)malloc(sizeof(double) * n);
    double* rhs = (double*)malloc(sizeof(double) * n);
    double* y = (double*)malloc(sizeof(double) * n);
    double* yr = (double*)malloc(sizeof(double) * n);
    double* pw = (double*)malloc(sizeof(double) * (k ? k : 1));
    double* mat = (double*)malloc(sizeof(double) * (k ? k * k : 1));
    if (!ex || !rhs || !y || !yr || !pw || !mat) {
        free(ex); free(rhs); free(y); free(yr); free(pw); free(mat);
        return -1;
    }
    sbo_fdm_exposure(f, h, ex);
    for (int t = 0; t < n; t++) {
        int64_t p = f->solved[t];
        rhs[t] = f->cap[t] * T[p] + input_q[p] + ambient * (f->dir[t] + ex[t]) + f->mcoup[t] * M[t];
    }
    sbo_fdm_lu_solve(f, rhs, y);
    if (k > 0 && air_g) {
        int active = 0;
        for (int i = 0; i < k; i++) if (air_g[i] != 0.0) { active = 1; break; }
        if (active) {
            for (int i = 0; i < k; i++) {
                double acc = 0.0;
                for (int p = f->sn_p[i]; p < f->sn_p[i + 1]; p++) acc += f->sn_x[p] * y[f->sn_i[p]];
                pw[i] = air_g[i] * (air_T[i] - acc);
            }
            for (int i = 0; i < k; i++)
                for (int j = 0; j < k; j++) mat[i * k + j] = (i == j ? 1.0 : 0.0) + air_g[i] * f->S[i * k + j];
            sbo_dense_solve(k, mat, pw);
            for (int t = 0; t < n; t++) rhs[t] = 0.0;
            for (int j = 0; j < k; j++) {
                double qj = pw[j];
                if (qj == 0.0) continue;
                for (int p = f->ap_p[j]; p < f->ap_p[j + 1]; p++) rhs[f->ap_i[p]] += f->ap_x[p] * qj;
            }
            sbo_fdm_lu_solve(f, rhs, yr);
            for (int t = 0; t < n; t++) y[t] += yr[t];
        }
    }
    for (int t = 0; t < n; t++) M[t] = M[t] * f->mret[t] + f->mgain[t] * y[t];
    for (int p = 0; p < f->n_cvs; p++) T[p] = ambient;
    for (int t = 0; t < n; t++) T[f->solved[t]] = y[t];
    free(ex); free(rhs); free(y); free(yr); free(pw); free(mat);
    return 0;
}

/* G envs sharing the factorization: T [G][n_cvs], M [G][n], input_q
 * [G][n_cvs], ambient / h [G], air_g / air_T [G][k]. */
int sbo_fdm_step_batch(const SboFdm* f, int G, double* T, double* M, const double* input_q, const double* ambient,
                       const double* h, const double* air_g, const double* air_T) {
    const size_t nc = (size_t)f->n_cvs, n = (size_t)f->n, k = (size_t)f->k;
    for (int g = 0; g < G; g++)
        if (sbo_fdm_step(f, T + g * nc, M + g * n, input_q + g * nc, ambient[g], h[g], air_g ? air_g + g * k : NULL,
                         air_T ? air_T + g * k : NULL) != 0)
            return -1;
    return 0;
}
