/* Driver for the reference csim core compiled from /root/reference (oracle/_ref).
 *
 * TEST INFRASTRUCTURE: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load the library this file is linked into.
 *
 * It drives csim's public API in the order the reference CPU env does
 * (complete_port/pufferlib_cpu_env.h:187-208 puf_reset, :211-257 puf_step), with
 * two documented additions for the synthetic scenarios:
 *   - solar gain, which csim has no input for: sb_sim_step (sb_sim.c:526-531) is
 *     run as its three public parts, and between sb_sim_step_pre and sb_fdm_step
 *     every solved cell's input_q gets coeff[t] * irradiance[kk] (added on room
 *     cells, which step_pre rewrote; assigned on the others, which csim never
 *     writes);
 *   - a calendar start offset per env: the calendar index is offset + step
 *     everywhere the reference uses step (sb_sim.c step_index, obs/occupancy/
 *     reward index j), and the occupancy prime reads occ_hour_m1[offset].
 * The occupancy generator is reseeded per env with sb_rng_seed (sb_rng.c:9-16).
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "sb_baked.h"
#include "sb_convect.h"
#include "sb_fdm.h"
#include "sb_obs.h"
#include "sb_occup.h"
#include "sb_reward.h"
#include "sb_sim.h"
#include "sbo_philox.h"

#define SB_OBS 1024
#define SB_CONT 256
#define SB_DISC 16

typedef struct {
    SbBlob blob;
    SbFdm fdm;
    SbConv conv;
    SbOccup occ;
    SbSim sim;
    const uint8_t* is_disc;
    int n_act, n_cont, n_disc, obs_len;
    int step, max_steps, start;
    double cont[SB_CONT], disc[SB_DISC], native[SB_CONT + SB_DISC], parts[12];
    float obs[SB_OBS];
    float log[6];          /* perf, score, episode_return, episode_length, reward_mean, n */
    double last_rew;       /* f64 reward of the last step (before the float cast) */
    const double* solar_i; /* per calendar step */
    const double* solar_c; /* per solved cell */
    uint8_t* is_room;      /* per cell */
    const int64_t* hour_m1;
    const uint8_t* work_m1;
} RefEnv;

static void write_obs(RefEnv* e, int j, float* out) {
    sb_obs(&e->sim, e->occ.V, j, e->obs);
    for (int i = e->obs_len; i < SB_OBS; i++) e->obs[i] = 0.0f;
    if (out) memcpy(out, e->obs, sizeof(float) * SB_OBS);
}

RefEnv* ref_open(const char* path, uint32_t occ_seed, uint32_t conv_seed, int start, int max_steps) {
    RefEnv* e = (RefEnv*)calloc(1, sizeof(RefEnv));
    if (!e) return NULL;
    if (sb_open(&e->blob, path) != 0) { free(e); return NULL; }
    if (sb_fdm_init(&e->fdm, &e->blob) || sb_conv_init(&e->conv, &e->blob) ||
        sb_occup_init(&e->occ, &e->blob) ||
        sb_sim_init(&e->sim, &e->blob, &e->fdm, &e->conv, &e->occ)) {
        fprintf(stderr, "ref_open: init failed for %s\n", path);
        free(e);
        return NULL;
    }
    sb_rng_seed(&e->occ.rng, occ_seed);
    sb_rng_seed(&e->conv.rng, conv_seed);
    e->is_disc = sb_u8(&e->blob, "act_is_discrete");
    e->n_act = e->sim.n_action;
    for (int i = 0; i < e->n_act; i++) {
        if (e->is_disc[i]) e->n_disc++; else e->n_cont++;
    }
    e->obs_len = e->sim.n_dev + e->sim.n_aux;
    e->max_steps = max_steps;
    e->start = start;
    e->solar_i = sb_f64(&e->blob, "solar_irradiance");
    e->solar_c = sb_f64(&e->blob, "solar_gain_coeff");
    e->hour_m1 = sb_i64(&e->blob, "occ_hour_m1");
    e->work_m1 = sb_u8(&e->blob, "occ_workday_m1");
    e->is_room = (uint8_t*)calloc((size_t)e->sim.n_cvs, 1);
    for (int rm = 0; rm < e->sim.n_rooms; rm++)
        for (int t = e->sim.room_off[rm]; t < e->sim.room_off[rm + 1]; t++)
            e->is_room[e->sim.room_cells[2 * t] * e->sim.nc + e->sim.room_cells[2 * t + 1]] = 1;
    return e;
}

void ref_close(RefEnv* e) {
    if (!e) return;
    sb_sim_free(&e->sim);
    sb_occup_free(&e->occ);
    sb_conv_free(&e->conv);
    sb_fdm_free(&e->fdm);
    sb_close(&e->blob);
    free(e->is_room);
    free(e);
}

int ref_obs_len(RefEnv* e) { return e->obs_len; }
int ref_n_cont(RefEnv* e) { return e->n_cont; }
int ref_n_disc(RefEnv* e) { return e->n_disc; }
int ref_n_cvs(RefEnv* e) { return e->sim.n_cvs; }

/* puf_reset (pufferlib_cpu_env.h:187-208) at the env's calendar offset. */
void ref_reset(RefEnv* e, float* obs_out) {
    sb_sim_reset(&e->sim, &e->blob);
    e->sim.step_index = e->start;
    if (e->hour_m1) e->occ.hour_m1 = (int)e->hour_m1[e->start];
    if (e->work_m1) e->occ.workday_m1 = e->work_m1[e->start];
    sb_occup_prime(&e->occ);
    e->step = 0;
    for (int i = 0; i < e->n_act; i++) e->native[i] = 0.0;
    write_obs(e, e->start, obs_out);
    sb_occup_advance(&e->occ, e->start);
}

static void step_with_solar(RefEnv* e) {
    SbSim* s = &e->sim;
    sb_sim_step_pre(s, e->occ.V);
    if (e->solar_i && e->solar_c) {
        double irr = e->solar_i[s->step_index];
        for (int t = 0; t < s->n_solved; t++) {
            int p = (int)s->fdm->solved[t];
            double q = e->solar_c[t] * irr;
            if (e->is_room[p]) s->input_q[p] += q;
            else s->input_q[p] = q;
        }
    }
    sb_fdm_step(s->fdm, s->input_q, s->amb[s->step_index], s->h, s->air_g, s->air_T);
    sb_sim_step_post(s);
}

/* puf_step (pufferlib_cpu_env.h:211-257). `actions` is one trainer row of
 * SB_CONT + SB_DISC floats. Returns 1 when the step ended an episode (the
 * observation then is the next episode's reset observation). */
int ref_step(RefEnv* e, const float* actions, float* obs_out, float* reward, float* terminal) {
    for (int i = 0; i < e->n_cont; i++) {
        double a = (double)actions[i];
        if (a > 1.0) a = 1.0;
        else if (a < -1.0) a = -1.0;
        e->cont[i] = a;
    }
    for (int i = 0; i < e->n_disc; i++) e->disc[i] = (double)actions[SB_CONT + i];
    sb_decode_native(e->n_act, e->is_disc, sb_f64(&e->blob, "act_min_native"),
                     sb_f64(&e->blob, "act_max_native"), sb_f64(&e->blob, "act_min_norm"),
                     sb_f64(&e->blob, "act_max_norm"), e->cont, e->disc, e->native);
    sb_sim_apply_native(&e->sim, e->native);
    step_with_solar(e);
    e->step += 1;
    int j = e->start + e->step;
    write_obs(e, j, NULL);
    sb_occup_advance(&e->occ, j);
    double rew = sb_reward(&e->sim, e->occ.V, j, e->parts);
    e->last_rew = rew;
    float r = (float)rew;
    int done = e->step >= e->max_steps;
    if (reward) *reward = r;
    if (terminal) *terminal = done ? 1.0f : 0.0f;
    e->log[2] += r;
    e->log[4] += (r - e->log[4]) / (float)e->step;
    if (done) {
        float mean = e->log[2] / (float)e->step;
        e->log[0] += mean;
        e->log[1] += mean;
        e->log[3] += (float)e->step;
        e->log[5] += 1.0f;
        ref_reset(e, NULL);
    }
    if (obs_out) memcpy(obs_out, e->obs, sizeof(float) * SB_OBS);
    return done;
}

double ref_last_reward_f64(RefEnv* e) { return e->last_rew; }

void ref_native(RefEnv* e, double* out) { memcpy(out, e->native, sizeof(double) * (size_t)e->n_act); }
void ref_parts(RefEnv* e, double* out) { memcpy(out, e->parts, sizeof(e->parts)); }
void ref_log(RefEnv* e, float* out) { memcpy(out, e->log, sizeof(e->log)); }
void ref_clear_log(RefEnv* e) { memset(e->log, 0, sizeof(e->log)); }

/* State snapshot: temp[n_cvs], mass_temp[n_solved], then per-VAV damper,
 * reheat, ratio, sensing, then per-AHU flow, sat, recirc, fan, then
 * air_g[k], air_T[k], occupancy V[nz], then boiler_current, boiler_return,
 * boiler_setpoint, pump_head, step_index. Returns the count written. */
int ref_state(RefEnv* e, double* out) {
    SbSim* s = &e->sim;
    int c = 0;
    for (int p = 0; p < s->n_cvs; p++) out[c++] = s->fdm->temp[p];
    for (int t = 0; t < s->n_solved; t++) out[c++] = s->fdm->mass_temp[t];
    for (int v = 0; v < s->n_vav; v++) out[c++] = s->vav_damper[v];
    for (int v = 0; v < s->n_vav; v++) out[c++] = s->vav_reheat[v];
    for (int v = 0; v < s->n_vav; v++) out[c++] = s->vav_ratio[v];
    for (int v = 0; v < s->n_vav; v++) out[c++] = s->sensing[v];
    for (int a = 0; a < s->n_ahu; a++) out[c++] = s->ahu_flow[a];
    for (int a = 0; a < s->n_ahu; a++) out[c++] = s->ahu_sat[a];
    for (int a = 0; a < s->n_ahu; a++) out[c++] = s->ahu_recirc[a];
    for (int a = 0; a < s->n_ahu; a++) out[c++] = s->ahu_fan[a];
    for (int i = 0; i < s->k; i++) out[c++] = s->air_g[i];
    for (int i = 0; i < s->k; i++) out[c++] = s->air_T[i];
    for (int z = 0; z < s->n_zones; z++) out[c++] = e->occ.V[z];
    out[c++] = s->boiler_current;
    out[c++] = s->boiler_return;
    out[c++] = s->boiler_setpoint;
    out[c++] = s->pump_head;
    out[c++] = (double)s->step_index;
    return c;
}

/* ---- batch runner: n envs, `steps` puf_steps each, Beta(2,2) actions ---- */
typedef struct {
    RefEnv** envs;
    const int* env_ids;
    int lo, hi, steps;
    uint64_t seed;
    double reward_sum;
} Job;

static void* run_job(void* arg) {
    Job* j = (Job*)arg;
    float row[SB_CONT + SB_DISC];
    float r, t;
    double acc = 0.0;
    for (int i = j->lo; i < j->hi; i++) {
        RefEnv* e = j->envs[i];
        for (int s = 0; s < j->steps; s++) {
            sbo_action_row_philox(j->seed, (uint32_t)j->env_ids[i], (uint32_t)s, e->n_cont, e->n_disc,
                           row, SB_CONT, SB_DISC);
            ref_step(e, row, NULL, &r, &t);
            acc += r;
        }
    }
    j->reward_sum = acc;
    return NULL;
}

/* Steps every env `steps` times on `nthreads` threads (whole envs per thread).
 * Returns wall seconds; *reward_sum receives the sum of all rewards. */
double ref_run_batch(RefEnv** envs, const int* env_ids, int n, int steps, uint64_t seed,
                     int nthreads, double* reward_sum) {
    if (nthreads < 1) nthreads = 1;
    if (nthreads > n) nthreads = n;
    Job* jobs = (Job*)calloc((size_t)nthreads, sizeof(Job));
    pthread_t* th = (pthread_t*)calloc((size_t)nthreads, sizeof(pthread_t));
    struct timespec t0, t1;
    clock_gettime(CLOCK_MONOTONIC, &t0);
    for (int i = 0; i < nthreads; i++) {
        jobs[i].envs = envs;
        jobs[i].env_ids = env_ids;
        jobs[i].lo = (int)((long)n * i / nthreads);
        jobs[i].hi = (int)((long)n * (i + 1) / nthreads);
        jobs[i].steps = steps;
        jobs[i].seed = seed;
        pthread_create(&th[i], NULL, run_job, &jobs[i]);
    }
    double acc = 0.0;
    for (int i = 0; i < nthreads; i++) {
        pthread_join(th[i], NULL);
        acc += jobs[i].reward_sum;
    }
    clock_gettime(CLOCK_MONOTONIC, &t1);
    if (reward_sum) *reward_sum = acc;
    free(jobs);
    free(th);
    return (double)(t1.tv_sec - t0.tv_sec) + 1e-9 * (double)(t1.tv_nsec - t0.tv_nsec);
}

void ref_action_row(uint64_t seed, uint32_t env, uint32_t step, int n_cont, int n_disc, float* row) {
    sbo_action_row_philox(seed, env, step, n_cont, n_disc, row, SB_CONT, SB_DISC);
}

/* ---- the reference's field model alone (sb_fdm.h), for the FDM-scale plans:
 * G envs of one blob, each its own SbFdm (sb_fdm_init, sb_fdm.c:40-118) over
 * the one loaded blob, stepped together by sb_fdm_step_batch (sb_fdm.c:190-270). */
typedef struct {
    SbBlob blob;
    int G;
    SbFdm* f;
    SbFdm** fp;
    double *rhs, *sol, *work;
} RefFdm;

void ref_fdm_close(RefFdm* r) {
    if (!r) return;
    for (int g = 0; g < r->G; g++) sb_fdm_free(&r->f[g]);
    free(r->f); free(r->fp); free(r->rhs); free(r->sol); free(r->work);
    free(r);
}

RefFdm* ref_fdm_open(const char* path, int G) {
    RefFdm* r = (RefFdm*)calloc(1, sizeof(RefFdm));
    if (!r || G < 1) { free(r); return NULL; }
    if (sb_open(&r->blob, path) != 0) { free(r); return NULL; }
    r->f = (SbFdm*)calloc((size_t)G, sizeof(SbFdm));
    r->fp = (SbFdm**)calloc((size_t)G, sizeof(SbFdm*));
    if (!r->f || !r->fp) { ref_fdm_close(r); return NULL; }
    for (int g = 0; g < G; g++) {
        if (sb_fdm_init(&r->f[g], &r->blob) != 0) { r->G = g; ref_fdm_close(r); return NULL; }
        r->G = g + 1;
        r->fp[g] = &r->f[g];
    }
    const size_t n = (size_t)r->f[0].n_solved;
    r->rhs = (double*)malloc(sizeof(double) * n * G);
    r->sol = (double*)malloc(sizeof(double) * n * G);
    r->work = (double*)malloc(sizeof(double) * n * G);
    if (!r->rhs || !r->sol || !r->work) { ref_fdm_close(r); return NULL; }
    return r;
}

void ref_fdm_dims(const RefFdm* r, int* out) {
    out[0] = r->f[0].n_cvs;
    out[1] = r->f[0].n_solved;
    out[2] = r->f[0].k;
    out[3] = r->f[0].nr;
    out[4] = r->f[0].nc;
}

void ref_fdm_sensed_response(const RefFdm* r, double* out) {
    const int k = r->f[0].k;
    memcpy(out, r->f[0].sensed_response, sizeof(double) * (size_t)k * k);
}

void ref_fdm_lu_solve(const RefFdm* r, const double* b, double* x) {
    sb_lu_solve(&r->f[0].lu, b, x, r->work);
}

/* env g's fields: T [n_cvs], M [n_solved] */
void ref_fdm_get(const RefFdm* r, int g, double* T, double* M) {
    memcpy(T, r->f[g].temp, sizeof(double) * (size_t)r->f[g].n_cvs);
    memcpy(M, r->f[g].mass_temp, sizeof(double) * (size_t)r->f[g].n_solved);
}

void ref_fdm_set(RefFdm* r, int g, const double* T, const double* M) {
    memcpy(r->f[g].temp, T, sizeof(double) * (size_t)r->f[g].n_cvs);
    memcpy(r->f[g].mass_temp, M, sizeof(double) * (size_t)r->f[g].n_solved);
}

/* input_q [G][n_cvs], ambient / h [G], air_g / air_T [G][k] */
void ref_fdm_step_batch(RefFdm* r, const double* input_q, const double* ambient, const double* h,
                        const double* air_g, const double* air_T) {
    const int G = r->G;
    const size_t nc = (size_t)r->f[0].n_cvs, k = (size_t)r->f[0].k;
    const double** q = (const double**)malloc(sizeof(double*) * G);
    const double** ag = (const double**)malloc(sizeof(double*) * G);
    const double** at = (const double**)malloc(sizeof(double*) * G);
    for (int g = 0; g < G; g++) {
        q[g] = input_q + g * nc;
        ag[g] = air_g + g * k;
        at[g] = air_T + g * k;
    }
    sb_fdm_step_batch(r->fp, G, q, ambient, h, ag, at, r->rhs, r->sol, r->work);
    free(q); free(ag); free(at);
}
