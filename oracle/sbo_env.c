/* Oracle batch runner and action stream (TEST INFRASTRUCTURE).
 * Whole envs per thread, as the reference CPU vec steps independent envs
 * (complete_port/config/smart_buildings.ini num_threads). */
#include <pthread.h>
#include <stdlib.h>
#include <time.h>

#include "sbo.h"
#include "sbo_philox.h"

void sbo_action_row(uint64_t seed, uint32_t env, uint32_t step, int n_cont, int n_disc, float* row) {
    sbo_action_row_philox(seed, env, step, n_cont, n_disc, row, SBO_CONT, SBO_DISC);
}

typedef struct {
    SboEnv** envs;
    const int* ids;
    int lo, hi, steps;
    uint64_t seed;
    double acc;
} Job;

static void* job_main(void* p) {
    Job* j = (Job*)p;
    float row[SBO_CONT + SBO_DISC], r, t;
    double acc = 0.0;
    for (int i = j->lo; i < j->hi; i++) {
        SboEnv* e = j->envs[i];
        for (int s = 0; s < j->steps; s++) {
            sbo_action_row(j->seed, (uint32_t)j->ids[i], (uint32_t)s, e->sc->n_cont, e->sc->n_disc, row);
            sbo_env_step(e, row, NULL, &r, &t);
            acc += r;
        }
    }
    j->acc = acc;
    return NULL;
}

double sbo_run_batch(SboEnv** envs, const int* ids, int n, int steps, uint64_t seed,
                     int nthreads, double* reward_sum) {
    if (nthreads < 1) nthreads = 1;
    if (nthreads > n) nthreads = n;
    Job* jobs = (Job*)calloc((size_t)nthreads, sizeof(Job));
    pthread_t* th = (pthread_t*)calloc((size_t)nthreads, sizeof(pthread_t));
    struct timespec t0, t1;
    clock_gettime(CLOCK_MONOTONIC, &t0);
    for (int i = 0; i < nthreads; i++) {
        jobs[i] = (Job){envs, ids, (int)((long)n * i / nthreads), (int)((long)n * (i + 1) / nthreads),
                        steps, seed, 0.0};
        pthread_create(&th[i], NULL, job_main, &jobs[i]);
    }
    double acc = 0.0;
    for (int i = 0; i < nthreads; i++) {
        pthread_join(th[i], NULL);
        acc += jobs[i].acc;
    }
    clock_gettime(CLOCK_MONOTONIC, &t1);
    if (reward_sum) *reward_sum = acc;
    free(jobs);
    free(th);
    return (double)(t1.tv_sec - t0.tv_sec) + 1e-9 * (double)(t1.tv_nsec - t0.tv_nsec);
}

/* Philox4x32-10 block function, exported for known-answer tests. */
void sbo_philox4x32_10_ext(uint32_t ctr[4], uint32_t k0, uint32_t k1) { sbo_philox4x32_10(ctr, k0, k1); }
