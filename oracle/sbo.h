/* sbo: a plain-C restatement of the reference CPU core ("csim") for the
 * Smart Buildings env step, used as the parity oracle of the HIP path.
 *
 * TEST INFRASTRUCTURE. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load liboracle.so; the product never links it.
 *
 * Scope: the synthetic RC scenarios of this repo (every cell solved, rooms made
 * of cells, air side given as applied/sensed sparse columns, convection off).
 * Each function cites the reference function it restates, and keeps that
 * function's floating-point operation order so that the result is bit-identical
 * to the reference compiled with the same compiler flags (checked against
 * oracle/_ref and the committed golden fixtures).
 */
#ifndef SBO_H
#define SBO_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SBO_OBS 1024
/* action row: SBO_CONT continuous slots, then SBO_DISC discrete ones; 320
 * continuous slots when built with SB_CONT_BIG (the reference GPU env's
 * SB_CONT_BIG layout, complete_port/gpu/smart_buildings.cu:35-40) */
#ifdef SB_CONT_BIG
#define SBO_CONT 320
#else
#define SBO_CONT 256
#endif
#define SBO_DISC 16

/* ---------------- blob ---------------- */
typedef struct {
    const char* name;
    uint32_t dtype;
    uint64_t count;
    const void* data;
} SboSec;

typedef struct {
    uint8_t* bytes;
    uint64_t size;
    int n;
    SboSec* sec;
} SboBlob;

int sbo_blob_load(SboBlob* b, const char* path);
void sbo_blob_free(SboBlob* b);
const SboSec* sbo_sec(const SboBlob* b, const char* name);
const double* sbo_f64(const SboBlob* b, const char* name);
const int64_t* sbo_i64(const SboBlob* b, const char* name);
const int32_t* sbo_i32(const SboBlob* b, const char* name);
const uint8_t* sbo_u8(const SboBlob* b, const char* name);
double sbo_f64_1(const SboBlob* b, const char* name, double dflt);
int64_t sbo_i64_1(const SboBlob* b, const char* name, int64_t dflt);

/* ---------------- scenario (read-only, shared by the envs of a blob) -------- */
typedef struct {
    SboBlob blob;
    int nr, nc, n_cvs, n, k, n_ahu, n_vav, n_zones, n_rooms, n_act, n_dev, n_aux;
    const int64_t* solved;
    const double *cap, *dir, *mcoup, *mret, *mgain, *temp_init, *mass_init;
    const double *horiz, *vert, *cond, *face0, *face1;
    double h;
    /* baked LU (SuperLU convention) */
    const int32_t *Lp, *Li, *Up, *Ui;
    const double *Lx, *Ux;
    int *Ldiag, *Udiag, *ir, *pc;
    /* air side */
    const int32_t *ap_p, *ap_i, *sn_p, *sn_i;
    const double *ap_x, *sn_x;
    double* S;        /* k x k sensed * A^-1 * applied */
    /* HVAC topology / constants */
    const int32_t *vz_off, *vz_idx, *vav_ahu, *coupled, *phys_room, *room_off, *room_cells;
    const int32_t *zv_off, *zv_idx;
    const double *zone_area, *ahu_c, *vav_c;
    double boiler_c[10], pump_head0, pump_eff, header_res;
    double internal_w_m2, standby_frac, occupant_w, cv_area, dt_sec;
    /* actions */
    const uint8_t *act_kind, *act_act, *act_disc;
    const int32_t* act_idx;
    const double *act_mn, *act_mx, *act_mnr, *act_mxr;
    int n_cont, n_disc;
    /* calendar / weather */
    const double *amb, *comfort, *heat_sp, *cool_sp, *solar_i, *solar_c, *aux_time;
    const int64_t *occ_hour, *hour_m1, *rew_hour, *rew_month;
    const uint8_t *occ_work, *work_m1, *rew_work;
    int occ_assign, occ_ea, occ_la, occ_ed, occ_ld;
    double p_arr, p_dep;
    int64_t occ_seed;
    /* observation */
    const uint8_t *f_kind, *f_id;
    const int32_t* f_idx;
    const double *f_mean, *f_var;
    /* reward */
    const double *rw, *elec_wk, *elec_we, *elec_co2, *gas_price;
    double gas_co2;
    uint8_t* is_room;
    int episode_steps;
    /* stochastic convection (sb_convect.h); off when conv_p == 0 or conv_dist == 0 */
    double conv_p;
    int conv_dist, cv_rooms, cv_max_room;
    int64_t conv_seed;
    const int32_t *cv_off, *cv_cells, *cv_coff, *cv_cidx;
} SboScen;

int sbo_scen_open(SboScen* s, const char* path);
void sbo_scen_close(SboScen* s);

/* ---------------- per-env state ---------------- */
typedef struct {
    uint32_t mt[624];
    int idx;
} SboMt;

typedef struct {
    const SboScen* sc;
    /* field */
    double *T, *M;
    /* AHU */
    int *ahu_run, *ahu_coolreq;
    double *ahu_recirc, *ahu_sat, *ahu_fan, *ahu_flow, *ahu_wsum, *ahu_atotal, *ahu_satv;
    /* VAV */
    double *damper, *reheat, *ratio, *heatsp, *coolsp, *dcmd, *rcmd, *sensing, *vav_area;
    int *mode, *prev_valid, *dcmd_set, *rcmd_set;
    /* zones / coupled columns */
    double *avg_temp, *zone_q, *input_q, *air_g, *air_T, *coil;
    /* plant */
    double flow_factor_sum, pump_head, total_reheat;
    int hws_requests, hws_run, pump_run;
    double boiler_sp, boiler_ret, boiler_cur, boiler_dstep;
    int step_index;
    /* occupancy */
    uint8_t* occ_state;
    double* occV;
    SboMt mt;
    /* convection stream and swap lists */
    SboMt cmt;
    int *cv_left, *cv_right;
    /* scratch */
    double *rhs, *y, *yr, *r, *work, *power, *mat;
    /* bookkeeping (pufferlib_cpu_env.h Env) */
    int step, max_steps, start;
    int first_steps, first_done;   /* first episode's length (desync truncation), 1 once it ended */
    float log[6];
    double native[SBO_CONT + SBO_DISC];
    double parts[16];   /* sb_reward's 12 (sb_reward.c:148-151), then the GPU env's comfort
                           diagnostics (mean, worst, out-of-band fraction) and the gas rate */
    double last_rew;
    float obs[SBO_OBS];
} SboEnv;

SboEnv* sbo_env_new(const SboScen* sc, uint32_t occ_seed, uint32_t conv_seed, int start, int max_steps);
void sbo_env_free(SboEnv* e);
void sbo_env_set_first_steps(SboEnv* e, int first_steps);
void sbo_env_reset(SboEnv* e, float* obs_out);
int sbo_env_step(SboEnv* e, const float* actions, float* obs_out, float* reward, float* terminal);
int sbo_env_state(const SboEnv* e, double* out);
double sbo_env_last_reward(const SboEnv* e);
int sbo_env_obs_len(const SboEnv* e);
int sbo_env_n_cont(const SboEnv* e);
int sbo_env_n_disc(const SboEnv* e);
void sbo_env_log(const SboEnv* e, float* out);
void sbo_env_parts(const SboEnv* e, double* out);

/* core pieces (exposed for unit tests) */
void sbo_mt_seed(SboMt* r, uint32_t seed);
uint32_t sbo_mt_u32(SboMt* r);
double sbo_mt_double(SboMt* r);
uint32_t sbo_mt_interval(SboMt* r, uint32_t max);
void sbo_conv_apply(const SboScen* sc, SboMt* r, int* left, int* right, double* temp);
void sbo_decode(const SboScen* sc, const double* cont, const double* disc, double* native);
void sbo_lu_solve(const SboScen* sc, const double* b, double* x, double* work);
int sbo_dense_solve(int k, double* M, double* b);

/* ---------------- canonical layout, pid_water base, residual decode ---------
 * (sbo_canon.c; slot constants of complete_port/gpu/sb_gpu_base.inc:31-45) */
#define SBO_CN_K 9
#define SBO_CN_ZPA 10
#define SBO_CN_ZS (SBO_CN_K * SBO_CN_ZPA)
#define SBO_CN_OBS 983
#define SBO_CN_ACT 219
typedef struct {
    int K, n_act, n_cont, n_disc;
    int zc[SBO_CN_K];
    /* zone slots: observation fields (temperature, heating / cooling setpoint,
     * damper / reheat command) and native actions (damper, reheat); -1 absent */
    int zT[SBO_CN_ZS], zH[SBO_CN_ZS], zC[SBO_CN_ZS], zD[SBO_CN_ZS], zR[SBO_CN_ZS], zAd[SBO_CN_ZS], zAr[SBO_CN_ZS];
    /* AHU k: fields outside-air temp, static pressure, supply flow, outside-air
     * flow, supply temp setpoint, recirculation, cooling requests, run command */
    int aObs[SBO_CN_K][8];
    int aT[SBO_CN_K], aP[SBO_CN_K], aRec[SBO_CN_K], aRun[SBO_CN_K];
    /* hot water: supply temp, its setpoint, dP, dP setpoint, run status, requests */
    int hObs[6];
    int hW, hDPa, hRun;
    int g[19];   /* hod sin x4, hod cos x4, dow sin x4, dow cos x4, comfort now, soon, occupants */
    float tmean, tstd;
    float fmean[SBO_OBS], fstd[SBO_OBS];
    double comfort_lo, comfort_hi, eco_lo, eco_hi;
    int morning, evening;
    int slot_of_action[SBO_CONT + SBO_DISC];
    int act_col[SBO_CONT + SBO_DISC];
    uint8_t act_disc[SBO_CONT + SBO_DISC];
} SboCanon;
/* 0 ok, -1 a section is missing, -2 the building exceeds the canonical slots */
int sbo_canon_open(SboCanon* c, const char* blob_path);
size_t sbo_canon_size(void);
int sbo_canon_slot(const SboCanon* c, int native_action);
void sbo_canon_base(const SboCanon* c, const float* obs, double* pid, float* base, float* ahu_info);
void sbo_canon_features(const SboCanon* c, const float* obs, const float* base, const float* ahu_info,
                        const double* pid, float* out);
void sbo_canon_trust(const SboCanon* c, const float* obs, float d0, float d1, int hot, float* trust);
void sbo_canon_decode(const SboCanon* c, const float* base, const float* p_row, const float* trust, int resid,
                      float scale, float dscale, float* native_row);

double sbo_run_batch(SboEnv** envs, const int* env_ids, int n, int steps, uint64_t seed,
                     int nthreads, double* reward_sum);
void sbo_action_row(uint64_t seed, uint32_t env, uint32_t step, int n_cont, int n_disc, float* row);

/* ---------------- building-scale field step (sbo_fdm.c) ---------------- */
typedef struct SboFdm SboFdm;
SboFdm* sbo_fdm_open(const char* path);
void sbo_fdm_close(SboFdm* f);
void sbo_fdm_dims(const SboFdm* f, int* out);   /* n_cvs, n_solved, k, rows, cols */
const double* sbo_fdm_sensed_response(const SboFdm* f);
void sbo_fdm_init_state(const SboFdm* f, double* T, double* M);
void sbo_fdm_lu_solve(const SboFdm* f, const double* b, double* x);
void sbo_fdm_exposure(const SboFdm* f, double h, double* out);
int sbo_fdm_step(const SboFdm* f, double* T, double* M, const double* input_q, double ambient, double h,
                 const double* air_g, const double* air_T);
int sbo_fdm_step_batch(const SboFdm* f, int G, double* T, double* M, const double* input_q, const double* ambient,
                       const double* h, const double* air_g, const double* air_T);

#ifdef __cplusplus
}
#endif
#endif
