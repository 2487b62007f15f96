/* sbo core: restatement of the reference csim step (TEST INFRASTRUCTURE).
 *
 * Every expression keeps the operand order of the reference function cited
 * next to it; C evaluates a*b*c as (a*b)*c and a+b+c as (a+b)+c, and this file
 * is compiled with -ffp-contract=off like oracle/_ref, so the results are
 * bit-identical to the reference core on the same inputs.
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "sbo.h"

#define RHO_AIR 1.2
#define CP_AIR 1006.0
#define RHO_W 1000.0
#define CP_W 4180.0
#define GRAV 9.8
#define PA_PER_BAR 100000.0
#define PI_D 3.14159265358979323846
enum { M_OFF = 0, M_HEAT = 1, M_COOL = 2, M_PASSIVE = 3 };

/* ------------------------------------------------------------------ MT19937 */
/* init_genrand / genrand_int32 of Matsumoto & Nishimura (1998), the stream
 * numpy's legacy RandomState draws; complete_port/csim/sb_rng.c:9-37. */
void sbo_mt_seed(SboMt* r, uint32_t seed) {
    r->mt[0] = seed;
    for (int i = 1; i < 624; i++)
        r->mt[i] = 1812433253u * (r->mt[i - 1] ^ (r->mt[i - 1] >> 30)) + (uint32_t)i;
    r->idx = 624;
}

static void mt_twist(SboMt* r) {
    for (int i = 0; i < 624; i++) {
        uint32_t x = (r->mt[i] & 0x80000000u) | (r->mt[(i + 1) % 624] & 0x7fffffffu);
        uint32_t xa = x >> 1;
        if (x & 1u) xa ^= 0x9908b0dfu;
        r->mt[i] = r->mt[(i + 397) % 624] ^ xa;
    }
    r->idx = 0;
}

uint32_t sbo_mt_u32(SboMt* r) {
    if (r->idx >= 624) mt_twist(r);
    uint32_t y = r->mt[r->idx++];
    y ^= y >> 11;
    y ^= (y << 7) & 0x9d2c5680u;
    y ^= (y << 15) & 0xefc60000u;
    y ^= y >> 18;
    return y;
}

/* random_sample: 53-bit double from two draws; sb_rng.c:39-43. */
double sbo_mt_double(SboMt* r) {
    uint32_t a = sbo_mt_u32(r) >> 5;
    uint32_t b = sbo_mt_u32(r) >> 6;
    return (a * 67108864.0 + b) / 9007199254740992.0;
}

/* Uniform integer in [0, max] by masked rejection (numpy's legacy
 * rk_interval); complete_port/csim/sb_rng.c:45-54. */
uint32_t sbo_mt_interval(SboMt* r, uint32_t max) {
    if (max == 0) return 0;
    uint32_t mask = max;
    mask |= mask >> 1;
    mask |= mask >> 2;
    mask |= mask >> 4;
    mask |= mask >> 8;
    mask |= mask >> 16;
    uint32_t v;
    do {
        v = sbo_mt_u32(r) & mask;
    } while (v > max);
    return v;
}

/* ------------------------------------------------------------ convection */
/* sb_conv_apply, complete_port/csim/sb_convect.c:39-73: per room, every cell
 * draws u and, when u <= p and it has candidates, picks one of them; the
 * (cell, candidate) pairs are shuffled by Fisher-Yates from the last pair
 * down and the temperatures of each pair are swapped in that order. */
void sbo_conv_apply(const SboScen* s, SboMt* r, int* left, int* right, double* temp) {
    if (s->conv_p == 0.0 || s->conv_dist == 0) return;
    for (int rm = 0; rm < s->cv_rooms; rm++) {
        const int base = s->cv_off[rm], n = s->cv_off[rm + 1] - base;
        int m = 0;
        for (int j = 0; j < n; j++) {
            if (sbo_mt_double(r) > s->conv_p) continue;
            const int cg = base + j, c0 = s->cv_coff[cg], c1 = s->cv_coff[cg + 1];
            if (c1 <= c0) continue;
            left[m] = cg;
            right[m] = s->cv_cidx[c0 + (int)sbo_mt_interval(r, (uint32_t)(c1 - c0 - 1))];
            m++;
        }
        for (int t = m - 1; t > 0; t--) {
            const int j2 = (int)sbo_mt_interval(r, (uint32_t)t);
            int x = left[t];
            left[t] = left[j2];
            left[j2] = x;
            x = right[t];
            right[t] = right[j2];
            right[j2] = x;
        }
        for (int t = 0; t < m; t++) {
            const int a = left[t], b = right[t];
            const int ia = s->cv_cells[2 * a] * s->nc + s->cv_cells[2 * a + 1];
            const int ib = s->cv_cells[2 * b] * s->nc + s->cv_cells[2 * b + 1];
            const double held = temp[ia];
            temp[ia] = temp[ib];
            temp[ib] = held;
        }
    }
}

/* ------------------------------------------------------------ LU replay */
/* complete_port/csim/sb_lu.c:5-33 (diagonal lookup, inverse row perm) */
static int lu_prepare(SboScen* s) {
    int n = s->n;
    const int32_t* pr = sbo_i32(&s->blob, "lu_perm_r");
    const int32_t* pcs = sbo_i32(&s->blob, "lu_perm_c");
    if (!pr || !pcs || !s->Lp || !s->Up) return -1;
    s->Ldiag = (int*)malloc(sizeof(int) * n);
    s->Udiag = (int*)malloc(sizeof(int) * n);
    s->ir = (int*)malloc(sizeof(int) * n);
    s->pc = (int*)malloc(sizeof(int) * n);
    for (int j = 0; j < n; j++) {
        s->Ldiag[j] = s->Udiag[j] = -1;
        for (int p = s->Lp[j]; p < s->Lp[j + 1] && s->Ldiag[j] < 0; p++)
            if (s->Li[p] == j) s->Ldiag[j] = p;
        for (int p = s->Up[j]; p < s->Up[j + 1] && s->Udiag[j] < 0; p++)
            if (s->Ui[p] == j) s->Udiag[j] = p;
        if (s->Ldiag[j] < 0 || s->Udiag[j] < 0) return -1;
    }
    for (int i = 0; i < n; i++) s->ir[pr[i]] = i;
    for (int j = 0; j < n; j++) s->pc[j] = pcs[j];
    return 0;
}

/* y = b[ir]; unit-L column push; U column push with /U_jj; x = w[pc]
 * (complete_port/csim/sb_lu.c:38-63). */
void sbo_lu_solve(const SboScen* s, const double* b, double* x, double* w) {
    int n = s->n;
    for (int i = 0; i < n; i++) w[i] = b[s->ir[i]];
    for (int j = 0; j < n; j++) {
        double v = w[j];
        for (int p = s->Lp[j]; p < s->Lp[j + 1]; p++)
            if (p != s->Ldiag[j]) w[s->Li[p]] -= s->Lx[p] * v;
    }
    for (int j = n - 1; j >= 0; j--) {
        double v = w[j] / s->Ux[s->Udiag[j]];
        w[j] = v;
        for (int p = s->Up[j]; p < s->Up[j + 1]; p++)
            if (p != s->Udiag[j]) w[s->Ui[p]] -= s->Ux[p] * v;
    }
    for (int i = 0; i < n; i++) x[i] = w[s->pc[i]];
}

/* Dense partial-pivot solve, row swap only on a strictly larger |pivot|, rows
 * with a zero multiplier skipped (complete_port/csim/sb_fdm.c:9-38). */
int sbo_dense_solve(int k, double* M, double* b) {
    for (int c = 0; c < k; c++) {
        int piv = c;
        double best = fabs(M[c * k + c]);
        for (int r = c + 1; r < k; r++) {
            double a = fabs(M[r * k + c]);
            if (a > best) { best = a; piv = r; }
        }
        if (best == 0.0) return -1;
        if (piv != c) {
            for (int j = c; j < k; j++) {
                double t = M[c * k + j];
                M[c * k + j] = M[piv * k + j];
                M[piv * k + j] = t;
            }
            double t = b[c]; b[c] = b[piv]; b[piv] = t;
        }
        double d = M[c * k + c];
        for (int r = c + 1; r < k; r++) {
            double f = M[r * k + c] / d;
            if (f == 0.0) continue;
            for (int j = c; j < k; j++) M[r * k + j] -= f * M[c * k + j];
            b[r] -= f * b[c];
        }
    }
    for (int r = k - 1; r >= 0; r--) {
        double acc = b[r];
        for (int j = r + 1; j < k; j++) acc -= M[r * k + j] * b[j];
        b[r] = acc / M[r * k + r];
    }
    return 0;
}

/* ------------------------------------------------------------ scenario */
int sbo_scen_open(SboScen* s, const char* path) {
    memset(s, 0, sizeof(*s));
    if (sbo_blob_load(&s->blob, path) != 0) return -1;
    const SboBlob* b = &s->blob;
    const int64_t* g = sbo_i64(b, "grid");
    const SboSec* solved = sbo_sec(b, "solved");
    const int64_t* sn_shape = sbo_i64(b, "sensed_shape");
    if (!g || !solved || !sn_shape) return -1;
    s->nr = (int)g[0];
    s->nc = (int)g[1];
    s->n_cvs = s->nr * s->nc;
    s->n = (int)solved->count;
    s->k = (int)sn_shape[0];
    s->solved = sbo_i64(b, "solved");
    s->cap = sbo_f64(b, "capacitance_rate");
    s->dir = sbo_f64(b, "dirichlet_conductance");
    s->mcoup = sbo_f64(b, "mass_coupling");
    s->mret = sbo_f64(b, "mass_retained");
    s->mgain = sbo_f64(b, "mass_gained");
    s->temp_init = sbo_f64(b, "temp_init");
    s->mass_init = sbo_f64(b, "mass_temp_init");
    s->horiz = sbo_f64(b, "horizontal");
    s->vert = sbo_f64(b, "vertical");
    s->cond = sbo_f64(b, "solver_conductivity");
    s->face0 = sbo_f64(b, "ambient_face_areas_0");
    s->face1 = sbo_f64(b, "ambient_face_areas_1");
    s->h = sbo_f64_1(b, "convection_coefficient", 8.8);
    s->Lp = sbo_i32(b, "lu_L_indptr"); s->Li = sbo_i32(b, "lu_L_indices"); s->Lx = sbo_f64(b, "lu_L_data");
    s->Up = sbo_i32(b, "lu_U_indptr"); s->Ui = sbo_i32(b, "lu_U_indices"); s->Ux = sbo_f64(b, "lu_U_data");
    if (lu_prepare(s) != 0) return -1;
    s->ap_p = sbo_i32(b, "applied_indptr"); s->ap_i = sbo_i32(b, "applied_indices");
    s->ap_x = sbo_f64(b, "applied_data");
    s->sn_p = sbo_i32(b, "sensed_indptr"); s->sn_i = sbo_i32(b, "sensed_indices");
    s->sn_x = sbo_f64(b, "sensed_data");
    if (!s->ap_p || !s->sn_p) return -1;
    /* S = sensed * A^-1 * applied, one column per LU solve (sb_fdm.c:103-114) */
    {
        int n = s->n, k = s->k;
        double* r = (double*)calloc((size_t)n, sizeof(double));
        double* yr = (double*)calloc((size_t)n, sizeof(double));
        double* w = (double*)calloc((size_t)n, sizeof(double));
        s->S = (double*)calloc((size_t)(k ? k * k : 1), sizeof(double));
        for (int j = 0; j < k; j++) {
            for (int t = 0; t < n; t++) r[t] = 0.0;
            for (int p = s->ap_p[j]; p < s->ap_p[j + 1]; p++) r[s->ap_i[p]] = s->ap_x[p];
            sbo_lu_solve(s, r, yr, w);
            for (int i = 0; i < k; i++) {
                double acc = 0.0;
                for (int p = s->sn_p[i]; p < s->sn_p[i + 1]; p++) acc += s->sn_x[p] * yr[s->sn_i[p]];
                s->S[i * k + j] = acc;
            }
        }
        free(r); free(yr); free(w);
    }
    const SboSec* ac = sbo_sec(b, "ahu_const");
    s->n_ahu = (int)(ac->count / 9);
    s->n_vav = (int)(sbo_sec(b, "vav_zone_offsets")->count - 1);
    s->n_zones = (int)sbo_sec(b, "zone_area")->count;
    s->n_rooms = (int)(sbo_sec(b, "room_offsets")->count - 1);
    s->n_act = (int)sbo_sec(b, "act_owner_kind")->count;
    s->vz_off = sbo_i32(b, "vav_zone_offsets"); s->vz_idx = sbo_i32(b, "vav_zone_idx");
    s->vav_ahu = sbo_i32(b, "vav_ahu_idx"); s->coupled = sbo_i32(b, "coupled_vav_idx");
    s->phys_room = sbo_i32(b, "phys_room_idx"); s->room_off = sbo_i32(b, "room_offsets");
    s->room_cells = sbo_i32(b, "room_cells");
    s->zv_off = sbo_i32(b, "zone_vav_offsets"); s->zv_idx = sbo_i32(b, "zone_vav_idx");
    s->zone_area = sbo_f64(b, "zone_area");
    s->ahu_c = sbo_f64(b, "ahu_const");
    s->vav_c = sbo_f64(b, "vav_const");
    {
        const double* bc = sbo_f64(b, "boiler_const");
        for (int i = 0; i < 10; i++) s->boiler_c[i] = bc ? bc[i] : 0.0;
        const double* pc = sbo_f64(b, "pump_const");
        s->pump_head0 = pc ? pc[0] : 0.0;
        s->pump_eff = pc ? pc[1] : 1.0;
    }
    s->header_res = sbo_f64_1(b, "hws_header_resistance", 0.0);
    s->internal_w_m2 = sbo_f64_1(b, "internal_gain_w_per_m2", 0.0);
    s->standby_frac = sbo_f64_1(b, "internal_gain_standby_fraction", 1.0);
    s->occupant_w = sbo_f64_1(b, "occupant_sensible_heat_w", 0.0);
    {
        double cv = sbo_f64_1(b, "cv_size_cm", 20.0) / 100.0;
        s->cv_area = cv * cv;
    }
    s->act_kind = sbo_u8(b, "act_owner_kind"); s->act_idx = sbo_i32(b, "act_owner_index");
    s->act_act = sbo_u8(b, "act_actuator"); s->act_disc = sbo_u8(b, "act_is_discrete");
    s->act_mn = sbo_f64(b, "act_min_native"); s->act_mx = sbo_f64(b, "act_max_native");
    s->act_mnr = sbo_f64(b, "act_min_norm"); s->act_mxr = sbo_f64(b, "act_max_norm");
    for (int i = 0; i < s->n_act; i++) {
        if (s->act_disc[i]) s->n_disc++; else s->n_cont++;
    }
    if (s->n_cont > SBO_CONT || s->n_disc > SBO_DISC) return -1;   /* the action row has no room for them */
    s->amb = sbo_f64(b, "weather_ambient");
    s->comfort = sbo_f64(b, "sched_comfort");
    s->heat_sp = sbo_f64(b, "sched_heat_sp");
    s->cool_sp = sbo_f64(b, "sched_cool_sp");
    s->solar_i = sbo_f64(b, "solar_irradiance");
    s->solar_c = sbo_f64(b, "solar_gain_coeff");
    s->aux_time = sbo_f64(b, "aux_time");
    s->occ_hour = sbo_i64(b, "occ_hour"); s->occ_work = sbo_u8(b, "occ_workday");
    s->hour_m1 = sbo_i64(b, "occ_hour_m1"); s->work_m1 = sbo_u8(b, "occ_workday_m1");
    s->rew_hour = sbo_i64(b, "rew_hour"); s->rew_month = sbo_i64(b, "rew_month");
    s->rew_work = sbo_u8(b, "rew_workday");
    {
        /* occupancy parameters, sb_occup.c:8-20 */
        const double* op = sbo_f64(b, "occ_params");
        if (!op) return -1;
        s->occ_assign = (int)op[0];
        s->occ_ea = (int)op[1]; s->occ_la = (int)op[2];
        s->occ_ed = (int)op[3]; s->occ_ld = (int)op[4];
        s->p_arr = 1.0 / ((s->occ_la - s->occ_ea) * 3600.0 / op[5] / 2.0);
        s->p_dep = 1.0 / ((s->occ_ld - s->occ_ed) * 3600.0 / op[5] / 2.0);
        s->dt_sec = op[5];
    }
    s->occ_seed = sbo_i64_1(b, "occ_seed", 17321);
    s->f_kind = sbo_u8(b, "f_dev_kind"); s->f_idx = sbo_i32(b, "f_dev_idx");
    s->f_id = sbo_u8(b, "f_obs_id"); s->f_mean = sbo_f64(b, "f_norm_mean");
    s->f_var = sbo_f64(b, "f_norm_var");
    s->n_dev = (int)sbo_i64_1(b, "n_dev", 0);
    s->n_aux = (int)sbo_i64_1(b, "n_aux", 0);
    s->rw = sbo_f64(b, "reward_scalars");
    s->elec_wk = sbo_f64(b, "elec_weekday_price"); s->elec_we = sbo_f64(b, "elec_weekend_price");
    s->elec_co2 = sbo_f64(b, "elec_carbon_rate"); s->gas_price = sbo_f64(b, "gas_month_price");
    s->gas_co2 = sbo_f64_1(b, "gas_carbon_rate", 0.0);
    {
        const double* meta = sbo_f64(b, "obs_meta");
        s->episode_steps = meta ? (int)meta[3] : 8640;
    }
    s->is_room = (uint8_t*)calloc((size_t)s->n_cvs, 1);
    for (int rm = 0; rm < s->n_rooms; rm++)
        for (int t = s->room_off[rm]; t < s->room_off[rm + 1]; t++)
            s->is_room[s->room_cells[2 * t] * s->nc + s->room_cells[2 * t + 1]] = 1;
    /* convection tables (sb_convect.c:6-31) */
    s->conv_p = sbo_f64_1(b, "conv_p", 0.0);
    s->conv_dist = (int)sbo_f64_1(b, "conv_distance", -1.0);
    s->conv_seed = sbo_i64_1(b, "conv_seed", 0);
    s->cv_off = sbo_i32(b, "conv_room_offsets");
    s->cv_cells = sbo_i32(b, "conv_room_cells");
    s->cv_coff = sbo_i32(b, "conv_cand_offsets");
    s->cv_cidx = sbo_i32(b, "conv_cand_idx");
    if (!s->cv_off || !s->cv_cells || !s->cv_coff || !s->cv_cidx) return -1;
    s->cv_rooms = (int)sbo_sec(b, "conv_room_offsets")->count - 1;
    s->cv_max_room = 0;
    for (int i = 0; i < s->cv_rooms; i++) {
        const int m = s->cv_off[i + 1] - s->cv_off[i];
        if (m > s->cv_max_room) s->cv_max_room = m;
    }
    return 0;
}

void sbo_scen_close(SboScen* s) {
    free(s->Ldiag); free(s->Udiag); free(s->ir); free(s->pc); free(s->S); free(s->is_room);
    sbo_blob_free(&s->blob);
    memset(s, 0, sizeof(*s));
}

/* ------------------------------------------------------------ decode */
/* Continuous dims: float32 affine map op by op; discrete dims: +-1 then a
 * double map (complete_port/csim/sb_sim.c:557-576). */
void sbo_decode(const SboScen* s, const double* cont, const double* disc, double* native) {
    int ci = 0, di = 0;
    for (int i = 0; i < s->n_act; i++) {
        if (s->act_disc[i]) {
            double m = (disc[di++] == 1.0) ? 1.0 : -1.0;
            native[i] = (m - s->act_mnr[i]) / (s->act_mxr[i] - s->act_mnr[i])
                        * (s->act_mx[i] - s->act_mn[i]) + s->act_mn[i];
        } else {
            float a = (float)cont[ci++];
            float span_in = (float)(s->act_mxr[i] - s->act_mnr[i]);
            float span_out = (float)(s->act_mx[i] - s->act_mn[i]);
            float v = (a - (float)s->act_mnr[i]) / span_in * span_out + (float)s->act_mn[i];
            native[i] = (double)v;
        }
    }
}

/* Routing of native values to devices (sb_sim.c:220-244). */
static void apply_native(SboEnv* e, const double* nat) {
    const SboScen* s = e->sc;
    for (int i = 0; i < s->n_act; i++) {
        double v = nat[i];
        int idx = s->act_idx[i], a = s->act_act[i];
        switch (s->act_kind[i]) {
        case 0:
            if (a == 0) e->ahu_sat[idx] = v;
            else if (a == 1) e->ahu_fan[idx] = v;
            else if (a == 2) {
                double hi = s->ahu_c[idx * 9 + 3];
                e->ahu_recirc[idx] = v < 0.0 ? 0.0 : (v > hi ? hi : v);
            } else e->ahu_run[idx] = (v == 1.0) ? 1 : 0;
            break;
        case 1: {
            double c = v < 0.0 ? 0.0 : (v > 1.0 ? 1.0 : v);
            if (a == 0) { e->dcmd[idx] = c; e->dcmd_set[idx] = 1; }
            else { e->rcmd[idx] = c; e->rcmd_set[idx] = 1; }
            break;
        }
        default:
            if (a == 0) e->boiler_sp = v;
            else if (a == 1) e->pump_head = v / (GRAV * RHO_W / PA_PER_BAR);
            else { int on = (v == 1.0) ? 1 : 0; e->hws_run = on; e->pump_run = on; }
        }
    }
}

/* ------------------------------------------------------------ HVAC helpers */
/* sb_sim.c:246-251 */
static double ahu_static(const SboEnv* e, int a) {
    if (e->ahu_run[a] != 1) return 0.0;
    double sp = e->ahu_fan[a], mn = e->sc->ahu_c[a * 9 + 2];
    return sp > mn ? sp : mn;
}

/* sb_sim.c:267-276 */
static double vav_unrestricted(const SboEnv* e, int v) {
    const double* c = &e->sc->vav_c[v * 9];
    double d = e->damper[v] * c[0] * sqrt(ahu_static(e, e->sc->vav_ahu[v]) / c[4]);
    return d > 0.00001 ? d : 0.00001;
}

static double vav_flow_demand(const SboEnv* e, int v) { return vav_unrestricted(e, v) * e->ratio[v]; }

/* sb_sim.c:278-287 */
static double total_flow_rate(const SboEnv* e) {
    double ff = e->flow_factor_sum;
    double dp = (e->pump_run != 1) ? 0.0 : GRAV * RHO_W * e->pump_head / PA_PER_BAR;
    return ff * sqrt(dp / (1.0 + ff * ff * e->sc->header_res)) / 3600.0;
}

/* reheat_flow_rate / reheat_eff / reheat_energy, sb_sim.c:289-314 */
static double reheat_energy(const SboEnv* e, int v, double sat, double iwt) {
    const double* c = &e->sc->vav_c[v * 9];
    double eff;
    double air_cap = CP_AIR * RHO_AIR * vav_flow_demand(e, v);
    if (air_cap <= 0.0) {
        eff = 0.0;
    } else {
        double wflow = 0.0;
        if (e->flow_factor_sum != 0.0)
            wflow = total_flow_rate(e) * ((e->reheat[v] * c[1]) / e->flow_factor_sum);
        double water_cap = CP_W * RHO_W * wflow;
        eff = water_cap / air_cap;
        if (eff > 1.0) eff = 1.0;
        double gap = iwt - sat;
        if (gap > 0.0) {
            double headroom = c[3] - sat;
            if (headroom <= 0.0) eff = 0.0;
            else {
                double hr = headroom / gap;
                if (hr < eff) eff = hr;
            }
        }
    }
    return eff * CP_AIR * RHO_AIR * vav_flow_demand(e, v) * (iwt - sat);
}

/* Thermostat + VAV settings, sb_sim.c:316-355 */
static int default_mode(int cur, double zt, double hsp, double csp) {
    double mid = 0.5 * (csp - hsp) + hsp;
    if (zt < hsp) return M_HEAT;
    if (zt > csp) return M_COOL;
    if (zt < mid && cur == M_HEAT) return M_HEAT;
    if (zt > mid && cur == M_COOL) return M_COOL;
    return M_OFF;
}

static void vav_settings(SboEnv* e, int v, double zt, int kk, int comfort) {
    const SboScen* s = e->sc;
    const double* c = &s->vav_c[v * 9];
    double hsp = s->heat_sp[kk], csp = s->cool_sp[kk];
    e->heatsp[v] = hsp;
    e->coolsp[v] = csp;
    int mode = e->mode[v];
    if (comfort) mode = default_mode(mode, zt, hsp, csp);
    else if (e->prev_valid[v] && s->comfort[kk - 1] != 0.0) mode = M_PASSIVE;
    else if (mode == M_PASSIVE && zt > hsp && zt < csp) mode = M_PASSIVE;
    else mode = default_mode(mode, zt, hsp, csp);
    e->mode[v] = mode;
    e->prev_valid[v] = 1;
    double damper, reheat;
    if (mode == M_HEAT) { damper = 1.0; reheat = 1.0; }
    else if (mode == M_COOL) { damper = 1.0; reheat = 0.0; }
    else { damper = c[2]; reheat = 0.0; }
    if (e->dcmd_set[v]) damper = e->dcmd[v];
    if (e->rcmd_set[v]) reheat = e->rcmd[v];
    e->damper[v] = damper > c[2] ? damper : c[2];
    e->reheat[v] = reheat;
}

/* zone means of room cells in ascending cell order, sb_sim.c:149-160 */
static void zone_means(SboEnv* e) {
    const SboScen* s = e->sc;
    for (int z = 0; z < s->n_zones; z++) {
        int rm = s->phys_room[z];
        int a = s->room_off[rm], b = s->room_off[rm + 1];
        double sum = 0.0;
        for (int t = a; t < b; t++) sum += e->T[s->room_cells[2 * t] * s->nc + s->room_cells[2 * t + 1]];
        e->avg_temp[z] = sum / (double)(b - a);
    }
}

/* area-weighted VAV sensing, sb_sim.c:163-175 */
static void vav_sensing(SboEnv* e) {
    const SboScen* s = e->sc;
    for (int v = 0; v < s->n_vav; v++) {
        double area = 0.0, wt = 0.0;
        for (int t = s->vz_off[v]; t < s->vz_off[v + 1]; t++) {
            int z = s->vz_idx[t];
            area += s->zone_area[z];
            wt += e->avg_temp[z] * s->zone_area[z];
        }
        e->vav_area[v] = area;
        e->sensing[v] = (area > 0.0) ? wt / area : 0.0;
    }
}

/* ------------------------------------------------------------ reset */
/* sb_sim_reset, sb_sim.c:177-218 (pump_head is not reset there) */
static void sim_reset(SboEnv* e) {
    const SboScen* s = e->sc;
    for (int a = 0; a < s->n_ahu; a++) {
        const double* c = &s->ahu_c[a * 9];
        e->ahu_run[a] = (int)c[8];
        e->ahu_recirc[a] = c[0];
        e->ahu_sat[a] = c[6];
        e->ahu_fan[a] = c[7];
        e->ahu_flow[a] = 0.0;
        e->ahu_coolreq[a] = 0;
    }
    for (int v = 0; v < s->n_vav; v++) {
        const double* c = &s->vav_c[v * 9];
        e->damper[v] = c[7];
        e->reheat[v] = c[8];
        e->ratio[v] = 1.0;
        e->heatsp[v] = c[5];
        e->coolsp[v] = c[6];
        e->mode[v] = M_OFF;
        e->prev_valid[v] = e->dcmd_set[v] = e->rcmd_set[v] = 0;
        e->dcmd[v] = e->rcmd[v] = 0.0;
    }
    e->flow_factor_sum = 0.0;
    e->hws_requests = 0;
    e->hws_run = e->pump_run = 1;
    e->boiler_sp = s->boiler_c[0];
    e->boiler_ret = s->boiler_c[1];
    e->boiler_cur = s->boiler_c[0];
    e->boiler_dstep = 0.0;
    e->step_index = 0;
    memcpy(e->T, s->temp_init, sizeof(double) * (size_t)s->n_cvs);
    memcpy(e->M, s->mass_init, sizeof(double) * (size_t)s->n);
    memset(e->input_q, 0, sizeof(double) * (size_t)s->n_cvs);
    zone_means(e);
    vav_sensing(e);
}

/* ------------------------------------------------------------ step pieces */
/* sb_sim_step_pre, sb_sim.c:357-457 */
static void step_pre(SboEnv* e) {
    const SboScen* s = e->sc;
    int kk = e->step_index;
    double ambient = s->amb[kk];
    int comfort = (s->comfort[kk] != 0.0);
    int na = s->n_ahu, nv = s->n_vav, nz = s->n_zones;
    e->hws_requests = nv;
    zone_means(e);
    for (int a = 0; a < na; a++) { e->ahu_wsum[a] = 0.0; e->ahu_atotal[a] = 0.0; }
    for (int v = 0; v < nv; v++) {
        double area = 0.0, wt = 0.0;
        for (int t = s->vz_off[v]; t < s->vz_off[v + 1]; t++) {
            int z = s->vz_idx[t];
            area += s->zone_area[z];
            wt += e->avg_temp[z] * s->zone_area[z];
        }
        e->vav_area[v] = area;
        if (area <= 0.0) { e->sensing[v] = 0.0; continue; }
        double sensing = wt / area;
        e->sensing[v] = sensing;
        vav_settings(e, v, sensing, kk, comfort);
        int a = s->vav_ahu[v];
        e->ahu_wsum[a] += sensing * area;
        e->ahu_atotal[a] += area;
    }
    for (int a = 0; a < na; a++) {
        double rt;
        if (e->ahu_atotal[a] > 0.0) rt = e->ahu_wsum[a] / e->ahu_atotal[a];
        else {
            double m = 0.0;
            for (int p = 0; p < s->n_cvs; p++) m += e->T[p];
            rt = m / (double)s->n_cvs;
        }
        double mixed = e->ahu_recirc[a] * rt + (1.0 - e->ahu_recirc[a]) * ambient;
        e->ahu_satv[a] = (mixed > e->ahu_sat[a] && e->ahu_run[a] == 1) ? e->ahu_sat[a] : mixed;
    }
    for (int a = 0; a < na; a++) { e->ahu_flow[a] = 0.0; e->ahu_coolreq[a] = 0; }
    e->flow_factor_sum = 0.0;
    for (int v = 0; v < nv; v++) e->flow_factor_sum += e->reheat[v] * s->vav_c[v * 9 + 1];
    double demand[256];
    for (int a = 0; a < na; a++) demand[a] = 0.0;
    for (int v = 0; v < nv; v++) demand[s->vav_ahu[v]] += vav_unrestricted(e, v);
    for (int v = 0; v < nv; v++) {
        int a = s->vav_ahu[v];
        if (demand[a] > 0.0) {
            double r = s->ahu_c[a * 9 + 1] / demand[a];
            e->ratio[v] = r < 1.0 ? r : 1.0;
        } else {
            e->ratio[v] = 1.0;
        }
    }
    for (int z = 0; z < nz; z++) e->zone_q[z] = 0.0;
    e->total_reheat = 0.0;
    for (int col = 0; col < s->k; col++) {
        int v = s->coupled[col];
        if (e->vav_area[v] <= 0.0) { e->air_g[col] = 0.0; e->air_T[col] = 0.0; continue; }
        int a = s->vav_ahu[v];
        double sat = e->ahu_satv[a];
        e->air_T[col] = sat;
        double rw = reheat_energy(e, v, sat, e->boiler_cur);
        e->total_reheat += rw;
        e->coil[col] = sat;
        double fd = vav_flow_demand(e, v);
        if (e->damper[v] > 0.0 && s->vav_c[v * 9] > 0.0) {
            e->air_g[col] = fd * RHO_AIR * CP_AIR;
            for (int t = s->vz_off[v]; t < s->vz_off[v + 1]; t++) {
                int z = s->vz_idx[t];
                e->zone_q[z] += rw * s->zone_area[z] / e->vav_area[v];
            }
        } else {
            e->air_g[col] = 0.0;
        }
        if (fd > 0.0) {
            e->ahu_flow[a] += fd;
            double mf = s->ahu_c[a * 9 + 1];
            if (e->ahu_flow[a] > mf) e->ahu_flow[a] = mf;
            e->ahu_coolreq[a] += 1;
        }
    }
    if (s->internal_w_m2 > 0.0) {
        double frac = comfort ? 1.0 : s->standby_frac;
        double wpc = s->internal_w_m2 * s->cv_area * frac;
        for (int z = 0; z < nz; z++) {
            int rm = s->phys_room[z];
            e->zone_q[z] += wpc * (double)(s->room_off[rm + 1] - s->room_off[rm]);
        }
    }
    if (s->occupant_w > 0.0)
        for (int z = 0; z < nz; z++) e->zone_q[z] += e->occV[z] * s->occupant_w;
    for (int z = 0; z < nz; z++) {
        int rm = s->phys_room[z];
        int a = s->room_off[rm], b = s->room_off[rm + 1];
        double q = e->zone_q[z] / (double)(b - a);
        for (int t = a; t < b; t++) e->input_q[s->room_cells[2 * t] * s->nc + s->room_cells[2 * t + 1]] = q;
    }
}

/* Solar gain on every solved cell (added on room cells, assigned on others);
 * the step-order injection the reference harness (oracle/ref_driver.c) uses. */
static void add_solar(SboEnv* e) {
    const SboScen* s = e->sc;
    if (!s->solar_i || !s->solar_c) return;
    double irr = s->solar_i[e->step_index];
    for (int t = 0; t < s->n; t++) {
        int p = (int)s->solved[t];
        double q = s->solar_c[t] * irr;
        if (s->is_room[p]) e->input_q[p] += q;
        else e->input_q[p] = q;
    }
}

/* Backward-Euler field step with the air-side coupling, sb_fdm.c:126-188 */
static void field_step(SboEnv* e) {
    const SboScen* s = e->sc;
    int n = s->n, k = s->k;
    double ambient = s->amb[e->step_index];
    for (int t = 0; t < n; t++) {
        int64_t p = s->solved[t];
        double ex = 0.0;
        double a0 = s->face0[p];
        if (a0 > 0.0) ex += s->h * a0 / (1.0 + s->h * 0.5 * s->horiz[p] / s->cond[p]);
        double a1 = s->face1[p];
        if (a1 > 0.0) ex += s->h * a1 / (1.0 + s->h * 0.5 * s->vert[p] / s->cond[p]);
        e->rhs[t] = s->cap[t] * e->T[p] + e->input_q[p] + ambient * (s->dir[t] + ex)
                    + s->mcoup[t] * e->M[t];
    }
    sbo_lu_solve(s, e->rhs, e->y, e->work);
    int active = 0;
    for (int i = 0; i < k; i++) if (e->air_g[i] != 0.0) { active = 1; break; }
    if (k > 0 && active) {
        for (int i = 0; i < k; i++) {
            double acc = 0.0;
            for (int p = s->sn_p[i]; p < s->sn_p[i + 1]; p++) acc += s->sn_x[p] * e->y[s->sn_i[p]];
            e->power[i] = e->air_g[i] * (e->air_T[i] - acc);
        }
        for (int i = 0; i < k; i++)
            for (int j = 0; j < k; j++)
                e->mat[i * k + j] = (i == j ? 1.0 : 0.0) + e->air_g[i] * s->S[i * k + j];
        sbo_dense_solve(k, e->mat, e->power);
        for (int t = 0; t < n; t++) e->r[t] = 0.0;
        for (int j = 0; j < k; j++) {
            double qj = e->power[j];
            if (qj == 0.0) continue;
            for (int p = s->ap_p[j]; p < s->ap_p[j + 1]; p++) e->r[s->ap_i[p]] += s->ap_x[p] * qj;
        }
        sbo_lu_solve(s, e->r, e->yr, e->work);
        for (int t = 0; t < n; t++) e->y[t] += e->yr[t];
    }
    for (int t = 0; t < n; t++) e->M[t] = e->M[t] * s->mret[t] + s->mgain[t] * e->y[t];
    for (int p = 0; p < s->n_cvs; p++) e->T[p] = ambient;
    for (int t = 0; t < n; t++) e->T[s->solved[t]] = e->y[t];
}

/* sb_sim_step_post, sb_sim.c:459-521. The post-solve sensed-mean block
 * (:462-487) writes only zone_q/input_q/sensed_mean, which the next step_pre
 * rewrites before any read, so it has no observable effect and is omitted.
 * Convection (sb_sim.c:489) permutes the new field within its rooms. */
static void step_post(SboEnv* e) {
    const SboScen* s = e->sc;
    sbo_conv_apply(s, &e->cmt, e->cv_left, e->cv_right, e->T);
    double wcap = CP_W * RHO_W * total_flow_rate(e);
    if (wcap > 0.0 && s->k > 0) {
        double supply = e->boiler_cur;
        double rt = supply - e->total_reheat / wcap;
        double at = e->coil[0];
        for (int c = 1; c < s->k; c++) {
            if (e->total_reheat >= 0.0) { if (e->coil[c] < at) at = e->coil[c]; }
            else { if (e->coil[c] > at) at = e->coil[c]; }
        }
        double lo = supply < at ? supply : at;
        double hi = supply > at ? supply : at;
        if (rt < lo) rt = lo;
        if (rt > hi) rt = hi;
        e->boiler_ret = rt;
    }
    double begin = e->boiler_cur, sp = e->boiler_sp;
    double dt_min = s->dt_sec / 60.0;
    if (sp > begin) {
        double v = begin + s->boiler_c[2] * dt_min;
        e->boiler_cur = v < sp ? v : sp;
    } else if (sp < begin) {
        double v = begin - s->boiler_c[3] * dt_min;
        e->boiler_cur = v > sp ? v : sp;
    } else {
        e->boiler_cur = sp;
    }
    e->boiler_dstep = e->boiler_cur - begin;
    e->step_index += 1;
}

/* ------------------------------------------------------------ observation */
/* obs_value + sb_obs, complete_port/csim/sb_obs.c:11-64 */
static double obs_value(const SboEnv* e, int kind, int idx, int id, int j) {
    const SboScen* s = e->sc;
    if (kind == 0) {
        switch (id) {
        case 0: return (double)e->ahu_coolreq[idx];
        case 1: return ahu_static(e, idx);
        case 2: return (e->ahu_run[idx] == 1) ? e->ahu_flow[idx] : 0.0;
        case 3: return e->ahu_sat[idx];
        case 4: return (double)e->ahu_run[idx];
        case 5: return e->ahu_flow[idx] / s->ahu_c[idx * 9 + 1];
        case 6: return (1.0 - e->ahu_recirc[idx]) * e->ahu_flow[idx];
        case 7: return (double)e->ahu_run[idx];
        case 8: return e->ahu_recirc[idx];
        default: return s->amb[j];
        }
    }
    if (kind == 1) {
        switch (id) {
        case 0: return e->reheat[idx];
        case 1: return e->damper[idx];
        case 2: return s->vav_c[idx * 9];
        case 3: return e->coolsp[idx];
        case 4: return e->heatsp[idx];
        default: return e->sensing[idx];
        }
    }
    double dp = (e->pump_run == 1) ? 9.8 * 1000.0 * e->pump_head / 100000.0 : 0.0;
    switch (id) {
    case 0: return dp;
    case 1: return e->boiler_cur;
    case 2: return dp;
    case 3: return (double)e->hws_run;
    case 4: return (double)e->hws_requests;
    case 5: return (double)e->hws_run;
    default: return e->boiler_sp;
    }
}

static void write_obs(SboEnv* e, int j) {
    const SboScen* s = e->sc;
    for (int i = 0; i < s->n_dev; i++) {
        double v = obs_value(e, s->f_kind[i], s->f_idx[i], s->f_id[i], j);
        double var = s->f_var[i];
        float v32 = (float)v;
        e->obs[i] = (float)((var > 0.0) ? ((double)v32 - s->f_mean[i]) / sqrt(var) : 0.0);
    }
    int na = s->n_aux;
    const double* aux = &s->aux_time[(size_t)j * (na - 1)];
    for (int c = 0; c < na - 1; c++) e->obs[s->n_dev + c] = (float)aux[c];
    double occ = 0.0;
    for (int z = 0; z < s->n_zones; z++) occ += e->occV[z];
    e->obs[s->n_dev + na - 1] = (float)(int)occ;
    for (int i = s->n_dev + na; i < SBO_OBS; i++) e->obs[i] = 0.0f;
}

/* ------------------------------------------------------------ occupancy */
/* RandomizedArrivalDeparture chains in zone order, sb_occup.c:36-61 */
static void occupancy_advance(SboEnv* e, int hour, int workday) {
    const SboScen* s = e->sc;
    for (int z = 0; z < s->n_zones; z++) {
        int cnt = 0;
        for (int a = 0; a < s->occ_assign; a++) {
            uint8_t* st = &e->occ_state[z * s->occ_assign + a];
            if (!workday) {
                *st = 0;
            } else if (*st == 0) {
                if (hour >= s->occ_ea && hour <= s->occ_la && sbo_mt_double(&e->mt) < s->p_arr) *st = 1;
            } else if (hour < s->occ_ed) {
                /* stays at work */
            } else if (hour >= s->occ_ld) {
                *st = 0;
            } else if (sbo_mt_double(&e->mt) < s->p_dep) {
                *st = 0;
            }
            cnt += *st;
        }
        e->occV[z] = (double)cnt;
    }
}

/* ------------------------------------------------------------ reward */
/* boiler gas rate, complete_port/csim/sb_reward.c:12-29 */
static double boiler_gas(const SboEnv* e, double rwt, double outside, double tf) {
    const double* c = e->sc->boiler_c;
    double supply = (e->boiler_sp > rwt) ? e->boiler_sp : rwt;
    double flow = CP_W * RHO_W * tf * (supply - rwt);
    double diss = 0.0;
    if (supply >= outside) {
        double num = c[5] * 2.0 * PI_D * (supply - outside);
        double r2 = c[6] + c[9];
        double cond = log(r2 / c[6]) / c[8];
        double conv = 1.0 / c[4] / r2;
        diss = num / (cond + conv);
    }
    double tank = 0.0;
    if (e->sc->dt_sec > 0.0) tank = CP_W * RHO_W * c[7] * e->boiler_dstep / e->sc->dt_sec;
    double tot = flow + diss + tank;
    return tot > 0.0 ? tot : 0.0;
}

/* 3C reward, sb_reward.c:31-155 (the zone flow diagnostics at :44-56 do not
 * enter the value and are omitted). */
static double reward(SboEnv* e, int kv) {
    const SboScen* s = e->sc;
    int nz = s->n_zones;
    double dt = s->dt_sec, inv_hour = 1.0 / 3600.0;
    zone_means(e);
    double ambient = s->amb[kv];
    int hour = (int)s->rew_hour[kv], month = (int)s->rew_month[kv], wd = (int)s->rew_work[kv];
    double intake = 0.0, exhaust = 0.0, cooling = 0.0;
    for (int a = 0; a < s->n_ahu; a++) { e->ahu_wsum[a] = 0.0; e->ahu_atotal[a] = 0.0; }
    for (int v = 0; v < s->n_vav; v++) {
        double area = 0.0, wt = 0.0;
        for (int t = s->vz_off[v]; t < s->vz_off[v + 1]; t++) {
            int z = s->vz_idx[t];
            area += s->zone_area[z];
            wt += e->avg_temp[z] * s->zone_area[z];
        }
        if (area > 0.0) {
            int a = s->vav_ahu[v];
            e->ahu_wsum[a] += (wt / area) * area;
            e->ahu_atotal[a] += area;
        }
    }
    double tmean = 0.0;
    for (int p = 0; p < s->n_cvs; p++) tmean += e->T[p];
    tmean /= (double)s->n_cvs;
    for (int a = 0; a < s->n_ahu; a++) {
        double rc = (e->ahu_atotal[a] > 0.0) ? e->ahu_wsum[a] / e->ahu_atotal[a] : tmean;
        double st = ahu_static(e, a);
        double fe = s->ahu_c[a * 9 + 5];
        double flow = (e->ahu_run[a] == 1) ? e->ahu_flow[a] : 0.0;
        intake += flow * st / fe;
        exhaust += flow * (1.0 - e->ahu_recirc[a]) * st / fe;
        double mixed = e->ahu_recirc[a] * rc + (1.0 - e->ahu_recirc[a]) * ambient;
        double sat = (mixed > e->ahu_sat[a] && e->ahu_run[a] == 1) ? e->ahu_sat[a] : mixed;
        cooling += flow * RHO_AIR * CP_AIR * (sat - mixed) / s->ahu_c[a * 9 + 4];
    }
    double blower = intake + exhaust;
    double tf = total_flow_rate(e);
    double gas_rate = boiler_gas(e, e->boiler_ret, ambient, tf);
    double pump_e = tf * RHO_W * GRAV * e->pump_head / s->pump_eff;
    double max_pph = s->rw[0], min_pph = s->rw[1], ref = s->rw[2];
    double total_occ = 0.0, cum = 0.0;
    double dsum = 0.0, dmax = 0.0;   /* comfort diagnostics of the reference GPU env */
    int n_oob = 0;                   /* (complete_port/gpu/sb_gpu_kernels.cuh:1409-1473) */
    for (int z = 0; z < nz; z++) {
        double occ = e->occV[z];
        total_occ += occ;
        double zt = e->avg_temp[z];
        double hsp = s->heat_sp[kv], csp = s->cool_sp[kv];
        double dev = zt - csp;
        if (hsp - zt > dev) dev = hsp - zt;
        if (dev < 0.0) dev = 0.0;
        dsum += dev;
        if (dev > dmax) dmax = dev;
        if (dev > 0.0) n_oob++;
        double sh = (dev <= ref) ? dev / ref : 1.0 + ((dev - ref) / ref) * ((dev - ref) / ref);
        cum += max_pph * (1.0 - sh) * occ * dt * inv_hour;
    }
    double max_prod = max_pph * total_occ * dt * inv_hour;
    double min_prod = min_pph * total_occ * dt * inv_hour;
    double npr = 0.0;
    if (total_occ > 0.0 && (max_prod - min_prod) != 0.0)
        npr = (cum - min_prod) / (max_prod - min_prod) - 1.0;
    double elec_rate = blower + fabs(cooling) + pump_e;
    double price = wd ? s->elec_wk[hour] : s->elec_we[hour];
    double crate = s->elec_co2[hour];
    double elec_cost = price * fabs(elec_rate) * dt;
    double elec_cost_max = price * s->rw[3] * dt;
    double elec_carb = crate * fabs(elec_rate) * dt;
    double elec_carb_max = crate * s->rw[3] * dt;
    double gprice = s->gas_price[month - 1];
    double g = gas_rate > 0.0 ? gas_rate : 0.0;
    double gas_cost = gprice * g * dt;
    double gas_cost_max = gprice * s->rw[4] * dt;
    double gas_carb = s->gas_co2 * g * dt;
    double gas_carb_max = s->gas_co2 * s->rw[4] * dt;
    double den_e = elec_cost_max + gas_cost_max;
    double nec = (den_e > 0.0) ? (elec_cost + gas_cost) / den_e : 0.0;
    double den_c = elec_carb_max + gas_carb_max;
    double ncar = (den_c > 0.0) ? (elec_carb + gas_carb) / den_c : 0.0;
    double* pt = e->parts;
    pt[0] = npr; pt[1] = nec; pt[2] = ncar; pt[3] = elec_cost; pt[4] = gas_cost;
    pt[5] = blower; pt[6] = cooling; pt[7] = pump_e; pt[8] = price; pt[9] = dt;
    pt[10] = (double)hour; pt[11] = (double)wd;
    /* the reference GPU env's per-step diagnostics (sb_gpu_kernels.cuh:1469-1473):
     * mean and worst zone deviation from the band, fraction of zones outside
     * it, and the gas rate behind pt[4] */
    pt[12] = nz > 0 ? dsum / nz : 0.0; pt[13] = dmax; pt[14] = nz > 0 ? (double)n_oob / nz : 0.0;
    pt[15] = g;
    double pw = s->rw[5], ew = s->rw[6], cw = s->rw[7];
    double raw = npr * pw - nec * ew - ncar * cw;
    return raw / (pw + ew + cw);
}

/* ------------------------------------------------------------ env API */
static void* zalloc(size_t n, size_t sz) { return calloc(n ? n : 1, sz); }

SboEnv* sbo_env_new(const SboScen* s, uint32_t occ_seed, uint32_t conv_seed, int start, int max_steps) {
    SboEnv* e = (SboEnv*)calloc(1, sizeof(SboEnv));
    if (!e) return NULL;
    int na = s->n_ahu, nv = s->n_vav, nz = s->n_zones, n = s->n, k = s->k;
    e->sc = s;
    e->T = zalloc((size_t)s->n_cvs, 8); e->M = zalloc((size_t)n, 8);
    e->ahu_run = zalloc(na, 4); e->ahu_coolreq = zalloc(na, 4);
    e->ahu_recirc = zalloc(na, 8); e->ahu_sat = zalloc(na, 8); e->ahu_fan = zalloc(na, 8);
    e->ahu_flow = zalloc(na, 8); e->ahu_wsum = zalloc(na, 8); e->ahu_atotal = zalloc(na, 8);
    e->ahu_satv = zalloc(na, 8);
    e->damper = zalloc(nv, 8); e->reheat = zalloc(nv, 8); e->ratio = zalloc(nv, 8);
    e->heatsp = zalloc(nv, 8); e->coolsp = zalloc(nv, 8); e->dcmd = zalloc(nv, 8);
    e->rcmd = zalloc(nv, 8); e->sensing = zalloc(nv, 8); e->vav_area = zalloc(nv, 8);
    e->mode = zalloc(nv, 4); e->prev_valid = zalloc(nv, 4); e->dcmd_set = zalloc(nv, 4);
    e->rcmd_set = zalloc(nv, 4);
    e->avg_temp = zalloc(nz, 8); e->zone_q = zalloc(nz, 8); e->input_q = zalloc((size_t)s->n_cvs, 8);
    e->air_g = zalloc(k, 8); e->air_T = zalloc(k, 8); e->coil = zalloc(k, 8);
    e->occ_state = zalloc((size_t)nz * (size_t)s->occ_assign, 1);
    e->occV = zalloc(nz, 8);
    e->rhs = zalloc(n, 8); e->y = zalloc(n, 8); e->yr = zalloc(n, 8); e->r = zalloc(n, 8);
    e->work = zalloc(n, 8); e->power = zalloc(k, 8); e->mat = zalloc((size_t)k * (size_t)k, 8);
    e->pump_head = s->pump_head0;
    sbo_mt_seed(&e->mt, occ_seed);
    sbo_mt_seed(&e->cmt, conv_seed);
    e->cv_left = zalloc((size_t)s->cv_max_room, 4);
    e->cv_right = zalloc((size_t)s->cv_max_room, 4);
    e->start = start;
    e->max_steps = max_steps;
    e->first_steps = max_steps;
    return e;
}

/* The GPU env's desync (complete_port/gpu/smart_buildings.cu:2808-2815): the
 * env's first episode ends after first_steps steps, a truncation that leaves
 * the episode log alone (:1990-1993); later episodes have max_steps. */
void sbo_env_set_first_steps(SboEnv* e, int first_steps) { e->first_steps = first_steps; }

void sbo_env_free(SboEnv* e) {
    if (!e) return;
    void* ptrs[] = {e->T, e->M, e->ahu_run, e->ahu_coolreq, e->ahu_recirc, e->ahu_sat, e->ahu_fan,
                    e->ahu_flow, e->ahu_wsum, e->ahu_atotal, e->ahu_satv, e->damper, e->reheat,
                    e->ratio, e->heatsp, e->coolsp, e->dcmd, e->rcmd, e->sensing, e->vav_area,
                    e->mode, e->prev_valid, e->dcmd_set, e->rcmd_set, e->avg_temp, e->zone_q,
                    e->input_q, e->air_g, e->air_T, e->coil, e->occ_state, e->occV, e->rhs, e->y,
                    e->yr, e->r, e->work, e->power, e->mat, e->cv_left, e->cv_right};
    for (size_t i = 0; i < sizeof(ptrs) / sizeof(ptrs[0]); i++) free(ptrs[i]);
    free(e);
}

/* puf_reset (complete_port/pufferlib_cpu_env.h:187-208) at the env's start. */
void sbo_env_reset(SboEnv* e, float* obs_out) {
    const SboScen* s = e->sc;
    sim_reset(e);
    e->step_index = e->start;
    occupancy_advance(e, (int)s->hour_m1[e->start], (int)s->work_m1[e->start]);
    e->step = 0;
    for (int i = 0; i < s->n_act; i++) e->native[i] = 0.0;
    write_obs(e, e->start);
    if (obs_out) memcpy(obs_out, e->obs, sizeof(float) * SBO_OBS);
    occupancy_advance(e, (int)s->occ_hour[e->start], (int)s->occ_work[e->start]);
}

/* puf_step (complete_port/pufferlib_cpu_env.h:211-257). */
int sbo_env_step(SboEnv* e, const float* act, float* obs_out, float* reward_out, float* term_out) {
    const SboScen* s = e->sc;
    double cont[SBO_CONT], disc[SBO_DISC];
    for (int i = 0; i < s->n_cont; i++) {
        double a = (double)act[i];
        cont[i] = a > 1.0 ? 1.0 : (a < -1.0 ? -1.0 : a);
    }
    for (int i = 0; i < s->n_disc; i++) disc[i] = (double)act[SBO_CONT + i];
    sbo_decode(s, cont, disc, e->native);
    apply_native(e, e->native);
    step_pre(e);
    add_solar(e);
    field_step(e);
    step_post(e);
    e->step += 1;
    int j = e->start + e->step;
    write_obs(e, j);
    occupancy_advance(e, (int)s->occ_hour[j], (int)s->occ_work[j]);
    double rew = reward(e, j);
    e->last_rew = rew;
    float r = (float)rew;
    const int cut = !e->first_done && e->first_steps < e->max_steps;
    int done = e->step >= (e->first_done ? e->max_steps : e->first_steps);
    if (reward_out) *reward_out = r;
    if (term_out) *term_out = done ? 1.0f : 0.0f;
    if (!cut) {
        e->log[2] += r;
        e->log[4] += (r - e->log[4]) / (float)e->step;
    }
    if (done) {
        if (!cut) {
            float mean = e->log[2] / (float)e->step;
            e->log[0] += mean;
            e->log[1] += mean;
            e->log[3] += (float)e->step;
            e->log[5] += 1.0f;
        }
        e->first_done = 1;
        sbo_env_reset(e, NULL);
    }
    if (obs_out) memcpy(obs_out, e->obs, sizeof(float) * SBO_OBS);
    return done;
}

/* Same layout as ref_state in oracle/ref_driver.c. */
int sbo_env_state(const SboEnv* e, double* out) {
    const SboScen* s = e->sc;
    int c = 0;
    for (int p = 0; p < s->n_cvs; p++) out[c++] = e->T[p];
    for (int t = 0; t < s->n; t++) out[c++] = e->M[t];
    for (int v = 0; v < s->n_vav; v++) out[c++] = e->damper[v];
    for (int v = 0; v < s->n_vav; v++) out[c++] = e->reheat[v];
    for (int v = 0; v < s->n_vav; v++) out[c++] = e->ratio[v];
    for (int v = 0; v < s->n_vav; v++) out[c++] = e->sensing[v];
    for (int a = 0; a < s->n_ahu; a++) out[c++] = e->ahu_flow[a];
    for (int a = 0; a < s->n_ahu; a++) out[c++] = e->ahu_sat[a];
    for (int a = 0; a < s->n_ahu; a++) out[c++] = e->ahu_recirc[a];
    for (int a = 0; a < s->n_ahu; a++) out[c++] = e->ahu_fan[a];
    for (int i = 0; i < s->k; i++) out[c++] = e->air_g[i];
    for (int i = 0; i < s->k; i++) out[c++] = e->air_T[i];
    for (int z = 0; z < s->n_zones; z++) out[c++] = e->occV[z];
    out[c++] = e->boiler_cur;
    out[c++] = e->boiler_ret;
    out[c++] = e->boiler_sp;
    out[c++] = e->pump_head;
    out[c++] = (double)e->step_index;
    return c;
}

double sbo_env_last_reward(const SboEnv* e) { return e->last_rew; }
int sbo_env_obs_len(const SboEnv* e) { return e->sc->n_dev + e->sc->n_aux; }
int sbo_env_n_cont(const SboEnv* e) { return e->sc->n_cont; }
int sbo_env_n_disc(const SboEnv* e) { return e->sc->n_disc; }
void sbo_env_log(const SboEnv* e, float* out) { memcpy(out, e->log, sizeof(e->log)); }
void sbo_env_parts(const SboEnv* e, double* out) { memcpy(out, e->parts, sizeof(e->parts)); }
