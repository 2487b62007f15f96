/* Canonical observation, pid_water base controller and residual decode, for
 * the oracle (TEST INFRASTRUCTURE: only tests/ load liboracle.so).
 *
 * Restates, for one env and one step:
 *   - the slot maps of complete_port/gpu/smart_buildings.cu:844-1000
 *     (sb_canon_setup: zones by the order their VAV temperature field appears
 *     in the observation, slot 10 k + j on AHU k; AHU / hot-water / time fields
 *     found by name; native action -> canonical action slot);
 *   - the base controller complete_port/submission/pidw_base.py
 *     PIDWaterResetPolicy (pid -> worst-zone -> economiser -> proportional
 *     reheat -> water reset), with each AHU's zones in observation order, in
 *     the precisions numpy 2 gives it: zone temperatures, the zone commands
 *     and the per-AHU mean in float32 (numpy's pairwise sum), the PID loop,
 *     economiser and water reset in float64; the building's mean heating
 *     shortfall is a float64 mean when some zone has none (the list then holds
 *     Python zeros) and a float32 mean when every zone has one;
 *   - the canonical features of complete_port/submission/residual_policy.py
 *     _features (= complete_port/gpu/sb_gpu_base.inc:287-369 canon_obs_k);
 *   - the comfort guard (residual_policy.py _trust, sb_gpu_base.inc:230-265);
 *   - the residual / absolute action decode of sb_gpu_base.inc:371-404
 *     (decode_res_k), written as the action row the plain env step decodes:
 *     a continuous action's value m in [-1, 1], a discrete action 1 or 0.
 * Compiled with -ffp-contract=off: every float operation rounds as numpy's. */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "sbo.h"

#define CN_K SBO_CN_K
#define CN_ZPA SBO_CN_ZPA
#define CN_ZS SBO_CN_ZS
#define CN_FZ 9
#define CN_FA 16
#define CN_FH 10
#define CN_FG 19
#define CN_OA (CN_ZS * CN_FZ)
#define CN_OH (CN_OA + CN_K * CN_FA)
#define CN_OG (CN_OH + CN_FH)
#define CN_AA (2 * CN_ZS)
#define CN_AH (CN_AA + 4 * CN_K)

static const char* kAhuMeas[8] = {"outside_air_temperature_sensor", "supply_air_static_pressure_sensor",
                                  "supply_air_flowrate_sensor", "outside_air_flowrate_sensor",
                                  "supply_air_temperature_setpoint", "recirculation_percentage_command",
                                  "cooling_request_count", "supervisor_run_command"};

typedef struct {
    char** names;
    int n;
} Names;

static int find_name(const Names* nm, const char* s) {
    for (int i = 0; i < nm->n; i++)
        if (strcmp(nm->names[i], s) == 0) return i;
    return -1;
}

int sbo_canon_open(SboCanon* c, const char* path) {
    memset(c, 0, sizeof(*c));
    SboBlob b;
    if (sbo_blob_load(&b, path) != 0) return -1;
    const SboSec* fs = sbo_sec(&b, "field_names");
    const uint8_t* fk = sbo_u8(&b, "f_dev_kind");
    const int32_t* fi = sbo_i32(&b, "f_dev_idx");
    const uint8_t* fo = sbo_u8(&b, "f_obs_id");
    const double* fmn = sbo_f64(&b, "f_norm_mean");
    const double* fvr = sbo_f64(&b, "f_norm_var");
    const int32_t* vai = sbo_i32(&b, "vav_ahu_idx");
    const double* sc = sbo_f64(&b, "sched_scalars");
    const uint8_t* ok_ = sbo_u8(&b, "act_owner_kind");
    const int32_t* oi = sbo_i32(&b, "act_owner_index");
    const uint8_t* oa = sbo_u8(&b, "act_actuator");
    const uint8_t* isd = sbo_u8(&b, "act_is_discrete");
    const SboSec* ahu = sbo_sec(&b, "ahu_const");
    if (!fs || fs->dtype != 7 || !fk || !fi || !fo || !fmn || !fvr || !vai || !sc || !ok_ || !oi || !oa || !isd ||
        !ahu) {
        sbo_blob_free(&b);
        return -1;
    }
    const int n_dev = (int)sbo_i64_1(&b, "n_dev", 0);
    c->n_act = (int)sbo_sec(&b, "act_owner_kind")->count;
    c->K = (int)(ahu->count / 9);
    /* names, newline separated */
    Names nm = {0};
    {
        const char* s = (const char*)fs->data;
        const uint64_t len = fs->count;
        nm.names = (char**)calloc(len + 1, sizeof(char*));
        uint64_t a = 0;
        for (uint64_t i = 0; i <= len; i++) {
            if (i == len || s[i] == '\n') {
                char* w = (char*)malloc(i - a + 1);
                memcpy(w, s + a, i - a);
                w[i - a] = 0;
                nm.names[nm.n++] = w;
                a = i + 1;
            }
        }
    }
    int rc = 0;
    if (c->K > CN_K) rc = -2;
    for (int i = 0; i < CN_ZS; i++) c->zT[i] = c->zH[i] = c->zC[i] = c->zD[i] = c->zR[i] = c->zAd[i] = c->zAr[i] = -1;
    for (int k = 0; k < CN_K; k++)
        for (int m = 0; m < 8; m++) c->aObs[k][m] = -1;
    for (int k = 0; k < CN_K; k++) c->aT[k] = c->aP[k] = c->aRec[k] = c->aRun[k] = -1;
    c->hW = c->hDPa = c->hRun = -1;
    int vav_slot[1024];
    for (int v = 0; v < 1024; v++) vav_slot[v] = -1;
    const char* zsuf = "zone_air_temperature_sensor";
    for (int i = 0; i < n_dev && i < nm.n && rc == 0; i++) {
        if (fk[i] != 1 || fo[i] != 5) continue;
        const int v = fi[i], a = vai[v];
        if (a < 0 || a >= CN_K || c->zc[a] >= CN_ZPA) { rc = -2; break; }
        const int sl = CN_ZPA * a + c->zc[a]++;
        if (v >= 0 && v < 1024) vav_slot[v] = sl;
        const char* full = nm.names[i];
        const size_t pl = strlen(full) - strlen(zsuf);
        char buf[256];
        c->zT[sl] = i;
#define FIND_Z(dst, suffix)                                              \
    do {                                                                 \
        snprintf(buf, sizeof buf, "%.*s%s", (int)pl, full, suffix);      \
        dst = find_name(&nm, buf);                                       \
    } while (0)
        FIND_Z(c->zH[sl], "zone_air_heating_temperature_setpoint_sensor");
        FIND_Z(c->zC[sl], "zone_air_cooling_temperature_setpoint_sensor");
        FIND_Z(c->zD[sl], "supply_air_damper_percentage_command");
        FIND_Z(c->zR[sl], "reheat_valve_percentage_command");
#undef FIND_Z
    }
    for (int k = 0; k < c->K && k < CN_K; k++)
        for (int m = 0; m < 8; m++) {
            char buf[256];
            snprintf(buf, sizeof buf, "ahs_ahu_%d_%s", k + 1, kAhuMeas[m]);
            c->aObs[k][m] = find_name(&nm, buf);
        }
    {
        static const char* hw[6] = {"hws_supply_water_temperature_sensor", "hws_supply_water_temperature_setpoint",
                                    "hws_differential_pressure_sensor", "hws_differential_pressure_setpoint",
                                    "hws_run_status", "hws_heating_request_count"};
        for (int m = 0; m < 6; m++) c->hObs[m] = find_name(&nm, hw[m]);
    }
    for (int h = 0; h < 4; h++) {
        char buf[32];
        snprintf(buf, sizeof buf, "hod_sin_%03d", h); c->g[h] = find_name(&nm, buf);
        snprintf(buf, sizeof buf, "hod_cos_%03d", h); c->g[4 + h] = find_name(&nm, buf);
        snprintf(buf, sizeof buf, "dow_sin_%03d", h); c->g[8 + h] = find_name(&nm, buf);
        snprintf(buf, sizeof buf, "dow_cos_%03d", h); c->g[12 + h] = find_name(&nm, buf);
    }
    c->g[16] = find_name(&nm, "comfort_mode_now");
    c->g[17] = find_name(&nm, "comfort_mode_soon");
    c->g[18] = find_name(&nm, "num_occupants");
    if (c->g[0] < 0 || c->g[4] < 0 || c->g[8] < 0 || c->g[12] < 0) rc = rc ? rc : -1;
    for (int i = 0; i < SBO_OBS; i++) {
        c->fmean[i] = 0.0f;
        c->fstd[i] = 1.0f;
    }
    for (int i = 0; i < n_dev && i < SBO_OBS; i++)
        if (fvr[i] > 0.0) {
            c->fmean[i] = (float)fmn[i];
            c->fstd[i] = (float)sqrt(fvr[i]);
        }
    for (int i = 0; i < CN_ZS; i++)
        if (c->zT[i] >= 0) {
            c->tmean = c->fmean[c->zT[i]];
            c->tstd = c->fstd[c->zT[i]];
            break;
        }
    c->morning = (int)sc[0];
    c->evening = (int)sc[1];
    c->comfort_lo = sc[2];
    c->comfort_hi = sc[3];
    c->eco_lo = sc[4];
    c->eco_hi = sc[5];
    int ncont = 0, ndisc = 0;
    for (int a = 0; a < c->n_act && a < SBO_CONT + SBO_DISC; a++) {
        c->act_disc[a] = isd[a];
        c->act_col[a] = isd[a] ? SBO_CONT + ndisc++ : ncont++;
        c->slot_of_action[a] = -1;
        if (ok_[a] == 1) {
            const int sl = (oi[a] >= 0 && oi[a] < 1024) ? vav_slot[oi[a]] : -1;
            if (sl < 0) continue;
            if (oa[a] == 0) { c->zAd[sl] = a; c->slot_of_action[a] = 2 * sl; }
            else { c->zAr[sl] = a; c->slot_of_action[a] = 2 * sl + 1; }
        } else if (ok_[a] == 0) {
            const int k = oi[a];
            if (k < 0 || k >= CN_K) continue;
            if (oa[a] == 0) c->aT[k] = a;
            else if (oa[a] == 1) c->aP[k] = a;
            else if (oa[a] == 2) c->aRec[k] = a;
            else c->aRun[k] = a;
            c->slot_of_action[a] = CN_AA + 4 * k + oa[a];
        } else {
            if (oa[a] == 0) c->hW = a;
            else if (oa[a] == 1) c->hDPa = a;
            else c->hRun = a;
            c->slot_of_action[a] = CN_AH + oa[a];
        }
    }
    c->n_cont = ncont;
    c->n_disc = ndisc;
    for (int i = 0; i < nm.n; i++) free(nm.names[i]);
    free(nm.names);
    sbo_blob_free(&b);
    return rc;
}

/* numpy's pairwise sum of n < 128 values (8 accumulators), then / n. */
static float mean_f32(const float* a, int n) {
    float r;
    if (n < 8) {
        r = 0.0f;
        for (int i = 0; i < n; i++) r = r + a[i];
    } else {
        float q[8];
        for (int j = 0; j < 8; j++) q[j] = a[j];
        int i = 8;
        for (; i < n - (n % 8); i += 8)
            for (int j = 0; j < 8; j++) q[j] = q[j] + a[i + j];
        r = ((q[0] + q[1]) + (q[2] + q[3])) + ((q[4] + q[5]) + (q[6] + q[7]));
        for (; i < n; i++) r = r + a[i];
    }
    return r / (float)n;
}

static double mean_f64(const double* a, int n) {
    double r;
    if (n < 8) {
        r = 0.0;
        for (int i = 0; i < n; i++) r = r + a[i];
    } else {
        double q[8];
        for (int j = 0; j < 8; j++) q[j] = a[j];
        int i = 8;
        for (; i < n - (n % 8); i += 8)
            for (int j = 0; j < 8; j++) q[j] = q[j] + a[i + j];
        r = ((q[0] + q[1]) + (q[2] + q[3])) + ((q[4] + q[5]) + (q[6] + q[7]));
        for (; i < n; i++) r = r + a[i];
    }
    return r / (double)n;
}

/* pidw_base.py _cyclic_feature_to_index: float32 arctan2, + 2 pi, period * angle / (2 pi) */
static int cyclic(float s, float c, int period) {
    float ang = (float)atan2((double)s, (double)c);
    if (ang < 0.0f) ang = ang + (float)(2.0 * 3.141592653589793);
    const float v = ((float)period * ang) / (float)(2.0 * 3.141592653589793);
    return (int)floorf(v);
}

static double clip(double x, double lo, double hi) { return x < lo ? lo : (x > hi ? hi : x); }

static int work_hours(const SboCanon* c, const float* o) {
    const int hour = cyclic(o[c->g[0]], o[c->g[4]], 24);
    const int day = cyclic(o[c->g[8]], o[c->g[12]], 7);
    return day < 5 && c->morning <= hour && hour < c->evening;
}

/* zone temperature in kelvin: obs * std + mean in float32 */
static float zone_temp(const SboCanon* c, const float* o, int s) { return o[c->zT[s]] * c->tstd + c->tmean; }

void sbo_canon_base(const SboCanon* c, const float* o, double* pid, float* base, float* ahu_info) {
    for (int i = 0; i < c->n_act; i++) base[i] = 0.0f;
    const int work = work_hours(c, o);
    const double lo = work ? c->comfort_lo : c->eco_lo, hi = work ? c->comfort_hi : c->eco_hi;
    const float lof = (float)lo, hif = (float)hi;
    for (int k = 0; k < c->K; k++)
        if (c->aRec[k] >= 0) base[c->aRec[k]] = 1.0f;
    int any_heating = 0, any_active = 0;
    double efforts[CN_K];
    int ne = 0;
    for (int k = 0; k < c->K; k++) {
        ahu_info[2 * k] = 0.0f;
        ahu_info[2 * k + 1] = 0.0f;
        const int nz = c->zc[k];
        if (nz == 0) continue;
        float T[CN_ZPA];
        for (int j = 0; j < nz; j++) {
            const int s = CN_ZPA * k + j;
            T[j] = zone_temp(c, o, s);
            /* PIDProportionalReheatPolicy._command_zones (float32) */
            float err = 0.0f;
            if (T[j] < lof) err = lof - T[j];
            else if (T[j] > hif) err = hif - T[j];
            const float damper = fminf(1.0f, fabsf(err) / 2.0f);
            if (c->zAd[s] >= 0) base[c->zAd[s]] = 2.0f * damper - 1.0f;
            const float opening = fminf(1.0f, fmaxf(0.0f, err) / 2.0f);
            if (c->zAr[s] >= 0) base[c->zAr[s]] = 2.0f * opening - 1.0f;
        }
        const double avg = (double)mean_f32(T, nz);
        ahu_info[2 * k + 1] = (float)avg;
        double error = 0.0;
        if (avg < lo) error = lo - avg;
        else if (avg > hi) error = hi - avg;
        double* st = pid + 2 * k;
        if (error == 0.0) {
            st[0] = st[0] * 0.5;
            st[1] = 0.0;
            if (c->aT[k] >= 0) base[c->aT[k]] = -1.0f;
            if (c->aP[k] >= 0) base[c->aP[k]] = -1.0f;
            if (c->aRec[k] >= 0) base[c->aRec[k]] = 1.0f;
            if (c->aRun[k] >= 0) base[c->aRun[k]] = 0.0f;
            continue;
        }
        st[0] = clip(st[0] + error, -10.0, 10.0);
        const double deriv = error - st[1];
        st[1] = error;
        const double u = clip(0.5 * error + 0.02 * st[0] + 0.1 * deriv, -1.0, 1.0);
        ahu_info[2 * k] = (float)u;
        efforts[ne++] = u;
        const double pressure = clip(2.0 * fabs(u) - 1.0, -1.0, 1.0);
        if (c->aT[k] >= 0) base[c->aT[k]] = (float)u;
        if (c->aP[k] >= 0) base[c->aP[k]] = (float)pressure;
        if (c->aRun[k] >= 0) base[c->aRun[k]] = 1.0f;
        if (c->aRec[k] >= 0) { /* PIDEconomizerPolicy._recirculation */
            double rec = 1.0;
            const int oat = c->aObs[k][0];
            if (!(u >= 0.0) && oat >= 0) {
                const double outside = (double)o[oat], inside = avg;
                if (isfinite(outside) && !(outside >= inside)) {
                    double pa = (pressure + 1.0) * 0.5 * 2000.0;
                    pa = pa > 200.0 ? pa : 200.0;
                    const double breakeven = pa * 0.00322;
                    if (!(inside - outside <= breakeven)) {
                        double target = 285.0 + (u + 1.0) * 0.5 * (305.0 - 285.0);
                        target = target > lo ? target : lo;
                        if (!(inside <= target)) {
                            const double f = (inside - target) / (inside - outside);
                            rec = 2.0 * clip(1.0 - f, 0.0, 1.0) - 1.0;
                        }
                    }
                }
            }
            base[c->aRec[k]] = (float)rec;
        }
        any_active = 1;
        if (error > 0.0) any_heating = 1;
    }
    if (c->hW >= 0) base[c->hW] = any_heating ? 1.0f : -1.0f;
    if (c->hDPa >= 0) base[c->hDPa] = any_active ? 1.0f : -1.0f;
    if (c->hRun >= 0) base[c->hRun] = any_active ? 1.0f : 0.0f;
    /* PIDWaterResetPolicy.get_action / _water_fraction (integral gain 0) */
    if (c->hW >= 0 && base[c->hW] > 0.0f) {
        float s32[CN_ZS];
        double s64[CN_ZS];
        int n = 0, all_pos = 1;
        for (int k = 0; k < c->K; k++)
            for (int j = 0; j < c->zc[k]; j++) {
                const float d = lof - zone_temp(c, o, CN_ZPA * k + j);
                s32[n] = d;
                s64[n] = d > 0.0f ? (double)d : 0.0;
                if (!(d > 0.0f)) all_pos = 0;
                n++;
            }
        double shortfall = 0.0;
        if (n > 0) shortfall = all_pos ? (double)mean_f32(s32, n) : mean_f64(s64, n);
        const double demand = shortfall / 4.0;
        double sat = 0.0;
        if (ne > 0) {
            double h[CN_K];
            for (int i = 0; i < ne; i++) h[i] = efforts[i] > 0.0 ? efforts[i] : 0.0;
            for (int i = 1; i < ne; i++) { /* sort, ascending */
                const double x = h[i];
                int j = i - 1;
                while (j >= 0 && h[j] > x) { h[j + 1] = h[j]; j--; }
                h[j + 1] = x;
            }
            /* np.quantile(method linear, q = 0.25): virtual index (n - 1) q, numpy's _lerp */
            const double vi = (double)(ne - 1) * 0.25;
            int i0 = (int)floor(vi), i1 = i0 + 1;
            if (vi >= (double)(ne - 1)) i0 = i1 = ne - 1;
            const double t = vi - floor(vi);
            const double a0 = h[i0], a1 = h[i1];
            const double diff = a1 - a0;
            sat = t >= 0.5 ? a1 - diff * (1.0 - t) : a0 + diff * t;
        }
        const double m = demand > sat ? demand : sat;   /* Python max(demand, saturation) */
        const double frac = clip(m + 0.0, 0.0, 1.0);
        base[c->hW] = (float)(2.0 * frac - 1.0);
    }
}

static float nat(const SboCanon* c, const float* o, int i) { return i >= 0 ? o[i] * c->fstd[i] + c->fmean[i] : 0.0f; }

void sbo_canon_features(const SboCanon* c, const float* o, const float* b, const float* ai, const double* pid,
                        float* x) {
    for (int i = 0; i < SBO_CN_OBS; i++) x[i] = 0.0f;
    for (int s = 0; s < CN_ZS; s++) {
        if (c->zT[s] < 0) continue;
        const float T = nat(c, o, c->zT[s]), Hs = nat(c, o, c->zH[s]), Cs = nat(c, o, c->zC[s]);
        float* f = x + CN_FZ * s;
        f[0] = 1.0f;
        f[1] = (T - 295.0f) / 5.0f;
        f[2] = (T - Hs) / 2.0f;
        f[3] = (Cs - T) / 2.0f;
        f[4] = (Hs - 294.0f) / 3.0f;
        f[5] = c->zD[s] >= 0 ? 2.0f * nat(c, o, c->zD[s]) - 1.0f : 0.0f;
        f[6] = c->zR[s] >= 0 ? 2.0f * nat(c, o, c->zR[s]) - 1.0f : 0.0f;
        f[7] = c->zAd[s] >= 0 ? b[c->zAd[s]] : 0.0f;
        f[8] = c->zAr[s] >= 0 ? b[c->zAr[s]] : 0.0f;
    }
    for (int k = 0; k < c->K && k < CN_K; k++) {
        float* f = x + CN_OA + CN_FA * k;
        const int* q = c->aObs[k];
        f[0] = 1.0f;
        f[1] = (nat(c, o, q[0]) - 283.0f) / 15.0f;
        f[2] = nat(c, o, q[1]) / 1000.0f;
        f[3] = nat(c, o, q[2]) / 10.0f;
        f[4] = nat(c, o, q[3]) / 10.0f;
        f[5] = q[4] >= 0 ? (nat(c, o, q[4]) - 295.0f) / 5.0f : 0.0f;
        f[6] = 2.0f * nat(c, o, q[5]) - 1.0f;
        f[7] = nat(c, o, q[6]) / 10.0f;
        f[8] = 2.0f * nat(c, o, q[7]) - 1.0f;
        f[9] = c->aT[k] >= 0 ? b[c->aT[k]] : 0.0f;
        f[10] = c->aP[k] >= 0 ? b[c->aP[k]] : 0.0f;
        f[11] = c->aRec[k] >= 0 ? b[c->aRec[k]] : 0.0f;
        f[12] = c->aRun[k] >= 0 ? 2.0f * b[c->aRun[k]] - 1.0f : 0.0f;
        f[13] = c->zc[k] > 0 ? (ai[2 * k + 1] - 295.0f) / 5.0f : 0.0f;
        f[14] = (float)(pid[2 * k] / 10.0);
        f[15] = ai[2 * k];
    }
    {
        float* f = x + CN_OH;
        const int* q = c->hObs;
        f[0] = 1.0f;
        f[1] = (nat(c, o, q[0]) - 330.0f) / 20.0f;
        f[2] = (nat(c, o, q[1]) - 330.0f) / 20.0f;
        f[3] = nat(c, o, q[2]) / 10.0f;
        f[4] = nat(c, o, q[3]) / 10.0f;
        f[5] = 2.0f * nat(c, o, q[4]) - 1.0f;
        f[6] = nat(c, o, q[5]) / 10.0f;
        f[7] = c->hW >= 0 ? b[c->hW] : 0.0f;
        f[8] = c->hDPa >= 0 ? b[c->hDPa] : 0.0f;
        f[9] = c->hRun >= 0 ? 2.0f * b[c->hRun] - 1.0f : 0.0f;
    }
    for (int j = 0; j < CN_FG; j++) x[CN_OG + j] = c->g[j] >= 0 ? o[c->g[j]] : 0.0f;
}

void sbo_canon_trust(const SboCanon* c, const float* o, float d0, float d1, int hot, float* w) {
    for (int i = 0; i < c->n_act; i++) w[i] = 1.0f;
    const int work = work_hours(c, o);
    const float lof = (float)(work ? c->comfort_lo : c->eco_lo), hif = (float)(work ? c->comfort_hi : c->eco_hi);
    float wb = 1.0f;
    for (int k = 0; k < c->K; k++) {
        float wk = 1.0f;
        for (int j = 0; j < c->zc[k]; j++) {
            const int s = CN_ZPA * k + j;
            const float T = zone_temp(c, o, s);
            const float dev = T < lof ? lof - T : (hot && T > hif ? T - hif : 0.0f);
            const float t = fminf(1.0f, fmaxf(0.0f, 1.0f - (dev - d0) / d1));
            if (c->zAd[s] >= 0) w[c->zAd[s]] = t;
            if (c->zAr[s] >= 0) w[c->zAr[s]] = t;
            wk = fminf(wk, t);
        }
        if (c->aT[k] >= 0) w[c->aT[k]] = wk;
        if (c->aP[k] >= 0) w[c->aP[k]] = wk;
        if (c->aRec[k] >= 0) w[c->aRec[k]] = wk;
        if (c->aRun[k] >= 0) w[c->aRun[k]] = wk;
        wb = fminf(wb, wk);
    }
    if (c->hW >= 0) w[c->hW] = wb;
    if (c->hDPa >= 0) w[c->hDPa] = wb;
    if (c->hRun >= 0) w[c->hRun] = wb;
}

void sbo_canon_decode(const SboCanon* c, const float* b, const float* prow, const float* trust, int resid,
                      float scale, float dscale, float* row) {
    for (int i = 0; i < SBO_CONT + SBO_DISC; i++) row[i] = 0.0f;
    for (int i = 0; i < c->n_act; i++) {
        const int sl = c->slot_of_action[i];
        float p = 0.0f;
        if (sl >= 0) {
            p = prow[sl];
            p = isfinite(p) ? fminf(1.0f, fmaxf(-1.0f, p)) : 0.0f;
            if (trust) p = p * trust[i];
        }
        if (c->act_disc[i]) {
            const int on = resid ? ((2.0f * b[i] - 1.0f) + dscale * p > 0.0f) : (p > -0.5f);
            row[c->act_col[i]] = on ? 1.0f : 0.0f;
        } else {
            float m = resid ? b[i] + scale * p : p;
            row[c->act_col[i]] = fminf(1.0f, fmaxf(-1.0f, m));
        }
    }
}

size_t sbo_canon_size(void) { return sizeof(SboCanon); }

int sbo_canon_slot(const SboCanon* c, int i) { return (i >= 0 && i < c->n_act) ? c->slot_of_action[i] : -1; }
