// Field envs (see field_env.h): the HVAC plant, actions, observation,
// occupancy, reward and episode bookkeeping of FDM-scale scenarios, one lane
// per env. Each env's work is O(zones + VAVs + observation fields) per step
// beside a field solve over 10^5-10^6 cells, so the lanes run csim's own
// sequential order: every sum keeps its operand order and this file is built
// with -ffp-contract=off, which makes the results bit-identical to the
// reference core (complete_port/csim/sb_sim.c, sb_obs.c, sb_occup.c,
// sb_reward.c, sb_rng.c; complete_port/pufferlib_cpu_env.h:187-257).
#include <hip/hip_runtime.h>

#include "sbenv.h"
#include "field_env.h"

namespace sbe {

#define RHO_AIR 1.2
#define CP_AIR 1006.0
#define RHO_W 1000.0
#define CP_W 4180.0
#define GRAV 9.8
#define PA_PER_BAR 100000.0
#define PI_D 3.14159265358979323846

enum { M_OFF = 0, M_HEAT = 1, M_COOL = 2, M_PASSIVE = 3 };

// One env's view of its record.
struct E {
    const Tabs* t;
    double *recirc, *sat, *fan, *flow, *wsum, *atotal, *satv;
    double *damper, *reheat, *ratio, *heatsp, *coolsp, *dcmd, *rcmd, *sensing, *vav_area;
    double *avg_temp, *zone_q, *occV;
    double *air_g, *air_T, *coil;
    double* pl;
    int *run, *coolreq, *mode, *prev_valid, *dcmd_set, *rcmd_set, *ip;
    uint8_t* occ_state;
    uint32_t* mt;
};

__device__ __forceinline__ E bind(const Args& a, int s) {
    const StateLayout& st = a.st;
    unsigned char* b = a.state + (size_t)s * st.bytes;
    E e;
    e.t = &a.t;
    e.recirc = (double*)(b + st.recirc);
    e.sat = (double*)(b + st.sat);
    e.fan = (double*)(b + st.fan);
    e.flow = (double*)(b + st.flow);
    e.wsum = (double*)(b + st.wsum);
    e.atotal = (double*)(b + st.atotal);
    e.satv = (double*)(b + st.satv);
    e.damper = (double*)(b + st.damper);
    e.reheat = (double*)(b + st.reheat);
    e.ratio = (double*)(b + st.ratio);
    e.heatsp = (double*)(b + st.heatsp);
    e.coolsp = (double*)(b + st.coolsp);
    e.dcmd = (double*)(b + st.dcmd);
    e.rcmd = (double*)(b + st.rcmd);
    e.sensing = (double*)(b + st.sensing);
    e.vav_area = (double*)(b + st.vav_area);
    e.avg_temp = (double*)(b + st.avg_temp);
    e.zone_q = (double*)(b + st.zone_q);
    e.occV = (double*)(b + st.occV);
    e.air_g = (double*)(b + st.air_g);
    e.air_T = (double*)(b + st.air_T);
    e.coil = (double*)(b + st.coil);
    e.pl = (double*)(b + st.plant);
    e.run = (int*)(b + st.run);
    e.coolreq = (int*)(b + st.coolreq);
    e.mode = (int*)(b + st.mode);
    e.prev_valid = (int*)(b + st.prev_valid);
    e.dcmd_set = (int*)(b + st.dcmd_set);
    e.rcmd_set = (int*)(b + st.rcmd_set);
    e.ip = (int*)(b + st.ip);
    e.occ_state = b + st.occ_state;
    e.mt = (uint32_t*)(b + st.mt);
    return e;
}

// ------------------------------------------------------------------ MT19937
// genrand_int32 / random_sample of Matsumoto & Nishimura (1998), the stream
// numpy's legacy RandomState draws (sb_rng.c:9-43).
__device__ void mt_seed(E& e, uint32_t seed) {
    e.mt[0] = seed;
    for (int i = 1; i < 624; i++) e.mt[i] = 1812433253u * (e.mt[i - 1] ^ (e.mt[i - 1] >> 30)) + (uint32_t)i;
    e.ip[IP_MT_IDX] = 624;
}

__device__ uint32_t mt_u32(E& e) {
    if (e.ip[IP_MT_IDX] >= 624) {
        for (int i = 0; i < 624; i++) {
            const uint32_t x = (e.mt[i] & 0x80000000u) | (e.mt[(i + 1) % 624] & 0x7fffffffu);
            uint32_t xa = x >> 1;
            if (x & 1u) xa ^= 0x9908b0dfu;
            e.mt[i] = e.mt[(i + 397) % 624] ^ xa;
        }
        e.ip[IP_MT_IDX] = 0;
    }
    uint32_t y = e.mt[e.ip[IP_MT_IDX]++];
    y ^= y >> 11;
    y ^= (y << 7) & 0x9d2c5680u;
    y ^= (y << 15) & 0xefc60000u;
    y ^= y >> 18;
    return y;
}

__device__ double mt_double(E& e) {
    const uint32_t a = mt_u32(e) >> 5;
    const uint32_t b = mt_u32(e) >> 6;
    return (a * 67108864.0 + b) / 9007199254740992.0;
}

// ------------------------------------------------------------------ HVAC
// sb_sim.c:246-251
__device__ double ahu_static(const E& e, int a) {
    if (e.run[a] != 1) return 0.0;
    const double sp = e.fan[a], mn = e.t->ahu_c[a * 9 + 2];
    return sp > mn ? sp : mn;
}

// sb_sim.c:267-276
__device__ double vav_unrestricted(const E& e, int v) {
    const double* c = &e.t->vav_c[v * 9];
    const double d = e.damper[v] * c[0] * sqrt(ahu_static(e, e.t->vav_ahu[v]) / c[4]);
    return d > 0.00001 ? d : 0.00001;
}

__device__ double vav_flow_demand(const E& e, int v) { return vav_unrestricted(e, v) * e.ratio[v]; }

// sb_sim.c:278-287
__device__ double total_flow_rate(const E& e) {
    const double ff = e.pl[PL_FFS];
    const double dp = (e.ip[IP_PUMP_RUN] != 1) ? 0.0 : GRAV * RHO_W * e.pl[PL_PUMP_HEAD] / PA_PER_BAR;
    return ff * sqrt(dp / (1.0 + ff * ff * e.t->header_res)) / 3600.0;
}

// reheat_flow_rate / reheat_eff / reheat_energy, sb_sim.c:289-314
__device__ double reheat_energy(const E& e, int v, double sat, double iwt) {
    const double* c = &e.t->vav_c[v * 9];
    double eff;
    const double air_cap = CP_AIR * RHO_AIR * vav_flow_demand(e, v);
    if (air_cap <= 0.0) {
        eff = 0.0;
    } else {
        double wflow = 0.0;
        if (e.pl[PL_FFS] != 0.0) wflow = total_flow_rate(e) * ((e.reheat[v] * c[1]) / e.pl[PL_FFS]);
        const double water_cap = CP_W * RHO_W * wflow;
        eff = water_cap / air_cap;
        if (eff > 1.0) eff = 1.0;
        const double gap = iwt - sat;
        if (gap > 0.0) {
            const double headroom = c[3] - sat;
            if (headroom <= 0.0) {
                eff = 0.0;
            } else {
                const double hr = headroom / gap;
                if (hr < eff) eff = hr;
            }
        }
    }
    return eff * CP_AIR * RHO_AIR * vav_flow_demand(e, v) * (iwt - sat);
}

// Thermostat and VAV settings, sb_sim.c:316-355
__device__ int default_mode(int cur, double zt, double hsp, double csp) {
    const double mid = 0.5 * (csp - hsp) + hsp;
    if (zt < hsp) return M_HEAT;
    if (zt > csp) return M_COOL;
    if (zt < mid && cur == M_HEAT) return M_HEAT;
    if (zt > mid && cur == M_COOL) return M_COOL;
    return M_OFF;
}

__device__ void vav_settings(E& e, int v, double zt, int kk, int comfort) {
    const Tabs& t = *e.t;
    const double* c = &t.vav_c[v * 9];
    const double hsp = t.heat_sp[kk], csp = t.cool_sp[kk];
    e.heatsp[v] = hsp;
    e.coolsp[v] = csp;
    int mode = e.mode[v];
    if (comfort) mode = default_mode(mode, zt, hsp, csp);
    else if (e.prev_valid[v] && t.comfort[kk - 1] != 0.0) mode = M_PASSIVE;
    else if (mode == M_PASSIVE && zt > hsp && zt < csp) mode = M_PASSIVE;
    else mode = default_mode(mode, zt, hsp, csp);
    e.mode[v] = mode;
    e.prev_valid[v] = 1;
    double damper, reheat;
    if (mode == M_HEAT) {
        damper = 1.0;
        reheat = 1.0;
    } else if (mode == M_COOL) {
        damper = 1.0;
        reheat = 0.0;
    } else {
        damper = c[2];
        reheat = 0.0;
    }
    if (e.dcmd_set[v]) damper = e.dcmd[v];
    if (e.rcmd_set[v]) reheat = e.rcmd[v];
    e.damper[v] = damper > c[2] ? damper : c[2];
    e.reheat[v] = reheat;
}

// area-weighted VAV sensing of the zone means, sb_sim.c:163-175
__device__ void vav_sensing(E& e) {
    const Tabs& t = *e.t;
    for (int v = 0; v < t.nv; v++) {
        double area = 0.0, wt = 0.0;
        for (int q = t.vz_off[v]; q < t.vz_off[v + 1]; q++) {
            const int z = t.vz_idx[q];
            area += t.zone_area[z];
            wt += e.avg_temp[z] * t.zone_area[z];
        }
        e.vav_area[v] = area;
        e.sensing[v] = (area > 0.0) ? wt / area : 0.0;
    }
}

// decode (sb_sim.c:557-576, after puf_step's clamp, pufferlib_cpu_env.h:218-232)
// and sb_sim_apply_native (sb_sim.c:220-244)
__device__ void decode_apply(E& e, const float* row) {
    const Tabs& t = *e.t;
    int ci = 0, di = 0;
    for (int i = 0; i < t.n_act; i++) {
        double v;
        if (t.act_disc[i]) {
            const double d = (double)row[SB_CONT + di++];
            const double m = (d == 1.0) ? 1.0 : -1.0;
            v = (m - t.act_mnr[i]) / (t.act_mxr[i] - t.act_mnr[i]) * (t.act_mx[i] - t.act_mn[i]) + t.act_mn[i];
        } else {
            const double a64 = (double)row[ci++];
            const double cl = a64 > 1.0 ? 1.0 : (a64 < -1.0 ? -1.0 : a64);
            const float a = (float)cl;
            const float span_in = (float)(t.act_mxr[i] - t.act_mnr[i]);
            const float span_out = (float)(t.act_mx[i] - t.act_mn[i]);
            const float r = (a - (float)t.act_mnr[i]) / span_in * span_out + (float)t.act_mn[i];
            v = (double)r;
        }
        const int idx = t.act_idx[i], act = t.act_act[i];
        switch (t.act_kind[i]) {
        case 0:
            if (act == 0) e.sat[idx] = v;
            else if (act == 1) e.fan[idx] = v;
            else if (act == 2) {
                const double hi = t.ahu_c[idx * 9 + 3];
                e.recirc[idx] = v < 0.0 ? 0.0 : (v > hi ? hi : v);
            } else e.run[idx] = (v == 1.0) ? 1 : 0;
            break;
        case 1: {
            const double c = v < 0.0 ? 0.0 : (v > 1.0 ? 1.0 : v);
            if (act == 0) {
                e.dcmd[idx] = c;
                e.dcmd_set[idx] = 1;
            } else {
                e.rcmd[idx] = c;
                e.rcmd_set[idx] = 1;
            }
            break;
        }
        default:
            if (act == 0) e.pl[PL_BOILER_SP] = v;
            else if (act == 1) e.pl[PL_PUMP_HEAD] = v / (GRAV * RHO_W / PA_PER_BAR);
            else {
                const int on = (v == 1.0) ? 1 : 0;
                e.ip[IP_HWS_RUN] = on;
                e.ip[IP_PUMP_RUN] = on;
            }
        }
    }
}

// sb_sim_step_pre (sb_sim.c:357-457) from the zone means in avg_temp; writes
// the field step's inputs of slot s. Every AHU serves zone area (the host
// checks it), so the all-cell mean of the AHU fallback is never read.
__device__ void step_pre(E& e, const Args& a, int s) {
    const Tabs& t = *e.t;
    const int kk = e.ip[IP_STEP_INDEX];
    const double ambient = t.amb[kk];
    const int comfort = (t.comfort[kk] != 0.0);
    const int na = t.na, nv = t.nv, nz = t.nz;
    e.ip[IP_HWS_REQ] = nv;
    for (int q = 0; q < na; q++) {
        e.wsum[q] = 0.0;
        e.atotal[q] = 0.0;
    }
    for (int v = 0; v < nv; v++) {
        double area = 0.0, wt = 0.0;
        for (int q = t.vz_off[v]; q < t.vz_off[v + 1]; q++) {
            const int z = t.vz_idx[q];
            area += t.zone_area[z];
            wt += e.avg_temp[z] * t.zone_area[z];
        }
        e.vav_area[v] = area;
        if (area <= 0.0) {
            e.sensing[v] = 0.0;
            continue;
        }
        const double sensing = wt / area;
        e.sensing[v] = sensing;
        vav_settings(e, v, sensing, kk, comfort);
        const int q = t.vav_ahu[v];
        e.wsum[q] += sensing * area;
        e.atotal[q] += area;
    }
    for (int q = 0; q < na; q++) {
        const double rt = e.wsum[q] / e.atotal[q];
        const double mixed = e.recirc[q] * rt + (1.0 - e.recirc[q]) * ambient;
        e.satv[q] = (mixed > e.sat[q] && e.run[q] == 1) ? e.sat[q] : mixed;
    }
    for (int q = 0; q < na; q++) {
        e.flow[q] = 0.0;
        e.coolreq[q] = 0;
    }
    double ffs = 0.0;
    for (int v = 0; v < nv; v++) ffs += e.reheat[v] * t.vav_c[v * 9 + 1];
    e.pl[PL_FFS] = ffs;
    // AHU demand in VAV order, then the VAV flow ratios (wsum is scratch here)
    for (int q = 0; q < na; q++) e.wsum[q] = 0.0;
    for (int v = 0; v < nv; v++) e.wsum[t.vav_ahu[v]] += vav_unrestricted(e, v);
    for (int v = 0; v < nv; v++) {
        const int q = t.vav_ahu[v];
        if (e.wsum[q] > 0.0) {
            const double r = t.ahu_c[q * 9 + 1] / e.wsum[q];
            e.ratio[v] = r < 1.0 ? r : 1.0;
        } else {
            e.ratio[v] = 1.0;
        }
    }
    for (int z = 0; z < nz; z++) e.zone_q[z] = 0.0;
    double total_rw = 0.0;
    const double iwt = e.pl[PL_BOILER_CUR];
    for (int col = 0; col < t.k; col++) {
        const int v = t.coupled[col];
        if (e.vav_area[v] <= 0.0) {
            e.air_g[col] = 0.0;
            e.air_T[col] = 0.0;
            continue;
        }
        const int q = t.vav_ahu[v];
        const double sat = e.satv[q];
        e.air_T[col] = sat;
        const double rw = reheat_energy(e, v, sat, iwt);
        total_rw += rw;
        e.coil[col] = sat;
        const double fd = vav_flow_demand(e, v);
        if (e.damper[v] > 0.0 && t.vav_c[v * 9] > 0.0) {
            e.air_g[col] = fd * RHO_AIR * CP_AIR;
            for (int w = t.vz_off[v]; w < t.vz_off[v + 1]; w++) {
                const int z = t.vz_idx[w];
                e.zone_q[z] += rw * t.zone_area[z] / e.vav_area[v];
            }
        } else {
            e.air_g[col] = 0.0;
        }
        if (fd > 0.0) {
            e.flow[q] += fd;
            const double mf = t.ahu_c[q * 9 + 1];
            if (e.flow[q] > mf) e.flow[q] = mf;
            e.coolreq[q] += 1;
        }
    }
    e.pl[PL_TOTAL_REHEAT] = total_rw;
    if (t.internal_w_m2 > 0.0) {
        const double frac = comfort ? 1.0 : t.standby_frac;
        const double wpc = t.internal_w_m2 * t.cv_area * frac;
        for (int z = 0; z < nz; z++) e.zone_q[z] += wpc * (double)(t.zoff[z + 1] - t.zoff[z]);
    }
    if (t.occupant_w > 0.0)
        for (int z = 0; z < nz; z++) e.zone_q[z] += e.occV[z] * t.occupant_w;
    // the field step's inputs (input_q of a zone's room cells = its heat per cell)
    for (int z = 0; z < nz; z++) a.qz[(size_t)s * nz + z] = e.zone_q[z] / (double)(t.zoff[z + 1] - t.zoff[z]);
    for (int col = 0; col < t.k; col++) {
        a.g[(size_t)s * t.k + col] = e.air_g[col];
        a.airT[(size_t)s * t.k + col] = e.air_T[col];
    }
    a.amb[s] = ambient;
    a.hh[s] = t.h;
}

// sb_sim_step_post, sb_sim.c:459-521 (no convection)
__device__ void step_post(E& e) {
    const Tabs& t = *e.t;
    const double wcap = CP_W * RHO_W * total_flow_rate(e);
    const double total_rw = e.pl[PL_TOTAL_REHEAT];
    if (wcap > 0.0 && t.k > 0) {
        const double supply = e.pl[PL_BOILER_CUR];
        double rt = supply - total_rw / wcap;
        double at = e.coil[0];
        for (int c = 1; c < t.k; c++) {
            if (total_rw >= 0.0) {
                if (e.coil[c] < at) at = e.coil[c];
            } else {
                if (e.coil[c] > at) at = e.coil[c];
            }
        }
        const double lo = supply < at ? supply : at;
        const double hi = supply > at ? supply : at;
        if (rt < lo) rt = lo;
        if (rt > hi) rt = hi;
        e.pl[PL_BOILER_RET] = rt;
    }
    const double begin = e.pl[PL_BOILER_CUR], sp = e.pl[PL_BOILER_SP];
    const double dt_min = t.dt_sec / 60.0;
    if (sp > begin) {
        const double v = begin + t.boiler_c[2] * dt_min;
        e.pl[PL_BOILER_CUR] = v < sp ? v : sp;
    } else if (sp < begin) {
        const double v = begin - t.boiler_c[3] * dt_min;
        e.pl[PL_BOILER_CUR] = v > sp ? v : sp;
    } else {
        e.pl[PL_BOILER_CUR] = sp;
    }
    e.pl[PL_BOILER_DSTEP] = e.pl[PL_BOILER_CUR] - begin;
    e.ip[IP_STEP_INDEX] += 1;
}

// ------------------------------------------------------------------ observation
// obs_value + sb_obs (complete_port/csim/sb_obs.c:11-64) at calendar row j
__device__ double obs_value(const E& e, int kind, int idx, int id, int j) {
    const Tabs& t = *e.t;
    if (kind == 0) {
        switch (id) {
        case 0: return (double)e.coolreq[idx];
        case 1: return ahu_static(e, idx);
        case 2: return (e.run[idx] == 1) ? e.flow[idx] : 0.0;
        case 3: return e.sat[idx];
        case 4: return (double)e.run[idx];
        case 5: return e.flow[idx] / t.ahu_c[idx * 9 + 1];
        case 6: return (1.0 - e.recirc[idx]) * e.flow[idx];
        case 7: return (double)e.run[idx];
        case 8: return e.recirc[idx];
        default: return t.amb[j];
        }
    }
    if (kind == 1) {
        switch (id) {
        case 0: return e.reheat[idx];
        case 1: return e.damper[idx];
        case 2: return t.vav_c[idx * 9];
        case 3: return e.coolsp[idx];
        case 4: return e.heatsp[idx];
        default: return e.sensing[idx];
        }
    }
    const double dp = (e.ip[IP_PUMP_RUN] == 1) ? 9.8 * 1000.0 * e.pl[PL_PUMP_HEAD] / 100000.0 : 0.0;
    switch (id) {
    case 0: return dp;
    case 1: return e.pl[PL_BOILER_CUR];
    case 2: return dp;
    case 3: return (double)e.ip[IP_HWS_RUN];
    case 4: return (double)e.ip[IP_HWS_REQ];
    case 5: return (double)e.ip[IP_HWS_RUN];
    default: return e.pl[PL_BOILER_SP];
    }
}

// The observation prefix (the row's zero tail is written by puf_reset only).
__device__ void write_obs(const E& e, float* row, int j) {
    const Tabs& t = *e.t;
    for (int i = 0; i < t.n_dev; i++) {
        const double v = obs_value(e, t.f_kind[i], t.f_idx[i], t.f_id[i], j);
        const double sd = t.f_sd[i];
        const float v32 = (float)v;
        row[i] = (float)((sd > 0.0) ? ((double)v32 - t.f_mean[i]) / sd : 0.0);
    }
    const int na = t.n_aux;
    const double* aux = &t.aux_time[(size_t)j * (na - 1)];
    for (int c = 0; c < na - 1; c++) row[t.n_dev + c] = (float)aux[c];
    double occ = 0.0;
    for (int z = 0; z < t.nz; z++) occ += e.occV[z];
    row[t.n_dev + na - 1] = (float)(int)occ;
}

// ------------------------------------------------------------------ occupancy
// RandomizedArrivalDeparture chains in zone order, sb_occup.c:36-61
__device__ void occupancy_advance(E& e, int hour, int workday) {
    const Tabs& t = *e.t;
    for (int z = 0; z < t.nz; z++) {
        int cnt = 0;
        for (int q = 0; q < t.nassign; q++) {
            uint8_t* st = &e.occ_state[z * t.nassign + q];
            if (!workday) {
                *st = 0;
            } else if (*st == 0) {
                if (hour >= t.occ_ea && hour <= t.occ_la && mt_double(e) < t.p_arr) *st = 1;
            } else if (hour < t.occ_ed) {
                // stays at work
            } else if (hour >= t.occ_ld) {
                *st = 0;
            } else if (mt_double(e) < t.p_dep) {
                *st = 0;
            }
            cnt += *st;
        }
        e.occV[z] = (double)cnt;
    }
}

// ------------------------------------------------------------------ reward
// 3C reward at calendar row kv from the zone means of the new field
// (sb_reward.c:12-155; gas dissipation denominator precomputed on the host)
__device__ double reward(E& e, int kv) {
    const Tabs& t = *e.t;
    const double dt = t.dt_sec, inv_hour = 1.0 / 3600.0;
    const double ambient = t.amb[kv];
    const int hour = (int)t.rew_hour[kv], month = (int)t.rew_month[kv], wd = (int)t.rew_work[kv];
    double intake = 0.0, exhaust = 0.0, cooling = 0.0;
    for (int q = 0; q < t.na; q++) {
        e.wsum[q] = 0.0;
        e.atotal[q] = 0.0;
    }
    for (int v = 0; v < t.nv; v++) {
        double area = 0.0, wt = 0.0;
        for (int w = t.vz_off[v]; w < t.vz_off[v + 1]; w++) {
            const int z = t.vz_idx[w];
            area += t.zone_area[z];
            wt += e.avg_temp[z] * t.zone_area[z];
        }
        if (area > 0.0) {
            const int q = t.vav_ahu[v];
            e.wsum[q] += (wt / area) * area;
            e.atotal[q] += area;
        }
    }
    for (int q = 0; q < t.na; q++) {
        const double rc = e.wsum[q] / e.atotal[q];
        const double st = ahu_static(e, q);
        const double fe = t.ahu_c[q * 9 + 5];
        const double flow = (e.run[q] == 1) ? e.flow[q] : 0.0;
        intake += flow * st / fe;
        exhaust += flow * (1.0 - e.recirc[q]) * st / fe;
        const double mixed = e.recirc[q] * rc + (1.0 - e.recirc[q]) * ambient;
        const double sat = (mixed > e.sat[q] && e.run[q] == 1) ? e.sat[q] : mixed;
        cooling += flow * RHO_AIR * CP_AIR * (sat - mixed) / t.ahu_c[q * 9 + 4];
    }
    const double blower = intake + exhaust;
    const double tf = total_flow_rate(e);
    double gas_rate;
    {
        const double* c = t.boiler_c;
        const double rwt = e.pl[PL_BOILER_RET], bsp = e.pl[PL_BOILER_SP];
        const double supply = (bsp > rwt) ? bsp : rwt;
        const double flow = CP_W * RHO_W * tf * (supply - rwt);
        double diss = 0.0;
        if (supply >= ambient) diss = c[5] * 2.0 * PI_D * (supply - ambient) / t.gas_den;
        double tank = 0.0;
        if (dt > 0.0) tank = CP_W * RHO_W * c[7] * e.pl[PL_BOILER_DSTEP] / dt;
        const double tot = flow + diss + tank;
        gas_rate = tot > 0.0 ? tot : 0.0;
    }
    const double pump_e = tf * RHO_W * GRAV * e.pl[PL_PUMP_HEAD] / t.pump_eff;
    const double max_pph = t.rw[0], min_pph = t.rw[1], ref = t.rw[2];
    double total_occ = 0.0, cum = 0.0;
    for (int z = 0; z < t.nz; z++) {
        const double occ = e.occV[z];
        total_occ += occ;
        const double zt = e.avg_temp[z];
        const double hsp = t.heat_sp[kv], csp = t.cool_sp[kv];
        double dev = zt - csp;
        if (hsp - zt > dev) dev = hsp - zt;
        if (dev < 0.0) dev = 0.0;
        const double sh = (dev <= ref) ? dev / ref : 1.0 + ((dev - ref) / ref) * ((dev - ref) / ref);
        cum += max_pph * (1.0 - sh) * occ * dt * inv_hour;
    }
    const double max_prod = max_pph * total_occ * dt * inv_hour;
    const double min_prod = min_pph * total_occ * dt * inv_hour;
    double npr = 0.0;
    if (total_occ > 0.0 && (max_prod - min_prod) != 0.0) npr = (cum - min_prod) / (max_prod - min_prod) - 1.0;
    const double elec_rate = blower + fabs(cooling) + pump_e;
    const double price = wd ? t.elec_wk[hour] : t.elec_we[hour];
    const double crate = t.elec_co2[hour];
    const double elec_cost = price * fabs(elec_rate) * dt;
    const double elec_cost_max = price * t.rw[3] * dt;
    const double elec_carb = crate * fabs(elec_rate) * dt;
    const double elec_carb_max = crate * t.rw[3] * dt;
    const double gprice = t.gas_price[month - 1];
    const double g = gas_rate > 0.0 ? gas_rate : 0.0;
    const double gas_cost = gprice * g * dt;
    const double gas_cost_max = gprice * t.rw[4] * dt;
    const double gas_carb = t.gas_co2 * g * dt;
    const double gas_carb_max = t.gas_co2 * t.rw[4] * dt;
    const double den_e = elec_cost_max + gas_cost_max;
    const double nec = (den_e > 0.0) ? (elec_cost + gas_cost) / den_e : 0.0;
    const double den_c = elec_carb_max + gas_carb_max;
    const double ncar = (den_c > 0.0) ? (elec_carb + gas_carb) / den_c : 0.0;
    const double pw = t.rw[5], ew = t.rw[6], cw = t.rw[7];
    const double raw = npr * pw - nec * ew - ncar * cw;
    return raw / (pw + ew + cw);
}

// ------------------------------------------------------------------ reset
// sb_sim_reset (sb_sim.c:177-218; pump_head is not reset there) and puf_reset's
// occupancy and observation at the env's start (pufferlib_cpu_env.h:187-208);
// the field itself is re-initialised by fe_field_reset_kernel, its zone means
// come from the host (the same sums).
__device__ void env_reset(E& e, const Slot& sl, float* obs_row) {
    const Tabs& t = *e.t;
    for (int q = 0; q < t.na; q++) {
        const double* c = &t.ahu_c[q * 9];
        e.run[q] = (int)c[8];
        e.recirc[q] = c[0];
        e.sat[q] = c[6];
        e.fan[q] = c[7];
        e.flow[q] = 0.0;
        e.coolreq[q] = 0;
    }
    for (int v = 0; v < t.nv; v++) {
        const double* c = &t.vav_c[v * 9];
        e.damper[v] = c[7];
        e.reheat[v] = c[8];
        e.ratio[v] = 1.0;
        e.heatsp[v] = c[5];
        e.coolsp[v] = c[6];
        e.mode[v] = M_OFF;
        e.prev_valid[v] = e.dcmd_set[v] = e.rcmd_set[v] = 0;
        e.dcmd[v] = e.rcmd[v] = 0.0;
    }
    e.pl[PL_FFS] = 0.0;
    e.ip[IP_HWS_REQ] = 0;
    e.ip[IP_HWS_RUN] = e.ip[IP_PUMP_RUN] = 1;
    e.pl[PL_BOILER_SP] = t.boiler_c[0];
    e.pl[PL_BOILER_RET] = t.boiler_c[1];
    e.pl[PL_BOILER_CUR] = t.boiler_c[0];
    e.pl[PL_BOILER_DSTEP] = 0.0;
    for (int z = 0; z < t.nz; z++) e.avg_temp[z] = t.zm_init[z];
    vav_sensing(e);
    e.ip[IP_STEP_INDEX] = sl.start;
    occupancy_advance(e, (int)t.hour_m1[sl.start], (int)t.work_m1[sl.start]);
    e.ip[IP_STEP] = 0;
    write_obs(e, obs_row, sl.start);
    occupancy_advance(e, (int)t.occ_hour[sl.start], (int)t.occ_work[sl.start]);
}

// ------------------------------------------------------------------ kernels
__global__ void fe_pre_kernel(Args a) {
    const int s = (int)(blockIdx.x * blockDim.x + threadIdx.x);
    if (s >= a.G) return;
    E e = bind(a, s);
    const Slot sl = a.slots[s];
    if (a.mode == FE_RESET) {
        // puf_reset: every env from its start (the pump head, the occupant
        // chains and the occupancy stream persist, as in the CPU env), and the
        // observation row's zero tail
        float* row = a.obs + (size_t)sl.env * SB_OBS;
        env_reset(e, sl, row);
        for (int i = a.t.n_dev + a.t.n_aux; i < SB_OBS; i++) row[i] = 0.0f;
        e.ip[IP_STEPS_TOTAL] = 0;
        e.ip[IP_EPISODES] = 0;
        e.pl[PL_REW_SUM] = 0.0;
        return;
    }
    decode_apply(e, a.actions + (size_t)sl.env * SB_ACT);
    step_pre(e, a, s);
}

// Zone means of the new field: lane per (zone, env), envs of one zone on
// adjacent lanes (they read the same cells), the room's cells in order, eight
// loads in flight ahead of the sequential sum.
__global__ void fe_means_kernel(Args a) {
    const int x = (int)(blockIdx.x * blockDim.x + threadIdx.x);
    const int nz = a.t.nz;
    if (x >= a.G * nz) return;
    const int z = x / a.G, s = x % a.G;
    const size_t b = (size_t)(s / a.Gl), l = (size_t)(s % a.Gl);
    const double* T = a.T + b * (size_t)a.t.n_cvs * a.Gl + l;
    const int* cells = a.t.zcells;
    const int c0 = a.t.zoff[z], c1 = a.t.zoff[z + 1];
    double sum = 0.0;
    int q = c0;
    constexpr int U = 8;
    for (; q + U <= c1; q += U) {
        double v[U];
#pragma unroll
        for (int u = 0; u < U; u++) v[u] = T[(size_t)cells[q + u] * a.Gl];
#pragma unroll
        for (int u = 0; u < U; u++) sum += v[u];
    }
    for (; q < c1; q++) sum += T[(size_t)cells[q] * a.Gl];
    unsigned char* rec = a.state + (size_t)s * a.st.bytes;
    reinterpret_cast<double*>(rec + a.st.avg_temp)[z] = sum / (double)(c1 - c0);
}

__global__ void fe_post_kernel(Args a) {
    const int s = (int)(blockIdx.x * blockDim.x + threadIdx.x);
    if (s >= a.G) return;
    E e = bind(a, s);
    const Slot sl = a.slots[s];
    const Tabs& t = a.t;
    step_post(e);
    const int step = e.ip[IP_STEP] + 1;
    e.ip[IP_STEP] = step;
    const int j = sl.start + step;
    float* obs_row = a.obs + (size_t)sl.env * SB_OBS;
    write_obs(e, obs_row, j);
    occupancy_advance(e, (int)t.occ_hour[j], (int)t.occ_work[j]);
    const double rew = reward(e, j);
    const float r = (float)rew;
    // the first episode after puf_vec_create may be cut short (desync); a cut
    // episode is a truncation and stays out of the episode log
    // (complete_port/gpu/smart_buildings.cu:1990-1993, 2043)
    const bool first = e.ip[IP_FIRST_DONE] == 0;
    const bool cut = first && sl.first_steps < sl.max_steps;
    const bool done = step >= (first ? sl.first_steps : sl.max_steps);
    a.rewards[sl.env] = r * a.reward_scale;
    a.terminals[sl.env] = done ? 1.0f : 0.0f;
    e.pl[PL_REW_SUM] += rew;
    e.ip[IP_STEPS_TOTAL] += 1;
    a.reset_mask[s] = done ? 1 : 0;
    if (a.host_env && !cut) {
        Log* lg = reinterpret_cast<Log*>(reinterpret_cast<unsigned char*>(a.host_env) + (size_t)sl.env * a.env_stride
                                         + a.log_offset);
        float* lf = reinterpret_cast<float*>(lg);
        const float ret = __hip_atomic_load(&lg->episode_return, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) + r;
        const float m0 = __hip_atomic_load(&lg->reward_mean, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        const float mean = m0 + (r - m0) / (float)step;
        __hip_atomic_store(&lg->episode_return, ret, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        __hip_atomic_store(&lg->reward_mean, mean, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        if (done) {
            const float m = ret / (float)step;
            const float perf = __hip_atomic_load(&lf[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            const float score = __hip_atomic_load(&lf[1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            const float elen = __hip_atomic_load(&lf[3], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            const float nn = __hip_atomic_load(&lf[5], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            __hip_atomic_store(&lf[0], perf + m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            __hip_atomic_store(&lf[1], score + m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            __hip_atomic_store(&lf[3], elen + (float)step, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            __hip_atomic_store(&lf[5], nn + 1.0f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        }
    }
    if (done) {
        e.ip[IP_EPISODES] += 1;
        e.ip[IP_FIRST_DONE] = 1;
        env_reset(e, sl, obs_row);
    }
}

// Seeds every env's occupancy stream (puf_vec_create).
__global__ void fe_seed_kernel(Args a) {
    const int s = (int)(blockIdx.x * blockDim.x + threadIdx.x);
    if (s >= a.G) return;
    E e = bind(a, s);
    mt_seed(e, a.slots[s].occ_seed);
    e.pl[PL_PUMP_HEAD] = a.t.pump_head0;
    e.ip[IP_FIRST_DONE] = 0;
}

// Adds the group's f64 reward sum, env-steps and episodes since puf_reset to
// live[0..2], in env order.
__global__ void fe_live_kernel(Args a) {
    if (blockIdx.x != 0 || threadIdx.x != 0) return;
    double rs = 0.0, st = 0.0, ep = 0.0;
    for (int s = 0; s < a.G; s++) {
        const unsigned char* rec = a.state + (size_t)s * a.st.bytes;
        rs += reinterpret_cast<const double*>(rec + a.st.plant)[PL_REW_SUM];
        const int* ip = reinterpret_cast<const int*>(rec + a.st.ip);
        st += (double)ip[IP_STEPS_TOTAL];
        ep += (double)ip[IP_EPISODES];
    }
    a.live[0] += rs;
    a.live[1] += st;
    a.live[2] += ep;
}

// temp_init / mass_temp_init into the fields of the envs marked in reset_mask.
__global__ void fe_field_reset_kernel(double* T, double* M, int n_cvs, int n, int G, int Gl, const int* mask,
                                      const double* temp_init, const double* mass_init) {
    const size_t total = (size_t)G * (size_t)(n_cvs > n ? n_cvs : n);
    for (size_t x = (size_t)blockIdx.x * blockDim.x + threadIdx.x; x < total; x += (size_t)gridDim.x * blockDim.x) {
        const int s = (int)(x % G);
        const int p = (int)(x / G);
        if (!mask[s]) continue;
        const size_t b = (size_t)(s / Gl), l = (size_t)(s % Gl);
        if (p < n_cvs) T[(b * n_cvs + p) * Gl + l] = temp_init[p];
        if (p < n) M[(b * n + p) * Gl + l] = mass_init[p];
    }
}

}  // namespace sbe

// ---------------------------------------------------------------- launchers
extern "C" int sbe_launch(const sbe::Args* a, int which, hipStream_t s) {
    using namespace sbe;
    const int G = a->G;
    switch (which) {
    case 0: hipLaunchKernelGGL(fe_pre_kernel, dim3((G + 63) / 64), dim3(64), 0, s, *a); break;
    case 1: {
        const int n = G * a->t.nz;
        hipLaunchKernelGGL(fe_means_kernel, dim3((n + 63) / 64), dim3(64), 0, s, *a);
        break;
    }
    case 2: hipLaunchKernelGGL(fe_post_kernel, dim3((G + 63) / 64), dim3(64), 0, s, *a); break;
    case 3: hipLaunchKernelGGL(fe_seed_kernel, dim3((G + 63) / 64), dim3(64), 0, s, *a); break;
    case 4: hipLaunchKernelGGL(fe_live_kernel, dim3(1), dim3(64), 0, s, *a); break;
    default: return (int)hipErrorInvalidValue;
    }
    return (int)hipGetLastError();
}

extern "C" int sbe_launch_field_reset(double* T, double* M, int n_cvs, int n, int G, int Gl, const int* mask,
                                      const double* temp_init, const double* mass_init, hipStream_t s) {
    hipLaunchKernelGGL(sbe::fe_field_reset_kernel, dim3(1024), dim3(256), 0, s, T, M, n_cvs, n, G, Gl, mask,
                       temp_init, mass_init);
    return (int)hipGetLastError();
}
