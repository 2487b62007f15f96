// Field envs (field_env.h): the HVAC plant, actions, observation, occupancy,
// reward, convection and episode bookkeeping of FDM-scale scenarios.
//
// One 64-lane wavefront (a one-wavefront workgroup) per env. Its record is
// staged into LDS in one burst and stored back in one burst; every phase runs
// with lanes over the phase's entities (actions, VAVs, AHUs, air-side columns,
// zones, observation fields, occupant chains). The reference core's sums run
// in a fixed operand order (complete_port/csim/sb_sim.c, sb_reward.c), so each
// such sum belongs to one lane, which walks its operands in that order from
// LDS: an AHU's sums over its VAVs and columns, a zone's over its columns, the
// building-wide sums over VAVs, columns, AHUs and zones. This file is built
// with -ffp-contract=off: every product is rounded before it is added, as the
// reference core computes on x86-64, so a field scenario's env is
// bit-identical to the reference core's when its field step is (exact mode).
#include <hip/hip_runtime.h>

#include "sbenv.h"
#include "field_env.h"

namespace sbe {
namespace {

constexpr int W = 64;
constexpr double kRhoAir = 1.2;
constexpr double kCpAir = 1006.0;
constexpr double kRhoW = 1000.0;
constexpr double kCpW = 4180.0;
constexpr double kGrav = 9.8;
constexpr double kPaPerBar = 100000.0;
constexpr double kPi = 3.14159265358979323846;
enum { MODE_OFF = 0, MODE_HEAT = 1, MODE_COOL = 2, MODE_PASSIVE = 3 };

__device__ __forceinline__ int lane() { return (int)threadIdx.x; }
// one-wavefront workgroups: orders the wavefront's LDS accesses across lanes
__device__ __forceinline__ void wsync() { __syncthreads(); }

__device__ __forceinline__ unsigned long long ballot(bool p) { return __ballot(p); }
__device__ __forceinline__ int first_lane(unsigned long long m) { return __ffsll((long long)m) - 1; }
__device__ __forceinline__ uint32_t lane_u32(uint32_t v, int l) {
    return (uint32_t)__builtin_amdgcn_readlane((int)v, l);
}
__device__ __forceinline__ int below_me(unsigned long long m) {
    return __popcll(m & ((1ull << lane()) - 1ull));
}

// The env's staged record, typed.
struct Rec {
    double *recirc, *sat, *fan, *flow, *satv;
    double *damper, *reheat, *ratio, *heatsp, *coolsp, *dcmd, *rcmd, *sensing, *vav_area, *unres;
    double *avg_temp, *zone_q, *occV;
    double *air_g, *air_T, *coil, *rwen;
    double* pl;
    int *run, *coolreq, *mode, *prev_valid, *dcmd_set, *rcmd_set, *ip;
    float* ep;
    uint8_t* occ;
    uint32_t* mt;
};

__device__ Rec view(unsigned char* b, const StateLayout& s) {
    Rec r;
    auto d = [&](int o) { return reinterpret_cast<double*>(b + o); };
    auto i = [&](int o) { return reinterpret_cast<int*>(b + o); };
    r.recirc = d(s.recirc); r.sat = d(s.sat); r.fan = d(s.fan); r.flow = d(s.flow); r.satv = d(s.satv);
    r.damper = d(s.damper); r.reheat = d(s.reheat); r.ratio = d(s.ratio); r.heatsp = d(s.heatsp);
    r.coolsp = d(s.coolsp); r.dcmd = d(s.dcmd); r.rcmd = d(s.rcmd); r.sensing = d(s.sensing);
    r.vav_area = d(s.vav_area); r.unres = d(s.unres);
    r.avg_temp = d(s.avg_temp); r.zone_q = d(s.zone_q); r.occV = d(s.occV);
    r.air_g = d(s.air_g); r.air_T = d(s.air_T); r.coil = d(s.coil); r.rwen = d(s.rwen);
    r.pl = d(s.plant);
    r.run = i(s.run); r.coolreq = i(s.coolreq); r.mode = i(s.mode); r.prev_valid = i(s.prev_valid);
    r.dcmd_set = i(s.dcmd_set); r.rcmd_set = i(s.rcmd_set); r.ip = i(s.ip);
    r.ep = reinterpret_cast<float*>(b + s.ep);
    r.occ = b + s.occ_state;
    r.mt = reinterpret_cast<uint32_t*>(b + s.mt);
    return r;
}

// The record image [0, bytes) between HBM and LDS, 16 bytes per lane.
__device__ void stage_in(unsigned char* l, const unsigned char* g, int bytes) {
    const uint4* src = reinterpret_cast<const uint4*>(g);
    uint4* dst = reinterpret_cast<uint4*>(l);
    for (int i = lane(); i < (bytes >> 4); i += W) dst[i] = src[i];
    wsync();
}

__device__ void stage_out(unsigned char* g, const unsigned char* l, int bytes) {
    wsync();
    const uint4* src = reinterpret_cast<const uint4*>(l);
    uint4* dst = reinterpret_cast<uint4*>(g);
    for (int i = lane(); i < (bytes >> 4); i += W) dst[i] = src[i];
}

// ------------------------------------------------------------------ MT19937
// Matsumoto & Nishimura (1998), the generator behind numpy's legacy
// RandomState (complete_port/csim/sb_rng.c). A block of 624 raw words yields
// the next block by x'[i] = x[i + 397] ^ twist(x[i], x[i + 1]); the far term
// is a word of the old block for i < 227 and of the new block beyond, so the
// wavefront fills the new block in three dependent ranges.
__device__ __forceinline__ uint32_t mt_mix(uint32_t cur, uint32_t nxt, uint32_t far) {
    const uint32_t y = (cur & 0x80000000u) | (nxt & 0x7fffffffu);
    return far ^ (y >> 1) ^ ((y & 1u) ? 0x9908b0dfu : 0u);
}

__device__ __forceinline__ uint32_t mt_temper(uint32_t y) {
    y ^= y >> 11;
    y ^= (y << 7) & 0x9d2c5680u;
    y ^= (y << 15) & 0xefc60000u;
    y ^= y >> 18;
    return y;
}

// Each range: every lane's loads (at most four words per lane) issued before
// its first store, so a range costs one LDS round trip. `tw`, if given,
// receives the tempered words of the new block as well.
__device__ void mt_next_block(const uint32_t* src, uint32_t* dst, uint32_t* tw = nullptr) {
    auto range = [&](int lo, int hi, bool far_new) {
        uint32_t a[4], b[4], f[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int i = lo + u * W + lane();
            const bool ok = i < hi;
            const int ic = ok ? i : lo;
            a[u] = src[ic];
            b[u] = ic + 1 < SBE_MT_N ? src[ic + 1] : dst[0];
            f[u] = far_new ? dst[ic - 227] : src[ic + 397];
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int i = lo + u * W + lane();
            if (i < hi) {
                const uint32_t x = mt_mix(a[u], b[u], f[u]);
                dst[i] = x;
                if (tw) tw[i] = mt_temper(x);
            }
        }
        wsync();
    };
    range(0, 227, false);
    range(227, 454, true);
    range(454, SBE_MT_N, true);
}

// numpy's random_sample from two consecutive words (sb_rng.c:39-43)
__device__ __forceinline__ double mt_unit(uint32_t a, uint32_t b) {
    return ((a >> 5) * 67108864.0 + (b >> 6)) / 9007199254740992.0;
}

// ------------------------------------------------------------------ decode
// Trainer row -> native command of each action (the CPU env's clamp,
// complete_port/pufferlib_cpu_env.h:218-232; sb_decode_native, sb_sim.c:557-576:
// continuous in float32 op by op, discrete in f64), then the command applied
// to its target (sb_sim_apply_native, sb_sim.c:220-244). Lanes over actions;
// an action the host marked as overwritten by a later one on the same target
// is decoded but not applied.
__device__ void decode_apply(const Tabs& t, Rec& r, const float* row) {
    for (int i = lane(); i < t.n_act; i += W) {
        const double mn = t.act_mn[i], mx = t.act_mx[i], mnr = t.act_mnr[i], mxr = t.act_mxr[i];
        const float x = row[t.act_col[i]];
        double v;
        if (t.act_disc[i]) {
            const double m = ((double)x == 1.0) ? 1.0 : -1.0;
            v = (m - mnr) / (mxr - mnr) * (mx - mn) + mn;
        } else {
            double c = (double)x;
            if (c > 1.0) c = 1.0;
            else if (c < -1.0) c = -1.0;
            const float f = (float)c;
            const float in = (float)(mxr - mnr), out = (float)(mx - mn);
            v = (double)((f - (float)mnr) / in * out + (float)mn);
        }
        if (!t.act_live[i]) continue;
        const int tg = t.act_tgt[i];
        const int kind = tg & 15, act = (tg >> 4) & 15, idx = tg >> 8;
        if (kind == 0) {
            if (act == 0) r.sat[idx] = v;
            else if (act == 1) r.fan[idx] = v;
            else if (act == 2) {
                const double hi = t.ahu_c[idx * 9 + 3];
                r.recirc[idx] = v < 0.0 ? 0.0 : (v > hi ? hi : v);
            } else r.run[idx] = (v == 1.0) ? 1 : 0;
        } else if (kind == 1) {
            const double c = v < 0.0 ? 0.0 : (v > 1.0 ? 1.0 : v);
            if (act == 0) {
                r.dcmd[idx] = c;
                r.dcmd_set[idx] = 1;
            } else {
                r.rcmd[idx] = c;
                r.rcmd_set[idx] = 1;
            }
        } else {
            if (act == 0) r.pl[PL_BOILER_SP] = v;
            else if (act == 1) r.pl[PL_PUMP_HEAD] = v / (kGrav * kRhoW / kPaPerBar);
            else {
                const int on = (v == 1.0) ? 1 : 0;
                r.ip[IP_HWS_RUN] = on;
                r.ip[IP_PUMP_RUN] = on;
            }
        }
    }
    wsync();
}

// ------------------------------------------------------------------ HVAC
__device__ __forceinline__ double static_pressure(const Tabs& t, const Rec& r, int a) {
    if (r.run[a] != 1) return 0.0;
    const double sp = r.fan[a], lo = t.ahu_c[a * 9 + 2];
    return sp > lo ? sp : lo;
}

// hot-water loop flow (sb_sim.c:278-287)
__device__ __forceinline__ double water_flow(const Tabs& t, const Rec& r) {
    const double ff = r.pl[PL_FFS];
    const double dp = (r.ip[IP_PUMP_RUN] != 1) ? 0.0 : kGrav * kRhoW * r.pl[PL_PUMP_HEAD] / kPaPerBar;
    return ff * sqrt(dp / (1.0 + ff * ff * t.header_res)) / 3600.0;
}

// thermostat mode of a VAV at sensed temperature zt (sb_sim.c:316-338)
__device__ __forceinline__ int thermostat(int cur, bool comfort, bool prev_comfort, bool valid, double zt,
                                          double hsp, double csp) {
    const bool passive = !comfort && ((valid && prev_comfort) || (cur == MODE_PASSIVE && zt > hsp && zt < csp));
    if (passive) return MODE_PASSIVE;
    const double mid = 0.5 * (csp - hsp) + hsp;
    if (zt < hsp) return MODE_HEAT;
    if (zt > csp) return MODE_COOL;
    if (zt < mid && cur == MODE_HEAT) return MODE_HEAT;
    if (zt > mid && cur == MODE_COOL) return MODE_COOL;
    return MODE_OFF;
}

// area-weighted mean of a VAV's zones (sb_sim.c:163-175): its area and the
// weighted sum, both in the VAV's zone order
__device__ __forceinline__ void vav_zone_sums(const Tabs& t, const double* zmean, int v, double& area, double& wt) {
    area = 0.0;
    wt = 0.0;
    for (int q = t.vz_off[v]; q < t.vz_off[v + 1]; q++) {
        const int z = t.vz_idx[q];
        area += t.zone_area[z];
        wt += zmean[z] * t.zone_area[z];
    }
}

// sb_sim_step_pre (sb_sim.c:357-457) from the zone means in the record, the
// boiler update of sb_sim_step_post (:489-521; it reads nothing the field
// step writes) and the field step's inputs of slot s. `scr` is f64 scratch
// of at least na + k.
__device__ void hvac_pre(const Tabs& t, Rec& r, double* scr, const Args& a, int s) {
    const int kk = r.ip[IP_STEP_INDEX];
    const double ambient = t.amb[kk];
    const bool comfort = t.comfort[kk] != 0.0;
    const bool prev_comfort = kk > 0 && t.comfort[kk - 1] != 0.0;
    const double hsp = t.heat_sp[kk], csp = t.cool_sp[kk];
    const int na = t.na, nv = t.nv, nz = t.nz, k = t.k;
    double* demand = scr;          // [na]
    double* fdem = scr + na;       // [k]

    // VAVs: sensed temperature, thermostat, damper and reheat settings
    for (int v = lane(); v < nv; v += W) {
        double area, wt;
        vav_zone_sums(t, r.avg_temp, v, area, wt);
        r.vav_area[v] = area;
        if (area <= 0.0) {
            r.sensing[v] = 0.0;
            continue;
        }
        const double zt = wt / area;
        r.sensing[v] = zt;
        const double* c = &t.vav_c[v * 9];
        const int md = thermostat(r.mode[v], comfort, prev_comfort, r.prev_valid[v] != 0, zt, hsp, csp);
        r.heatsp[v] = hsp;
        r.coolsp[v] = csp;
        r.mode[v] = md;
        r.prev_valid[v] = 1;
        double dmp = (md == MODE_HEAT || md == MODE_COOL) ? 1.0 : c[2];
        double rht = (md == MODE_HEAT) ? 1.0 : 0.0;
        if (r.dcmd_set[v]) dmp = r.dcmd[v];
        if (r.rcmd_set[v]) rht = r.rcmd[v];
        r.damper[v] = dmp > c[2] ? dmp : c[2];
        r.reheat[v] = rht;
    }
    wsync();
    // AHUs (one lane each, its VAVs ascending): return-air mean and supply
    // temperature; lane 0 meanwhile sums the flow factors over every VAV
    for (int q = lane(); q < na; q += W) {
        double ws = 0.0, at = 0.0;
        for (int i = t.av_off[q]; i < t.av_off[q + 1]; i++) {
            const int v = t.av_idx[i];
            if (r.vav_area[v] > 0.0) {
                ws += r.sensing[v] * r.vav_area[v];
                at += r.vav_area[v];
            }
        }
        const double rt = ws / at;
        const double mixed = r.recirc[q] * rt + (1.0 - r.recirc[q]) * ambient;
        r.satv[q] = (mixed > r.sat[q] && r.run[q] == 1) ? r.sat[q] : mixed;
    }
    if (lane() == 0) {
        double ffs = 0.0;
        for (int v = 0; v < nv; v++) ffs += r.reheat[v] * t.vav_c[v * 9 + 1];
        r.pl[PL_FFS] = ffs;
        r.ip[IP_HWS_REQ] = nv;
    }
    // VAVs: unrestricted flow at the new damper (sb_sim.c:267-276)
    for (int v = lane(); v < nv; v += W) {
        const double* c = &t.vav_c[v * 9];
        const double d = r.damper[v] * c[0] * sqrt(static_pressure(t, r, t.vav_ahu[v]) / c[4]);
        r.unres[v] = d > 0.00001 ? d : 0.00001;
    }
    wsync();
    // AHUs: demand over all their VAVs in order; VAVs: flow ratio
    for (int q = lane(); q < na; q += W) {
        double dm = 0.0;
        for (int i = t.av_off[q]; i < t.av_off[q + 1]; i++) dm += r.unres[t.av_idx[i]];
        demand[q] = dm;
    }
    wsync();
    for (int v = lane(); v < nv; v += W) {
        const int q = t.vav_ahu[v];
        const double d = demand[q];
        double ratio = 1.0;
        if (d > 0.0) {
            const double x = t.ahu_c[q * 9 + 1] / d;
            ratio = x < 1.0 ? x : 1.0;
        }
        r.ratio[v] = ratio;
    }
    wsync();
    // coupled columns: supply temperature, reheat energy (sb_sim.c:289-314),
    // air-side conductance; a column whose VAV serves no zone area keeps its
    // coil temperature
    const double tf = water_flow(t, r);
    const double iwt = r.pl[PL_BOILER_CUR];
    const double ffs = r.pl[PL_FFS];
    for (int col = lane(); col < k; col += W) {
        const int v = t.coupled[col];
        if (r.vav_area[v] <= 0.0) {
            r.air_g[col] = 0.0;
            r.air_T[col] = 0.0;
            r.rwen[col] = 0.0;
            fdem[col] = 0.0;
            continue;
        }
        const double* c = &t.vav_c[v * 9];
        const double sat = r.satv[t.vav_ahu[v]];
        const double fd = r.unres[v] * r.ratio[v];
        double eff = 0.0;
        const double air_cap = kCpAir * kRhoAir * fd;
        if (air_cap > 0.0) {
            const double wflow = (ffs == 0.0) ? 0.0 : tf * ((r.reheat[v] * c[1]) / ffs);
            const double water_cap = kCpW * kRhoW * wflow;
            eff = water_cap / air_cap;
            if (eff > 1.0) eff = 1.0;
            const double gap = iwt - sat;
            if (gap > 0.0) {
                const double headroom = c[3] - sat;
                if (headroom <= 0.0) eff = 0.0;
                else {
                    const double hr = headroom / gap;
                    eff = eff < hr ? eff : hr;
                }
            }
        }
        r.air_T[col] = sat;
        r.coil[col] = sat;
        r.rwen[col] = eff * kCpAir * kRhoAir * fd * (iwt - sat);
        r.air_g[col] = (r.damper[v] > 0.0 && c[0] > 0.0) ? fd * kRhoAir * kCpAir : 0.0;
        fdem[col] = fd;
    }
    wsync();
    // AHUs: delivered flow (clamped to the maximum after every column, as the
    // reference accumulates it) and cooling requests, over their columns in order
    for (int q = lane(); q < na; q += W) {
        const double mf = t.ahu_c[q * 9 + 1];
        double f = 0.0;
        int req = 0;
        for (int i = t.ac_off[q]; i < t.ac_off[q + 1]; i++) {
            const int col = t.ac_idx[i];
            const double fd = fdem[col];
            if (r.vav_area[t.coupled[col]] > 0.0 && fd > 0.0) {
                f += fd;
                if (f > mf) f = mf;
                req++;
            }
        }
        r.flow[q] = f;
        r.coolreq[q] = req;
    }
    // zones: reheat share of the columns that heat them, in column order, then
    // internal and occupant gains, per room cell (sb_sim.c:416-457)
    const double wpc = t.internal_w_m2 * t.cv_area * (comfort ? 1.0 : t.standby_frac);
    for (int z = lane(); z < nz; z += W) {
        double q = 0.0;
        for (int i = t.zc_off[z]; i < t.zc_off[z + 1]; i++) {
            const int col = t.zc_idx[i];
            const int v = t.coupled[col];
            if (r.vav_area[v] > 0.0 && r.damper[v] > 0.0 && t.vav_c[v * 9] > 0.0)
                q += r.rwen[col] * t.zone_area[z] / r.vav_area[v];
        }
        const double cells = (double)(t.zoff[z + 1] - t.zoff[z]);
        if (t.internal_w_m2 > 0.0) q += wpc * cells;
        if (t.occupant_w > 0.0) q += r.occV[z] * t.occupant_w;
        r.zone_q[z] = q;
        a.qz[(size_t)s * nz + z] = q / cells;
    }
    // coil extremes for the boiler's return temperature (exact in any order)
    double cmin = 1.0e308, cmax = -1.0e308;
    for (int col = lane(); col < k; col += W) {
        cmin = fmin(cmin, r.coil[col]);
        cmax = fmax(cmax, r.coil[col]);
    }
    for (int o = 32; o > 0; o >>= 1) {
        cmin = fmin(cmin, __shfl_xor(cmin, o));
        cmax = fmax(cmax, __shfl_xor(cmax, o));
    }
    for (int col = lane(); col < k; col += W) {
        a.g[(size_t)s * k + col] = r.air_g[col];
        a.airT[(size_t)s * k + col] = r.air_T[col];
    }
    if (lane() == 0) {
        double total = 0.0;
        for (int col = 0; col < k; col++)
            if (r.vav_area[t.coupled[col]] > 0.0) total += r.rwen[col];
        r.pl[PL_TOTAL_REHEAT] = total;
        // boiler return temperature and setpoint ramp (sb_sim.c:491-521)
        const double wcap = kCpW * kRhoW * tf;
        if (wcap > 0.0 && k > 0) {
            const double supply = r.pl[PL_BOILER_CUR];
            double rt = supply - total / wcap;
            const double at = total >= 0.0 ? cmin : cmax;
            const double lo = supply < at ? supply : at, hi = supply > at ? supply : at;
            if (rt < lo) rt = lo;
            if (rt > hi) rt = hi;
            r.pl[PL_BOILER_RET] = rt;
        }
        const double begin = r.pl[PL_BOILER_CUR], sp = r.pl[PL_BOILER_SP];
        const double dt_min = t.dt_sec / 60.0;
        double cur = sp;
        if (sp > begin) {
            const double x = begin + t.boiler_c[2] * dt_min;
            cur = x < sp ? x : sp;
        } else if (sp < begin) {
            const double x = begin - t.boiler_c[3] * dt_min;
            cur = x > sp ? x : sp;
        }
        r.pl[PL_BOILER_CUR] = cur;
        r.pl[PL_BOILER_DSTEP] = cur - begin;
        r.ip[IP_STEP_INDEX] = kk + 1;
        a.amb[s] = ambient;
        a.hh[s] = t.h;
    }
    wsync();
}

// ------------------------------------------------------------------ observation
// One observed device value (sb_obs.c:11-47) at calendar row j.
__device__ double device_value(const Tabs& t, const Rec& r, int kind, int idx, int id, int j) {
    if (kind == 0) {
        switch (id) {
        case 0: return (double)r.coolreq[idx];
        case 1: return static_pressure(t, r, idx);
        case 2: return (r.run[idx] == 1) ? r.flow[idx] : 0.0;
        case 3: return r.sat[idx];
        case 4: return (double)r.run[idx];
        case 5: return r.flow[idx] / t.ahu_c[idx * 9 + 1];
        case 6: return (1.0 - r.recirc[idx]) * r.flow[idx];
        case 7: return (double)r.run[idx];
        case 8: return r.recirc[idx];
        default: return t.amb[j];
        }
    }
    if (kind == 1) {
        switch (id) {
        case 0: return r.reheat[idx];
        case 1: return r.damper[idx];
        case 2: return t.vav_c[idx * 9];
        case 3: return r.coolsp[idx];
        case 4: return r.heatsp[idx];
        default: return r.sensing[idx];
        }
    }
    const double dp = (r.ip[IP_PUMP_RUN] == 1) ? 9.8 * 1000.0 * r.pl[PL_PUMP_HEAD] / 100000.0 : 0.0;
    switch (id) {
    case 0: return dp;
    case 1: return r.pl[PL_BOILER_CUR];
    case 2: return dp;
    case 3: return (double)r.ip[IP_HWS_RUN];
    case 4: return (double)r.ip[IP_HWS_REQ];
    case 5: return (double)r.ip[IP_HWS_RUN];
    default: return r.pl[PL_BOILER_SP];
    }
}

// The observation prefix at calendar row j (sb_obs.c:49-64): lanes over the
// device fields (float32-quantised, then normalised), the time features and
// the occupant count (integers: any summation order is exact).
__device__ void write_obs(const Tabs& t, const Rec& r, float* row, int j) {
    for (int i = lane(); i < t.n_dev; i += W) {
        const double v = device_value(t, r, t.f_kind[i], t.f_idx[i], t.f_id[i], j);
        const double sd = t.f_sd[i];
        const float v32 = (float)v;
        row[i] = (float)((sd > 0.0) ? ((double)v32 - t.f_mean[i]) / sd : 0.0);
    }
    const int nx = t.n_aux - 1;
    for (int c = lane(); c < nx; c += W) row[t.n_dev + c] = (float)t.aux_time[(size_t)j * nx + c];
    double occ = 0.0;
    for (int z = lane(); z < t.nz; z += W) occ += r.occV[z];
    for (int o = 32; o > 0; o >>= 1) occ += __shfl_xor(occ, o);
    if (lane() == 0) row[t.n_dev + nx] = (float)(int)occ;
}

// ------------------------------------------------------------------ occupancy
// One interval of the occupant chains (sb_occup.c:36-61) at (hour, workday).
// Chain c = z * nassign + q draws one numpy double (two words) when it is
// away inside the arrival window or at work inside the departure window; the
// draws are taken from the stream in chain order, so a chunk of 64 chains
// places its draws by a wavefront prefix sum. `blk` is LDS scratch of 624 words.
__device__ void occupancy(const Tabs& t, Rec& r, int hour, int workday, uint32_t* blk) {
    const int nch = t.nz * t.nassign;
    int idx = r.ip[IP_MT_IDX];
    for (int base = 0; base < nch; base += W) {
        const int c = base + lane();
        const bool ok = c < nch;
        int st = ok ? r.occ[c] : 0;
        const bool arrive = st == 0 && hour >= t.occ_ea && hour <= t.occ_la;
        const bool depart = st == 1 && hour >= t.occ_ed && hour < t.occ_ld;
        const bool draw = ok && workday && (arrive || depart);
        const unsigned long long m = ballot(draw);
        const int cnt = __popcll(m);
        const int p0 = idx + 2 * below_me(m), p1 = p0 + 1;
        uint32_t w0 = 0, w1 = 0;
        if (draw && p0 < SBE_MT_N) w0 = r.mt[p0];
        if (draw && p1 < SBE_MT_N) w1 = r.mt[p1];
        if (idx + 2 * cnt > SBE_MT_N) {
            // the chunk's draws run past the block: the next block, in place
            mt_next_block(r.mt, blk);
            for (int i = lane(); i < SBE_MT_N; i += W) r.mt[i] = blk[i];
            wsync();
            if (draw && p0 >= SBE_MT_N) w0 = r.mt[p0 - SBE_MT_N];
            if (draw && p1 >= SBE_MT_N) w1 = r.mt[p1 - SBE_MT_N];
            idx -= SBE_MT_N;
        }
        idx += 2 * cnt;
        if (ok) {
            if (!workday) st = 0;
            else if (draw) {
                const double u = mt_unit(mt_temper(w0), mt_temper(w1));
                if (arrive) st = (u < t.p_arr) ? 1 : 0;
                else st = (u < t.p_dep) ? 0 : 1;
            } else if (st == 1 && hour >= t.occ_ld) st = 0;
            r.occ[c] = (uint8_t)st;
        }
        wsync();
    }
    for (int z = lane(); z < t.nz; z += W) {
        int cnt = 0;
        for (int q = 0; q < t.nassign; q++) cnt += r.occ[z * t.nassign + q];
        r.occV[z] = (double)cnt;
    }
    if (lane() == 0) r.ip[IP_MT_IDX] = idx;
    wsync();
}

// ------------------------------------------------------------------ reward
// 3C reward at calendar row kv from the zone means of the new field
// (sb_reward.c:31-155; the tank dissipation's denominator precomputed on the
// host), and in `dg` (lane 0) the reference GPU env's 8 per-step diagnostics
// (complete_port/gpu/sb_gpu_kernels.cuh:1409-1473). `scr` is f64 scratch of
// at least nv + 3 na + 2 nz.
__device__ double reward(const Tabs& t, Rec& r, double* scr, int kv, double (&dg)[8]) {
    const int na = t.na, nv = t.nv, nz = t.nz;
    double* vwt = scr;                 // [nv] VAV mean * area (area > 0)
    double* ahu_terms = scr + nv;      // [3 na] intake, exhaust, cooling
    double* zterm = ahu_terms + 3 * na;   // [nz] productivity term
    double* zdev = zterm + nz;            // [nz] deviation from the comfort band
    const double dt = t.dt_sec, inv_hour = 1.0 / 3600.0;
    const double ambient = t.amb[kv];
    for (int v = lane(); v < nv; v += W) {
        double area, wt;
        vav_zone_sums(t, r.avg_temp, v, area, wt);
        vwt[v] = (area > 0.0) ? (wt / area) * area : 0.0;
    }
    const double max_pph = t.rw[0], min_pph = t.rw[1], ref = t.rw[2];
    const double hsp = t.heat_sp[kv], csp = t.cool_sp[kv];
    for (int z = lane(); z < nz; z += W) {
        const double zt = r.avg_temp[z];
        double dev = zt - csp;
        if (hsp - zt > dev) dev = hsp - zt;
        if (dev < 0.0) dev = 0.0;
        const double sh = (dev <= ref) ? dev / ref : 1.0 + ((dev - ref) / ref) * ((dev - ref) / ref);
        zterm[z] = max_pph * (1.0 - sh) * r.occV[z] * dt * inv_hour;
        zdev[z] = dev;
    }
    wsync();
    for (int q = lane(); q < na; q += W) {
        double ws = 0.0, at = 0.0;
        for (int i = t.av_off[q]; i < t.av_off[q + 1]; i++) {
            const int v = t.av_idx[i];
            if (r.vav_area[v] > 0.0) {
                ws += vwt[v];
                at += r.vav_area[v];
            }
        }
        const double rc = ws / at;
        const double st = static_pressure(t, r, q);
        const double fe = t.ahu_c[q * 9 + 5];
        const double fl = (r.run[q] == 1) ? r.flow[q] : 0.0;
        const double mixed = r.recirc[q] * rc + (1.0 - r.recirc[q]) * ambient;
        const double sat = (mixed > r.sat[q] && r.run[q] == 1) ? r.sat[q] : mixed;
        ahu_terms[3 * q] = fl * st / fe;
        ahu_terms[3 * q + 1] = fl * (1.0 - r.recirc[q]) * st / fe;
        ahu_terms[3 * q + 2] = fl * kRhoAir * kCpAir * (sat - mixed) / t.ahu_c[q * 9 + 4];
    }
    wsync();
    double rew = 0.0;
    if (lane() == 0) {
        double intake = 0.0, exhaust = 0.0, cooling = 0.0;
        for (int q = 0; q < na; q++) {
            intake += ahu_terms[3 * q];
            exhaust += ahu_terms[3 * q + 1];
            cooling += ahu_terms[3 * q + 2];
        }
        double total_occ = 0.0, cum = 0.0, dsum = 0.0, dmax = 0.0;
        int n_oob = 0;
        for (int z = 0; z < nz; z++) {
            total_occ += r.occV[z];
            cum += zterm[z];
            dsum += zdev[z];
            if (zdev[z] > dmax) dmax = zdev[z];
            if (zdev[z] > 0.0) n_oob++;
        }
        const double tf = water_flow(t, r);
        const double* bc = t.boiler_c;
        const double rwt = r.pl[PL_BOILER_RET], bsp = r.pl[PL_BOILER_SP];
        const double supply = (bsp > rwt) ? bsp : rwt;
        double diss = 0.0;
        if (supply >= ambient) diss = bc[5] * 2.0 * kPi * (supply - ambient) / t.gas_den;
        const double tank = (dt > 0.0) ? kCpW * kRhoW * bc[7] * r.pl[PL_BOILER_DSTEP] / dt : 0.0;
        const double gtot = kCpW * kRhoW * tf * (supply - rwt) + diss + tank;
        const double gas = gtot > 0.0 ? gtot : 0.0;
        const double pump_e = tf * kRhoW * kGrav * r.pl[PL_PUMP_HEAD] / t.pump_eff;
        const double max_prod = max_pph * total_occ * dt * inv_hour;
        const double min_prod = min_pph * total_occ * dt * inv_hour;
        double npr = 0.0;
        if (total_occ > 0.0 && (max_prod - min_prod) != 0.0) npr = (cum - min_prod) / (max_prod - min_prod) - 1.0;
        const int hour = (int)t.rew_hour[kv], month = (int)t.rew_month[kv];
        const double elec = (intake + exhaust) + fabs(cooling) + pump_e;
        const double price = t.rew_work[kv] ? t.elec_wk[hour] : t.elec_we[hour];
        const double crate = t.elec_co2[hour], gprice = t.gas_price[month - 1];
        const double den_e = price * t.rw[3] * dt + gprice * t.rw[4] * dt;
        const double nec = (den_e > 0.0) ? (price * fabs(elec) * dt + gprice * gas * dt) / den_e : 0.0;
        const double den_c = crate * t.rw[3] * dt + t.gas_co2 * t.rw[4] * dt;
        const double ncar = (den_c > 0.0) ? (crate * fabs(elec) * dt + t.gas_co2 * gas * dt) / den_c : 0.0;
        const double pw = t.rw[5], ew = t.rw[6], cw = t.rw[7];
        rew = (npr * pw - nec * ew - ncar * cw) / (pw + ew + cw);
        dg[0] = npr;
        dg[1] = nec;
        dg[2] = ncar;
        dg[3] = nz > 0 ? dsum / nz : 0.0;
        dg[4] = dmax;
        dg[5] = nz > 0 ? (double)n_oob / nz : 0.0;
        dg[6] = fabs(elec) * dt / 3.6e6;
        dg[7] = gas * dt / 3.6e6;
    }
    wsync();
    return rew;
}

// ------------------------------------------------------------------ reset
// sb_sim_reset (sb_sim.c:177-218; the pump head, coil temperatures and the
// random streams persist) with the zone means of temp_init from the host, then
// puf_reset's occupancy prime, observation and first interval at the env's
// start (complete_port/pufferlib_cpu_env.h:187-208). `field`: also write
// temp_init / mass_temp_init into the env's field (an auto-reset; puf_reset
// initialises the whole group's field itself).
__device__ void env_reset(const Tabs& t, Rec& r, const Slot& sl, float* obs_row, uint32_t* blk, const Args& a,
                          int s, bool field) {
    for (int q = lane(); q < t.na; q += W) {
        const double* c = &t.ahu_c[q * 9];
        r.run[q] = (int)c[8];
        r.recirc[q] = c[0];
        r.sat[q] = c[6];
        r.fan[q] = c[7];
        r.flow[q] = 0.0;
        r.coolreq[q] = 0;
    }
    for (int z = lane(); z < t.nz; z += W) r.avg_temp[z] = t.zm_init[z];
    for (int v = lane(); v < t.nv; v += W) {
        const double* c = &t.vav_c[v * 9];
        r.damper[v] = c[7];
        r.reheat[v] = c[8];
        r.ratio[v] = 1.0;
        r.heatsp[v] = c[5];
        r.coolsp[v] = c[6];
        r.mode[v] = MODE_OFF;
        r.prev_valid[v] = 0;
        r.dcmd_set[v] = 0;
        r.rcmd_set[v] = 0;
        r.dcmd[v] = 0.0;
        r.rcmd[v] = 0.0;
    }
    if (lane() == 0) {
        r.pl[PL_FFS] = 0.0;
        r.ip[IP_HWS_REQ] = 0;
        r.ip[IP_HWS_RUN] = 1;
        r.ip[IP_PUMP_RUN] = 1;
        r.pl[PL_BOILER_SP] = t.boiler_c[0];
        r.pl[PL_BOILER_RET] = t.boiler_c[1];
        r.pl[PL_BOILER_CUR] = t.boiler_c[0];
        r.pl[PL_BOILER_DSTEP] = 0.0;
        r.ip[IP_STEP_INDEX] = sl.start;
        r.ip[IP_STEP] = 0;
    }
    wsync();
    for (int v = lane(); v < t.nv; v += W) {
        double area, wt;
        vav_zone_sums(t, r.avg_temp, v, area, wt);
        r.vav_area[v] = area;
        r.sensing[v] = (area > 0.0) ? wt / area : 0.0;
    }
    wsync();
    occupancy(t, r, (int)t.hour_m1[sl.start], (int)t.work_m1[sl.start], blk);
    write_obs(t, r, obs_row, sl.start);
    wsync();
    occupancy(t, r, (int)t.occ_hour[sl.start], (int)t.occ_work[sl.start], blk);
    if (field) {
        const size_t b = (size_t)(s / a.Gl), l = (size_t)(s % a.Gl), Gl = (size_t)a.Gl;
        double* T = a.T + b * (size_t)t.n_cvs * Gl + l;
        for (int p = lane(); p < t.n_cvs; p += W) T[(size_t)p * Gl] = t.temp_init[p];
        double* M = a.M + b * (size_t)t.n_solved * Gl + l;
        for (int q = lane(); q < t.n_solved; q += W) M[(size_t)q * Gl] = t.mass_init[q];
    }
}

// A whole episode's sums added to the env's host-visible Log (the reference
// GPU env's finalize_k, complete_port/gpu/smart_buildings.cu:2002-2036), each
// field read and written with system-scope accesses (the trainer may clear
// the Log between steps). ep: EP_* running sums, st: the episode's length.
__device__ void log_episode(const Args& a, int env, const float* ep, int st) {
    float* f = reinterpret_cast<float*>(reinterpret_cast<unsigned char*>(a.host_env) + (size_t)env * a.env_stride
                                        + a.log_offset);
    const float s = (float)st;
    const float mean = ep[EP_RET] / s;
    const float add[13] = {mean, mean, ep[EP_RET], s,
                           ep[EP_PART + 3] / s, ep[EP_WORST], ep[EP_PART + 5] / s,
                           ep[EP_PART + 0] / s, ep[EP_PART + 1] / s, ep[EP_PART + 2] / s,
                           ep[EP_PART + 6], ep[EP_PART + 7], 1.0f};
    // every read issued before the first write: one round trip over the host link
    float x[13];
#pragma unroll
    for (int i = 0; i < 13; i++) x[i] = __hip_atomic_load(&f[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
#pragma unroll
    for (int i = 0; i < 13; i++) __hip_atomic_store(&f[i], x[i] + add[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
static_assert(sizeof(Log) == 52 && offsetof(Log, n) == 48, "log_episode writes the reference GPU env's Log");

}  // namespace

// ------------------------------------------------------------------ kernels
// Before the field step: puf_reset of every env (mode FE_RESET), or decode,
// pre-step and boiler update with the field step's inputs.
__global__ __launch_bounds__(W) void fe_pre_kernel(Args a) {
    const int s = (int)blockIdx.x;
    if (s >= a.G) return;
    extern __shared__ __align__(16) unsigned char lds[];
    unsigned char* g = a.state + (size_t)s * a.st.record;
    stage_in(lds, g, a.st.bytes);
    Rec r = view(lds, a.st);
    double* scr = reinterpret_cast<double*>(lds + a.st.bytes);
    const Slot sl = a.slots[s];
    if (a.mode == FE_RESET) {
        float* row = a.obs + (size_t)sl.env * SB_OBS;
        uint32_t* blk = reinterpret_cast<uint32_t*>(scr);
        env_reset(a.t, r, sl, row, blk, a, s, false);
        for (int i = a.t.n_dev + a.t.n_aux + lane(); i < SB_OBS; i += W) row[i] = 0.0f;
        if (lane() == 0) {
            r.ip[IP_STEPS_TOTAL] = 0;
            r.ip[IP_EPISODES] = 0;
            r.pl[PL_REW_SUM] = 0.0;
            r.pl[PL_DEV_SUM] = 0.0;
            for (int i = 0; i < EP_COUNT; i++) r.ep[i] = 0.0f;
        }
    } else {
        decode_apply(a.t, r, a.actions + (size_t)sl.env * SB_ACT);
        hvac_pre(a.t, r, scr, a, s);
    }
    stage_out(g, lds, a.st.bytes);
}

// Zone means of the new field: one wavefront per (zone, env), the pairs
// zone-major (the envs of a zone read the same cell list). The lanes load
// 8 x 64 consecutive entries of the room's cell list a round (the next round's
// in flight while the current one is summed). In exact mode lane 0 adds them
// from LDS in the list's order, so the sum is the sequential one over the
// room's cells (csim's); otherwise each lane sums its own entries and a
// wavefront tree combines the lanes (reassociated, as the default mode's
// field solve is: its results agree with the reference within rounding).
constexpr int kMeansWaves = 4, kMeansChunks = 8;
__device__ __forceinline__ void means_load(double (&v)[kMeansChunks], const double* T, const int* cells, int q,
                                           int c1, int ln, int Gl) {
    int c[kMeansChunks];
#pragma unroll
    for (int u = 0; u < kMeansChunks; u++) {
        const int i = q + 64 * u + ln;
        c[u] = i < c1 ? cells[i] : -1;
    }
#pragma unroll
    for (int u = 0; u < kMeansChunks; u++) v[u] = c[u] >= 0 ? T[(size_t)c[u] * Gl] : 0.0;
}
__device__ __forceinline__ void wave_order() {
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
}
__global__ __launch_bounds__(64 * kMeansWaves) void fe_means_kernel(Args a) {
    constexpr int R = 64 * kMeansChunks;
    __shared__ __align__(16) double buf[kMeansWaves][R];
    const int w = (int)(threadIdx.x >> 6), ln = (int)(threadIdx.x & 63);
    const int p = (int)blockIdx.x * kMeansWaves + w;
    const int nz = a.t.nz;
    if (p >= a.G * nz) return;   // wave-uniform; the kernel has no workgroup barrier
    const int z = p / a.G, s = p % a.G;
    const size_t b = (size_t)(s / a.Gl), l = (size_t)(s % a.Gl);
    const double* T = a.T + b * (size_t)a.t.n_cvs * a.Gl + l;
    const int* cells = a.t.zcells;
    const int c0 = a.t.zoff[z], c1 = a.t.zoff[z + 1];
    double* bw = buf[w];
    double sum = 0.0;
    double v[kMeansChunks], vn[kMeansChunks];
    means_load(v, T, cells, c0, c1, ln, a.Gl);
    if (!a.exact) {
        for (int q = c0; q < c1; q += R) {
            if (q + R < c1) means_load(vn, T, cells, q + R, c1, ln, a.Gl);
#pragma unroll
            for (int u = 0; u < kMeansChunks; u++) sum += v[u];
#pragma unroll
            for (int u = 0; u < kMeansChunks; u++) v[u] = vn[u];
        }
        for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o);
        if (ln == 0) {
            unsigned char* rec = a.state + (size_t)s * a.st.record;
            reinterpret_cast<double*>(rec + a.st.avg_temp)[z] = sum / (double)(c1 - c0);
        }
        return;
    }
    for (int q = c0; q < c1; q += R) {
        if (q + R < c1) means_load(vn, T, cells, q + R, c1, ln, a.Gl);
#pragma unroll
        for (int u = 0; u < kMeansChunks; u++) bw[64 * u + ln] = v[u];
        wave_order();
        if (ln == 0) {
            const int m = c1 - q;
            if (m >= R) {
#pragma unroll 8
                for (int i = 0; i < R; i += 2) {
                    const double2 t = *reinterpret_cast<const double2*>(bw + i);
                    sum += t.x;
                    sum += t.y;
                }
            } else {
                for (int i = 0; i < m; i++) sum += bw[i];
            }
        }
        wave_order();
#pragma unroll
        for (int u = 0; u < kMeansChunks; u++) v[u] = vn[u];
    }
    if (ln == 0) {
        unsigned char* rec = a.state + (size_t)s * a.st.record;
        reinterpret_cast<double*>(rec + a.st.avg_temp)[z] = sum / (double)(c1 - c0);
    }
}

// After the field step and the zone means: observation, occupancy, reward,
// bookkeeping, Log and the auto-reset.
__global__ __launch_bounds__(W) void fe_post_kernel(Args a) {
    const int s = (int)blockIdx.x;
    if (s >= a.G) return;
    extern __shared__ __align__(16) unsigned char lds[];
    unsigned char* g = a.state + (size_t)s * a.st.record;
    stage_in(lds, g, a.st.bytes);
    Rec r = view(lds, a.st);
    double* scr = reinterpret_cast<double*>(lds + a.st.bytes);
    uint32_t* blk = reinterpret_cast<uint32_t*>(scr);
    const Tabs& t = a.t;
    const Slot sl = a.slots[s];
    const int step = r.ip[IP_STEP] + 1;
    const int j = sl.start + step;
    float* obs_row = a.obs + (size_t)sl.env * SB_OBS;
    write_obs(t, r, obs_row, j);
    wsync();
    occupancy(t, r, (int)t.occ_hour[j], (int)t.occ_work[j], blk);
    double dg[8];
    const double rew = reward(t, r, scr, j, dg);
    // the first episode after puf_vec_create may be cut short (desync); a cut
    // episode is a truncation and stays out of the episode log
    // (complete_port/gpu/smart_buildings.cu:1990-1993, 2043)
    const bool first = r.ip[IP_FIRST_DONE] == 0;
    const bool cut = first && sl.first_steps < sl.max_steps;
    const bool done = step >= (first ? sl.first_steps : sl.max_steps);
    if (lane() == 0) {
        const float rf = (float)rew;
        a.rewards[sl.env] = rf * a.reward_scale;
        a.terminals[sl.env] = done ? 1.0f : 0.0f;
        r.ip[IP_STEP] = step;
        r.pl[PL_REW_SUM] += rew;
        r.pl[PL_DEV_SUM] += dg[3];
        r.ip[IP_STEPS_TOTAL] += 1;
        // the episode's running sums in float (smart_buildings.cu:1965-1971),
        // into the host Log when a whole episode ends
        r.ep[EP_RET] += rf;
        for (int k = 0; k < 8; k++) r.ep[EP_PART + k] += (float)dg[k];
        if ((float)dg[4] > r.ep[EP_WORST]) r.ep[EP_WORST] = (float)dg[4];
        if (done) {
            r.ip[IP_EPISODES] += 1;
            r.ip[IP_FIRST_DONE] = 1;
            if (a.host_env && !cut) log_episode(a, sl.env, r.ep, step);
            for (int k = 0; k < EP_COUNT; k++) r.ep[k] = 0.0f;
        }
    }
    wsync();
    if (done) env_reset(t, r, sl, obs_row, blk, a, s, true);
    stage_out(g, lds, a.st.bytes);
}

// ------------------------------------------------------------------ convection
// The step's stochastic convection (complete_port/csim/sb_convect.c:39-73)
// planned from the env's convection stream alone: per room, each cell draws
// u, and a cell with u <= p and candidates draws one of them (numpy's masked
// rejection, sb_rng.c:45-54); the room's pairs are shuffled (Fisher-Yates
// from the top) and swapped in order. None of this reads a temperature, so the
// plan runs before the field step and leaves a list of moves.
//
// Stream: raw blocks in LDS, two at a time (the current one and, once a read
// reaches past it, the next), each with its tempered copy. A round reads the u
// of up to 64 cells at the positions they have if no cell before them swaps,
// and with it the word each would start its candidate draw with; the first
// cell that swaps ends the round. Fisher-Yates draws take 64 words at a time
// and resolve one draw per ballot. Each final pair t (known once the shuffle
// has passed t, from the top) is composed into the room's inverse
// permutation q (q <- q o (a b)), so after the room T_new[q[i]] = T_old[i]
// for every cell i of the room: the moves are the cells with q[i] != i.
namespace {

struct Stream {
    uint32_t* raw;     // [2][624]
    uint32_t* tw;      // [2][624] tempered
    long long base;    // stream position of the current block's word 0
    long long pos;     // next word to consume
    int cur;
    bool have_next;

    __device__ uint32_t word(long long q) const {
        const int d = (int)(q - base);
        const int b = d >= SBE_MT_N ? cur ^ 1 : cur;
        return tw[b * SBE_MT_N + (d >= SBE_MT_N ? d - SBE_MT_N : d)];
    }
    // words up to position q (q - pos < 624) readable
    __device__ void ensure(long long q) {
        while (q >= base + SBE_MT_N * (have_next ? 2 : 1)) {
            if (!have_next) {
                const int nb = cur ^ 1;
                mt_next_block(raw + cur * SBE_MT_N, raw + nb * SBE_MT_N, tw + nb * SBE_MT_N);
                have_next = true;
            } else {
                base += SBE_MT_N;
                cur ^= 1;
                have_next = false;
            }
        }
    }
};

__device__ __forceinline__ uint32_t smear(uint32_t x) {
    x |= x >> 1;
    x |= x >> 2;
    x |= x >> 4;
    x |= x >> 8;
    x |= x >> 16;
    return x;
}

}  // namespace

__global__ __launch_bounds__(W) void fe_conv_plan_kernel(Args a) {
    const int s = (int)blockIdx.x;
    if (s >= a.G) return;
    const Tabs& t = a.t;
    extern __shared__ __align__(16) unsigned char lds[];
    Stream S;
    S.raw = reinterpret_cast<uint32_t*>(lds);
    S.tw = S.raw + 2 * SBE_MT_N;
    uint32_t* pr = S.tw + 2 * SBE_MT_N;                           // [cv_lds_pairs]
    uint16_t* qinv = reinterpret_cast<uint16_t*>(pr + a.cv_lds_pairs);   // [cv_max_room]
    uint8_t* ncand = reinterpret_cast<uint8_t*>(qinv + t.cv_max_room);    // [cv_max_room]
    unsigned char* g = a.state + (size_t)s * a.st.record;
    uint32_t* gmt = reinterpret_cast<uint32_t*>(g + a.st.cmt);
    int* gidx = reinterpret_cast<int*>(gmt + SBE_MT_N);   // the stream's position in its block
    unsigned int* spill = a.cv_spill + (size_t)s * 2 * t.cv_max_room;
    const int cap = a.cv_lds_pairs;
    // the room's Fisher-Yates draws: u16 in LDS beside the pairs, past the
    // LDS pairs in the HBM overflow area's second half
    uint16_t* jd = reinterpret_cast<uint16_t*>(lds + ((ncand + t.cv_max_room - lds + 3) & ~3));
    unsigned int* jspill = spill + t.cv_max_room;
    auto jd_st = [&](int i, uint32_t v) {
        if (i < cap) jd[i] = (uint16_t)v;
        else jspill[i - cap] = v;
    };
    auto jd_ld = [&](int i) -> uint32_t { return i < cap ? (uint32_t)jd[i] : jspill[i - cap]; };
    auto pr_ld = [&](int i) -> uint32_t { return i < cap ? pr[i] : spill[i - cap]; };
    auto pr_st = [&](int i, uint32_t v) {
        if (i < cap) pr[i] = v;
        else spill[i - cap] = v;
    };
    for (int i = lane(); i < SBE_MT_N; i += W) {
        const uint32_t w = gmt[i];
        S.raw[i] = w;
        S.tw[i] = mt_temper(w);
    }
    S.base = 0;
    S.pos = *gidx;
    S.cur = 0;
    S.have_next = false;
    wsync();
    const uint64_t thr = ((uint64_t)t.cv_thr_hi << 32) | t.cv_thr_lo;
    const bool never = t.cv_thr_hi == 0xFFFFFFFFu;
    unsigned long long* moves = a.cv_moves + (size_t)s * t.cv_cells;
    int count = 0;
    for (int rm = 0; rm < t.cv_rooms; rm++) {
        const int b0 = t.cv_off[rm], n = t.cv_off[rm + 1] - b0;
        // the room's candidate counts, eight loads in flight per lane
        for (int i0 = 0; i0 < n; i0 += 8 * W) {
            uint8_t c8[8];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int i = i0 + u * W + lane();
                c8[u] = i < n ? t.cv_ncand[b0 + i] : 0;
            }
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int i = i0 + u * W + lane();
                if (i < n) {
                    ncand[i] = c8[u];
                    qinv[i] = (uint16_t)i;
                }
            }
        }
        wsync();
        // cells, in windows of 128 stream words: lane i holds the words at
        // offsets 2i, 2i + 1, 2i + 2 of the window, so for either parity of the
        // drift (the words the window's swapping cells have taken beyond two
        // per cell) the swap bit of cell i is one ballot (P0, P1), and a drift
        // of 2t + par shifts those bits by t cells; each swap's candidate
        // draw reads its words from the same registers
        int m = 0;
        for (int j = 0; j < n;) {
            S.ensure(S.pos + 2 * W);
            const long long p = S.pos + 2 * lane();
            const uint32_t w0 = S.word(p), w1 = S.word(p + 1), w2 = S.word(p + 2);
            const int nc = (j + lane() < n) ? ncand[j + lane()] : 0;
            const uint64_t u0 = ((uint64_t)(w0 >> 5) << 26) | (uint64_t)(w1 >> 6);
            const uint64_t u1 = ((uint64_t)(w1 >> 5) << 26) | (uint64_t)(w2 >> 6);
            const unsigned long long P0 = ballot(!never && u0 <= thr), P1 = ballot(!never && u1 <= thr);
            const unsigned long long HC = ballot(nc > 0);
            // the window's pairs collect in one register (lane k: its k-th pair)
            uint32_t wp = 0;
            int npair = 0;
            int c = 0, drift = 0;
            bool slow = false;           // a candidate draw ran past the window
            uint32_t smax = 0;
            while (true) {
                const int tt = drift >> 1, par = drift & 1;
                if (c + tt >= W) break;
                const unsigned long long cand = ((par ? P1 : P0) >> tt) & HC & (~0ull << c);
                if (cand == 0ull) {
                    c = W - tt;
                    break;
                }
                const int cc = first_lane(cand);
                const uint32_t mx = (uint32_t)__builtin_amdgcn_readlane(nc, cc) - 1u;
                int q = 2 * (cc + tt) + par + 2;   // the candidate draw's first word
                uint32_t pick = 0;
                if (mx != 0u) {
                    const uint32_t mask = smear(mx);
                    for (;;) {
                        if (q >= 2 * W) {
                            slow = true;
                            break;
                        }
                        const uint32_t wa = lane_u32(w0, q >> 1), wb = lane_u32(w1, q >> 1);
                        const uint32_t v = ((q & 1) ? wb : wa) & mask;
                        q++;
                        if (v <= mx) {
                            pick = v;
                            break;
                        }
                    }
                }
                if (slow) {
                    // the draw continues past the window: finish it from LDS
                    S.pos += q;
                    j += cc;
                    smax = mx;
                    break;
                }
                wp = lane() == npair ? ((uint32_t)(j + cc) | (pick << 16)) : wp;
                npair++;
                drift = q - 2 * (cc + 1);
                c = cc + 1;
            }
            if (npair > 0) {
                if (m + W <= cap) {
                    if (lane() < npair) pr[m + lane()] = wp;
                } else if (lane() < npair) {
                    pr_st(m + lane(), wp);
                }
                m += npair;
            }
            if (slow) {
                const uint32_t mask = smear(smax);
                uint32_t pick = 0;
                for (;;) {
                    S.ensure(S.pos + W - 1);
                    const uint32_t v = S.word(S.pos + lane()) & mask;
                    const unsigned long long okm = ballot(v <= smax);
                    if (okm) {
                        const int gl = first_lane(okm);
                        pick = lane_u32(v, gl);
                        S.pos += gl + 1;
                        break;
                    }
                    S.pos += W;
                }
                if (lane() == 0) pr_st(m, (uint32_t)j | (pick << 16));
                m++;
                j += 1;
                continue;
            }
            const int ce = min(c, n - j);   // the window's cells past the room draw nothing
            S.pos += 2 * ce + drift;
            j += ce;
        }
        wsync();
        // each pair's candidate as a room-local cell
        for (int i = lane(); i < m; i += W) {
            const uint32_t x = pr_ld(i);
            const int cell = (int)(x & 0xffffu), pick = (int)(x >> 16);
            const uint32_t right = t.cv_cidx[t.cv_coff[b0 + cell] + pick];
            pr_st(i, (uint32_t)cell | (right << 16));
        }
        wsync();
        // Fisher-Yates from the top: every draw resolved first (64 stream
        // words per ballot pass; draw t into jd[t]), then lane 0 applies them,
        // each final pair composed into q (q <- q o (a b)); the composition of
        // one pair overlaps the loads of the next, one LDS round trip a draw
        for (int tt = m - 1; tt > 0;) {
            S.ensure(S.pos + W - 1);
            const uint32_t w = S.word(S.pos + lane());
            int kx = 0;
            while (tt > 0 && kx < W) {
                const uint32_t mask = smear((uint32_t)tt);
                const unsigned long long okm = ballot((w & mask) <= (uint32_t)tt) & (~0ull << kx);
                if (okm == 0ull) {
                    kx = W;
                    break;
                }
                const int gl = first_lane(okm);
                if (lane() == 0) jd_st(tt, (lane_u32(w, gl) & mask));
                kx = gl + 1;
                tt--;
            }
            S.pos += kx;
        }
        wsync();
        for (int top = m - 1; top > 0; top -= W) {
            const int mine = top - lane();
            const uint32_t jl = mine > 0 ? jd_ld(mine) : 0u;
            if (lane() == 0) {
                const int cnt = min(W, top);
                uint32_t held = 0;
                bool have = false;
                for (int l = 0; l < cnt; l++) {
                    const int t2 = top - l;
                    const int j2 = (int)lane_u32(jl, l);
                    const uint32_t x = pr_ld(t2), y = pr_ld(j2);
                    if (have) {
                        const int ca = (int)(held & 0xffffu), cb = (int)(held >> 16);
                        const uint16_t qa = qinv[ca], qb = qinv[cb];
                        qinv[ca] = qb;
                        qinv[cb] = qa;
                    }
                    pr_st(j2, x);
                    held = y;
                    have = true;
                }
                if (have) {
                    const int ca = (int)(held & 0xffffu), cb = (int)(held >> 16);
                    const uint16_t qa = qinv[ca], qb = qinv[cb];
                    qinv[ca] = qb;
                    qinv[cb] = qa;
                }
            }
            wsync();
        }
        if (m > 0 && lane() == 0) {
            const uint32_t y = pr_ld(0);
            const int ca = (int)(y & 0xffffu), cb = (int)(y >> 16);
            const uint16_t qa = qinv[ca], qb = qinv[cb];
            qinv[ca] = qb;
            qinv[cb] = qa;
        }
        wsync();
        // moves: cell i's value goes to cell q[i] (convection-cell indices;
        // the move kernels map them to field cells)
        for (int i0 = 0; i0 < n; i0 += W) {
            const int i = i0 + lane();
            const int q = i < n ? (int)qinv[i] : i;
            const bool mv = i < n && q != i;
            const unsigned long long mm = ballot(mv);
            if (mv) moves[count + below_me(mm)] = ((unsigned long long)(unsigned)(b0 + q) << 32) | (unsigned)(b0 + i);
            count += __popcll(mm);
        }
        wsync();
    }
    // the stream state: the block holding the last word consumed
    const long long d = S.pos - S.base;
    const int blkx = d > SBE_MT_N ? (S.cur ^ 1) : S.cur;
    for (int i = lane(); i < SBE_MT_N; i += W) gmt[i] = S.raw[blkx * SBE_MT_N + i];
    if (lane() == 0) {
        *gidx = (int)(d > SBE_MT_N ? d - SBE_MT_N : d);
        a.cv_count[s] = count;
    }
}

// The moves of the step, read then written (two launches: every value is read
// before any cell is overwritten). Blocks y = env, x strides its moves.
__global__ void fe_conv_gather_kernel(Args a) {
    const int s = (int)blockIdx.y;
    const int cnt = a.cv_count[s];
    const size_t b = (size_t)(s / a.Gl), l = (size_t)(s % a.Gl), Gl = (size_t)a.Gl;
    const double* T = a.T + b * (size_t)a.t.n_cvs * Gl + l;
    const unsigned long long* mv = a.cv_moves + (size_t)s * a.t.cv_cells;
    double* val = a.cv_vals + (size_t)s * a.t.cv_cells;
    for (int i = (int)(blockIdx.x * blockDim.x + threadIdx.x); i < cnt; i += (int)(gridDim.x * blockDim.x))
        val[i] = T[(size_t)(unsigned)a.t.cv_cell[(unsigned)(mv[i] & 0xffffffffull)] * Gl];
}

__global__ void fe_conv_scatter_kernel(Args a) {
    const int s = (int)blockIdx.y;
    const int cnt = a.cv_count[s];
    const size_t b = (size_t)(s / a.Gl), l = (size_t)(s % a.Gl), Gl = (size_t)a.Gl;
    double* T = a.T + b * (size_t)a.t.n_cvs * Gl + l;
    const unsigned long long* mv = a.cv_moves + (size_t)s * a.t.cv_cells;
    const double* val = a.cv_vals + (size_t)s * a.t.cv_cells;
    for (int i = (int)(blockIdx.x * blockDim.x + threadIdx.x); i < cnt; i += (int)(gridDim.x * blockDim.x))
        T[(size_t)(unsigned)a.t.cv_cell[(unsigned)(mv[i] >> 32)] * Gl] = val[i];
}

// Adds the group's f64 reward sum, env-steps and episodes since puf_reset to
// live[0..2]: lane l sums envs l, l + 64, ... in order, lane 0 the lanes' sums
// in lane order (independent of timing).
__global__ __launch_bounds__(W) void fe_live_kernel(Args a) {
    __shared__ double part[4][W];
    double rs = 0.0, st = 0.0, ep = 0.0, dv = 0.0;
    for (int s = lane(); s < a.G; s += W) {
        const unsigned char* rec = a.state + (size_t)s * a.st.record;
        const double* pl = reinterpret_cast<const double*>(rec + a.st.plant);
        rs += pl[PL_REW_SUM];
        dv += pl[PL_DEV_SUM];
        const int* ip = reinterpret_cast<const int*>(rec + a.st.ip);
        st += (double)ip[IP_STEPS_TOTAL];
        ep += (double)ip[IP_EPISODES];
    }
    part[0][lane()] = rs;
    part[1][lane()] = st;
    part[2][lane()] = ep;
    part[3][lane()] = dv;
    __syncthreads();
    if (lane() < 4) {
        double x = 0.0;
        for (int i = 0; i < W; i++) x += part[lane()][i];
        if (lane() < 3) a.live[lane()] += x;
        if (a.live_scen >= 0) {
            // the scenario's (reward sum, deviation sum, env-steps)
            const int slot = lane() == 0 ? 0 : (lane() == 3 ? 1 : (lane() == 1 ? 2 : -1));
            if (slot >= 0) a.live[3 + 3 * a.live_scen + slot] += x;
        }
    }
}

}  // namespace sbe

// ---------------------------------------------------------------- launchers
// which: 0 pre (or puf_reset), 1 zone means, 2 post, 3 live sums, 4 convection
// plan, 5 convection moves (gather then scatter)
extern "C" int sbe_launch(const sbe::Args* a, int which, hipStream_t s) {
    using namespace sbe;
    const int G = a->G;
    switch (which) {
    case 0: hipLaunchKernelGGL(fe_pre_kernel, dim3(G), dim3(64), a->lds_bytes, s, *a); break;
    case 1: {
        const int n = G * a->t.nz;   // (zone, env) pairs, one wavefront each
        hipLaunchKernelGGL(fe_means_kernel, dim3((n + kMeansWaves - 1) / kMeansWaves), dim3(64 * kMeansWaves), 0, s, *a);
        break;
    }
    case 2: hipLaunchKernelGGL(fe_post_kernel, dim3(G), dim3(64), a->lds_bytes, s, *a); break;
    case 3: hipLaunchKernelGGL(fe_live_kernel, dim3(1), dim3(64), 0, s, *a); break;
    case 4: {
        const size_t lds = 4 * 4 * SBE_MT_N + 6 * (size_t)a->cv_lds_pairs + 3 * (size_t)a->t.cv_max_room + 16;
        hipLaunchKernelGGL(fe_conv_plan_kernel, dim3(G), dim3(64), lds, s, *a);
        break;
    }
    case 5: {
        const dim3 grid(32, G);
        hipLaunchKernelGGL(fe_conv_gather_kernel, grid, dim3(256), 0, s, *a);
        hipLaunchKernelGGL(fe_conv_scatter_kernel, grid, dim3(256), 0, s, *a);
        break;
    }
    default: return (int)hipErrorInvalidValue;
    }
    return (int)hipGetLastError();
}

// Dynamic LDS the env kernels may use (the plan kernel's and the HVAC kernels').
extern "C" int sbe_lds_limit(int bytes) {
    using namespace sbe;
    const void* fns[3] = {(const void*)fe_pre_kernel, (const void*)fe_post_kernel, (const void*)fe_conv_plan_kernel};
    for (const void* f : fns) {
        const hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
        if (e != hipSuccess) return (int)e;
    }
    return 0;
}
