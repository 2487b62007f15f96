// Host side of the field envs: reads an FDM-scale scenario's HVAC, calendar,
// observation and reward tables (the sections csim reads, complete_port/csim/
// sb_sim.c:23-98, sb_occup.c:8-29, sb_reward.c), checks them, uploads them
// once, opens the scenario's field group (fdm.cpp) and launches each step's
// kernels (field_env_kernel.hip, fdm_kernel.hip) on the vec's stream.
#include <hip/hip_runtime_api.h>
#include <math.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <string>
#include <vector>

#include "fdm_host.h"
#include "field_host.h"
#include "sbb_reader.h"
#include "sbenv.h"

extern "C" int sbe_launch(const sbe::Args* a, int which, hipStream_t s);
extern "C" int sbe_lds_limit(int bytes);
extern "C" SbxFdm* sbx_fdm_open(const char* blob_path, int n_envs, int envs_per_block, int flags);
extern "C" void sbx_fdm_close(SbxFdm* f);
extern "C" const char* sbx_last_error(void);

namespace {

constexpr int kFieldMinSolved = 2048;   // the RC kernel's LDS plans stop well below this

struct Arena {
    std::vector<unsigned char> host;
    size_t add(const void* p, size_t bytes) {
        size_t off = (host.size() + 255) & ~(size_t)255;
        host.resize(off + bytes + 8, 0);
        if (p && bytes) memcpy(host.data() + off, p, bytes);
        return off;
    }
    template <class T>
    size_t vec(const std::vector<T>& v) { return add(v.data(), v.size() * sizeof(T)); }
};

bool hip_ok(hipError_t e, const char* what, std::string* err) {
    if (e == hipSuccess) return true;
    *err = std::string(what) + ": " + hipGetErrorString(e);
    return false;
}

}  // namespace

struct FieldScen {
    FieldCounts c{};
    sbe::Tabs t{};                 // device pointers patched at attach
    sbe::StateLayout st{};
    Arena A;
    std::vector<std::pair<const void**, size_t>> fix;
    unsigned char* d_tables = nullptr;
    // per env
    int G = 0;
    std::vector<sbe::Slot> slots;
    sbe::Slot* d_slots = nullptr;
    unsigned char* d_state = nullptr;
    double *d_qz = nullptr, *d_amb = nullptr, *d_hh = nullptr, *d_g = nullptr, *d_airT = nullptr;
    int lds_bytes = 0;            // the HVAC kernels' dynamic LDS
    // convection: the step's moves, their count and values, pair overflow
    unsigned long long* d_moves = nullptr;
    int* d_count = nullptr;
    double* d_vals = nullptr;
    unsigned int* d_spill = nullptr;
    int lds_pairs = 0;
    double conv_p = 0.0;
    // the plan kernel runs on its own stream, forked from the bound stream at
    // the start of a step and joined before the moves (it reads no field)
    hipStream_t side = nullptr;
    hipEvent_t fork = nullptr, join = nullptr;
    SbxFdm* fdm = nullptr;
    int exact = 0;                // SBX_FDM_EXACT: the zone means sum in the reference's order too
};

bool field_blob(const sbh::Blob& b) {
    uint64_t n = 0;
    if (!b.i64("solved", &n)) return false;
    if ((int64_t)n > kFieldMinSolved) return true;
    // air side: one applied and one sensed entry per column, unit weight, on
    // the same node, no node twice (what the RC plans fold into diag(g))
    uint64_t nss = 0, nap = 0, nai = 0, nsp = 0, nsi = 0, nax = 0, nsx = 0;
    const int64_t* ss = b.i64("sensed_shape", &nss);
    const int k = (ss && nss >= 1) ? (int)ss[0] : 0;
    const int32_t *ap = b.i32("applied_indptr", &nap), *ai = b.i32("applied_indices", &nai);
    const int32_t *sp = b.i32("sensed_indptr", &nsp), *si = b.i32("sensed_indices", &nsi);
    const double *ax = b.f64("applied_data", &nax), *sx = b.f64("sensed_data", &nsx);
    if (k <= 0) return false;
    // a malformed air side goes to the field path, whose open checks it with
    // a message (the tests below read only inside the sections)
    if (!ap || !ai || !sp || !si || !ax || !sx) return true;
    if (nap != (uint64_t)k + 1 || nsp != (uint64_t)k + 1 || nax < nai || nsx < nsi) return true;
    for (int c = 0; c < k; c++)
        if (ap[c] < 0 || ap[c + 1] < ap[c] || (uint64_t)ap[c + 1] > nai || sp[c] < 0 || sp[c + 1] < sp[c]
            || (uint64_t)sp[c + 1] > nsi)
            return true;
    std::vector<char> seen(n, 0);
    for (int c = 0; c < k; c++) {
        if (ap[c + 1] - ap[c] != 1 || sp[c + 1] - sp[c] != 1) return true;
        const int t = ai[ap[c]];
        if (si[sp[c]] != t || ax[ap[c]] != 1.0 || sx[sp[c]] != 1.0 || t < 0 || t >= (int)n || seen[t]) return true;
        seen[t] = 1;
    }
    return false;
}

FieldScen* field_open(const sbh::Blob& b, std::string* err) {
    auto F = new FieldScen();
    FieldScen& f = *F;
    auto bad = [&](const std::string& m) {
        *err = m;
        delete F;
        return (FieldScen*)nullptr;
    };
    uint64_t c = 0;
    const int64_t* grid = b.i64("grid", &c);
    if (!grid || c != 2) return bad("grid missing");
    const int nr = (int)grid[0], ncol = (int)grid[1];
    f.t.n_cvs = nr * ncol;
    uint64_t n_solved = 0;
    if (!b.i64("solved", &n_solved)) return bad("solved missing");
    f.c.n_cvs = f.t.n_cvs;
    f.c.n_solved = (int)n_solved;
    // ---- HVAC topology
    const double* ahu_c = b.f64("ahu_const", &c);
    if (!ahu_c || c % 9 || c == 0) return bad("ahu_const missing");
    const int na = (int)(c / 9);
    const int32_t* vz_off = b.i32("vav_zone_offsets", &c);
    if (!vz_off || c < 2) return bad("vav_zone_offsets missing");
    const int nv = (int)c - 1;
    const double* zone_area = b.f64("zone_area", &c);
    const int nz = (int)c;
    uint64_t nvz = 0, nro = 0, nrc = 0, ncp = 0;
    const int32_t* vz_idx = b.i32("vav_zone_idx", &nvz);
    const int32_t* vav_ahu = b.i32("vav_ahu_idx");
    const int32_t* coupled = b.i32("coupled_vav_idx", &ncp);
    const int32_t* phys = b.i32("phys_room_idx");
    const int32_t* room_off = b.i32("room_offsets", &nro);
    const int32_t* room_cells = b.i32("room_cells", &nrc);
    const double* vav_c = b.f64("vav_const");
    if (!zone_area || nz < 1 || !vz_idx || !vav_ahu || !coupled || !phys || !room_off || !room_cells || !vav_c)
        return bad("HVAC topology sections missing");
    const int64_t* ss = b.i64("sensed_shape");
    const int k = ss ? (int)ss[0] : 0;
    if ((int)ncp != k) return bad("coupled_vav_idx does not match the air side's columns");
    for (int q = 0; q < k; q++)
        if (coupled[q] < 0 || coupled[q] >= nv) return bad("coupled_vav_idx out of range");
    if ((uint64_t)vz_off[nv] > nvz) return bad("vav_zone_offsets past vav_zone_idx");
    for (int v = 0; v < nv; v++) {
        if (vav_ahu[v] < 0 || vav_ahu[v] >= na) return bad("vav_ahu_idx out of range");
        if (vz_off[v + 1] < vz_off[v]) return bad("vav_zone_offsets decrease");
        for (int q = vz_off[v]; q < vz_off[v + 1]; q++)
            if (vz_idx[q] < 0 || vz_idx[q] >= nz) return bad("vav_zone_idx out of range");
    }
    // every AHU serves zone area (its return air is then a VAV mean: the all-cell
    // mean csim falls back to is never read)
    {
        std::vector<double> at(na, 0.0);
        for (int v = 0; v < nv; v++) {
            double a = 0.0;
            for (int q = vz_off[v]; q < vz_off[v + 1]; q++) a += zone_area[vz_idx[q]];
            if (a > 0.0) at[vav_ahu[v]] += a;
        }
        for (int q = 0; q < na; q++)
            if (!(at[q] > 0.0)) return bad("an AHU serves no zone area (not supported for field scenarios)");
    }
    // each AHU's VAVs and columns in ascending order; each zone's heating
    // columns in column order (a column heats every zone of its VAV)
    std::vector<int> av_off(1, 0), av_idx, ac_off(1, 0), ac_idx, zc_off(1, 0), zc_idx;
    {
        std::vector<std::vector<int>> zc(nz);
        for (int col = 0; col < k; col++) {
            const int v = coupled[col];
            for (int q = vz_off[v]; q < vz_off[v + 1]; q++) zc[vz_idx[q]].push_back(col);
        }
        for (int q = 0; q < na; q++) {
            for (int v = 0; v < nv; v++)
                if (vav_ahu[v] == q) av_idx.push_back(v);
            av_off.push_back((int)av_idx.size());
            for (int col = 0; col < k; col++)
                if (vav_ahu[coupled[col]] == q) ac_idx.push_back(col);
            ac_off.push_back((int)ac_idx.size());
        }
        for (int z = 0; z < nz; z++) {
            zc_idx.insert(zc_idx.end(), zc[z].begin(), zc[z].end());
            zc_off.push_back((int)zc_idx.size());
        }
    }
    // zones -> their room's cells, in the room's order; zone means of temp_init
    const double* tinit = b.f64("temp_init", &c);
    if (!tinit || (int64_t)c != f.t.n_cvs) return bad("temp_init missing");
    std::vector<int> zoff(1, 0), zcells;
    std::vector<double> zm(nz);
    const int nrooms = (int)nro - 1;
    for (int z = 0; z < nz; z++) {
        const int rm = phys[z];
        if (rm < 0 || rm >= nrooms || room_off[rm + 1] <= room_off[rm] || 2 * (uint64_t)room_off[rm + 1] > nrc)
            return bad("zone room out of range or empty");
        double sum = 0.0;
        for (int q = room_off[rm]; q < room_off[rm + 1]; q++) {
            const int r = room_cells[2 * q], cc = room_cells[2 * q + 1];
            if (r < 0 || r >= nr || cc < 0 || cc >= ncol) return bad("room cell outside the grid");
            const int p = r * ncol + cc;
            zcells.push_back(p);
            sum += tinit[p];
        }
        zoff.push_back((int)zcells.size());
        zm[z] = sum / (double)(zoff[z + 1] - zoff[z]);
    }
    // ---- stochastic convection (sb_convect.c:5-31, applied at :39-73): on
    // when conv_p != 0 and conv_distance != 0; the rooms' candidates must lie
    // in their own room (the reference baker's tables, bake_scenario.py:162-186)
    std::vector<int> cv_off(1, 0), cv_cell, cv_coff;
    std::vector<uint8_t> cv_ncand;
    std::vector<uint16_t> cv_cidx;
    const double conv_p = b.f64_1("conv_p", 0.0);
    const int conv_dist = (int)b.f64_1("conv_distance", -1.0);
    f.t.cv_max_room = 0;
    if (conv_p != 0.0 && conv_dist != 0) {
        uint64_t nco = 0, ncc = 0, ncf = 0, nci = 0;
        const int32_t* co = b.i32("conv_room_offsets", &nco);
        const int32_t* cc = b.i32("conv_room_cells", &ncc);
        const int32_t* cf = b.i32("conv_cand_offsets", &ncf);
        const int32_t* ci = b.i32("conv_cand_idx", &nci);
        if (!co || !cc || !cf || !ci || nco < 1) return bad("convection tables missing");
        const int rooms = (int)nco - 1, cells = co[rooms];
        if (co[0] != 0 || cells < 0 || 2 * (uint64_t)cells > ncc || ncf != (uint64_t)cells + 1)
            return bad("convection room tables inconsistent");
        for (int rm = 0; rm < rooms; rm++) {
            const int r0 = co[rm], r1 = co[rm + 1];
            if (r1 < r0) return bad("convection room offsets decrease");
            if (r1 - r0 > 65535) return bad("a convection room has more than 65535 cells");
            f.t.cv_max_room = std::max(f.t.cv_max_room, r1 - r0);
            for (int q = r0; q < r1; q++) {
                const int r = cc[2 * q], c2 = cc[2 * q + 1];
                if (r < 0 || r >= nr || c2 < 0 || c2 >= ncol) return bad("convection cell outside the grid");
                cv_cell.push_back(r * ncol + c2);
                const int a0 = cf[q], a1 = cf[q + 1];
                if (a0 < 0 || a1 < a0 || (uint64_t)a1 > nci) return bad("convection candidate offsets inconsistent");
                if (a1 - a0 > 255) return bad("a convection cell has more than 255 candidates");
                cv_ncand.push_back((uint8_t)(a1 - a0));
                for (int x = a0; x < a1; x++) {
                    if (ci[x] < r0 || ci[x] >= r1) return bad("a convection candidate lies outside its room");
                    cv_cidx.push_back((uint16_t)(ci[x] - r0));
                }
            }
            cv_off.push_back(r1);
        }
        cv_coff.assign(cf, cf + cells + 1);
        f.t.cv_rooms = rooms;
        f.t.cv_cells = cells;
        // csim swaps when its 53-bit draw u / 2^53 <= p (sb_convect.c:47)
        if (!(conv_p > 0.0)) {
            f.t.cv_thr_hi = 0xFFFFFFFFu;   // never (p < 0; NaN is refused below)
            f.t.cv_thr_lo = 0;
        } else {
            const uint64_t thr = conv_p >= 1.0 ? (1ull << 53) : (uint64_t)floor(conv_p * 9007199254740992.0);
            f.t.cv_thr_hi = (uint32_t)(thr >> 32);
            f.t.cv_thr_lo = (uint32_t)thr;
        }
        if (conv_p != conv_p) return bad("conv_p is NaN");
    }
    if (cv_coff.empty()) cv_coff.push_back(0);
    f.conv_p = conv_p;
    f.c.conv_seed = b.i64_1("conv_seed", 0);
    // ---- features this path does not carry
    {
        uint64_t cs = 0;
        const double* sc = b.f64("solar_gain_coeff", &cs);
        for (uint64_t i = 0; sc && i < cs; i++)
            if (sc[i] != 0.0) return bad("solar gain is not supported for field scenarios");
    }
    // ---- actions
    uint64_t n_act = 0;
    const uint8_t* kind = b.u8("act_owner_kind", &n_act);
    const uint8_t* act = b.u8("act_actuator");
    const uint8_t* disc = b.u8("act_is_discrete");
    const int32_t* aidx = b.i32("act_owner_index");
    const double *mn = b.f64("act_min_native"), *mx = b.f64("act_max_native");
    const double *mnr = b.f64("act_min_norm"), *mxr = b.f64("act_max_norm");
    if (!kind || !act || !disc || !aidx || !mn || !mx || !mnr || !mxr) return bad("action tables missing");
    int ncont = 0, ndisc = 0;
    for (uint64_t i = 0; i < n_act; i++) {
        if (disc[i]) ndisc++;
        else ncont++;
        const int lim = kind[i] == 0 ? na : (kind[i] == 1 ? nv : 1);
        if (kind[i] > 1 && aidx[i] != 0 && kind[i] != 2) return bad("action owner kind out of range");
        if (kind[i] < 2 && (aidx[i] < 0 || aidx[i] >= lim)) return bad("action owner index out of range");
    }
    if (ncont > SB_CONT || ndisc > SB_DISC) return bad("scenario has more actions than SB_CONT/SB_DISC");
    // each action's trainer column and target; the sequential apply
    // (sb_sim.c:220-244) keeps the last action written to a target
    std::vector<int> act_col(std::max<uint64_t>(n_act, 1), 0), act_tgt(std::max<uint64_t>(n_act, 1), 0);
    std::vector<uint8_t> act_live(std::max<uint64_t>(n_act, 1), 0);
    {
        int ci = 0, di = 0;
        std::map<int, int> last;
        for (uint64_t i = 0; i < n_act; i++) {
            act_col[i] = disc[i] ? SB_CONT + di++ : ci++;
            const int kd = kind[i] > 2 ? 2 : kind[i];
            const int ac = kd == 0 ? std::min<int>(act[i], 3) : (kd == 1 ? (act[i] == 0 ? 0 : 1) : std::min<int>(act[i], 2));
            const int ix = kd == 2 ? 0 : aidx[i];
            act_tgt[i] = kd | (ac << 4) | (ix << 8);
            last[act_tgt[i]] = (int)i;
        }
        for (auto& kv : last) act_live[kv.second] = 1;
    }
    // ---- observation
    const int n_dev = (int)b.i64_1("n_dev", 0), n_aux = (int)b.i64_1("n_aux", 0);
    if (n_aux < 1 || n_dev < 0 || n_dev + n_aux > SB_OBS) return bad("observation size out of range");
    const uint8_t *fk = b.u8("f_dev_kind"), *fo = b.u8("f_obs_id");
    const int32_t* fi = b.i32("f_dev_idx");
    const double *fm = b.f64("f_norm_mean"), *fv = b.f64("f_norm_var");
    if (n_dev && (!fk || !fo || !fi || !fm || !fv)) return bad("observation map missing");
    std::vector<double> fsd(std::max(n_dev, 1), 0.0);
    for (int i = 0; i < n_dev; i++) {
        fsd[i] = fv[i] > 0.0 ? sqrt(fv[i]) : 0.0;
        const int lim = fk[i] == 0 ? na : (fk[i] == 1 ? nv : 1);
        if (fk[i] < 2 && (fi[i] < 0 || fi[i] >= lim)) return bad("observation device index out of range");
    }
    // ---- calendar
    uint64_t n1 = 0;
    const double* amb = b.f64("weather_ambient", &n1);
    if (!amb) return bad("weather_ambient missing");
    auto rows = [&](uint64_t cnt) { n1 = std::min(n1, cnt); };
    const double *comf = b.f64("sched_comfort", &c);
    if (!comf) return bad("sched_comfort missing");
    rows(c);
    const double* hsp = b.f64("sched_heat_sp", &c);
    if (!hsp) return bad("sched_heat_sp missing");
    rows(c);
    const double* csp = b.f64("sched_cool_sp", &c);
    if (!csp) return bad("sched_cool_sp missing");
    rows(c);
    const int64_t* occ_hour = b.i64("occ_hour", &c);
    if (!occ_hour) return bad("occ_hour missing");
    rows(c);
    const uint8_t* occ_work = b.u8("occ_workday", &c);
    if (!occ_work) return bad("occ_workday missing");
    rows(c);
    const int64_t* rew_hour = b.i64("rew_hour", &c);
    if (!rew_hour) return bad("rew_hour missing");
    rows(c);
    const int64_t* rew_month = b.i64("rew_month", &c);
    if (!rew_month) return bad("rew_month missing");
    rows(c);
    const uint8_t* rew_work = b.u8("rew_workday", &c);
    if (!rew_work) return bad("rew_workday missing");
    rows(c);
    const double* aux = b.f64("aux_time", &c);
    if (n_aux > 1) {
        if (!aux) return bad("aux_time missing");
        rows(c / (uint64_t)(n_aux - 1));
    }
    uint64_t cm1 = 0, cw1 = 0;
    const int64_t* hm1 = b.i64("occ_hour_m1", &cm1);
    const uint8_t* wm1 = b.u8("occ_workday_m1", &cw1);
    if (!hm1 || !wm1) return bad("occ_hour_m1/occ_workday_m1 missing");
    for (uint64_t i = 0; i < n1; i++) {
        if (rew_hour[i] < 0 || rew_hour[i] > 23) return bad("rew_hour out of range");
        if (rew_month[i] < 1 || rew_month[i] > 12) return bad("rew_month out of range");
    }
    // ---- occupancy (sb_occup.c:8-20)
    const double* op = b.f64("occ_params", &c);
    if (!op || c < 6) return bad("occ_params missing");
    const int nassign = (int)op[0];
    if (nassign < 0 || nassign > 64) return bad("occupants per zone out of range");
    f.t.occ_ea = (int)op[1];
    f.t.occ_la = (int)op[2];
    f.t.occ_ed = (int)op[3];
    f.t.occ_ld = (int)op[4];
    f.t.p_arr = 1.0 / ((f.t.occ_la - f.t.occ_ea) * 3600.0 / op[5] / 2.0);
    f.t.p_dep = 1.0 / ((f.t.occ_ld - f.t.occ_ed) * 3600.0 / op[5] / 2.0);
    f.t.dt_sec = op[5];
    // ---- plant and reward constants
    const double* bc = b.f64("boiler_const", &c);
    std::vector<double> boiler(10, 0.0);
    for (int i = 0; i < 10 && bc && i < (int)c; i++) boiler[i] = bc[i];
    const double* pc = b.f64("pump_const");
    f.t.pump_head0 = pc ? pc[0] : 0.0;
    f.t.pump_eff = pc ? pc[1] : 1.0;
    f.t.header_res = b.f64_1("hws_header_resistance", 0.0);
    f.t.internal_w_m2 = b.f64_1("internal_gain_w_per_m2", 0.0);
    f.t.standby_frac = b.f64_1("internal_gain_standby_fraction", 1.0);
    f.t.occupant_w = b.f64_1("occupant_sensible_heat_w", 0.0);
    {
        const double cv = b.f64_1("cv_size_cm", 20.0) / 100.0;
        f.t.cv_area = cv * cv;
    }
    f.t.h = b.f64_1("convection_coefficient", 8.8);
    {
        // the tank's dissipation denominator, sb_reward.c:19-23
        const double r2 = boiler[6] + boiler[9];
        const double cond = log(r2 / boiler[6]) / boiler[8];
        const double conv = 1.0 / boiler[4] / r2;
        f.t.gas_den = cond + conv;
    }
    const double* rw = b.f64("reward_scalars", &c);
    if (!rw || c < 8) return bad("reward_scalars missing");
    const double *ewk = b.f64("elec_weekday_price"), *ewe = b.f64("elec_weekend_price");
    const double *eco2 = b.f64("elec_carbon_rate"), *gp = b.f64("gas_month_price");
    if (!ewk || !ewe || !eco2 || !gp) return bad("price tables missing");
    f.t.gas_co2 = b.f64_1("gas_carbon_rate", 0.0);

    // ---- counts and the state record
    f.t.nz = nz;
    f.t.nv = nv;
    f.t.na = na;
    f.t.k = k;
    f.t.n_act = (int)n_act;
    f.t.n_dev = n_dev;
    f.t.n_aux = n_aux;
    f.t.nassign = nassign;
    f.t.n1 = (int)n1;
    f.c.n_act = (int)n_act;
    f.c.n_cont = ncont;
    f.c.n_disc = ndisc;
    f.c.n1 = (int)n1;
    {
        const double* meta = b.f64("obs_meta", &c);
        f.c.episode_steps = (meta && c >= 4) ? (int)meta[3] : 0;
    }
    f.c.hour_m1_rows = (int)std::min(cm1, cw1);
    f.c.occ_seed = b.i64_1("occ_seed", 17321);
    f.c.nz = nz;
    f.c.n_obs = n_dev + n_aux;
    sbe::StateLayout& S = f.st;
    int o = 0;
    auto f64a = [&](int count) { const int r = o; o += 8 * std::max(count, 1); return r; };
    S.recirc = f64a(na); S.sat = f64a(na); S.fan = f64a(na); S.flow = f64a(na); S.satv = f64a(na);
    S.damper = f64a(nv); S.reheat = f64a(nv); S.ratio = f64a(nv); S.heatsp = f64a(nv); S.coolsp = f64a(nv);
    S.dcmd = f64a(nv); S.rcmd = f64a(nv); S.sensing = f64a(nv); S.vav_area = f64a(nv); S.unres = f64a(nv);
    S.avg_temp = f64a(nz); S.zone_q = f64a(nz); S.occV = f64a(nz);
    S.air_g = f64a(k); S.air_T = f64a(k); S.coil = f64a(k); S.rwen = f64a(k);
    S.plant = f64a(sbe::PL_COUNT);
    auto i32a = [&](int count) { const int r = o; o += 4 * std::max(count, 1); return r; };
    S.run = i32a(na); S.coolreq = i32a(na);
    S.mode = i32a(nv); S.prev_valid = i32a(nv); S.dcmd_set = i32a(nv); S.rcmd_set = i32a(nv);
    S.ip = i32a(sbe::IP_COUNT);
    S.ep = i32a(sbe::EP_COUNT);
    S.occ_state = o;
    o += std::max(nz * nassign, 1);
    o = (o + 15) & ~15;
    S.mt = o;
    o += 4 * SBE_MT_N;
    S.bytes = (o + 15) & ~15;
    S.cmt = f.t.cv_rooms > 0 ? S.bytes : 0;
    S.record = (S.bytes + (S.cmt ? 4 * (SBE_MT_N + 4) : 0) + 255) & ~255;
    // the HVAC kernels' LDS: the image, then f64 scratch for the pre-step
    // (AHU demand, column flow demand), the reward (VAV sums, AHU terms, zone
    // terms) or one MT block
    {
        const int scratch = std::max({8 * (na + k), 8 * (nv + 3 * na + 2 * nz), 4 * SBE_MT_N});
        f.lds_bytes = S.bytes + ((scratch + 15) & ~15);
        if (f.lds_bytes > 160 * 1024) return bad("an env's HVAC state does not fit in LDS");
    }

    // ---- device tables (host image; pointers patched at attach)
    Arena& A = f.A;
    auto put = [&](const void** dst, size_t off) { f.fix.push_back({dst, off}); };
    auto sec = [&](const void** dst, const void* p, size_t bytes) { put(dst, A.add(p, bytes)); };
    sec((const void**)&f.t.zoff, zoff.data(), 4 * zoff.size());
    sec((const void**)&f.t.zcells, zcells.data(), 4 * zcells.size());
    sec((const void**)&f.t.zone_area, zone_area, 8 * (size_t)nz);
    sec((const void**)&f.t.zm_init, zm.data(), 8 * (size_t)nz);
    sec((const void**)&f.t.vz_off, vz_off, 4 * (size_t)(nv + 1));
    sec((const void**)&f.t.vz_idx, vz_idx, 4 * std::max<uint64_t>(nvz, 1));
    sec((const void**)&f.t.vav_ahu, vav_ahu, 4 * (size_t)nv);
    sec((const void**)&f.t.coupled, coupled, 4 * (size_t)std::max(k, 1));
    sec((const void**)&f.t.av_off, av_off.data(), 4 * av_off.size());
    sec((const void**)&f.t.av_idx, av_idx.data(), 4 * std::max<size_t>(av_idx.size(), 1));
    sec((const void**)&f.t.ac_off, ac_off.data(), 4 * ac_off.size());
    sec((const void**)&f.t.ac_idx, ac_idx.data(), 4 * std::max<size_t>(ac_idx.size(), 1));
    sec((const void**)&f.t.zc_off, zc_off.data(), 4 * zc_off.size());
    sec((const void**)&f.t.zc_idx, zc_idx.data(), 4 * std::max<size_t>(zc_idx.size(), 1));
    sec((const void**)&f.t.vav_c, vav_c, 8 * 9 * (size_t)nv);
    sec((const void**)&f.t.ahu_c, ahu_c, 8 * 9 * (size_t)na);
    sec((const void**)&f.t.boiler_c, boiler.data(), 8 * boiler.size());
    sec((const void**)&f.t.act_col, act_col.data(), 4 * act_col.size());
    sec((const void**)&f.t.act_tgt, act_tgt.data(), 4 * act_tgt.size());
    sec((const void**)&f.t.act_live, act_live.data(), act_live.size());
    sec((const void**)&f.t.act_disc, disc, n_act);
    sec((const void**)&f.t.act_mn, mn, 8 * n_act);
    sec((const void**)&f.t.act_mx, mx, 8 * n_act);
    sec((const void**)&f.t.act_mnr, mnr, 8 * n_act);
    sec((const void**)&f.t.act_mxr, mxr, 8 * n_act);
    sec((const void**)&f.t.f_kind, n_dev ? fk : nullptr, (size_t)std::max(n_dev, 1));
    sec((const void**)&f.t.f_id, n_dev ? fo : nullptr, (size_t)std::max(n_dev, 1));
    sec((const void**)&f.t.f_idx, n_dev ? fi : nullptr, 4 * (size_t)std::max(n_dev, 1));
    sec((const void**)&f.t.f_mean, n_dev ? fm : nullptr, 8 * (size_t)std::max(n_dev, 1));
    sec((const void**)&f.t.f_sd, fsd.data(), 8 * fsd.size());
    sec((const void**)&f.t.amb, amb, 8 * n1);
    sec((const void**)&f.t.comfort, comf, 8 * n1);
    sec((const void**)&f.t.heat_sp, hsp, 8 * n1);
    sec((const void**)&f.t.cool_sp, csp, 8 * n1);
    sec((const void**)&f.t.aux_time, aux, 8 * n1 * (size_t)std::max(n_aux - 1, 0));
    sec((const void**)&f.t.occ_hour, occ_hour, 8 * n1);
    sec((const void**)&f.t.occ_work, occ_work, n1);
    sec((const void**)&f.t.hour_m1, hm1, 8 * (size_t)f.c.hour_m1_rows);
    sec((const void**)&f.t.work_m1, wm1, (size_t)f.c.hour_m1_rows);
    sec((const void**)&f.t.rew_hour, rew_hour, 8 * n1);
    sec((const void**)&f.t.rew_month, rew_month, 8 * n1);
    sec((const void**)&f.t.rew_work, rew_work, n1);
    sec((const void**)&f.t.rw, rw, 8 * 8);
    sec((const void**)&f.t.elec_wk, ewk, 8 * 24);
    sec((const void**)&f.t.elec_we, ewe, 8 * 24);
    sec((const void**)&f.t.elec_co2, eco2, 8 * 24);
    sec((const void**)&f.t.gas_price, gp, 8 * 12);
    sec((const void**)&f.t.temp_init, tinit, 8 * (size_t)f.t.n_cvs);
    {
        const double* mi = b.f64("mass_temp_init", &c);
        if (!mi || c != n_solved) return bad("mass_temp_init missing");
        sec((const void**)&f.t.mass_init, mi, 8 * (size_t)n_solved);
    }
    f.t.n_solved = (int)n_solved;
    sec((const void**)&f.t.cv_off, cv_off.data(), 4 * cv_off.size());
    sec((const void**)&f.t.cv_cell, cv_cell.data(), 4 * std::max<size_t>(cv_cell.size(), 1));
    sec((const void**)&f.t.cv_ncand, cv_ncand.data(), std::max<size_t>(cv_ncand.size(), 1));
    sec((const void**)&f.t.cv_coff, cv_coff.data(), 4 * cv_coff.size());
    sec((const void**)&f.t.cv_cidx, cv_cidx.data(), 2 * std::max<size_t>(cv_cidx.size(), 1));
    return F;
}

FieldCounts field_counts(const FieldScen* f) { return f->c; }

namespace {

// MT19937 initialisation (sb_rng.c:9-16)
void mt_seed(uint32_t* mt, uint32_t seed) {
    mt[0] = seed;
    for (int i = 1; i < SBE_MT_N; i++) mt[i] = 1812433253u * (mt[i - 1] ^ (mt[i - 1] >> 30)) + (uint32_t)i;
}

sbe::Args base_args(const FieldScen* f) {
    sbe::Args a{};
    a.t = f->t;
    a.st = f->st;
    a.state = f->d_state;
    a.slots = f->d_slots;
    a.G = f->G;
    a.lds_bytes = f->lds_bytes;
    a.qz = f->d_qz;
    a.amb = f->d_amb;
    a.hh = f->d_hh;
    a.g = f->d_g;
    a.airT = f->d_airT;
    a.T = f->fdm->grp.T;
    a.M = f->fdm->grp.M;
    a.Gl = f->fdm->grp.Gl;
    a.cv_moves = f->d_moves;
    a.cv_count = f->d_count;
    a.cv_vals = f->d_vals;
    a.cv_spill = f->d_spill;
    a.cv_lds_pairs = f->lds_pairs;
    a.exact = f->exact;
    return a;
}

}  // namespace

bool field_attach(FieldScen* f, const std::string& path, const std::vector<sbe::Slot>& slots, int flags,
                  int envs_per_block, std::string* err) {
    f->slots = slots;
    f->G = (int)slots.size();
    const int G = f->G;
    if (!hip_ok(hipMalloc(&f->d_tables, f->A.host.size()), "hipMalloc(field env tables)", err)
        || !hip_ok(hipMemcpy(f->d_tables, f->A.host.data(), f->A.host.size(), hipMemcpyHostToDevice),
                   "upload field env tables", err))
        return false;
    for (auto& e : f->fix) *e.first = f->d_tables + e.second;
    f->A.host.clear();
    f->A.host.shrink_to_fit();
    f->exact = (flags & SBX_FDM_EXACT) ? 1 : 0;
    f->fdm = sbx_fdm_open(path.c_str(), G, envs_per_block, flags);
    if (!f->fdm) return (*err = std::string("field group: ") + sbx_last_error()), false;
    if (f->fdm->tab.k != f->t.k || f->fdm->tab.nz != f->t.nz || f->fdm->tab.n != f->t.n_solved)
        return (*err = "the field's air side, zones or solved cells do not match the HVAC tables"), false;
    // the records: zero, the streams seeded (sb_rng.c:9-16; position 624: the
    // first draw twists), the pump head at its constant
    const sbe::StateLayout& S = f->st;
    std::vector<unsigned char> rec((size_t)S.record * G, 0);
    for (int s = 0; s < G; s++) {
        unsigned char* r = rec.data() + (size_t)s * S.record;
        int* ip = reinterpret_cast<int*>(r + S.ip);
        mt_seed(reinterpret_cast<uint32_t*>(r + S.mt), slots[s].occ_seed);
        ip[sbe::IP_MT_IDX] = SBE_MT_N;
        if (S.cmt) {
            uint32_t* cmt = reinterpret_cast<uint32_t*>(r + S.cmt);
            mt_seed(cmt, slots[s].conv_seed);
            cmt[SBE_MT_N] = SBE_MT_N;   // position: the first draw twists
        }
        reinterpret_cast<double*>(r + S.plant)[sbe::PL_PUMP_HEAD] = f->t.pump_head0;
    }
    const size_t nz = (size_t)f->t.nz, k = (size_t)std::max(f->t.k, 1);
    if (!hip_ok(hipMalloc(&f->d_slots, sizeof(sbe::Slot) * G), "hipMalloc(field slots)", err)
        || !hip_ok(hipMemcpy(f->d_slots, slots.data(), sizeof(sbe::Slot) * G, hipMemcpyHostToDevice), "upload", err)
        || !hip_ok(hipMalloc(&f->d_state, rec.size()), "hipMalloc(field env state)", err)
        || !hip_ok(hipMemcpy(f->d_state, rec.data(), rec.size(), hipMemcpyHostToDevice), "upload", err)
        || !hip_ok(hipMalloc(&f->d_qz, 8 * nz * G), "hipMalloc", err)
        || !hip_ok(hipMalloc(&f->d_amb, 8 * (size_t)G), "hipMalloc", err)
        || !hip_ok(hipMalloc(&f->d_hh, 8 * (size_t)G), "hipMalloc", err)
        || !hip_ok(hipMalloc(&f->d_g, 8 * k * G), "hipMalloc", err)
        || !hip_ok(hipMalloc(&f->d_airT, 8 * k * G), "hipMalloc", err))
        return false;
    int lds = f->lds_bytes;
    if (f->t.cv_rooms > 0) {
        // the plan kernel keeps two MT blocks (raw and tempered), the room's
        // inverse permutation (u16) and candidate counts (u8) in LDS, and the
        // room's first pairs (the rest in HBM): room for 1.5 times the
        // expected count of the largest room, at least 2,048, so that two plan
        // wavefronts and a field-solve workgroup fit on one compute unit
        const int fixed = 4 * 4 * SBE_MT_N + 3 * f->t.cv_max_room + 16;
        const int room = 160 * 1024 - fixed;
        if (room < 6 * 1024) return (*err = "a convection room is too large for the plan kernel's LDS"), false;
        const double expect = 1.5 * std::min(std::max(f->conv_p, 0.0), 1.0) * f->t.cv_max_room;
        f->lds_pairs = std::min({f->t.cv_max_room, room / 6, std::max(2048, (int)expect)});
        lds = std::max(lds, fixed + 6 * f->lds_pairs);
        const size_t cells = (size_t)std::max(f->t.cv_cells, 1), mr = (size_t)std::max(f->t.cv_max_room, 1);
        if (!hip_ok(hipMalloc(&f->d_moves, 8 * cells * G), "hipMalloc(convection moves)", err)
            || !hip_ok(hipMalloc(&f->d_vals, 8 * cells * G), "hipMalloc(convection values)", err)
            || !hip_ok(hipMalloc(&f->d_count, 4 * (size_t)G), "hipMalloc", err)
            || !hip_ok(hipMemset(f->d_count, 0, 4 * (size_t)G), "clear", err)
            || !hip_ok(hipMalloc(&f->d_spill, 8 * mr * G), "hipMalloc(convection pairs)", err)
            || !hip_ok(hipStreamCreateWithFlags(&f->side, hipStreamNonBlocking), "convection stream", err)
            || !hip_ok(hipEventCreateWithFlags(&f->fork, hipEventDisableTiming), "event", err)
            || !hip_ok(hipEventCreateWithFlags(&f->join, hipEventDisableTiming), "event", err))
            return false;
    }
    if (lds > 64 * 1024 && !hip_ok((hipError_t)sbe_lds_limit(lds), "field env LDS limit", err)) return false;
    return true;
}

bool field_step(FieldScen* f, const FieldIo& io, bool reset, hipStream_t s, std::string* err) {
    sbe::Args a = base_args(f);
    a.mode = reset ? sbe::FE_RESET : sbe::FE_STEP;
    a.actions = io.actions;
    a.obs = io.obs;
    a.rewards = io.rewards;
    a.terminals = io.terminals;
    a.host_env = io.host_env;
    a.env_stride = io.env_stride;
    a.log_offset = io.log_offset;
    a.reward_scale = io.reward_scale;
    const sbf::Tables& T = f->fdm->tab;
    const sbf::Group& g = f->fdm->grp;
    if (reset) {
        return hip_ok((hipError_t)sbf_launch_init(&T, &g, f->fdm->d_temp_init, f->fdm->d_mass_init, s),
                      "field init", err)
               && hip_ok((hipError_t)sbe_launch(&a, 0, s), "field env reset", err);
    }
    const bool conv = f->t.cv_rooms > 0;
    const sbf::StepIn in{nullptr, f->d_amb, f->d_hh, f->d_g, f->d_airT, f->d_qz};
    // convection plan on the side stream, beside the pre-step and the field
    // step; the bound stream waits for it before the moves
    if (conv && !(hip_ok(hipEventRecord(f->fork, s), "fork", err)
                  && hip_ok(hipStreamWaitEvent(f->side, f->fork, 0), "fork", err)
                  && hip_ok((hipError_t)sbe_launch(&a, 4, f->side), "convection plan", err)
                  && hip_ok(hipEventRecord(f->join, f->side), "join", err)))
        return false;
    return hip_ok((hipError_t)sbe_launch(&a, 0, s), "field env pre-step", err)
           && hip_ok((hipError_t)sbf_launch_step(&T, &g, &in, s), "field step", err)
           && (!conv || hip_ok(hipStreamWaitEvent(s, f->join, 0), "join", err))
           && (!conv || hip_ok((hipError_t)sbe_launch(&a, 5, s), "convection moves", err))
           && hip_ok((hipError_t)sbe_launch(&a, 1, s), "field zone means", err)
           && hip_ok((hipError_t)sbe_launch(&a, 2, s), "field env post-step", err);
}

int field_state(FieldScen* f, int slot, double* out, int cap) {
    if (slot < 0 || slot >= f->G) return -1;
    const sbe::StateLayout& S = f->st;
    const sbe::Tabs& t = f->t;
    const sbf::Group& g = f->fdm->grp;
    const int n_cvs = t.n_cvs, n = f->fdm->tab.n;
    std::vector<unsigned char> r(S.bytes);
    const size_t b = (size_t)(slot / g.Gl), l = (size_t)(slot % g.Gl);
    std::vector<double> blk((size_t)std::max(n_cvs, n) * g.Gl);
    if (hipDeviceSynchronize() != hipSuccess) return -1;
    if (hipMemcpy(r.data(), f->d_state + (size_t)slot * S.record, S.bytes, hipMemcpyDeviceToHost) != hipSuccess)
        return -1;
    std::vector<double> o;
    if (hipMemcpy(blk.data(), g.T + b * n_cvs * g.Gl, 8 * (size_t)n_cvs * g.Gl, hipMemcpyDeviceToHost) != hipSuccess)
        return -1;
    for (int p = 0; p < n_cvs; p++) o.push_back(blk[(size_t)p * g.Gl + l]);
    if (hipMemcpy(blk.data(), g.M + b * n * g.Gl, 8 * (size_t)n * g.Gl, hipMemcpyDeviceToHost) != hipSuccess)
        return -1;
    for (int q = 0; q < n; q++) o.push_back(blk[(size_t)q * g.Gl + l]);
    const unsigned char* s = r.data();
    auto d = [&](int off) { return reinterpret_cast<const double*>(s + off); };
    for (int v = 0; v < t.nv; v++) o.push_back(d(S.damper)[v]);
    for (int v = 0; v < t.nv; v++) o.push_back(d(S.reheat)[v]);
    for (int v = 0; v < t.nv; v++) o.push_back(d(S.ratio)[v]);
    for (int v = 0; v < t.nv; v++) o.push_back(d(S.sensing)[v]);
    for (int q = 0; q < t.na; q++) o.push_back(d(S.flow)[q]);
    for (int q = 0; q < t.na; q++) o.push_back(d(S.sat)[q]);
    for (int q = 0; q < t.na; q++) o.push_back(d(S.recirc)[q]);
    for (int q = 0; q < t.na; q++) o.push_back(d(S.fan)[q]);
    for (int q = 0; q < t.k; q++) o.push_back(d(S.air_g)[q]);
    for (int q = 0; q < t.k; q++) o.push_back(d(S.air_T)[q]);
    for (int z = 0; z < t.nz; z++) o.push_back(d(S.occV)[z]);
    const double* pl = d(S.plant);
    const int* ip = reinterpret_cast<const int*>(s + S.ip);
    o.push_back(pl[sbe::PL_BOILER_CUR]);
    o.push_back(pl[sbe::PL_BOILER_RET]);
    o.push_back(pl[sbe::PL_BOILER_SP]);
    o.push_back(pl[sbe::PL_PUMP_HEAD]);
    o.push_back((double)ip[sbe::IP_STEP_INDEX]);
    o.push_back(pl[sbe::PL_REW_SUM]);
    o.push_back((double)ip[sbe::IP_STEPS_TOTAL]);
    if ((int)o.size() > cap) return -1;
    memcpy(out, o.data(), o.size() * sizeof(double));
    return (int)o.size();
}

bool field_live(FieldScen* f, double* out, int scen, hipStream_t s) {
    sbe::Args a = base_args(f);
    a.live = out;
    a.live_scen = scen;
    return sbe_launch(&a, 3, s) == 0;
}

double field_bytes_per_step(const FieldScen* f) {
    // the field group's step, plus per env its record read and written and
    // its action row, observation prefix, reward and terminal
    const double per_env = 2.0 * f->st.bytes + 4.0 * f->c.n_act + 4.0 * (f->t.n_dev + f->t.n_aux) + 8.0;
    return f->fdm->info.bytes_per_step + per_env * f->G;
}

double field_flops_per_step(const FieldScen* f) { return f->fdm->info.flops_per_step; }

void field_close(FieldScen* f) {
    if (!f) return;
    (void)hipDeviceSynchronize();
    if (f->fork) (void)hipEventDestroy(f->fork);
    if (f->join) (void)hipEventDestroy(f->join);
    if (f->side) (void)hipStreamDestroy(f->side);
    for (void* p : {(void*)f->d_tables, (void*)f->d_slots, (void*)f->d_state, (void*)f->d_qz, (void*)f->d_amb,
                    (void*)f->d_hh, (void*)f->d_g, (void*)f->d_airT, (void*)f->d_moves, (void*)f->d_count,
                    (void*)f->d_vals, (void*)f->d_spill})
        (void)hipFree(p);
    if (f->fdm) sbx_fdm_close(f->fdm);
    delete f;
}
