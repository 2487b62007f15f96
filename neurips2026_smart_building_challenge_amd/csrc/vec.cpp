// PufferLib env ABI for the MI355X env step (host side).
//
// puf_vec_create mirrors the reference GPU vec (complete_port/gpu/
// smart_buildings.cu:2497-2880): scenarios come from env.blob or every *.sbb of
// env.blob_dir (sorted, then round-robin over buildings, :2435-2459), G groups
// (env.groups, default n/32) get n/G envs each, and every env then steps in one
// fused kernel launch per puf_step. Unlike the reference there is no per-group
// solver (no SB_NE cap, no weather merging): envs of different layouts and
// climates share one launch and read their own tables.
#include <dirent.h>
#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <cmath>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "canon.h"
#include "field_host.h"
#include "plan.h"
#include "sbb_reader.h"
#include "sbenv.h"
#include "sbenv_internal.h"

static_assert(sbh::kPlanKmax == SBK_KMAX && sbh::kPlanDepth == SBK_PLAN_DEPTH && sbh::kWordTail >= SBK_KMAX,
              "the kernel's pass registers and prefetch depth match the planner's");

extern "C" int sbk_launch_step(const sbk::KParams* p, int n_blocks, int threads, int lds_bytes, int variant,
                               hipStream_t s);
extern "C" int sbk_set_lds_limit(int width, int bytes);
extern "C" int sbk_launch_policy(const float* obs, const float* w1, const float* b1, const float* w2,
                                 const float* b2, const float* w3, const float* b3, float* h1, float* h2, float* y,
                                 float* actions, const int* n_cont, const int* n_disc, int n, uint64_t seed,
                                 uint32_t step, float* draws, float* hlp, float* hent, float* logp, float* entropy,
                                 float floor, int obs_cols, hipStream_t s);
extern "C" int sbk_launch_beta_eval(const float* y, const float* draws, const int* n_cont, const int* n_disc, int n,
                                    float* hlp, float* hent, float* grad, float* logp, float* entropy, float floor,
                                    hipStream_t s);
extern "C" int sbk_launch_ppo_beta(const float* y_new, const float* y_old, const float* draws, const float* logp_old,
                                   const float* adv, const int* n_cont, const int* n_disc, int n, float floor,
                                   float clip, float ent_coef, int per_dim, float* out, float* grad, hipStream_t s);
extern "C" int sbk_launch_beta_sample(const float* alpha, const float* beta, float* out, int n, uint64_t seed,
                                      hipStream_t s);
extern "C" int sbk_noalloc_max_envs(void);
extern "C" int sbk_launch_policy_noalloc(const float* obs, const float* w1, const float* b1, const float* w2,
                                         const float* b2, const float* w3, const float* b3, float* actions,
                                         const int* n_cont, const int* n_disc, int n, uint64_t seed, uint32_t step,
                                         float floor, int obs_cols, hipStream_t s);
extern "C" int sbk_launch_canon(const sbk::CanonArgs* a, int post, hipStream_t s);
extern "C" int sbk_launch_live_sums(const sbk::EnvDesc* envs, const sbk::DevLayout* layouts,
                                    const unsigned char* state, int n, int n_scen, double* out, hipStream_t s);
extern "C" int sbk_launch_gen_actions(float* actions, const int* n_cont, const int* n_disc, int n_envs,
                                      uint64_t seed, uint32_t step, hipStream_t s);

namespace {

hipStream_t g_stream = nullptr;
std::string g_err;
struct Vec;
Vec* g_last = nullptr;

[[noreturn]] void die(const std::string& msg) {
    fprintf(stderr, "smart_buildings: %s\n", msg.c_str());
    abort();
}

void hip_ok(hipError_t e, const char* what) {
    if (e != hipSuccess) die(std::string(what) + ": " + hipGetErrorString(e));
}

// ---------------------------------------------------------------- arena
struct Arena {
    std::vector<unsigned char> host;
    size_t add(const void* p, size_t bytes) {
        size_t off = (host.size() + 255) & ~(size_t)255;
        host.resize(off + bytes + 1, 0);
        if (bytes) memcpy(host.data() + off, p, bytes);
        return off;
    }
    template <class T>
    size_t vec(const std::vector<T>& v) { return add(v.data(), v.size() * sizeof(T)); }
};

template <class T>
const T* at(unsigned char* base, size_t off) { return reinterpret_cast<const T*>(base + off); }

int align_up(int x, int a) { return (x + a - 1) / a * a; }

uint64_t splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

// ---------------------------------------------------------------- layouts
// Host-side tables of one layout; offsets into the arena.
struct HostLayout {
    std::string key;
    sbh::SolvePlan plan;
    sbh::RelaxPlan relax;
    sbh::BlockPlan block;
    sbk::DevLayout dev{};   // sizes + layouts; pointers patched after upload
    std::map<std::string, size_t> off;
    std::unique_ptr<sbk::CanonTab> canon;   // canonical maps (canonical mode only)
    int field = -1;         // a field scenario's stand-in (counts only; its envs are not tiled)
};

struct HostScen {
    std::string path;
    int layout = -1;
    sbk::DevScen dev{};
    std::map<std::string, size_t> off;
    int n1 = 0;
    int episode_steps = 0;
    int64_t occ_seed = 17321;
    int64_t conv_seed = 0;
    int hour_m1_rows = 0;
    int n_cont = 0, n_disc = 0;
    int field = -1;         // index into Vec::fields (FDM-scale scenario)
};

const char* kStructural[] = {
    "grid", "solved", "A_system_indptr", "A_system_indices", "A_system_data", "lu_perm_r", "lu_perm_c",
    "lu_L_indptr", "lu_L_indices", "lu_U_indptr", "lu_U_indices", "capacitance_rate", "mass_coupling",
    "mass_retained", "mass_gained", "solar_gain_coeff", "applied_indptr", "applied_indices", "applied_data",
    "sensed_indptr", "sensed_indices", "sensed_data", "zone_area", "phys_room_idx", "room_offsets",
    "room_cells", "vav_zone_offsets", "vav_zone_idx", "vav_ahu_idx", "coupled_vav_idx", "ahu_const",
    "vav_const", "act_owner_kind", "act_owner_index", "act_actuator", "act_is_discrete", "act_min_native",
    "act_max_native", "act_min_norm", "act_max_norm", "f_dev_kind", "f_dev_idx", "f_obs_id", "f_norm_mean",
    "f_norm_var", "n_dev", "n_aux", "occ_params", "conv_room_offsets", "conv_room_cells", "conv_cand_offsets",
    "conv_cand_idx", "field_names", "sched_scalars", nullptr};

std::string structural_key(const sbh::Blob& b) {
    std::string k;
    for (int i = 0; kStructural[i]; i++) {
        std::string s = b.bytes(kStructural[i]);
        k += std::to_string(s.size()) + ":" + s;
    }
    return k;
}

// The canonical maps of one layout, found by name in the blob's observation
// field names and its action owner tables as the reference does
// (complete_port/gpu/smart_buildings.cu:844-1000 sb_canon_setup): zone slots
// in the order the VAV temperature fields appear, slot 10 k + j on AHU k.
bool make_canon(const sbh::Blob& b, sbk::CanonTab* C, std::string* err) {
    memset(C, 0, sizeof(*C));
    const sbh::Section* fs = b.find("field_names");
    uint64_t cnt = 0;
    const uint8_t* fk = b.u8("f_dev_kind");
    const int32_t* fi = b.i32("f_dev_idx");
    const uint8_t* fo = b.u8("f_obs_id");
    const double* fmn = b.f64("f_norm_mean");
    const double* fvr = b.f64("f_norm_var");
    const int32_t* vai = b.i32("vav_ahu_idx", &cnt);
    const int nv = (int)cnt;
    const double* sc = b.f64("sched_scalars", &cnt);
    if (!fs || fs->dtype != sbh::STR || !fk || !fi || !fo || !fmn || !fvr || !vai || !sc || cnt < 6)
        return (*err = "canonical mode needs the blob's field_names and sched_scalars"), false;
    const uint8_t* ok_ = b.u8("act_owner_kind", &cnt);
    const int n_act = (int)cnt;
    const int32_t* oi = b.i32("act_owner_index");
    const uint8_t* oa = b.u8("act_actuator");
    const uint8_t* isd = b.u8("act_is_discrete");
    const double* ahu = b.f64("ahu_const", &cnt);
    if (!ok_ || !oi || !oa || !isd || !ahu) return (*err = "action tables missing"), false;
    const int n_dev = (int)b.i64_1("n_dev", 0);
    std::vector<std::string> names;
    {
        std::string cur;
        for (uint64_t i = 0; i < fs->count; i++) {
            const char ch = (char)fs->data[i];
            if (ch == '\n') { names.push_back(cur); cur.clear(); } else cur += ch;
        }
        names.push_back(cur);
    }
    auto find = [&](const std::string& nm) -> int {
        for (size_t i = 0; i < names.size(); i++)
            if (names[i] == nm) return (int)i;
        return -1;
    };
    C->K = (int)(cnt / 9);
    C->n_act = n_act;
    if (C->K > SBC_K) return (*err = "more AHUs than the canonical slots (9)"), false;
    for (int i = 0; i < SBC_ZS; i++) C->zT[i] = C->zH[i] = C->zC[i] = C->zD[i] = C->zR[i] = C->zAd[i] = C->zAr[i] = -1;
    for (int k = 0; k < SBC_K; k++) {
        for (int m = 0; m < 8; m++) C->aObs[k][m] = -1;
        C->aT[k] = C->aP[k] = C->aRec[k] = C->aRun[k] = -1;
    }
    C->hW = C->hDPa = C->hRun = -1;
    std::vector<int> vav_slot(nv, -1);
    const std::string zsuf = "zone_air_temperature_sensor";
    for (int i = 0; i < n_dev && i < (int)names.size(); i++) {
        if (fk[i] != 1 || fo[i] != 5) continue;
        const int v = fi[i];
        if (v < 0 || v >= nv) return (*err = "observation field of an unknown VAV"), false;
        const int a = vai[v];
        if (a < 0 || a >= SBC_K || C->zc[a] >= SBC_ZPA)
            return (*err = "an AHU serves more zones than the canonical slots (10)"), false;
        const int sl = SBC_ZPA * a + C->zc[a]++;
        vav_slot[v] = sl;
        const std::string& full = names[i];
        if (full.size() < zsuf.size()) return (*err = "bad zone temperature field name"), false;
        const std::string pre = full.substr(0, full.size() - zsuf.size());
        C->zT[sl] = i;
        C->zH[sl] = find(pre + "zone_air_heating_temperature_setpoint_sensor");
        C->zC[sl] = find(pre + "zone_air_cooling_temperature_setpoint_sensor");
        C->zD[sl] = find(pre + "supply_air_damper_percentage_command");
        C->zR[sl] = find(pre + "reheat_valve_percentage_command");
    }
    static const char* ahu_meas[8] = {"outside_air_temperature_sensor", "supply_air_static_pressure_sensor",
                                      "supply_air_flowrate_sensor", "outside_air_flowrate_sensor",
                                      "supply_air_temperature_setpoint", "recirculation_percentage_command",
                                      "cooling_request_count", "supervisor_run_command"};
    for (int k = 0; k < C->K; k++)
        for (int m = 0; m < 8; m++) C->aObs[k][m] = find("ahs_ahu_" + std::to_string(k + 1) + "_" + ahu_meas[m]);
    static const char* hws[6] = {"hws_supply_water_temperature_sensor", "hws_supply_water_temperature_setpoint",
                                 "hws_differential_pressure_sensor", "hws_differential_pressure_setpoint",
                                 "hws_run_status", "hws_heating_request_count"};
    for (int m = 0; m < 6; m++) C->hObs[m] = find(hws[m]);
    for (int h = 0; h < 4; h++) {
        char buf[32];
        snprintf(buf, sizeof buf, "hod_sin_%03d", h); C->g[h] = find(buf);
        snprintf(buf, sizeof buf, "hod_cos_%03d", h); C->g[4 + h] = find(buf);
        snprintf(buf, sizeof buf, "dow_sin_%03d", h); C->g[8 + h] = find(buf);
        snprintf(buf, sizeof buf, "dow_cos_%03d", h); C->g[12 + h] = find(buf);
    }
    C->g[16] = find("comfort_mode_now");
    C->g[17] = find("comfort_mode_soon");
    C->g[18] = find("num_occupants");
    if (C->g[0] < 0 || C->g[4] < 0 || C->g[8] < 0 || C->g[12] < 0)
        return (*err = "canonical mode needs the hod/dow time features"), false;
    for (int i = 0; i < SB_OBS; i++) {
        C->fmean[i] = 0.0f;
        C->fstd[i] = 1.0f;
    }
    for (int i = 0; i < n_dev && i < SB_OBS; i++)
        if (fvr[i] > 0.0) {
            C->fmean[i] = (float)fmn[i];
            C->fstd[i] = (float)sqrt(fvr[i]);
        }
    for (int sl = 0; sl < SBC_ZS; sl++)
        if (C->zT[sl] >= 0) {
            C->tmean = C->fmean[C->zT[sl]];
            C->tstd = C->fstd[C->zT[sl]];
            break;
        }
    C->morning = (int)sc[0];
    C->evening = (int)sc[1];
    C->comfort_lo = sc[2];
    C->comfort_hi = sc[3];
    C->eco_lo = sc[4];
    C->eco_hi = sc[5];
    for (int c = 0; c < SB_ACT; c++) C->act_of_col[c] = -1;
    int nc = 0, nd = 0;
    for (int a = 0; a < n_act; a++) {
        C->act_disc[a] = isd[a] ? 1 : 0;
        const int col = isd[a] ? SB_CONT + nd++ : nc++;
        if (col >= SB_ACT || (isd[a] && nd > SB_DISC) || (!isd[a] && nc > SB_CONT))
            return (*err = "too many actions"), false;
        C->act_of_col[col] = a;
        C->slot_of_action[a] = -1;
        if (ok_[a] == 1) {
            const int sl = (oi[a] >= 0 && oi[a] < nv) ? vav_slot[oi[a]] : -1;
            if (sl < 0) continue;
            if (oa[a] == 0) { C->zAd[sl] = a; C->slot_of_action[a] = 2 * sl; }
            else { C->zAr[sl] = a; C->slot_of_action[a] = 2 * sl + 1; }
        } else if (ok_[a] == 0) {
            const int k = oi[a];
            if (k < 0 || k >= SBC_K || oa[a] > 3) continue;
            if (oa[a] == 0) C->aT[k] = a;
            else if (oa[a] == 1) C->aP[k] = a;
            else if (oa[a] == 2) C->aRec[k] = a;
            else C->aRun[k] = a;
            C->slot_of_action[a] = SBC_AA + 4 * k + oa[a];
        } else if (oa[a] <= 2) {
            if (oa[a] == 0) C->hW = a;
            else if (oa[a] == 1) C->hDPa = a;
            else C->hRun = a;
            C->slot_of_action[a] = SBC_AH + oa[a];
        }
    }
    return true;
}

template <class T>
std::vector<T> take(const T* p, uint64_t n) { return p ? std::vector<T>(p, p + n) : std::vector<T>(); }

// Packs tables into one byte image with 16-byte aligned sections (the LDS
// images the step kernel stages in one burst).
struct ImgBuilder {
    std::vector<unsigned char> bytes;
    template <class T>
    int add(const std::vector<T>& v) {
        const size_t off = (bytes.size() + 15) & ~(size_t)15;
        bytes.resize(off + v.size() * sizeof(T), 0);
        if (!v.empty()) memcpy(bytes.data() + off, v.data(), v.size() * sizeof(T));
        return (int)off;
    }
    int finish() {
        bytes.resize((bytes.size() + 15) & ~(size_t)15, 0);
        return (int)bytes.size();
    }
};

enum { SOLVE_AUTO = 0, SOLVE_LU = 1, SOLVE_RELAX = 2, SOLVE_POINT = 3 };

// Builds one layout's tables (everything shared by its scenarios). `solve`
// picks the field solver: AUTO takes block-Jacobi relaxation where it is
// certified, else point Jacobi where that is, else the LU plan; RELAX the
// same without the LU fallback; POINT and LU force those forms.
bool make_layout(const sbh::Blob& b, int width, int solve, HostLayout* H, Arena& A, std::string* err) {
    if (!sbh::build_plan(b, width, &H->plan, err)) return false;
    const sbh::SolvePlan& P = H->plan;
    sbh::build_relax(b, P, &H->relax);
    sbh::build_block(b, P, &H->block);
    const sbh::RelaxPlan& R = H->relax;
    const sbh::BlockPlan& BP = H->block;
    const bool use_block = (solve == SOLVE_AUTO || solve == SOLVE_RELAX) && BP.ok && (!R.ok || BP.rho < R.rho);
    if (solve == SOLVE_RELAX && !BP.ok && !R.ok)
        return (*err = "relaxation solver not applicable: " + R.why + "; " + BP.why), false;
    if (solve == SOLVE_POINT && !R.ok) return (*err = "point relaxation not applicable: " + R.why), false;
    const bool relax = use_block || solve == SOLVE_POINT || ((solve == SOLVE_AUTO || solve == SOLVE_RELAX) && R.ok);
    sbk::DevLayout& D = H->dev;
    uint64_t cnt = 0;
    const int n = P.n;
    const int64_t* grid = b.i64("grid");
    const int nc_grid = (int)grid[1];
    const double* ahu_c = b.f64("ahu_const", &cnt);
    if (!ahu_c || cnt % 9) return (*err = "ahu_const missing"), false;
    const int na = (int)(cnt / 9);
    const int32_t* vz_off = b.i32("vav_zone_offsets", &cnt);
    if (!vz_off) return (*err = "vav_zone_offsets missing"), false;
    const int nv = (int)cnt - 1;
    const double* zone_area = b.f64("zone_area", &cnt);
    const int nz = (int)cnt;
    const int32_t* vz_idx = b.i32("vav_zone_idx");
    const int32_t* vav_ahu = b.i32("vav_ahu_idx");
    const int32_t* coupled = b.i32("coupled_vav_idx");
    const int32_t* phys = b.i32("phys_room_idx");
    const int32_t* room_off = b.i32("room_offsets");
    const int32_t* room_cells = b.i32("room_cells");
    const double* vav_c = b.f64("vav_const");
    if (!zone_area || !vz_idx || !vav_ahu || !phys || !room_off || !room_cells || !vav_c)
        return (*err = "HVAC topology sections missing"), false;
    if (na > SBK_MAX_AHU) return (*err = "too many AHUs"), false;
    const int k = P.k;
    if (k > 0 && !coupled) return (*err = "coupled_vav_idx missing"), false;
    if (k > nv) return (*err = "more coupled columns than VAVs"), false;
    if (nv > 64 * SBK_VPL) return (*err = "more than 256 VAVs per building"), false;
    if (nz > 64 * SBK_VPL) return (*err = "more than 256 zones per building"), false;
    for (int c = 0; c < k; c++)
        if (coupled[c] < 0 || coupled[c] >= nv) return (*err = "coupled_vav_idx out of range"), false;
    for (int v = 0; v < nv; v++)
        if (vav_ahu[v] < 0 || vav_ahu[v] >= na) return (*err = "vav_ahu_idx out of range"), false;
    // zones -> cells
    std::vector<int> zoff(1, 0), zcells;
    std::vector<uint8_t> is_room(n, 0);
    int max_cells = 0;
    for (int z = 0; z < nz; z++) {
        int rm = phys[z];
        for (int t = room_off[rm]; t < room_off[rm + 1]; t++) {
            int p = room_cells[2 * t] * nc_grid + room_cells[2 * t + 1];
            if (p < 0 || p >= n) return (*err = "room cell outside the grid"), false;
            zcells.push_back(p);
            is_room[p] = 1;
        }
        zoff.push_back((int)zcells.size());
        max_cells = std::max(max_cells, zoff[z + 1] - zoff[z]);
        if (zoff[z + 1] == zoff[z]) return (*err = "zone without cells"), false;
    }
    std::vector<double> vav_area(nv, 0.0);
    for (int v = 0; v < nv; v++) {
        double a = 0.0;
        for (int t = vz_off[v]; t < vz_off[v + 1]; t++) a += zone_area[vz_idx[t]];
        vav_area[v] = a;
        if (!(a > 0.0)) return (*err = "VAVs without zone area are not supported"), false;
    }
    // zone -> coupled columns feeding it, ascending column
    std::vector<int> zcol_off(1, 0), zcols;
    {
        std::vector<std::vector<int>> per(nz);
        for (int c = 0; c < k; c++) {
            int v = coupled[c];
            for (int t = vz_off[v]; t < vz_off[v + 1]; t++) per[vz_idx[t]].push_back(c);
        }
        for (int z = 0; z < nz; z++) {
            zcols.insert(zcols.end(), per[z].begin(), per[z].end());
            zcol_off.push_back((int)zcols.size());
        }
    }
    // actions
    const uint8_t* kind = b.u8("act_owner_kind", &cnt);
    const int n_act = (int)cnt;
    const uint8_t* act = b.u8("act_actuator");
    const uint8_t* disc = b.u8("act_is_discrete");
    const int32_t* aidx = b.i32("act_owner_index");
    const double* mn = b.f64("act_min_native");
    const double* mx = b.f64("act_max_native");
    const double* mnr = b.f64("act_min_norm");
    const double* mxr = b.f64("act_max_norm");
    if (!kind || !act || !disc || !aidx || !mn || !mx || !mnr || !mxr) return (*err = "action tables missing"), false;
    std::vector<int> src(n_act);
    int ncont = 0, ndisc = 0;
    std::map<long long, int> targets;
    for (int i = 0; i < n_act; i++) {
        src[i] = disc[i] ? SB_CONT + ndisc++ : ncont++;
        long long key = ((long long)kind[i] << 40) | ((long long)aidx[i] << 8) | act[i];
        if (targets.count(key)) return (*err = "two actions drive the same actuator"), false;
        targets[key] = i;
    }
    if (ncont > SB_CONT || ndisc > SB_DISC) return (*err = "scenario has more actions than SB_CONT/SB_DISC"), false;
    // observation
    const int n_dev = (int)b.i64_1("n_dev", 0), n_aux = (int)b.i64_1("n_aux", 0);
    if (n_aux < 1 || n_aux > SBK_NAUX_MAX) return (*err = "n_aux out of range"), false;
    if (n_dev + n_aux > SB_OBS) return (*err = "observation larger than OBS_SIZE"), false;
    const uint8_t* fk = b.u8("f_dev_kind");
    const uint8_t* fo = b.u8("f_obs_id");
    const int32_t* fi = b.i32("f_dev_idx");
    const double* fm = b.f64("f_norm_mean");
    const double* fv = b.f64("f_norm_var");
    if (n_dev && (!fk || !fo || !fi || !fm || !fv)) return (*err = "observation map missing"), false;
    std::vector<double> fsd(n_dev);
    for (int i = 0; i < n_dev; i++) fsd[i] = fv[i] > 0.0 ? sqrt(fv[i]) : 0.0;
    // occupancy
    const double* op = b.f64("occ_params");
    if (!op) return (*err = "occ_params missing"), false;
    const int nassign = (int)op[0];
    if (nassign < 0 || nz * nassign > 312 || nz * nassign > 5 * width)
        return (*err = "too many occupants per env"), false;
    // convection rooms (complete_port/csim/sb_convect.c:6-31): cells -> nodes,
    // candidates as positions in the cell list
    std::vector<int> cv_off, cv_node, cv_coff, cv_cidx;
    int cv_max_room = 0;
    {
        uint64_t c_off = 0, c_cells = 0, c_coff = 0, c_idx = 0;
        const int32_t* ro = b.i32("conv_room_offsets", &c_off);
        const int32_t* rc = b.i32("conv_room_cells", &c_cells);
        const int32_t* co = b.i32("conv_cand_offsets", &c_coff);
        const int32_t* ci = b.i32("conv_cand_idx", &c_idx);
        if (!ro || !co || c_off < 1 || c_coff < 1) return (*err = "convection tables missing"), false;
        const int nrooms = (int)c_off - 1, ncells = (int)c_coff - 1;
        if (ro[0] != 0 || ro[nrooms] != ncells || (int)c_cells != 2 * ncells || co[0] != 0 || co[ncells] != (int)c_idx)
            return (*err = "convection tables inconsistent"), false;
        if (ncells > 0) {
            cv_off.assign(ro, ro + nrooms + 1);
            cv_coff.assign(co, co + ncells + 1);
            for (int r = 0; r < nrooms; r++) {
                if (ro[r + 1] < ro[r]) return (*err = "convection room offsets decrease"), false;
                cv_max_room = std::max(cv_max_room, ro[r + 1] - ro[r]);
            }
            if (cv_max_room > SBK_CV_ROOM) return (*err = "convection room with more than 64 cells"), false;
            if (ncells > 4 * 64) return (*err = "more than 256 convection cells per building"), false;
            if (nrooms > 64) return (*err = "more than 64 convection rooms per building"), false;
            for (int j = 0; j < ncells; j++) {
                const int p = rc[2 * j] * nc_grid + rc[2 * j + 1];
                if (p < 0 || p >= n) return (*err = "convection cell outside the solved field"), false;
                cv_node.push_back(p);
                if (co[j + 1] < co[j]) return (*err = "convection candidate offsets decrease"), false;
            }
            for (uint64_t j = 0; j < c_idx; j++) {
                if (ci[j] < 0 || ci[j] >= ncells) return (*err = "convection candidate out of range"), false;
                cv_cidx.push_back(ci[j]);
            }
        }
    }

    D.n = n; D.nz = nz; D.nv = nv; D.na = na; D.k = k; D.n_act = n_act; D.n_cont = ncont; D.n_disc = ndisc;
    D.n_dev = n_dev; D.n_aux = n_aux; D.nassign = nassign;
    D.n_slots = P.n_slots; D.vec_base = P.vec_base; D.n_pass = P.n_pass(); D.width = width;
    D.lu_sbase = P.term_bits == 12 ? P.scale_base : 0;
    D.max_room_cells = max_cells;
    D.solver = relax ? sbk::SOLVER_RELAX : sbk::SOLVER_LU;
    D.rx_block = use_block ? (BP.n_blocks > 64 ? 2 : 1) : 0;
    D.rx_terms = use_block ? BP.terms : (relax ? R.terms : 0);
    D.rx_stop = use_block ? BP.rho / (1.0 - BP.rho) : (relax ? R.rho / (1.0 - R.rho) : 0.0);
    if (relax) D.n_pass = 0;
    // state record
    sbk::StateLayout& S = D.st;
    int o = 0;
    auto f64a = [&](int count) { int r = o; o += 8 * count; return r; };
    S.T = f64a(n); S.M = f64a(n);
    S.damper = f64a(nv); S.reheat = f64a(nv); S.ratio = f64a(nv); S.heatsp = f64a(nv);
    S.coolsp = f64a(nv); S.dcmd = f64a(nv); S.rcmd = f64a(nv); S.sensing = f64a(nv);
    S.recirc = f64a(na); S.sat = f64a(na); S.fan = f64a(na); S.flow = f64a(na);
    S.plant = f64a(sbk::PF_COUNT);
    S.cal_n = sbk::RW_COUNT + std::max(n_aux - 1, 0);
    S.cal = f64a(2 * S.cal_n);
    S.run = o; o += 4 * na; S.coolreq = o; o += 4 * na; S.iplant = o; o += 4 * sbk::PI_COUNT;
    S.mode = o; o += nv; S.prev_valid = o; o += nv; S.dcmd_set = o; o += nv; S.rcmd_set = o; o += nv;
    S.occ_state = o; o += nz * nassign; S.occV = o; o += nz;
    S.bytes = align_up(o, 16);
    // HBM record: the image, then (convection) the convection stream state,
    // which the staging burst copies with the image into the env's MT scratch
    // in LDS (it follows the image there too), then the occupancy stream state
    S.cmt = cv_node.empty() ? 0 : S.bytes;
    S.mt = S.bytes + (cv_node.empty() ? 0 : 4 * SBK_MT_N);
    S.record_bytes = align_up(S.bytes + 4 * SBK_MT_N * (cv_node.empty() ? 1 : 2), 256);
    // per-env LDS region: record image, MT words (filled when a draw twists),
    // scenario image, action row, then scratch
    sbk::LdsLayout& Ls = D.lds;
    int l = 0;
    Ls.state = 0; l = S.bytes;
    Ls.mt = l; l += 4 * SBK_MT_N; l = align_up(l, 16);
    Ls.scen = l; l += align_up(8 * n, 16) + 8 * 84;
    Ls.act = l; l += 4 * SB_ACT;
    // slots: the LU entries and vector, or (relaxation) the node heat inputs
    Ls.slots = l; l += 8 * (relax ? n : P.n_slots); l = align_up(l, 16);
    Ls.zq = l; l += 8 * nz;
    Ls.vtmp = l; l += 8 * 4 * nv;
    Ls.g = l; l += 8 * std::max(k, 1);
    Ls.tair = l; l += 8 * std::max(k, 1);
    Ls.atmp = l; l += 8 * 8 * na;
    Ls.red = l; l += 8 * 64;
    Ls.misc = l; l += 8 * sbk::MS_SIZE;
    Ls.obsx = l; l += 8 * (sbk::OX_AHU + 4 * na);
    Ls.iscr = l; l += 4 * (width / 64 + 8);
    l = align_up(l, 16);
    Ls.occn = l; l += nz * nassign + nz;
    l = align_up(l, 16);
    Ls.hzq = l; l += 8 * nz;
    l = align_up(l, 16);
    Ls.sync = l; l += 4 * sbk::SY_WORDS;
    l = align_up(l, 16);
    Ls.stamps = l; l += 8 * SBK_NSTAMP;
    Ls.prec = l; l += 16 * D.n_pass;
    Ls.cvwin = Ls.cvsig = Ls.cvl = Ls.cvr = 0;
    if (!cv_node.empty()) {
        l = align_up(l, 16);
        Ls.cvwin = l; l += 4 * SBK_CV_WIN;
        Ls.cvsig = l; l += 4 * (int)cv_node.size();
        Ls.cvl = l; l += 4 * cv_max_room;
        Ls.cvr = l; l += 4 * cv_max_room;
    }
    Ls.bytes = align_up(l, 16);
    D.cv_rooms = cv_node.empty() ? 0 : (int)cv_off.size() - 1;
    D.cv_cells = (int)cv_node.size();
    D.cv_max_room = cv_max_room;
    // algorithmic bytes of one env-step: the persistent state a step must read
    // and write (T [8n], per VAV 7 f64 and a flag byte [57 nv], per AHU 3 f64
    // and a flag byte [25 na], 48 B of plant scalars, occupant counts [nz] and
    // chain bits [nz * nassign / 8]; interior mass [8n] where any node has
    // it), the action row read, the observation prefix (n_dev + n_aux floats),
    // reward and terminal written; shared per-layout and per-scenario tables
    // are not counted (one copy serves every env of the layout or scenario)
    {
        bool mass = false;
        const double* mc = b.f64("mass_coupling");
        const double* mg = b.f64("mass_gained");
        for (int t = 0; t < n && !mass; t++) mass = mc[t] != 0.0 || mg[t] != 0.0;
        const double state = 8.0 * n + 57.0 * nv + 25.0 * na + 48.0 + nz + (nz * nassign + 7) / 8 + (mass ? 8.0 * n : 0.0);
        D.bytes_per_step = 2.0 * state + 4.0 * n_act + 4.0 * (n_dev + n_aux) + 8.0;
        if (S.cmt) D.bytes_per_step += 4.0 * SBK_MT_N;   // the convection stream state, read every step
    }
    // what this kernel actually moves for it: the record image (without the
    // calendar prefetch, a copy of shared per-scenario tables) read and
    // written, the action row, the observation prefix, reward and terminal
    D.record_bytes_per_step = 2.0 * (S.bytes - 16.0 * S.cal_n) + 4.0 * (ncont + ndisc) + 4.0 * (n_dev + n_aux) + 8.0;
    if (S.cmt) D.record_bytes_per_step += 4.0 * SBK_MT_N;
    D.solve_flops = 2.0 * (double)P.n_pairs + (double)P.n_divs;
    if (use_block) {   // per sweep: off-block multiply-subtracts, then each block's inverse applied
        long long nnz = 0, dense = 0;
        for (double x : BP.val) nnz += x != 0.0;
        for (const auto& blk : BP.blocks) dense += (long long)blk.size() * (long long)blk.size();
        D.solve_flops = 2.0 * (double)(nnz + dense);
    } else if (relax) {   // per sweep: one multiply-subtract per off-diagonal entry, one scaling per row
        long long nnz = 0;
        for (int i = 0; i < n; i++)
            for (int m = 0; m < sbh::kRelaxTerms; m++) nnz += R.val[(size_t)m * sbh::kRelaxRows + i] != 0.0;
        D.solve_flops = 2.0 * (double)nnz + (double)n;
    }

    auto& O = H->off;
    O["rx_diag"] = A.vec(R.ok ? R.diag : std::vector<double>(sbh::kRelaxRows, 1.0));
    O["rx_air"] = A.vec(R.ok ? R.air_col : std::vector<int>(sbh::kRelaxRows, -1));
    O["rx_val"] = A.vec(R.ok ? R.val : std::vector<double>((size_t)sbh::kRelaxTerms * sbh::kRelaxRows, 0.0));
    O["rx_col"] = A.vec(R.ok ? R.col : std::vector<int>((size_t)sbh::kRelaxTerms * sbh::kRelaxRows, 0));
    O["pinfo"] = A.add(P.passes.data(), P.passes.size() * sizeof(sbh::PassInfo));
    O["hdr"] = A.vec(P.hdr);
    O["words"] = A.vec(P.words);
    O["slot_init"] = A.vec(P.slot_init);
    O["pos"] = A.vec(P.pos);
    O["air_slot"] = A.vec(P.air_slot);
    O["air_node"] = A.vec(P.air_node);
    O["cap"] = A.vec(take(b.f64("capacitance_rate"), n));
    O["mcoup"] = A.vec(take(b.f64("mass_coupling"), n));
    O["mret"] = A.vec(take(b.f64("mass_retained"), n));
    O["mgain"] = A.vec(take(b.f64("mass_gained"), n));
    {
        uint64_t c2 = 0;
        const double* sc = b.f64("solar_gain_coeff", &c2);
        std::vector<double> v(n, 0.0);
        if (sc && (int)c2 == n) v.assign(sc, sc + n);
        O["solar_c"] = A.vec(v);
    }
    if (!b.f64("capacitance_rate") || !b.f64("mass_coupling") || !b.f64("mass_retained") || !b.f64("mass_gained"))
        return (*err = "field sections missing"), false;
    O["is_room"] = A.vec(is_room);
    O["zone_cell_off"] = A.vec(zoff);
    O["zone_cells"] = A.vec(zcells);
    O["zone_area"] = A.vec(take(zone_area, nz));
    O["vz_off"] = A.vec(take(vz_off, nv + 1));
    O["vz_idx"] = A.vec(take(vz_idx, vz_off[nv]));
    O["vav_area"] = A.vec(vav_area);
    O["vav_ahu"] = A.vec(take(vav_ahu, nv));
    O["coupled"] = A.vec(take(coupled, k));
    O["zone_col_off"] = A.vec(zcol_off);
    O["zone_cols"] = A.vec(zcols);
    O["vav_c"] = A.vec(take(vav_c, 9 * nv));
    O["ahu_c"] = A.vec(take(ahu_c, 9 * na));
    O["act_kind"] = A.vec(take(kind, n_act));
    O["act_act"] = A.vec(take(act, n_act));
    O["act_disc"] = A.vec(take(disc, n_act));
    O["act_idx"] = A.vec(take(aidx, n_act));
    O["act_src"] = A.vec(src);
    O["act_mn"] = A.vec(take(mn, n_act));
    O["act_mx"] = A.vec(take(mx, n_act));
    O["act_mnr"] = A.vec(take(mnr, n_act));
    O["act_mxr"] = A.vec(take(mxr, n_act));
    O["f_kind"] = A.vec(take(fk, n_dev));
    O["f_id"] = A.vec(take(fo, n_dev));
    O["f_idx"] = A.vec(take(fi, n_dev));
    O["f_mean"] = A.vec(take(fm, n_dev));
    O["f_sd"] = A.vec(fsd);
    // the layout image the step kernel stages into LDS (one copy per workgroup)
    {
        ImgBuilder I;
        sbk::ImgLayout& G = D.img;
        uint64_t c2 = 0;
        const double* sc = b.f64("solar_gain_coeff", &c2);
        std::vector<double> solar(n, 0.0);
        if (sc && (int)c2 == n) solar.assign(sc, sc + n);
        G.cap = I.add(take(b.f64("capacitance_rate"), n));
        G.mcoup = I.add(take(b.f64("mass_coupling"), n));
        G.mret = I.add(take(b.f64("mass_retained"), n));
        G.mgain = I.add(take(b.f64("mass_gained"), n));
        G.solar_c = I.add(solar);
        G.rx_diag = I.add(R.ok ? std::vector<double>(R.diag.begin(), R.diag.begin() + n) : std::vector<double>(n, 1.0));
        G.zone_area = I.add(take(zone_area, nz));
        G.vav_area = I.add(vav_area);
        G.vav_c = I.add(take(vav_c, 9 * nv));
        G.ahu_c = I.add(take(ahu_c, 9 * na));
        G.act_mn = I.add(take(mn, n_act));
        G.act_mx = I.add(take(mx, n_act));
        G.act_mnr = I.add(take(mnr, n_act));
        G.act_mxr = I.add(take(mxr, n_act));
        // action targets (complete_port/csim/sb_sim.c:220-244): AHU supply
        // temperature / fan static / recirculation (clamped to its maximum) /
        // run; VAV damper / reheat commands (clamped to [0, 1], with their set
        // flags); boiler setpoint / pump head (bar -> m) / HWS and pump run
        std::vector<uint32_t> adst(n_act), aaux(n_act, 0u);
        std::vector<double> ahi(n_act, 0.0);
        std::vector<uint8_t> aflag(n_act, 0);
        for (int i = 0; i < n_act; i++) {
            const int ix = aidx[i], ak = act[i];
            if (kind[i] == 0) {
                if (ix < 0 || ix >= na) return (*err = "action AHU index out of range"), false;
                if (ak == 0) adst[i] = (uint32_t)(S.sat + 8 * ix);
                else if (ak == 1) adst[i] = (uint32_t)(S.fan + 8 * ix);
                else if (ak == 2) {
                    adst[i] = (uint32_t)(S.recirc + 8 * ix);
                    aflag[i] = sbk::ACT_CLAMP;
                    ahi[i] = ahu_c[ix * 9 + 3];
                } else adst[i] = (uint32_t)(S.run + 4 * ix) | ACT_I32;
            } else if (kind[i] == 1) {
                if (ix < 0 || ix >= nv) return (*err = "action VAV index out of range"), false;
                aflag[i] = sbk::ACT_CLAMP;
                ahi[i] = 1.0;
                if (ak == 0) { adst[i] = (uint32_t)(S.dcmd + 8 * ix); aaux[i] = (uint32_t)(S.dcmd_set + ix) | ACT_AUX_U8; }
                else { adst[i] = (uint32_t)(S.rcmd + 8 * ix); aaux[i] = (uint32_t)(S.rcmd_set + ix) | ACT_AUX_U8; }
            } else {
                if (ak == 0) adst[i] = (uint32_t)(S.plant + 8 * sbk::PF_BOILER_SP);
                else if (ak == 1) { adst[i] = (uint32_t)(S.plant + 8 * sbk::PF_PUMP_HEAD); aflag[i] = sbk::ACT_PUMP_HEAD; }
                else {
                    adst[i] = (uint32_t)(S.iplant + 4 * sbk::PI_HWS_RUN) | ACT_I32;
                    aaux[i] = (uint32_t)(S.iplant + 4 * sbk::PI_PUMP_RUN) | ACT_AUX_I32;
                }
            }
        }
        G.act_hi = I.add(ahi);
        G.act_dst = I.add(adst);
        G.act_aux = I.add(aaux);
        G.act_flags = I.add(aflag);
        G.f_mean = I.add(take(fm, n_dev));
        G.f_sd = I.add(fsd);
        G.rx_air = I.add(R.ok ? std::vector<int>(R.air_col.begin(), R.air_col.begin() + n) : std::vector<int>(n, -1));
        G.pos = I.add(P.pos);
        G.zone_cell_off = I.add(zoff);
        G.zone_cells = I.add(zcells);
        G.vz_off = I.add(take(vz_off, nv + 1));
        G.vz_idx = I.add(take(vz_idx, vz_off[nv]));
        G.vav_ahu = I.add(take(vav_ahu, nv));
        G.coupled = I.add(take(coupled, k));
        G.zone_col_off = I.add(zcol_off);
        G.zone_cols = I.add(zcols);
        {
            std::vector<int> voff(1, 0), vl, coff(1, 0), cl;
            for (int a = 0; a < na; a++) {
                for (int v = 0; v < nv; v++)
                    if (vav_ahu[v] == a) vl.push_back(v);
                voff.push_back((int)vl.size());
                for (int c = 0; c < k; c++)
                    if (vav_ahu[coupled[c]] == a) cl.push_back(c);
                coff.push_back((int)cl.size());
            }
            G.ahu_vav_off = I.add(voff);
            G.ahu_vavs = I.add(vl);
            G.ahu_col_off = I.add(coff);
            G.ahu_cols = I.add(cl);
            // each entry's position in its AHU's list (the step writes per-AHU
            // sum terms there, so an AHU's terms are contiguous), and each
            // AHU's VAV area in the order the step would sum it
            std::vector<int> vpos(nv, -1), cpos(k, -1);
            for (int t = 0; t < (int)vl.size(); t++) vpos[vl[t]] = t;
            for (int t = 0; t < (int)cl.size(); t++) cpos[cl[t]] = t;
            for (int v = 0; v < nv; v++)
                if (vpos[v] < 0) return (*err = "VAV without an AHU"), false;
            for (int c = 0; c < k; c++)
                if (cpos[c] < 0) return (*err = "coupled column without an AHU"), false;
            std::vector<double> aarea(na, 0.0);
            for (int a = 0; a < na; a++)
                for (int t = voff[a]; t < voff[a + 1]; t++) aarea[a] += vav_area[vl[t]];
            G.vav_lpos = I.add(vpos);
            G.col_lpos = I.add(cpos);
            G.ahu_area = I.add(aarea);
        }
        G.act_src = I.add(src);
        G.air_slot = I.add(P.air_slot);
        G.air_node = I.add(P.air_node);
        G.bx_d = G.bx_i = 0;
        D.bx_nb = use_block ? BP.n_blocks : 0;
        if (use_block) {
            const int nb = BP.n_blocks, R = sbh::kBlockRows, T = sbh::kBlockTerms;
            static_assert(sbh::kBlockRows == 3 && sbh::kBlockTerms == 8, "chunk layout of the block tables");
            std::vector<double> bd((size_t)18 * nb, 0.0);
            std::vector<int32_t> bi((size_t)12 * nb, 0);
            for (int kb = 0; kb < nb; kb++) {
                const int q = kb / 64, ln = kb % 64;
                double rec[18] = {0.0};
                int32_t irec[12] = {0};
                static const int in_pairs[6][2] = {{0, 1}, {0, 2}, {1, 0}, {1, 2}, {2, 0}, {2, 1}};
                for (int p = 0; p < R; p++) {
                    const size_t at = (size_t)(q * R + p) * 64 + ln;
                    rec[p] = BP.diag[at];
                    irec[p] = (int32_t)(((uint32_t)BP.row[at] & 0xffffu) | ((uint32_t)BP.air[at] << 16));
                }
                for (int j = 0; j < 6; j++)
                    rec[3 + j] = BP.in[((size_t)(q * R + in_pairs[j][0]) * R + in_pairs[j][1]) * 64 + ln];
                for (int t = 0; t < T; t++) {
                    const size_t e = (size_t)(q * T + t) * 64 + ln;
                    rec[9 + t] = BP.val[e];
                    irec[4 + t] = (int32_t)((uint32_t)BP.col[e] | ((uint32_t)BP.trow[e] << 16));
                }
                for (int j = 0; j < 9; j++) {
                    bd[((size_t)j * nb + kb) * 2 + 0] = rec[2 * j];
                    bd[((size_t)j * nb + kb) * 2 + 1] = rec[2 * j + 1];
                }
                for (int j = 0; j < 3; j++)
                    for (int e = 0; e < 4; e++) bi[((size_t)j * nb + kb) * 4 + e] = irec[4 * j + e];
            }
            G.bx_d = I.add(bd);
            G.bx_i = I.add(bi);
        }
        G.cv_off = I.add(cv_off);
        G.cv_node = I.add(cv_node);
        G.cv_coff = I.add(cv_coff);
        G.cv_cidx = I.add(cv_cidx);
        G.is_room = I.add(is_room);
        G.act_disc = I.add(take(disc, n_act));
        // observation sources (the value each field reads; sb_obs.c:49-64 and
        // the device kinds of bake_env.py:228-248): AHU, VAV, then plant fields
        std::vector<uint32_t> fsrc(n_dev);
        for (int i = 0; i < n_dev; i++) {
            const int kd = fk[i], id = fo[i], ix = fi[i];
            auto env_f64 = [&](int off) { return (uint32_t)off; };
            auto env_i32 = [&](int off) { return (uint32_t)off | OBS_SRC_I32; };
            const int ox = Ls.obsx;
            uint32_t v;
            if (kd == 0) {
                if (ix < 0 || ix >= na) return (*err = "observation AHU index out of range"), false;
                const int ax = ox + 8 * (sbk::OX_AHU + 4 * ix);
                switch (id) {
                case 0: v = env_i32(S.coolreq + 4 * ix); break;
                case 1: v = env_f64(ax); break;
                case 2: v = env_f64(ax + 8); break;
                case 3: v = env_f64(S.sat + 8 * ix); break;
                case 4: case 7: v = env_i32(S.run + 4 * ix); break;
                case 5: v = env_f64(ax + 16); break;
                case 6: v = env_f64(ax + 24); break;
                case 8: v = env_f64(S.recirc + 8 * ix); break;
                default: v = env_f64(ox + 8 * sbk::OX_AMB);
                }
            } else if (kd == 1) {
                if (ix < 0 || ix >= nv) return (*err = "observation VAV index out of range"), false;
                switch (id) {
                case 0: v = env_f64(S.reheat + 8 * ix); break;
                case 1: v = env_f64(S.damper + 8 * ix); break;
                case 2: v = (uint32_t)(G.vav_c + 8 * 9 * ix) | OBS_SRC_IMG; break;
                case 3: v = env_f64(S.coolsp + 8 * ix); break;
                case 4: v = env_f64(S.heatsp + 8 * ix); break;
                default: v = env_f64(S.sensing + 8 * ix);
                }
            } else {
                switch (id) {
                case 0: case 2: v = env_f64(ox + 8 * sbk::OX_DP); break;
                case 1: v = env_f64(S.plant + 8 * sbk::PF_BOILER_CUR); break;
                case 3: case 5: v = env_i32(S.iplant + 4 * sbk::PI_HWS_RUN); break;
                case 4: v = env_i32(S.iplant + 4 * sbk::PI_HWS_REQ); break;
                default: v = env_f64(S.plant + 8 * sbk::PF_BOILER_SP);
                }
            }
            fsrc[i] = v;
        }
        G.f_src = I.add(fsrc);
        G.bytes = I.finish();
        O["img"] = A.vec(I.bytes);
    }
    return true;
}

void patch_layout(HostLayout* H, unsigned char* d) {
    sbk::DevLayout& D = H->dev;
    auto& O = H->off;
    D.img_src = at<unsigned char>(d, O["img"]);
    D.rx_diag = at<double>(d, O["rx_diag"]);
    D.rx_air = at<int>(d, O["rx_air"]);
    D.rx_val = at<double>(d, O["rx_val"]);
    D.rx_col = at<int>(d, O["rx_col"]);
    D.pinfo = at<int>(d, O["pinfo"]);
    D.hdr = at<uint64_t>(d, O["hdr"]);
    D.words = at<uint32_t>(d, O["words"]);
    D.slot_init = at<double>(d, O["slot_init"]);
    D.pos = at<int>(d, O["pos"]);
    D.air_slot = at<int>(d, O["air_slot"]);
    D.air_node = at<int>(d, O["air_node"]);
    D.cap = at<double>(d, O["cap"]);
    D.mcoup = at<double>(d, O["mcoup"]);
    D.mret = at<double>(d, O["mret"]);
    D.mgain = at<double>(d, O["mgain"]);
    D.solar_c = at<double>(d, O["solar_c"]);
    D.is_room = at<uint8_t>(d, O["is_room"]);
    D.zone_cell_off = at<int>(d, O["zone_cell_off"]);
    D.zone_cells = at<int>(d, O["zone_cells"]);
    D.zone_area = at<double>(d, O["zone_area"]);
    D.vz_off = at<int>(d, O["vz_off"]);
    D.vz_idx = at<int>(d, O["vz_idx"]);
    D.vav_area = at<double>(d, O["vav_area"]);
    D.vav_ahu = at<int>(d, O["vav_ahu"]);
    D.coupled = at<int>(d, O["coupled"]);
    D.zone_col_off = at<int>(d, O["zone_col_off"]);
    D.zone_cols = at<int>(d, O["zone_cols"]);
    D.vav_c = at<double>(d, O["vav_c"]);
    D.ahu_c = at<double>(d, O["ahu_c"]);
    D.act_kind = at<uint8_t>(d, O["act_kind"]);
    D.act_act = at<uint8_t>(d, O["act_act"]);
    D.act_disc = at<uint8_t>(d, O["act_disc"]);
    D.act_idx = at<int>(d, O["act_idx"]);
    D.act_src = at<int>(d, O["act_src"]);
    D.act_mn = at<double>(d, O["act_mn"]);
    D.act_mx = at<double>(d, O["act_mx"]);
    D.act_mnr = at<double>(d, O["act_mnr"]);
    D.act_mxr = at<double>(d, O["act_mxr"]);
    D.f_kind = at<uint8_t>(d, O["f_kind"]);
    D.f_id = at<uint8_t>(d, O["f_id"]);
    D.f_idx = at<int>(d, O["f_idx"]);
    D.f_mean = at<double>(d, O["f_mean"]);
    D.f_sd = at<double>(d, O["f_sd"]);
}

std::vector<uint8_t> to_u8(const int64_t* p, uint64_t n) {
    std::vector<uint8_t> v(n);
    for (uint64_t i = 0; i < n; i++) v[i] = (uint8_t)p[i];
    return v;
}

// Builds one scenario's tables (calendar, weather, prices, scalars).
bool make_scen(const sbh::Blob& b, const HostLayout& Lh, HostScen* H, Arena& A, std::string* err) {
    const sbk::DevLayout& L = Lh.dev;
    sbk::DevScen& D = H->dev;
    uint64_t c_amb = 0, c = 0;
    const double* amb = b.f64("weather_ambient", &c_amb);
    if (!amb) return (*err = "weather_ambient missing"), false;
    uint64_t n1 = c_amb;
    const char* f64_rows[] = {"sched_comfort", "sched_heat_sp", "sched_cool_sp", nullptr};
    for (int i = 0; f64_rows[i]; i++) {
        if (!b.f64(f64_rows[i], &c)) return (*err = std::string(f64_rows[i]) + " missing"), false;
        n1 = std::min(n1, c);
    }
    const char* i64_rows[] = {"occ_hour", "rew_hour", "rew_month", nullptr};
    for (int i = 0; i64_rows[i]; i++) {
        if (!b.i64(i64_rows[i], &c)) return (*err = std::string(i64_rows[i]) + " missing"), false;
        n1 = std::min(n1, c);
    }
    const char* u8_rows[] = {"occ_workday", "rew_workday", nullptr};
    for (int i = 0; u8_rows[i]; i++) {
        if (!b.u8(u8_rows[i], &c)) return (*err = std::string(u8_rows[i]) + " missing"), false;
        n1 = std::min(n1, c);
    }
    const double* aux = b.f64("aux_time", &c);
    if (!aux && L.n_aux > 1) return (*err = "aux_time missing"), false;
    if (L.n_aux > 1) n1 = std::min(n1, c / (uint64_t)(L.n_aux - 1));
    H->n1 = (int)n1;
    uint64_t c_solar = 0;
    const double* solar = b.f64("solar_irradiance", &c_solar);
    std::vector<double> sol(n1, 0.0);
    if (solar) for (uint64_t i = 0; i < n1 && i < c_solar; i++) sol[i] = solar[i];
    uint64_t cm1 = 0;
    const int64_t* hm1 = b.i64("occ_hour_m1", &cm1);
    uint64_t cw1 = 0;
    const uint8_t* wm1 = b.u8("occ_workday_m1", &cw1);
    if (!hm1 || !wm1) return (*err = "occ_hour_m1/occ_workday_m1 missing"), false;
    H->hour_m1_rows = (int)std::min(cm1, cw1);
    const int n = L.n;
    // Dirichlet + ambient exposure at the scenario's convection coefficient
    // (complete_port/csim/sb_fdm.c:126-140)
    const double* dir = b.f64("dirichlet_conductance");
    const double* f0 = b.f64("ambient_face_areas_0");
    const double* f1 = b.f64("ambient_face_areas_1");
    const double* hz = b.f64("horizontal");
    const double* vt = b.f64("vertical");
    const double* cd = b.f64("solver_conductivity");
    if (!dir || !f0 || !f1 || !hz || !vt || !cd) return (*err = "field sections missing"), false;
    const double h = b.f64_1("convection_coefficient", 8.8);
    std::vector<double> dirx(n);
    for (int t = 0; t < n; t++) {
        double e = 0.0;
        if (f0[t] > 0.0) e += h * f0[t] / (1.0 + h * 0.5 * hz[t] / cd[t]);
        if (f1[t] > 0.0) e += h * f1[t] / (1.0 + h * 0.5 * vt[t] / cd[t]);
        dirx[t] = dir[t] + e;
    }
    const double* ti = b.f64("temp_init");
    const double* mi = b.f64("mass_temp_init");
    if (!ti || !mi) return (*err = "temp_init/mass_temp_init missing"), false;
    const double* rw = b.f64("reward_scalars", &c);
    if (!rw || c < 8) return (*err = "reward_scalars missing"), false;
    const double* ewk = b.f64("elec_weekday_price");
    const double* ewe = b.f64("elec_weekend_price");
    const double* eco = b.f64("elec_carbon_rate");
    const double* gp = b.f64("gas_month_price");
    if (!ewk || !ewe || !eco || !gp) return (*err = "price tables missing"), false;
    auto& O = H->off;
    O["amb"] = A.vec(take(amb, n1));
    O["solar_i"] = A.vec(sol);
    O["comfort"] = A.vec(take(b.f64("sched_comfort"), n1));
    O["heat_sp"] = A.vec(take(b.f64("sched_heat_sp"), n1));
    O["cool_sp"] = A.vec(take(b.f64("sched_cool_sp"), n1));
    O["aux_time"] = A.vec(take(aux, n1 * (uint64_t)std::max(L.n_aux - 1, 0)));
    O["occ_hour"] = A.vec(to_u8(b.i64("occ_hour"), n1));
    O["occ_work"] = A.vec(take(b.u8("occ_workday"), n1));
    O["hour_m1"] = A.vec(to_u8(hm1, H->hour_m1_rows));
    O["work_m1"] = A.vec(take(wm1, (uint64_t)H->hour_m1_rows));
    O["rew_hour"] = A.vec(to_u8(b.i64("rew_hour"), n1));
    O["rew_month"] = A.vec(to_u8(b.i64("rew_month"), n1));
    O["rew_work"] = A.vec(take(b.u8("rew_workday"), n1));
    O["dirx"] = A.vec(dirx);
    O["temp_init"] = A.vec(take(ti, n));
    O["mass_init"] = A.vec(take(mi, n));
    O["elec_wk"] = A.vec(take(ewk, 24));
    O["elec_we"] = A.vec(take(ewe, 24));
    O["elec_co2"] = A.vec(take(eco, 24));
    O["gas_price"] = A.vec(take(gp, 12));
    {
        ImgBuilder I;
        D.img.dirx = I.add(dirx);
        D.img.elec_wk = I.add(take(ewk, 24));
        D.img.elec_we = I.add(take(ewe, 24));
        D.img.elec_co2 = I.add(take(eco, 24));
        D.img.gas_price = I.add(take(gp, 12));
        D.img.bytes = I.finish();
        if (D.img.bytes > align_up(8 * n, 16) + 8 * 84) return (*err = "scenario image larger than its LDS region"), false;
        O["img"] = A.vec(I.bytes);
    }
    D.n1 = (int)n1;
    D.gas_co2 = b.f64_1("gas_carbon_rate", 0.0);
    for (int i = 0; i < 8; i++) D.rw[i] = rw[i];
    const double* bc = b.f64("boiler_const");
    for (int i = 0; i < 10; i++) D.boiler_c[i] = bc ? bc[i] : 0.0;
    {
        // log(r2/c6)/c8 + 1/c4/r2 of the boiler tank loss (sb_reward.c:20-24)
        const double* q = D.boiler_c;
        double r2 = q[6] + q[9];
        double cond = log(r2 / q[6]) / q[8];
        double conv = 1.0 / q[4] / r2;
        D.diss_den = cond + conv;
    }
    const double* pc = b.f64("pump_const");
    D.pump_head0 = pc ? pc[0] : 0.0;
    D.pump_eff = pc ? pc[1] : 1.0;
    D.header_res = b.f64_1("hws_header_resistance", 0.0);
    D.internal_w_m2 = b.f64_1("internal_gain_w_per_m2", 0.0);
    D.standby_frac = b.f64_1("internal_gain_standby_fraction", 1.0);
    D.occupant_w = b.f64_1("occupant_sensible_heat_w", 0.0);
    {
        double cv = b.f64_1("cv_size_cm", 20.0) / 100.0;
        D.cv_area = cv * cv;
    }
    const double* op = b.f64("occ_params");
    D.dt_sec = op[5];
    D.inv_nz = 1.0 / L.nz;
    D.kwh_per_w = op[5] / 3.6e6;
    D.ea = (int)op[1]; D.la = (int)op[2]; D.ed = (int)op[3]; D.ld = (int)op[4];
    D.p_arr = 1.0 / ((D.la - D.ea) * 3600.0 / op[5] / 2.0);
    D.p_dep = 1.0 / ((D.ld - D.ed) * 3600.0 / op[5] / 2.0);
    {
        // the field mean is needed only when an AHU serves no zone area
        const int32_t* vav_ahu = b.i32("vav_ahu_idx");
        std::vector<int> has(L.na, 0);
        for (int v = 0; v < L.nv; v++) has[vav_ahu[v]] = 1;
        D.conv_tmean = 0;
        for (int a = 0; a < L.na; a++) if (!has[a]) D.conv_tmean = 1;
    }
    const double* meta = b.f64("obs_meta", &c);
    H->episode_steps = (meta && c >= 4) ? (int)meta[3] : 0;
    H->occ_seed = b.i64_1("occ_seed", 17321);
    // stochastic convection (sb_convect.c:12-14, :40): on when p != 0 and the
    // distance is not 0; the stream is seeded per env from conv_seed
    D.conv_p = b.f64_1("conv_p", 0.0);
    D.conv_on = (D.conv_p != 0.0 && (int)b.f64_1("conv_distance", -1.0) != 0) ? 1 : 0;
    if (D.conv_on && L.cv_cells == 0) D.conv_on = 0;   // no rooms: nothing to draw (sb_convect.c:42)
    H->conv_seed = b.i64_1("conv_seed", 0);
    H->n_cont = L.n_cont;
    H->n_disc = L.n_disc;
    return true;
}

void patch_scen(HostScen* H, unsigned char* d) {
    sbk::DevScen& D = H->dev;
    auto& O = H->off;
    D.img_src = at<unsigned char>(d, O["img"]);
    D.amb = at<double>(d, O["amb"]);
    D.solar_i = at<double>(d, O["solar_i"]);
    D.comfort = at<double>(d, O["comfort"]);
    D.heat_sp = at<double>(d, O["heat_sp"]);
    D.cool_sp = at<double>(d, O["cool_sp"]);
    D.aux_time = at<double>(d, O["aux_time"]);
    D.occ_hour = at<uint8_t>(d, O["occ_hour"]);
    D.occ_work = at<uint8_t>(d, O["occ_work"]);
    D.hour_m1 = at<uint8_t>(d, O["hour_m1"]);
    D.work_m1 = at<uint8_t>(d, O["work_m1"]);
    D.rew_hour = at<uint8_t>(d, O["rew_hour"]);
    D.rew_month = at<uint8_t>(d, O["rew_month"]);
    D.rew_work = at<uint8_t>(d, O["rew_work"]);
    D.dirx = at<double>(d, O["dirx"]);
    D.temp_init = at<double>(d, O["temp_init"]);
    D.mass_init = at<double>(d, O["mass_init"]);
    D.elec_wk = at<double>(d, O["elec_wk"]);
    D.elec_we = at<double>(d, O["elec_we"]);
    D.elec_co2 = at<double>(d, O["elec_co2"]);
    D.gas_price = at<double>(d, O["gas_price"]);
}

// ---------------------------------------------------------------- vec
struct TileGroup {
    int variant, first, count;
};

int kernel_variant(const sbk::DevLayout& d) {
    if (d.solver == sbk::SOLVER_LU) return sbk::KV_LU;
    return d.rx_block ? sbk::KV_BLOCK : sbk::KV_POINT;
}

struct Vec {
    int n = 0, width = 64, lds_bytes = 0;
    int epb = 4;                              // envs (wavefronts) per workgroup
    int img_lds = 0;                          // LDS bytes of the largest layout image
    std::vector<sbk::Tile> tiles;
    std::vector<TileGroup> groups;            // consecutive tiles of one kernel variant
    sbk::Tile* d_tiles = nullptr;
    float reward_scale = 1.0f;
    Env* envs = nullptr;
    std::vector<std::string> paths;           // ordered scenario list
    std::vector<HostLayout> layouts;
    std::vector<HostScen> scens;
    std::vector<sbk::EnvDesc> desc;
    std::vector<int> order;
    std::vector<uint32_t> seeds;
    std::vector<uint32_t> conv_seeds;
    std::vector<int> env_scen_local;
    unsigned char* d_arena = nullptr;
    unsigned char* d_state = nullptr;
    size_t state_bytes = 0;
    sbk::DevLayout* d_layouts = nullptr;
    sbk::DevScen* d_scens = nullptr;
    sbk::EnvDesc* d_envs = nullptr;
    int* d_order = nullptr;
    int* d_ncont = nullptr;
    int* d_ndisc = nullptr;
    float* obs = nullptr;
    float* actions = nullptr;
    float* rewards = nullptr;
    float* terminals = nullptr;
    double bytes_per_step = 0.0, record_bytes_per_step = 0.0, flops_per_step = 0.0;
    // step-kernel timer: an event pair around each puf_step launch while on
    std::vector<hipEvent_t> tev;
    int t_on = 0, t_used = 0, t_seen = 0;   // t_on: sampling period (0 = off)
    // shared policy (sbx_policy_bind): caller-owned weights, library-owned activations
    SbxPolicy pol{};
    float *p_h1 = nullptr, *p_h2 = nullptr, *p_y = nullptr;
    float *p_hlp = nullptr, *p_hent = nullptr;   // per-head log-densities and entropies [n][SB_ACT]
    int obs_cols = SB_OBS;                       // observation rows are zero from this column on (every env)
    double* d_air = nullptr;                     // kwarg trace_air: [n][2][air_stride] each step's air_g, air_T
    int air_stride = 0;
    double* d_live = nullptr;                    // puf_live_log totals (device: 3 f64, then 3 per scenario)
    double* h_live = nullptr;                    // and their pinned host copy
    std::vector<double> live_prev;               // per scenario: the totals at the previous puf_live_log
    std::vector<std::string> live_keys;          // per scenario: its two live keys (Dict keeps the pointers)
    // canonical policy interface (kwargs canonical / residual / res_* / guard_*)
    int canonical = 0, resid = 0, guard = 0, guard_hot = 0;
    float res_scale = 0.5f, res_dscale = 1.5f, guard_d0 = 1.0f, guard_d1 = 0.0f;
    sbk::CanonTab* d_canon = nullptr;            // per layout
    float* d_raw = nullptr;                      // [n][SB_OBS] the env's own observation rows
    float* d_native = nullptr;                   // [n][SB_ACT] native action rows the step decodes
    float* d_cbase = nullptr;                    // [n][SB_ACT] base proposal per native action
    float* d_ctrust = nullptr;                   // [n][SB_ACT] guard trust per native action
    double* d_cpid = nullptr;                    // [n][2 * SBC_K] PID state
    float* d_cinfo = nullptr;                    // [n][2 * SBC_K] effort, mean zone temperature per AHU
    // field scenarios (FDM-scale fields): one per scenario, its envs as slots
    std::vector<FieldScen*> fields;
    std::vector<std::vector<sbe::Slot>> field_slots;
    std::vector<int> field_of;                   // [n] field scenario of env i, or -1
    std::vector<int> slot_of;                    // [n] its slot there
};

constexpr int kTimerPairs = 16384;

sbk::KParams params(Vec* v, int mode) {
    sbk::KParams p{};
    p.envs = v->d_envs;
    p.order = v->d_order;
    p.tiles = v->d_tiles;
    p.img_lds = v->img_lds;
    p.layouts = v->d_layouts;
    p.scens = v->d_scens;
    p.state = v->d_state;
    p.actions = v->actions;
    p.obs = v->obs;
    p.rewards = v->rewards;
    p.terminals = v->terminals;
    p.host_env = v->envs;
    p.env_stride = (int)sizeof(Env);
    p.log_offset = (int)offsetof(Env, log);
    p.n_envs = v->n;
    p.mode = mode;
    p.reward_scale = v->reward_scale;
    p.air_trace = v->d_air;
    p.air_stride = v->air_stride;
    return p;
}

// One launch per kernel variant present (tiles are grouped by variant).
void launch_params(Vec* v, const sbk::KParams& p) {
    for (const TileGroup& g : v->groups) {
        sbk::KParams q = p;
        q.tiles = v->d_tiles + g.first;
        int rc = sbk_launch_step(&q, g.count, 2 * v->width * v->epb, v->lds_bytes, g.variant, g_stream);
        if (rc != 0) die(std::string("step kernel launch failed: ") + hipGetErrorString((hipError_t)rc));
    }
}

// The canonical interface's kernels around a step or reset (post) / before a
// step (pre, reading the trainer's canonical action rows `actions`).
void launch_canon(Vec* v, int post, int reset, const float* actions) {
    sbk::CanonArgs a{};
    a.tabs = v->d_canon;
    a.envs = v->d_envs;
    a.raw_obs = v->d_raw;
    a.obs = v->obs;
    a.actions = actions;
    a.native = v->d_native;
    a.terminals = v->terminals;
    a.pid = v->d_cpid;
    a.base = v->d_cbase;
    a.trust = v->d_ctrust;
    a.ainfo = v->d_cinfo;
    a.n = v->n;
    a.reset = reset;
    a.resid = v->resid;
    a.scale = v->res_scale;
    a.dscale = v->res_dscale;
    a.guard = v->guard;
    a.d0 = v->guard_d0;
    a.d1 = v->guard_d1;
    a.hot = v->guard_hot;
    const int rc = sbk_launch_canon(&a, post, g_stream);
    if (rc != 0) die(std::string("canonical kernel launch failed: ") + hipGetErrorString((hipError_t)rc));
}

// One step or reset of every env: in canonical mode the step kernels (RC
// tiles and field scenarios) read the native action rows the pre kernel
// decoded and write the envs' own observation rows, from which the post
// kernel then makes the canonical ones.
void run_env(Vec* v, sbk::KParams p, const float* actions) {
    const bool reset = p.mode == sbk::KMODE_RESET;
    if (v->canonical) {
        if (!reset) launch_canon(v, 0, 0, actions ? actions : v->actions);
        p.actions = v->d_native;
        p.obs = v->d_raw;
    } else if (actions) {
        p.actions = actions;
    }
    launch_params(v, p);
    if (!v->fields.empty()) {
        FieldIo io{p.actions, p.obs, p.rewards, p.terminals, p.host_env, p.env_stride, p.log_offset, p.reward_scale};
        std::string err;
        for (FieldScen* f : v->fields)
            if (!field_step(f, io, reset, g_stream, &err)) die("field scenario step: " + err);
    }
    if (v->canonical) launch_canon(v, 1, reset ? 1 : 0, nullptr);
}

void launch(Vec* v, int mode) { run_env(v, params(v, mode), nullptr); }

Vec* vec_of(Env* envs) {
    if (!envs || !envs[0].vec) die("env array was not created by puf_vec_create");
    return static_cast<Vec*>(envs[0].vec);
}

bool ends_with(const std::string& s, const std::string& suf) {
    return s.size() >= suf.size() && s.compare(s.size() - suf.size(), suf.size(), suf) == 0;
}

std::vector<std::string> list_blobs(const std::string& dir) {
    std::vector<std::string> out;
    DIR* d = opendir(dir.c_str());
    if (!d) return out;
    while (dirent* e = readdir(d)) {
        std::string nm = e->d_name;
        if (ends_with(nm, ".sbb")) out.push_back(dir + "/" + nm);
    }
    closedir(d);
    std::sort(out.begin(), out.end());
    return out;
}

// all buildings' first weather, then all buildings' second weather, ...
// (building = file name up to "__"), complete_port/gpu/smart_buildings.cu:2435-2459
std::vector<std::string> round_robin(const std::vector<std::string>& p) {
    std::vector<std::string> keys, blds, out;
    for (auto& f : p) {
        std::string base = f.substr(f.find_last_of('/') + 1);
        std::string b = base.substr(0, base.find("__"));
        keys.push_back(b);
        if (std::find(blds.begin(), blds.end(), b) == blds.end()) blds.push_back(b);
    }
    std::vector<int> used(p.size(), 0);
    while (out.size() < p.size())
        for (auto& b : blds)
            for (size_t i = 0; i < p.size(); i++)
                if (!used[i] && keys[i] == b) { out.push_back(p[i]); used[i] = 1; break; }
    return out;
}

float kw(Dict* d, const char* key, float dflt) {
    DictItem* it = d ? dict_find(d, key) : nullptr;
    return it ? it->value : dflt;
}

const char* kws(Dict* d, const char* key) {
    DictItem* it = d ? dict_find(d, key) : nullptr;
    return (it && it->str && it->str[0]) ? it->str : nullptr;
}

// [env] keys of the reference GPU env (complete_port/gpu/smart_buildings.cu:
// 2590-2720, complete_port/config/smart_buildings.ini [env]) whose behaviour
// this build does not have: each is accepted at its inert value (0, as the
// reference ini ships them) and aborts with a message otherwise, so a trainer
// config never gets a different environment without notice. Keys that only
// parameterise one of these (center_beta, plant_eps, shape_gamma,
// random_start_seed) and merge_weathers (how the reference groups scenarios
// for its solver: no effect on results) are accepted at any value. The
// canonical interface (canonical, residual, res_scale, res_dscale, guard_*)
// is implemented.
void check_env_keys(Dict* d) {
    static const char* const unsupported[] = {
        "random_start", "rew_norm", "rew_center", "plant_pair", "comfort_shape", "zone_memory", "interleave",
        "zone_adv", "zone_critic", "ahu_critic",
        "zone_command", "prestart_explore", "probe", "zone_signed", "zone_night_share",
    };
    if (!d) return;
    for (const char* k : unsupported) {
        DictItem* it = dict_find(d, k);
        if (it && it->value != 0.0f)
            die(std::string("env.") + k + " = " + std::to_string(it->value)
                + " is not supported by this env (only its default, 0)");
    }
}

void mt_seed(uint32_t* mt, uint32_t seed) {
    mt[0] = seed;
    for (int i = 1; i < SBK_MT_N; i++) mt[i] = 1812433253u * (mt[i - 1] ^ (mt[i - 1] >> 30)) + (uint32_t)i;
}

}  // namespace

// ================================================================== C ABI
extern "C" {

DictItem* dict_find(Dict* d, const char* key) {
    if (!d || !key) return nullptr;
    for (int i = 0; i < d->size; i++)
        if (d->items[i].key && strcmp(d->items[i].key, key) == 0) return &d->items[i];
    return nullptr;
}

void dict_set(Dict* d, const char* key, float value) {
    if (!d) return;
    DictItem* it = dict_find(d, key);
    if (it) { it->value = value; return; }
    if (d->size < d->capacity) {
        d->items[d->size].key = key;
        d->items[d->size].value = value;
        d->items[d->size].str = nullptr;
        d->size++;
    }
}

Env* puf_vec_create(int n, Dict* kwargs, obs_t* observations, float* actions, float* rewards, float* terminals) {
    if (n <= 0) die("puf_vec_create: n must be positive");
    if (!observations || !actions || !rewards || !terminals) die("puf_vec_create: null trainer buffer");
    auto v = std::make_unique<Vec>();
    v->n = n;
    v->obs = observations;
    v->actions = actions;
    v->rewards = rewards;
    v->terminals = terminals;
    v->width = (int)kw(kwargs, "block", 64.0f);
    if (v->width != 64) die("env.block must be 64 (one wavefront per env)");
    // a reward_scale <= 0 means 1 (complete_port/gpu/smart_buildings.cu:2595-2596)
    {
        const float rs = kw(kwargs, "reward_scale", 1.0f);
        v->reward_scale = rs > 0.0f ? rs : 1.0f;
    }
    // the Log is filled at episode ends (the reference GPU env's form); the
    // key of earlier versions that chose it is accepted at 1 only
    if (kw(kwargs, "log_at_end", 1.0f) != 1.0f)
        die("env.log_at_end: the per-step Log is not supported (the Log fills at episode ends)");
    check_env_keys(kwargs);
    // ---- scenario list
    std::vector<std::string> files;
    if (const char* one = kws(kwargs, "blob")) {
        files.push_back(one);
    } else {
        const char* dir = kws(kwargs, "blob_dir");
        if (!dir) dir = getenv("SB_BLOB_DIR");
        if (dir && dir[0]) files = round_robin(list_blobs(dir));
        if (files.empty()) die("no scenario. Set env.blob or env.blob_dir (or SB_BLOB_DIR).");
    }
    int G = (int)kw(kwargs, "groups", 0.0f);
    if (G <= 0) G = n / 32;
    G = std::min(G, (int)files.size());
    G = std::max(G, 1);
    G = std::min(G, n);
    files.resize(G);
    v->paths = files;
    std::vector<int> scnt(G);
    for (int i = 0; i < G; i++) scnt[i] = n / G + (i < n % G ? 1 : 0);
    // ---- canonical policy interface (complete_port/gpu/smart_buildings.cu:2611-2660, 2717)
    v->canonical = (int)kw(kwargs, "canonical", 0.0f) != 0;
    v->resid = (int)kw(kwargs, "residual", 0.0f) != 0;
    if (v->resid && !v->canonical) die("env.residual needs env.canonical = 1");
    {
        const float rs = kw(kwargs, "res_scale", 0.5f), rd = kw(kwargs, "res_dscale", 1.5f);
        if (rs > 0.0f) v->res_scale = rs;
        if (rd > 0.0f) v->res_dscale = rd;
        const float d0 = kw(kwargs, "guard_d0", 1.0f);
        if (d0 >= 0.0f) v->guard_d0 = d0;
        v->guard_d1 = kw(kwargs, "guard_d1", 0.0f);
        v->guard_hot = (int)kw(kwargs, "guard_hot", 0.0f) != 0;
        if (!v->resid) v->guard_d1 = 0.0f;     // the guard scales residuals only
        v->guard = v->guard_d1 > 0.0f;
        if ((v->guard_d1 != 0.0f || v->guard_hot) && !v->canonical)
            die("env.guard_d1 / env.guard_hot need env.canonical = 1 and env.residual = 1");
    }
    // ---- field solver: "auto" (relaxation where certified), "lu" or "relax"
    int solve = SOLVE_AUTO;
    if (const char* sv = kws(kwargs, "solver")) {
        if (!strcmp(sv, "lu")) solve = SOLVE_LU;
        else if (!strcmp(sv, "relax")) solve = SOLVE_RELAX;
        else if (!strcmp(sv, "point")) solve = SOLVE_POINT;
        else if (strcmp(sv, "auto")) die(std::string("env.solver must be auto, lu, relax or point, not ") + sv);
    }
    // ---- layouts + scenarios
    Arena A;
    std::map<std::string, int> layout_of_key;
    for (int i = 0; i < G; i++) {
        sbh::Blob b;
        std::string err;
        if (!b.open(files[i], &err)) die(err);
        if (field_blob(b)) {
            // FDM-scale field: HVAC lanes around the field group's solve
            FieldScen* F = field_open(b, &err);
            if (!F) die(files[i] + ": " + err);
            const FieldCounts fc = field_counts(F);
            HostLayout H;
            H.key = "field:" + files[i];
            H.field = (int)v->fields.size();
            if (v->canonical) {
                // the canonical maps read only the blob's observation map and topology
                H.canon = std::make_unique<sbk::CanonTab>();
                if (!make_canon(b, H.canon.get(), &err)) die(files[i] + ": canonical layout: " + err);
            }
            H.dev.n_act = fc.n_act;
            H.dev.n_cont = fc.n_cont;
            H.dev.n_disc = fc.n_disc;
            H.dev.nz = fc.nz;
            const int li = (int)v->layouts.size();
            v->layouts.push_back(std::move(H));
            HostScen S;
            S.path = files[i];
            S.layout = li;
            S.field = (int)v->fields.size();
            S.n1 = fc.n1;
            S.episode_steps = fc.episode_steps;
            S.occ_seed = fc.occ_seed;
            S.conv_seed = fc.conv_seed;
            S.hour_m1_rows = fc.hour_m1_rows;
            S.dev.layout = li;
            v->scens.push_back(std::move(S));
            v->fields.push_back(F);
            v->field_slots.emplace_back();
            continue;
        }
        std::string key = structural_key(b);
        int li;
        auto it = layout_of_key.find(key);
        if (it == layout_of_key.end()) {
            HostLayout H;
            H.key = key;
            if (!make_layout(b, v->width, solve, &H, A, &err)) die(files[i] + ": " + err);
            if (v->canonical) {
                H.canon = std::make_unique<sbk::CanonTab>();
                if (!make_canon(b, H.canon.get(), &err)) die(files[i] + ": canonical layout: " + err);
            }
            li = (int)v->layouts.size();
            v->layouts.push_back(std::move(H));
            layout_of_key[key] = li;
        } else {
            li = it->second;
        }
        HostScen S;
        S.path = files[i];
        S.layout = li;
        if (!make_scen(b, v->layouts[li], &S, A, &err)) die(files[i] + ": " + err);
        S.dev.layout = li;
        v->scens.push_back(std::move(S));
    }
    // ---- envs
    const int max_steps_kw = (int)kw(kwargs, "max_steps", 0.0f);
    // desync = 1: every env's first episode ends at a hashed step in
    // [1, episode length]; later episodes have the full length
    // (complete_port/gpu/smart_buildings.cu:2583-2590, 2808-2815)
    const int desync = (int)kw(kwargs, "desync", 0.0f);
    // start_offsets = 1: every env starts its episodes at its own seeded
    // calendar offset (the BASELINE's desynchronised starts; no reference key)
    const int start_offsets = (int)kw(kwargs, "start_offsets", 0.0f);
    const uint64_t start_seed = (uint64_t)kw(kwargs, "start_seed", 7.0f);
    // shard_base: index of this vec's first env in a batch sharded over
    // several vecs, so env-keyed draws (desync, start offsets) match the whole
    // batch's
    const int shard_base = (int)kw(kwargs, "shard_base", 0.0f);
    if (shard_base < 0) die("env.shard_base must be >= 0");
    const int per_env_seed = (int)kw(kwargs, "per_env_seed", 1.0f);
    size_t state_off = 0;
    int e = 0;
    for (int i = 0; i < G; i++) {
        const HostScen& S = v->scens[i];
        const HostLayout& L = v->layouts[S.layout];
        int ms = max_steps_kw > 0 ? max_steps_kw : S.episode_steps;
        if (ms <= 0) ms = S.n1 - 1;
        for (int j = 0; j < scnt[i]; j++, e++) {
            sbk::EnvDesc d{};
            d.scen = i;
            d.layout = S.layout;
            d.max_steps = ms;
            d.state_off = (long long)state_off;
            const uint64_t gid = (uint64_t)shard_base + (uint64_t)e;   // env index in the whole batch
            int start = 0;
            if (start_offsets) {
                int range = S.n1 - 1 - ms + 1;
                if (range < 1) die(S.path + ": calendar too short for start offsets");
                range = std::min(range, std::max(S.episode_steps, 1));
                start = (int)(splitmix64(start_seed * 0x100000001B3ull + gid) % (uint64_t)range);
            }
            d.first_steps = ms;
            if (desync) {
                uint64_t h = 0x9E3779B97F4A7C15ull * (gid + 1);
                h ^= h >> 31;
                h *= 0xBF58476D1CE4E5B9ull;
                h ^= h >> 29;
                d.first_steps = 1 + (int)(h % (uint64_t)ms);
            }
            if (start + ms > S.n1 - 1) die(S.path + ": calendar tables shorter than the episode");
            if (start >= S.hour_m1_rows) die(S.path + ": occ_hour_m1 has no row for the start offset");
            d.start = start;
            if (S.field >= 0) {
                v->field_of.push_back(S.field);
                v->slot_of.push_back((int)v->field_slots[S.field].size());
                v->field_slots[S.field].push_back(
                    sbe::Slot{e, start, ms, d.first_steps, (uint32_t)(S.occ_seed + (per_env_seed ? j : 0)),
                              (uint32_t)(S.conv_seed + (per_env_seed ? j : 0)), {0, 0}});
            } else {
                v->field_of.push_back(-1);
                v->slot_of.push_back(-1);
            }
            v->desc.push_back(d);
            v->seeds.push_back((uint32_t)(S.occ_seed + (per_env_seed ? j : 0)));
            v->conv_seeds.push_back((uint32_t)(S.conv_seed + (per_env_seed ? j : 0)));
            v->env_scen_local.push_back(j);
            state_off += (size_t)L.dev.st.record_bytes;
        }
    }
    v->state_bytes = state_off;
    // tiles: envs of one layout share a workgroup (two wavefronts each) and the
    // layout image it stages; largest layouts first, then by scenario
    for (int i = 0; i < n; i++)
        if (v->field_of[i] < 0) v->order.push_back(i);
    const int n_rc = (int)v->order.size();
    std::stable_sort(v->order.begin(), v->order.end(), [&](int a, int b) {
        const sbk::EnvDesc &da = v->desc[a], &db = v->desc[b];
        const int ka = kernel_variant(v->layouts[da.layout].dev), kb = kernel_variant(v->layouts[db.layout].dev);
        if (ka != kb) return ka > kb;
        const int na_ = v->layouts[da.layout].dev.n, nb_ = v->layouts[db.layout].dev.n;
        if (na_ != nb_) return na_ > nb_;
        if (da.layout != db.layout) return da.layout < db.layout;
        return da.scen < db.scen;
    });
    {
        const int epb_kw = (int)kw(kwargs, "envs_per_block", 4.0f);
        if (epb_kw < 1 || epb_kw > 4) die("env.envs_per_block must be 1..4");
        // every workgroup holds the largest layout image, then its envs'
        // regions; a layout's tiles take as many envs as fit (at most
        // envs_per_block), the launch is shaped for the largest tile
        int img = 0;
        for (auto& L : v->layouts) img = std::max(img, L.dev.img.bytes);
        const int limit = 160 * 1024;
        std::vector<int> per(v->layouts.size(), 1);
        int epb = 1, lds = 0;
        for (size_t li = 0; li < v->layouts.size(); li++) {
            if (v->layouts[li].field >= 0) continue;
            const int reg = v->layouts[li].dev.lds.bytes;
            if (img + reg > limit) die("layout needs more LDS than a workgroup has");
            per[li] = std::min(epb_kw, (limit - img) / reg);
            epb = std::max(epb, per[li]);
            lds = std::max(lds, img + per[li] * reg);
        }
        v->epb = epb;
        v->img_lds = img;
        v->lds_bytes = lds;
        for (int i = 0; i < n_rc;) {
            const int lay = v->desc[v->order[i]].layout;
            int j = i;
            while (j < n_rc && j - i < per[lay] && v->desc[v->order[j]].layout == lay) j++;
            v->tiles.push_back(sbk::Tile{lay, i, j - i, 0});
            const int kv = kernel_variant(v->layouts[lay].dev);
            if (v->groups.empty() || v->groups.back().variant != kv)
                v->groups.push_back(TileGroup{kv, (int)v->tiles.size() - 1, 0});
            v->groups.back().count++;
            i = j;
        }
    }
    // ---- upload tables
    hip_ok(hipMalloc(&v->d_arena, A.host.size()), "hipMalloc(tables)");
    hip_ok(hipMemcpy(v->d_arena, A.host.data(), A.host.size(), hipMemcpyHostToDevice), "upload tables");
    std::vector<sbk::DevLayout> dl;
    for (auto& L : v->layouts) {
        patch_layout(&L, v->d_arena);
        dl.push_back(L.dev);
    }
    std::vector<sbk::DevScen> ds;
    for (auto& S : v->scens) {
        patch_scen(&S, v->d_arena);
        ds.push_back(S.dev);
    }
    // burst inputs of the tiles and env records (device pointers now known)
    for (auto& t : v->tiles) {
        const sbk::DevLayout& D = v->layouts[t.layout].dev;
        t.lds_bytes = D.lds.bytes;
        t.img16 = D.img.bytes >> 4;
        t.rec16 = (D.st.bytes + (D.st.cmt ? 4 * SBK_MT_N : 0)) >> 4;   // the image (and the convection state)
        t.lds_state = D.lds.state;
        t.lds_scen = D.lds.scen;
        t.lds_act = D.lds.act;
        t.st_iplant = D.st.iplant;
        t.img_src = D.img_src;
    }
    for (auto& d : v->desc) {
        const sbk::DevScen& S = v->scens[d.scen].dev;
        d.scn16 = S.img.bytes >> 4;
        d.scen_src = S.img_src;
    }
    for (auto& t : v->tiles)
        for (int sl = 0; sl < 4; sl++) {
            t.env[sl] = v->order[t.first + (sl < t.count ? sl : 0)];
            t.desc[sl] = v->desc[t.env[sl]];
        }
    if (v->lds_bytes > 64 * 1024) hip_ok((hipError_t)sbk_set_lds_limit(v->width, v->lds_bytes), "LDS limit");
    hip_ok(hipMalloc(&v->d_layouts, sizeof(sbk::DevLayout) * dl.size()), "hipMalloc(layouts)");
    hip_ok(hipMemcpy(v->d_layouts, dl.data(), sizeof(sbk::DevLayout) * dl.size(), hipMemcpyHostToDevice), "upload");
    hip_ok(hipMalloc(&v->d_scens, sizeof(sbk::DevScen) * ds.size()), "hipMalloc(scens)");
    hip_ok(hipMemcpy(v->d_scens, ds.data(), sizeof(sbk::DevScen) * ds.size(), hipMemcpyHostToDevice), "upload");
    // the longest observation prefix: the shared policy's first layer skips the zero tail past it
    v->obs_cols = 1;
    for (int i = 0; i < n; i++) {
        const int w = v->canonical ? SB_OBS
                      : v->field_of[i] >= 0 ? field_counts(v->fields[v->field_of[i]]).n_obs
                                            : v->layouts[v->desc[i].layout].dev.n_dev + v->layouts[v->desc[i].layout].dev.n_aux;
        v->obs_cols = std::max(v->obs_cols, std::min(w, SB_OBS));
    }
    hip_ok(hipMalloc(&v->d_envs, sizeof(sbk::EnvDesc) * n), "hipMalloc(envs)");
    hip_ok(hipMemcpy(v->d_envs, v->desc.data(), sizeof(sbk::EnvDesc) * n, hipMemcpyHostToDevice), "upload");
    hip_ok(hipMalloc(&v->d_order, sizeof(int) * std::max(n_rc, 1)), "hipMalloc(order)");
    hip_ok(hipMemcpy(v->d_order, v->order.data(), sizeof(int) * n_rc, hipMemcpyHostToDevice), "upload");
    hip_ok(hipMalloc(&v->d_tiles, sizeof(sbk::Tile) * v->tiles.size()), "hipMalloc(tiles)");
    hip_ok(hipMemcpy(v->d_tiles, v->tiles.data(), sizeof(sbk::Tile) * v->tiles.size(), hipMemcpyHostToDevice),
           "upload");
    {
        // the trainer's heads: the native actions, or (canonical) the canonical slots
        std::vector<int> nc(n), nd(n);
        for (int i = 0; i < n; i++) {
            nc[i] = v->canonical ? SBC_ACT : v->layouts[v->desc[i].layout].dev.n_cont;
            nd[i] = v->canonical ? 0 : v->layouts[v->desc[i].layout].dev.n_disc;
        }
        hip_ok(hipMalloc(&v->d_ncont, sizeof(int) * n), "hipMalloc");
        hip_ok(hipMalloc(&v->d_ndisc, sizeof(int) * n), "hipMalloc");
        hip_ok(hipMemcpy(v->d_ncont, nc.data(), sizeof(int) * n, hipMemcpyHostToDevice), "upload");
        hip_ok(hipMemcpy(v->d_ndisc, nd.data(), sizeof(int) * n, hipMemcpyHostToDevice), "upload");
    }
    if (kw(kwargs, "trace_air", 0.0f) != 0.0f) {
        // every step also stores each env's air side, so state snapshots hold it
        for (const HostLayout& L : v->layouts) v->air_stride = std::max(v->air_stride, L.dev.k);
        v->air_stride = std::max(v->air_stride, 1);
        const size_t bytes = sizeof(double) * 2 * (size_t)v->air_stride * n;
        hip_ok(hipMalloc(&v->d_air, bytes), "hipMalloc(air trace)");
        hip_ok(hipMemset(v->d_air, 0, bytes), "memset(air trace)");
    }
    // ---- initial state records: pump head, seeded MT19937 (index 624)
    {
        std::vector<unsigned char> rec(v->state_bytes, 0);
        for (int i = 0; i < n; i++) {
            if (v->field_of[i] >= 0) continue;
            const sbk::EnvDesc& d = v->desc[i];
            const sbk::DevLayout& L = v->layouts[d.layout].dev;
            unsigned char* r = rec.data() + d.state_off;
            reinterpret_cast<double*>(r + L.st.plant)[sbk::PF_PUMP_HEAD] = v->scens[d.scen].dev.pump_head0;
            reinterpret_cast<int*>(r + L.st.iplant)[sbk::PI_MT_IDX] = SBK_MT_N;
            mt_seed(reinterpret_cast<uint32_t*>(r + L.st.mt), v->seeds[i]);
            if (L.st.cmt) {
                reinterpret_cast<int*>(r + L.st.iplant)[sbk::PI_CONV_IDX] = SBK_MT_N;
                mt_seed(reinterpret_cast<uint32_t*>(r + L.st.cmt), v->conv_seeds[i]);
            }
            v->bytes_per_step += L.bytes_per_step;
            v->record_bytes_per_step += L.record_bytes_per_step;
            v->flops_per_step += L.solve_flops;
        }
        hip_ok(hipMalloc(&v->d_state, std::max<size_t>(v->state_bytes, 16)), "hipMalloc(state)");
        hip_ok(hipMemcpy(v->d_state, rec.data(), v->state_bytes, hipMemcpyHostToDevice), "upload state");
    }
    if (v->canonical) {
        std::vector<sbk::CanonTab> tabs(v->layouts.size());
        for (size_t li = 0; li < v->layouts.size(); li++) tabs[li] = *v->layouts[li].canon;
        hip_ok(hipMalloc(&v->d_canon, sizeof(sbk::CanonTab) * tabs.size()), "hipMalloc(canonical maps)");
        hip_ok(hipMemcpy(v->d_canon, tabs.data(), sizeof(sbk::CanonTab) * tabs.size(), hipMemcpyHostToDevice),
               "upload");
        const size_t na = (size_t)n * SB_ACT, ns = (size_t)n * 2 * SBC_K;
        hip_ok(hipMalloc(&v->d_raw, sizeof(float) * (size_t)n * SB_OBS), "hipMalloc(canonical)");
        hip_ok(hipMalloc(&v->d_native, sizeof(float) * na), "hipMalloc(canonical)");
        hip_ok(hipMalloc(&v->d_cbase, sizeof(float) * na), "hipMalloc(canonical)");
        hip_ok(hipMalloc(&v->d_ctrust, sizeof(float) * na), "hipMalloc(canonical)");
        hip_ok(hipMalloc(&v->d_cpid, sizeof(double) * ns), "hipMalloc(canonical)");
        hip_ok(hipMalloc(&v->d_cinfo, sizeof(float) * ns), "hipMalloc(canonical)");
        hip_ok(hipMemset(v->d_raw, 0, sizeof(float) * (size_t)n * SB_OBS), "clear");
        hip_ok(hipMemset(v->d_native, 0, sizeof(float) * na), "clear");
        hip_ok(hipMemset(v->d_cbase, 0, sizeof(float) * na), "clear");
        hip_ok(hipMemset(v->d_ctrust, 0, sizeof(float) * na), "clear");
        hip_ok(hipMemset(v->d_cpid, 0, sizeof(double) * ns), "clear");
        hip_ok(hipMemset(v->d_cinfo, 0, sizeof(float) * ns), "clear");
    }
    {
        const size_t nl = 3 + 3 * v->scens.size();
        hip_ok(hipMalloc(&v->d_live, nl * sizeof(double)), "hipMalloc(live log)");
        hip_ok(hipHostMalloc(&v->h_live, nl * sizeof(double), hipHostMallocDefault), "hipHostMalloc(live log)");
        v->live_prev.assign(3 * v->scens.size(), 0.0);
        for (const HostScen& S : v->scens) {
            std::string name = S.path.substr(S.path.find_last_of('/') + 1);
            if (ends_with(name, ".sbb")) name.resize(name.size() - 4);
            v->live_keys.push_back("scenario/" + name + "/reward");
            v->live_keys.push_back("scenario/" + name + "/comfort_dev_K");
        }
    }
    // ---- Env array (host memory the device can write: logs)
    void* envmem = nullptr;
    hip_ok(hipHostMalloc(&envmem, sizeof(Env) * (size_t)n, hipHostMallocCoherent), "hipHostMalloc(envs)");
    memset(envmem, 0, sizeof(Env) * (size_t)n);
    v->envs = static_cast<Env*>(envmem);
    for (int i = 0; i < n; i++) {
        Env& E = v->envs[i];
        const sbk::DevLayout& L = v->layouts[v->desc[i].layout].dev;
        E.agents[0].observations = observations + (size_t)i * SB_OBS;
        E.agents[0].actions = actions + (size_t)i * SB_ACT;
        E.agents[0].rewards = rewards + i;
        E.agents[0].terminals = terminals + i;
        E.num_agents = 1;
        E.max_steps = v->desc[i].max_steps;
        E.start_offset = v->desc[i].start;
        E.n_act = v->canonical ? SBC_ACT : L.n_act;
        E.n_cont = v->canonical ? SBC_ACT : L.n_cont;
        E.n_disc = v->canonical ? 0 : L.n_disc;
        E.loaded = 1;
        E.index = i;
        E.vec = v.get();
    }
    // field scenarios: tables, field group, per-env records
    {
        const int fexact = (int)kw(kwargs, "field_exact", 0.0f) != 0;
        const int fepb = (int)kw(kwargs, "field_envs_per_block", 0.0f);
        if (fepb < 0) die("env.field_envs_per_block must be >= 0");
        // (every scenario holds at least one env: G <= n)
        for (size_t fi = 0; fi < v->fields.size(); fi++) {
            std::string err, path;
            for (auto& S : v->scens)
                if (S.field == (int)fi) path = S.path;
            if (!field_attach(v->fields[fi], path, v->field_slots[fi], fexact ? SBX_FDM_EXACT : 0, fepb, &err))
                die(path + ": " + err);
            v->bytes_per_step += field_bytes_per_step(v->fields[fi]);
            v->record_bytes_per_step += field_bytes_per_step(v->fields[fi]);
            v->flops_per_step += field_flops_per_step(v->fields[fi]);
        }
    }
    hip_ok(hipDeviceSynchronize(), "sync after create");
    g_last = v.get();
    Env* out = v->envs;
    v.release();
    return out;
}

// The reference ignores a NULL stream (smart_buildings.cu:2887-2890); here
// NULL binds the null stream, the binding before any call, so a caller that
// bound another stream (a graph capture's, say) can return to the default one.
void puf_bind_stream(void* s) { g_stream = (hipStream_t)s; }

void puf_init(Env* env, Dict* kwargs) {
    (void)kwargs;
    if (!env) return;
    memset(&env->log, 0, sizeof(env->log));
}

void puf_reset(Env* envs) {
    Vec* v = vec_of(envs);
    for (int i = 0; i < v->n; i++) {
        v->envs[i].step = 0;
        unsigned char* m = v->envs[i].agents[0].action_mask;
        if (m) {
            for (int h = 0; h < SB_CONT; h++) m[h] = (h < v->envs[i].n_cont) ? 1 : 0;
            for (int h = 0; h < SB_DISC; h++) {
                unsigned char b = (h < v->envs[i].n_disc) ? 1 : 0;
                m[SB_CONT + 2 * h] = b;
                m[SB_CONT + 2 * h + 1] = b;
            }
        }
    }
    launch(v, sbk::KMODE_RESET);
    hip_ok(hipStreamSynchronize(g_stream), "reset");
    std::fill(v->live_prev.begin(), v->live_prev.end(), 0.0);   // the per-env sums restart at 0
}

// One step reading its action rows from `actions` (the bound buffer when null).
void step_from(Vec* v, const float* actions) {
    const sbk::KParams p = params(v, sbk::KMODE_STEP);
    if (v->t_on && v->t_seen++ % v->t_on == 0 && v->t_used < kTimerPairs) {
        hip_ok(hipEventRecord(v->tev[2 * v->t_used], g_stream), "timer event");
        run_env(v, p, actions);
        hip_ok(hipEventRecord(v->tev[2 * v->t_used + 1], g_stream), "timer event");
        v->t_used++;
        return;
    }
    run_env(v, p, actions);
}

void puf_step(Env* envs) { step_from(vec_of(envs), nullptr); }

void puf_render(Env* env) { (void)env; }

void puf_close(Env* envs) {
    if (!envs) return;
    Vec* v = vec_of(envs);
    (void)hipStreamSynchronize(g_stream);
    (void)hipFree(v->d_arena);
    (void)hipFree(v->d_state);
    (void)hipFree(v->d_layouts);
    (void)hipFree(v->d_scens);
    (void)hipFree(v->d_envs);
    (void)hipFree(v->d_order);
    (void)hipFree(v->d_tiles);
    for (hipEvent_t e : v->tev) (void)hipEventDestroy(e);
    (void)hipFree(v->p_h1);
    (void)hipFree(v->p_h2);
    (void)hipFree(v->p_y);
    (void)hipFree(v->p_hlp);
    (void)hipFree(v->p_hent);
    (void)hipFree(v->d_ncont);
    (void)hipFree(v->d_ndisc);
    (void)hipFree(v->d_live);
    (void)hipFree(v->d_air);
    (void)hipHostFree(v->h_live);
    for (void* p : {(void*)v->d_canon, (void*)v->d_raw, (void*)v->d_native, (void*)v->d_cbase, (void*)v->d_ctrust,
                    (void*)v->d_cpid, (void*)v->d_cinfo})
        (void)hipFree(p);
    for (FieldScen* f : v->fields) field_close(f);
    (void)hipHostFree(v->envs);
    if (g_last == v) g_last = nullptr;
    delete v;
}

void puf_log(Log* log, Dict* out) {
    dict_set(out, "perf", log->perf);
    dict_set(out, "score", log->score);
    dict_set(out, "episode_return", log->episode_return);
    dict_set(out, "episode_length", log->episode_length);
    dict_set(out, "comfort_dev_K", log->comfort_dev_K);
    dict_set(out, "worst_dev_K", log->worst_dev_K);
    dict_set(out, "out_of_band_frac", log->out_of_band_frac);
    dict_set(out, "productivity", log->productivity);
    dict_set(out, "energy_cost_norm", log->energy_cost_norm);
    dict_set(out, "carbon_norm", log->carbon_norm);
    dict_set(out, "elec_kwh", log->elec_kwh);
    dict_set(out, "gas_kwh", log->gas_kwh);
    dict_set(out, "n", log->n);
}

// Totals over every env since puf_reset (env_steps, episodes, reward_mean)
// and, for a vec of several scenarios, each scenario's mean reward and mean
// zone deviation per env-step since the previous call (the reference's
// scenario/<name>/* keys, complete_port/gpu/smart_buildings.cu:3069-3100):
// one device reduction and one copy on the bound stream, then a sync.
void puf_live_log(Env* envs, Dict* out) {
    Vec* v = vec_of(envs);
    const int ns = (int)v->scens.size();
    int rc = sbk_launch_live_sums(v->d_envs, v->d_layouts, v->d_state, v->n, ns, v->d_live, g_stream);
    if (rc != 0) die("live log kernel launch failed");
    for (size_t fi = 0; fi < v->fields.size(); fi++) {
        int scen = -1;
        for (int g = 0; g < ns; g++)
            if (v->scens[g].field == (int)fi) scen = g;
        if (!field_live(v->fields[fi], v->d_live, scen, g_stream)) die("live log kernel launch failed (field scenario)");
    }
    const size_t nl = 3 + 3 * (size_t)ns;
    hip_ok(hipMemcpyAsync(v->h_live, v->d_live, nl * sizeof(double), hipMemcpyDeviceToHost, g_stream), "live log");
    hip_ok(hipStreamSynchronize(g_stream), "live log");
    const double rs = v->h_live[0], st = v->h_live[1], eps = v->h_live[2];
    dict_set(out, "env_steps", (float)st);
    dict_set(out, "episodes", (float)eps);
    dict_set(out, "reward_mean", st > 0.0 ? (float)(rs / st) : 0.0f);
    for (int g = 0; g < ns; g++) {
        const double* cur = v->h_live + 3 + 3 * g;
        double* prev = v->live_prev.data() + 3 * g;
        const double dn = cur[2] - prev[2];
        if (ns > 1 && dn > 0.0) {
            dict_set(out, v->live_keys[2 * g].c_str(), (float)((cur[0] - prev[0]) / dn));
            dict_set(out, v->live_keys[2 * g + 1].c_str(), (float)((cur[1] - prev[1]) / dn));
        }
        for (int q = 0; q < 3; q++) prev[q] = cur[q];
    }
}

// The action mask of every agent (complete_port/gpu/smart_buildings.cu:3230-
// 3300): the env's continuous heads and both categories of its discrete heads,
// or (canonical) the canonical slots the building has. The mask may be device
// or host memory: it is built on the host and copied.
void puf_mask_init(unsigned char* mask, int width, int nagents) {
    Vec* v = g_last;
    if (!v || !mask || nagents <= 0) return;
    if (width < 1 || width > SB_MASK_WIDTH) die("puf_mask_init: width " + std::to_string(width) + " out of range");
    std::vector<unsigned char> host((size_t)nagents * width, 0);
    for (int a = 0; a < nagents; a++) {
        unsigned char* m = host.data() + (size_t)a * width;
        const int i = a < v->n ? a : v->n - 1;
        const Env& E = v->envs[i];
        if (v->canonical) {
            const sbk::CanonTab& C = *v->layouts[v->desc[i].layout].canon;
            for (int j = 0; j < C.n_act; j++) {
                const int sl = C.slot_of_action[j];
                if (sl >= 0 && sl < width) m[sl] = 1;
            }
            continue;
        }
        for (int h = 0; h < SB_CONT && h < width; h++) m[h] = (h < E.n_cont) ? 1 : 0;
        for (int h = 0; h < SB_DISC && SB_CONT + 2 * h + 1 < width; h++) {
            unsigned char b = (h < E.n_disc) ? 1 : 0;
            m[SB_CONT + 2 * h] = b;
            m[SB_CONT + 2 * h + 1] = b;
        }
    }
    hip_ok(hipMemcpy(mask, host.data(), host.size(), hipMemcpyDefault), "puf_mask_init copy");
}

void sbx_gen_actions(Env* envs, uint64_t seed, uint32_t step) {
    Vec* v = vec_of(envs);
    int rc = sbk_launch_gen_actions(v->actions, v->d_ncont, v->d_ndisc, v->n, seed, step, g_stream);
    if (rc != 0) die("action kernel launch failed");
}

void sbx_vec_info(Env* envs, SbxVecInfo* out) {
    Vec* v = vec_of(envs);
    memset(out, 0, sizeof(*out));
    out->n_envs = v->n;
    out->n_layouts = (int)v->layouts.size();
    out->n_scenarios = (int)v->scens.size();
    out->block = 2 * v->width * v->epb;
    out->lds_bytes = v->lds_bytes;
    out->envs_per_block = v->epb;
    for (auto& L : v->layouts) out->max_nodes = std::max(out->max_nodes, L.dev.n);
    out->bytes_per_step = v->bytes_per_step;
    out->record_bytes_per_step = v->record_bytes_per_step;
    out->flops_per_step = v->flops_per_step;
}

int sbx_env_state(Env* envs, int i, double* out, int cap) {
    Vec* v = vec_of(envs);
    if (i < 0 || i >= v->n) return -1;
    if (v->field_of[i] >= 0) {
        hip_ok(hipStreamSynchronize(g_stream), "state sync");
        return field_state(v->fields[v->field_of[i]], v->slot_of[i], out, cap);
    }
    const sbk::EnvDesc& d = v->desc[i];
    const sbk::DevLayout& L = v->layouts[d.layout].dev;
    std::vector<unsigned char> r(L.st.bytes);
    hip_ok(hipStreamSynchronize(g_stream), "state sync");
    hip_ok(hipMemcpy(r.data(), v->d_state + d.state_off, r.size(), hipMemcpyDeviceToHost), "state copy");
    const unsigned char* s = r.data();
    auto f = [&](int off) { return reinterpret_cast<const double*>(s + off); };
    std::vector<double> o;
    for (int t = 0; t < L.n; t++) o.push_back(f(L.st.T)[t]);
    for (int t = 0; t < L.n; t++) o.push_back(f(L.st.M)[t]);
    for (int x = 0; x < L.nv; x++) o.push_back(f(L.st.damper)[x]);
    for (int x = 0; x < L.nv; x++) o.push_back(f(L.st.reheat)[x]);
    for (int x = 0; x < L.nv; x++) o.push_back(f(L.st.ratio)[x]);
    for (int x = 0; x < L.nv; x++) o.push_back(f(L.st.sensing)[x]);
    for (int a = 0; a < L.na; a++) o.push_back(f(L.st.flow)[a]);
    for (int a = 0; a < L.na; a++) o.push_back(f(L.st.sat)[a]);
    for (int a = 0; a < L.na; a++) o.push_back(f(L.st.recirc)[a]);
    for (int a = 0; a < L.na; a++) o.push_back(f(L.st.fan)[a]);
    if (v->d_air) {
        // the last step's air side (zero before the first step, as in a new reference env)
        std::vector<double> at(2 * (size_t)v->air_stride);
        hip_ok(hipMemcpy(at.data(), v->d_air + (size_t)i * at.size(), at.size() * sizeof(double),
                         hipMemcpyDeviceToHost), "air copy");
        for (int c = 0; c < L.k; c++) o.push_back(at[c]);
        for (int c = 0; c < L.k; c++) o.push_back(at[v->air_stride + c]);
    } else {
        for (int c = 0; c < 2 * L.k; c++) o.push_back(NAN);   // kept only under trace_air
    }
    for (int z = 0; z < L.nz; z++) o.push_back((double)s[L.st.occV + z]);
    const double* pf = f(L.st.plant);
    const int* ip = reinterpret_cast<const int*>(s + L.st.iplant);
    o.push_back(pf[sbk::PF_BOILER_CUR]);
    o.push_back(pf[sbk::PF_BOILER_RET]);
    o.push_back(pf[sbk::PF_BOILER_SP]);
    o.push_back(pf[sbk::PF_PUMP_HEAD]);
    o.push_back((double)ip[sbk::PI_STEP_INDEX]);
    // extras after the oracle's layout: f64 reward sum since puf_reset, steps since puf_reset
    o.push_back(pf[sbk::PF_REW_SUM]);
    o.push_back((double)ip[sbk::PI_STEPS_TOTAL]);
    if ((int)o.size() > cap) return -1;
    memcpy(out, o.data(), o.size() * sizeof(double));
    return (int)o.size();
}

int sbx_phase_times(Env* envs, double* mean_us, double* max_us, int n_phases) {
    Vec* v = vec_of(envs);
    if (n_phases > SBK_NSTAMP - 1) n_phases = SBK_NSTAMP - 1;
    unsigned long long* d = nullptr;
    const size_t count = (size_t)v->n * SBK_NSTAMP;
    hip_ok(hipMalloc(&d, count * sizeof(unsigned long long)), "hipMalloc(stamps)");
    hip_ok(hipMemset(d, 0, count * sizeof(unsigned long long)), "memset(stamps)");
    sbk::KParams p = params(v, sbk::KMODE_STEP);
    p.phase_ts = d;
    run_env(v, p, nullptr);
    hip_ok(hipStreamSynchronize(g_stream), "stamps sync");
    std::vector<unsigned long long> h(count);
    hip_ok(hipMemcpy(h.data(), d, count * sizeof(unsigned long long), hipMemcpyDeviceToHost), "stamps copy");
    (void)hipFree(d);
    int dev = 0, khz = 0;
    (void)hipGetDevice(&dev);
    hip_ok(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev), "wall clock rate");
    const double us_per_tick = 1e3 / (double)khz;
    for (int k = 0; k < n_phases; k++) {
        double sum = 0.0, mx = 0.0;
        for (int b = 0; b < v->n; b++) {
            const unsigned long long* t = &h[(size_t)b * SBK_NSTAMP];
            double dt = (t[k + 1] >= t[k]) ? (double)(t[k + 1] - t[k]) * us_per_tick : 0.0;
            sum += dt;
            mx = std::max(mx, dt);
        }
        mean_us[k] = sum / v->n;
        max_us[k] = mx;
    }
    return n_phases;
}

int sbx_phase_stamps(Env* envs, unsigned long long* out, int cap) {
    Vec* v = vec_of(envs);
    const size_t count = (size_t)v->n * SBK_NSTAMP;
    if (!out || cap < (int)count) return -1;
    unsigned long long* d = nullptr;
    hip_ok(hipMalloc(&d, count * sizeof(unsigned long long)), "hipMalloc(stamps)");
    hip_ok(hipMemset(d, 0, count * sizeof(unsigned long long)), "memset(stamps)");
    sbk::KParams p = params(v, sbk::KMODE_STEP);
    p.phase_ts = d;
    run_env(v, p, nullptr);
    hip_ok(hipStreamSynchronize(g_stream), "stamps sync");
    hip_ok(hipMemcpy(out, d, count * sizeof(unsigned long long), hipMemcpyDeviceToHost), "stamps copy");
    (void)hipFree(d);
    return (int)count;
}

int sbx_pass_times(Env* envs, int env, long long* cycles, int cap) {
    Vec* v = vec_of(envs);
    if (env < 0 || env >= v->n || v->field_of[env] >= 0) return -1;
    const bool relax = v->layouts[v->desc[env].layout].dev.solver == sbk::SOLVER_RELAX;
    // relaxation: a stamp at entry, after the setup and after every sweep
    const int np = relax ? SBK_RX_MAXIT + 1 : v->layouts[v->desc[env].layout].dev.n_pass;
    if (cap < np) return -1;
    unsigned long long* d = nullptr;
    hip_ok(hipMalloc(&d, (size_t)(np + 1) * sizeof(unsigned long long)), "hipMalloc(pass stamps)");
    hip_ok(hipMemset(d, 0, (size_t)(np + 1) * sizeof(unsigned long long)), "memset(pass stamps)");
    sbk::KParams p = params(v, sbk::KMODE_STEP);
    p.pass_ts = d;
    p.pass_ts_env = env;
    run_env(v, p, nullptr);
    hip_ok(hipStreamSynchronize(g_stream), "pass stamps sync");
    std::vector<unsigned long long> h(np + 1);
    hip_ok(hipMemcpy(h.data(), d, h.size() * sizeof(unsigned long long), hipMemcpyDeviceToHost), "copy");
    (void)hipFree(d);
    if (relax) {
        int m = 0;
        while (m < np && h[m + 1] != 0) {
            cycles[m] = (long long)(h[m + 1] - h[m]);
            m++;
        }
        return m;
    }
    // stamps are taken every SBK_PLAN_DEPTH passes (and after the last):
    // split each interval evenly
    for (int i = 0; i < np; i += SBK_PLAN_DEPTH) {
        const int j = std::min(i + SBK_PLAN_DEPTH, np);
        const long long dt = (long long)(h[j] - h[i]);
        for (int k = i; k < j; k++) cycles[k] = dt / (j - i);
    }
    return np;
}

double sbx_kernel_timer(Env* envs, int on, int* count) {
    Vec* v = vec_of(envs);
    if (on) {
        if (v->tev.empty()) {
            v->tev.resize(2 * kTimerPairs);
            for (auto& e : v->tev) hip_ok(hipEventCreate(&e), "event");
        }
        v->t_used = 0;
        v->t_seen = 0;
        v->t_on = on;
        if (count) *count = 0;
        return 0.0;
    }
    v->t_on = 0;
    if (count) *count = v->t_used;
    if (v->t_used == 0) return 0.0;
    hip_ok(hipEventSynchronize(v->tev[2 * v->t_used - 1]), "timer sync");
    double sum = 0.0;
    for (int i = 0; i < v->t_used; i++) {
        float ms = 0.f;
        hip_ok(hipEventElapsedTime(&ms, v->tev[2 * i], v->tev[2 * i + 1]), "elapsed");
        sum += ms;
    }
    return sum * 1e3 / v->t_used;
}

int sbx_step_actions(Env* envs, const float* actions) {
    if (!actions) { g_err = "sbx_step_actions: null action rows"; return -1; }
    step_from(vec_of(envs), actions);
    return 0;
}

float sbx_time_step(Env* envs, int iters) {
    Vec* v = vec_of(envs);
    hipEvent_t a, b;
    hip_ok(hipEventCreate(&a), "event");
    hip_ok(hipEventCreate(&b), "event");
    hip_ok(hipEventRecord(a, g_stream), "event");
    for (int i = 0; i < iters; i++) launch(v, sbk::KMODE_STEP);
    hip_ok(hipEventRecord(b, g_stream), "event");
    hip_ok(hipEventSynchronize(b), "event sync");
    float ms = 0.f;
    hip_ok(hipEventElapsedTime(&ms, a, b), "elapsed");
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    return ms;
}

static bool policy_ok(const SbxPolicy* p) {
    if (!p || !p->w1 || !p->b1 || !p->w2 || !p->b2 || !p->w3 || !p->b3) { g_err = "null policy weight"; return false; }
    // the reference trainer aborts unless policy.beta_floor > 0
    // (complete_port/patches/pufferlib_core.diff:5204-5208): at 0 a shape can
    // underflow to exactly 0, where lgamma and the boosted draw give inf/NaN
    if (!(p->beta_floor > 0.0f) || !std::isfinite(p->beta_floor)) {
        g_err = "policy beta_floor must be finite and > 0";
        return false;
    }
    return true;
}

int sbx_policy_bind(Env* envs, const SbxPolicy* p) {
    if (!policy_ok(p)) return -1;
    Vec* v = vec_of(envs);
    v->pol = *p;
    if (!v->p_h1) {
        hip_ok(hipMalloc(&v->p_h1, sizeof(float) * (size_t)v->n * SBX_POLICY_HIDDEN), "hipMalloc(policy)");
        hip_ok(hipMalloc(&v->p_h2, sizeof(float) * (size_t)v->n * SBX_POLICY_HIDDEN), "hipMalloc(policy)");
        hip_ok(hipMalloc(&v->p_y, sizeof(float) * (size_t)v->n * SBX_POLICY_HEADS), "hipMalloc(policy)");
        hip_ok(hipMalloc(&v->p_hlp, sizeof(float) * (size_t)v->n * SB_ACT), "hipMalloc(policy)");
        hip_ok(hipMalloc(&v->p_hent, sizeof(float) * (size_t)v->n * SB_ACT), "hipMalloc(policy)");
    }
    return 0;
}

int sbx_policy_act(Env* envs, uint64_t seed, uint32_t step) {
    Vec* v = vec_of(envs);
    if (!v->p_h1) { g_err = "sbx_policy_act before sbx_policy_bind"; return -1; }
    const SbxPolicy& p = v->pol;
    int rc = sbk_launch_policy(v->obs, p.w1, p.b1, p.w2, p.b2, p.w3, p.b3, v->p_h1, v->p_h2, v->p_y, v->actions,
                               v->d_ncont, v->d_ndisc, v->n, seed, step, nullptr, nullptr, nullptr, nullptr, nullptr,
                               p.beta_floor, v->obs_cols, g_stream);
    if (rc != 0) die(std::string("policy launch failed: ") + hipGetErrorString((hipError_t)rc));
    return 0;
}

int sbx_policy_act_noalloc(Env* envs, const SbxPolicy* p, uint64_t seed, uint32_t step) {
    if (!policy_ok(p)) return -1;
    Vec* v = vec_of(envs);
    if (v->n > sbk_noalloc_max_envs()) {
        g_err = "sbx_policy_act_noalloc: " + std::to_string(v->n) + " envs, at most "
                + std::to_string(sbk_noalloc_max_envs());
        return -1;
    }
    int rc = sbk_launch_policy_noalloc(v->obs, p->w1, p->b1, p->w2, p->b2, p->w3, p->b3, v->actions, v->d_ncont,
                                       v->d_ndisc, v->n, seed, step, p->beta_floor, v->obs_cols, g_stream);
    if (rc != 0) {
        g_err = std::string("sbx_policy_act_noalloc: ") + hipGetErrorString((hipError_t)rc);
        return -1;
    }
    return 0;
}

int sbx_policy_act_logp(Env* envs, uint64_t seed, uint32_t step, float* draws, float* logp, float* entropy) {
    Vec* v = vec_of(envs);
    if (!v->p_h1) { g_err = "sbx_policy_act_logp before sbx_policy_bind"; return -1; }
    if (!draws || !logp || !entropy) { g_err = "sbx_policy_act_logp: null output"; return -1; }
    const SbxPolicy& p = v->pol;
    int rc = sbk_launch_policy(v->obs, p.w1, p.b1, p.w2, p.b2, p.w3, p.b3, v->p_h1, v->p_h2, v->p_y, v->actions,
                               v->d_ncont, v->d_ndisc, v->n, seed, step, draws, v->p_hlp, v->p_hent, logp, entropy,
                               p.beta_floor, v->obs_cols, g_stream);
    if (rc != 0) die(std::string("policy launch failed: ") + hipGetErrorString((hipError_t)rc));
    return 0;
}

int sbx_beta_eval(Env* envs, const float* y, const float* draws, float* logp, float* entropy, float* grad) {
    Vec* v = vec_of(envs);
    if (!v->p_hlp) { g_err = "sbx_beta_eval before sbx_policy_bind"; return -1; }
    if (!y || !draws || !logp || !entropy) { g_err = "sbx_beta_eval: null argument"; return -1; }
    int rc = sbk_launch_beta_eval(y, draws, v->d_ncont, v->d_ndisc, v->n, v->p_hlp, v->p_hent, grad, logp, entropy,
                                  v->pol.beta_floor, g_stream);
    if (rc != 0) die(std::string("beta eval launch failed: ") + hipGetErrorString((hipError_t)rc));
    return 0;
}

int sbx_ppo_beta(Env* envs, const float* y_new, const float* y_old, const float* draws, const float* logp_old,
                 const float* adv, const SbxPpo* args, float* out, float* grad) {
    if (!y_new || !y_old || !draws || !logp_old || !adv || !args || !out) {
        g_err = "sbx_ppo_beta: null argument";
        return -1;
    }
    if (!(args->beta_floor > 0.0f) || !std::isfinite(args->beta_floor) || !(args->clip_coef >= 0.0f)) {
        g_err = "sbx_ppo_beta: beta_floor must be finite and > 0, clip_coef >= 0";
        return -1;
    }
    Vec* v = vec_of(envs);
    int rc = sbk_launch_ppo_beta(y_new, y_old, draws, logp_old, adv, v->d_ncont, v->d_ndisc, v->n, args->beta_floor,
                                 args->clip_coef, args->ent_coef, args->ratio_per_dim, out, grad, g_stream);
    if (rc != 0) die(std::string("ppo beta launch failed: ") + hipGetErrorString((hipError_t)rc));
    return 0;
}

int sbx_policy_heads(Env* envs, float* out, int cap) {
    Vec* v = vec_of(envs);
    const size_t count = (size_t)v->n * SBX_POLICY_HEADS;
    if (!v->p_y || !out || cap < (int)count) return -1;
    hip_ok(hipStreamSynchronize(g_stream), "policy sync");
    hip_ok(hipMemcpy(out, v->p_y, count * sizeof(float), hipMemcpyDeviceToHost), "policy heads copy");
    return (int)count;
}

int sbx_beta_sample(const float* alpha, const float* beta, float* out, int n, uint64_t seed, void* stream) {
    if (!alpha || !beta || !out || n <= 0) return -1;
    int rc = sbk_launch_beta_sample(alpha, beta, out, n, seed, (hipStream_t)stream);
    if (rc != 0) die(std::string("beta sample launch failed: ") + hipGetErrorString((hipError_t)rc));
    return 0;
}

int sbx_solve_info(Env* envs, int i, double* out) {
    Vec* v = vec_of(envs);
    if (i < 0 || i >= v->n || !out || v->field_of[i] >= 0) return -1;
    const sbk::EnvDesc& d = v->desc[i];
    const HostLayout& H = v->layouts[d.layout];
    double pf[8];
    hip_ok(hipStreamSynchronize(g_stream), "state sync");
    hip_ok(hipMemcpy(pf, v->d_state + d.state_off + H.dev.st.plant, sizeof(pf), hipMemcpyDeviceToHost), "copy");
    const bool relax = H.dev.solver == sbk::SOLVER_RELAX;
    out[0] = relax ? (H.dev.rx_block ? 2.0 : 1.0) : 0.0;
    out[1] = relax ? (H.dev.rx_block ? H.block.rho : H.relax.rho) : 0.0;
    out[2] = pf[sbk::PF_SWEEPS];
    out[3] = pf[sbk::PF_CAPPED];
    return 4;
}

int sbx_canon_state(Env* envs, int i, float* raw_obs, float* base, double* pid) {
    Vec* v = vec_of(envs);
    if (!v->canonical || i < 0 || i >= v->n) return -1;
    hip_ok(hipStreamSynchronize(g_stream), "canonical state");
    if (raw_obs)
        hip_ok(hipMemcpy(raw_obs, v->d_raw + (size_t)i * SB_OBS, sizeof(float) * SB_OBS, hipMemcpyDeviceToHost), "copy");
    if (base)
        hip_ok(hipMemcpy(base, v->d_cbase + (size_t)i * SB_ACT, sizeof(float) * SB_ACT, hipMemcpyDeviceToHost), "copy");
    if (pid)
        hip_ok(hipMemcpy(pid, v->d_cpid + (size_t)i * 2 * SBC_K, sizeof(double) * 2 * SBC_K, hipMemcpyDeviceToHost),
               "copy");
    return v->layouts[v->desc[i].layout].canon->n_act;
}

int sbx_env_meta(Env* envs, int i, int* scenario, int* start, uint32_t* occ_seed) {
    Vec* v = vec_of(envs);
    if (i < 0 || i >= v->n) return -1;
    if (scenario) *scenario = v->desc[i].scen;
    if (start) *start = v->desc[i].start;
    if (occ_seed) *occ_seed = v->seeds[i];
    return 0;
}

const char* sbx_scenario_path(Env* envs, int s) {
    Vec* v = vec_of(envs);
    if (s < 0 || s >= (int)v->paths.size()) return nullptr;
    return v->paths[s].c_str();
}

struct PlanHolder {
    sbh::SolvePlan plan;
    sbh::RelaxPlan relax;
    sbh::BlockPlan block;
};
static std::map<const void*, PlanHolder*> g_plans;

int sbx_plan_layout(const char* blob_path, int width, SbxPlan* out) {
    if (!blob_path || !out) return -1;
    if (width != 64 && width != 128 && width != 256) { g_err = "width must be 64, 128 or 256"; return -1; }
    sbh::Blob b;
    std::string err;
    if (!b.open(blob_path, &err)) { g_err = err; return -1; }
    auto* h = new PlanHolder();
    if (!sbh::build_plan(b, width, &h->plan, &err)) { g_err = err; delete h; return -2; }
    const sbh::SolvePlan& P = h->plan;
    memset(out, 0, sizeof(*out));
    out->n = P.n;
    out->width = P.width;
    out->n_slots = P.n_slots;
    out->vec_base = P.vec_base;
    out->inv_base = P.inv_base;
    out->term_bits = P.term_bits;
    out->scale_base = P.scale_base;
    out->n_pass = P.n_pass();
    out->n_levels = P.n_levels;
    out->n_tasks = P.n_tasks;
    out->n_pairs = P.n_pairs;
    out->kmax = sbh::kPlanKmax;
    out->n_hdr = (int)P.hdr.size();
    out->n_words = (int)P.words.size();
    out->pass_info = reinterpret_cast<const int*>(P.passes.data());
    out->hdr = P.hdr.data();
    out->words = P.words.data();
    out->slot_init = P.slot_init.data();
    out->pos = P.pos.data();
    out->air_slot = P.air_slot.data();
    out->air_node = P.air_node.data();
    out->k = P.k;
    sbh::build_relax(b, P, &h->relax);
    const sbh::RelaxPlan& R = h->relax;
    out->rx_ok = R.ok ? 1 : 0;
    out->rx_rows = sbh::kRelaxRows;
    out->rx_terms_max = sbh::kRelaxTerms;
    out->rx_terms = R.terms;
    out->rx_rho = R.rho;
    if (R.ok) {
        out->rx_diag = R.diag.data();
        out->rx_air = R.air_col.data();
        out->rx_val = R.val.data();
        out->rx_col = R.col.data();
    }
    sbh::build_block(b, P, &h->block);
    const sbh::BlockPlan& BP = h->block;
    out->bx_ok = BP.ok ? 1 : 0;
    out->bx_rows = sbh::kBlockRows;
    out->bx_slots = sbh::kBlockSlots;
    out->bx_terms_max = sbh::kBlockTerms;
    out->bx_terms = BP.terms;
    out->bx_blocks = BP.n_blocks;
    out->bx_rho = BP.rho;
    if (BP.ok) {
        out->bx_row = BP.row.data();
        out->bx_diag = BP.diag.data();
        out->bx_air = BP.air.data();
        out->bx_in = BP.in.data();
        out->bx_val = BP.val.data();
        out->bx_col = BP.col.data();
        out->bx_trow = BP.trow.data();
    }
    g_plans[out->hdr] = h;
    return 0;
}

void sbx_plan_free(SbxPlan* p) {
    if (!p) return;
    auto it = g_plans.find(p->hdr);
    if (it != g_plans.end()) {
        delete it->second;
        g_plans.erase(it);
    }
    memset(p, 0, sizeof(*p));
}

const char* sbx_last_error(void) { return g_err.c_str(); }

const char* sbx_version(void) { return SB_CONT == 256 ? "sbenv 0.1 gfx950" : "sbenv 0.1 gfx950 cont320"; }

int sbx_cont_width(void) { return SB_CONT; }

}  // extern "C"

// Error text for the other host files of the library (field step).
void sbx_set_error(const std::string& msg) { g_err = msg; }
