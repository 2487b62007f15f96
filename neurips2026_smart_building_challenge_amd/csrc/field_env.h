// Field envs: scenarios whose field is FDM-scale (10^5-10^6 cells, general
// area-weighted air side), stepped behind the same PufferLib ABI as the RC
// envs. The HVAC plant, actions, observation, occupancy, reward and episode
// bookkeeping run in field_env_kernel.hip, one lane per env (O(zones + VAVs +
// fields) work per env-step); the field solve runs in fdm_kernel.hip on the
// scenario's group of envs (envs as lanes of its level-ordered row solves).
// Shared by the host (vec.cpp) and the device; not part of the public ABI.
//
// One env-step of a field scenario, on the bound stream:
//   fe_pre    decode + sb_sim_apply_native + sb_sim_step_pre from the zone
//             means of the current field (kept per env): each zone's heat per
//             room cell, the air-side conductance and supply temperature per
//             coupled column, the ambient temperature and h, into the field
//             step's inputs (complete_port/csim/sb_sim.c:357-457);
//   field     the FDM step (forcing, LU replay, air side, mass, field update;
//             complete_port/csim/sb_fdm.c:126-188) on every env of the group;
//   fe_means  each zone's mean over its room's cells of the new field, in the
//             room's cell order (sb_sim.c:149-160);
//   fe_post   sb_sim_step_post (boiler), the observation, the occupancy
//             interval, the 3C reward from the new zone means, the Log and
//             the auto-reset (complete_port/pufferlib_cpu_env.h:211-257); an
//             env that resets marks its field for re-initialisation;
//   fe_field_reset  temp_init / mass_temp_init into the marked envs' fields.
#pragma once
#include <stddef.h>
#include <stdint.h>

namespace sbe {

// Per-env state record (one block per env, envs of a scenario back to back),
// byte offsets. f64 arrays first, then i32, then u8, then the MT19937 words.
struct StateLayout {
    int bytes;
    // f64 [na]
    int recirc, sat, fan, flow, wsum, atotal, satv;
    // f64 [nv]
    int damper, reheat, ratio, heatsp, coolsp, dcmd, rcmd, sensing, vav_area;
    // f64 [nz]
    int avg_temp, zone_q, occV;
    // f64 [k]
    int air_g, air_T, coil;
    int plant;        // f64 [PL_COUNT]
    // i32
    int run, coolreq;                         // [na]
    int mode, prev_valid, dcmd_set, rcmd_set; // [nv]
    int ip;                                   // [IP_COUNT]
    int occ_state;                            // u8 [nz * nassign]
    int mt;                                   // u32 [624]
};

enum {
    PL_FFS = 0,          // flow factor sum
    PL_TOTAL_REHEAT,
    PL_BOILER_SP,
    PL_BOILER_RET,
    PL_BOILER_CUR,
    PL_BOILER_DSTEP,
    PL_PUMP_HEAD,
    PL_REW_SUM,          // f64 sum of rewards since puf_reset
    PL_COUNT
};

enum {
    IP_HWS_REQ = 0,
    IP_HWS_RUN,
    IP_PUMP_RUN,
    IP_STEP_INDEX,       // calendar row of the next step
    IP_STEP,             // steps into the episode
    IP_FIRST_DONE,       // the first episode after puf_vec_create has ended
    IP_MT_IDX,
    IP_STEPS_TOTAL,      // env-steps since puf_reset
    IP_EPISODES,         // episodes ended since puf_reset
    IP_COUNT
};

// Read-only tables of one field scenario (device pointers).
struct Tabs {
    int n_cvs, nz, nv, na, k, n_act, n_dev, n_aux, nassign, n1;
    // zone z's room cells (cell ids r * cols + c, the room's order) are
    // zcells[zoff[z] .. zoff[z + 1])
    const int* zoff;
    const int* zcells;
    const double* zone_area;      // [nz]
    const double* zm_init;        // [nz] zone means of temp_init (host, the same order)
    const int* vz_off;            // [nv + 1] VAV -> zones
    const int* vz_idx;
    const int* vav_ahu;           // [nv]
    const int* coupled;           // [k] column -> VAV
    const double* vav_c;          // [nv * 9]
    const double* ahu_c;          // [na * 9]
    const double* boiler_c;       // [10]
    double pump_head0, pump_eff, header_res, internal_w_m2, standby_frac, occupant_w, cv_area, dt_sec, h;
    double gas_den;               // log(r2 / c6) / c8 + 1 / c4 / r2 (sb_reward.c:19-23)
    // actions
    const uint8_t* act_kind;
    const uint8_t* act_act;
    const uint8_t* act_disc;
    const int* act_idx;
    const double* act_mn;
    const double* act_mx;
    const double* act_mnr;
    const double* act_mxr;
    // observation
    const uint8_t* f_kind;
    const uint8_t* f_id;
    const int* f_idx;
    const double* f_mean;
    const double* f_sd;           // sqrt(var) where var > 0, else 0
    // calendar
    const double* amb;
    const double* comfort;
    const double* heat_sp;
    const double* cool_sp;
    const double* aux_time;       // [n1][n_aux - 1]
    const int64_t* occ_hour;
    const uint8_t* occ_work;
    const int64_t* hour_m1;
    const uint8_t* work_m1;
    const int64_t* rew_hour;
    const int64_t* rew_month;
    const uint8_t* rew_work;
    // occupancy (sb_occup.c:8-20)
    int occ_ea, occ_la, occ_ed, occ_ld;
    double p_arr, p_dep;
    // reward
    const double* rw;             // [8]
    const double* elec_wk;
    const double* elec_we;
    const double* elec_co2;
    const double* gas_price;
    double gas_co2;
};

// One env of a field group: its index in the vec, its calendar start, episode
// lengths and its occupancy stream seed.
struct Slot {
    int env;
    int start;
    int max_steps;
    int first_steps;
    uint32_t occ_seed;
    int pad[3];
};

enum { FE_STEP = 0, FE_RESET = 1 };

struct Args {
    Tabs t;
    StateLayout st;
    unsigned char* state;         // [G][st.bytes]
    const Slot* slots;            // [G]
    int G;
    int mode;
    // the trainer's buffers (rows of 1024 / 272 floats)
    const float* actions;
    float* obs;
    float* rewards;
    float* terminals;
    void* host_env;               // Env array (host-coherent), or null
    int env_stride, log_offset;
    float reward_scale;
    // the field step's inputs: per env the heat per room cell of each zone,
    // the ambient temperature, h, per column the air-side conductance and
    // supply temperature
    double* qz;                   // [G][nz]
    double* amb;                  // [G]
    double* hh;                   // [G]
    double* g;                    // [G][k]
    double* airT;                 // [G][k]
    int* reset_mask;              // [G] fe_post marks envs whose field is re-initialised
    // the group's field: cell p of env b * Gl + l at T[(b * n_cvs + p) * Gl + l]
    const double* T;
    int Gl;
    double* live;                 // fe_live adds the totals since puf_reset to live[0..2]
};

// The host (g++) and the device (hipcc) compile these structs separately and
// exchange them byte for byte: both builds check the same sizes and offsets.
static_assert(sizeof(Tabs) == 488 && offsetof(Tabs, gas_co2) == 480, "Tabs layout");
static_assert(sizeof(StateLayout) == 132 && sizeof(Slot) == 32, "StateLayout / Slot layout");
static_assert(sizeof(Args) == 776 && offsetof(Args, st) == 488 && offsetof(Args, state) == 624
              && offsetof(Args, live) == 768, "Args layout");

}  // namespace sbe
