// Field envs: scenarios whose field is FDM-scale (10^5-10^6 cells, general
// area-weighted air side), stepped behind the same PufferLib ABI as the RC
// envs. Shared by the host (field_env.cpp, vec.cpp) and the device
// (field_env_kernel.hip); not part of the public ABI.
//
// Work split of one env-step of a field scenario (G envs), on the bound stream:
//   hvac(pre)   one 64-lane wavefront per env, its record staged in LDS:
//               actions decoded and applied, VAV / AHU / column / zone
//               passes with lanes over the entities and every csim
//               accumulation kept in its operand order by giving each sum to
//               one lane (per AHU over its VAVs, per zone over its columns),
//               the boiler update (it reads only pre-step values), and the
//               field step's inputs: heat per room cell of each zone, air-side
//               conductance and supply temperature per column, ambient, h;
//   conv plan   (stochastic convection on) one wavefront per env: the
//               convection stream's swap decisions of the step, which depend
//               on no temperature, composed per room into a permutation and
//               listed as (cell, source cell) moves;
//   field       the FDM step on the whole group (fdm_kernel.hip);
//   conv apply  the listed moves, gathered then scattered;
//   means       each zone's mean over its room's cells, lane per (zone, env);
//   hvac(post)  one wavefront per env: observation (lanes over fields),
//               occupancy draws (lanes over chains, positions in the MT
//               stream from a wavefront prefix sum), 3C reward, bookkeeping,
//               the Log at episode ends and the auto-reset (which also
//               re-initialises the env's field).
#pragma once
#include <stddef.h>
#include <stdint.h>

#define SBE_MT_N 624

namespace sbe {

// Per-env record (HBM, envs of a scenario back to back, stride `record`).
// [0, bytes) is the image the HVAC kernels stage into LDS and store back;
// the convection stream follows it (624 words, then its position in the
// block), read and written only by the plan kernel, which may run beside the
// HVAC kernels on another stream.
struct StateLayout {
    int bytes;        // staged image (16-byte multiple)
    int record;       // record stride (256-byte multiple)
    // f64 [na]
    int recirc, sat, fan, flow, satv;
    // f64 [nv]
    int damper, reheat, ratio, heatsp, coolsp, dcmd, rcmd, sensing, vav_area, unres;
    // f64 [nz]
    int avg_temp, zone_q, occV;
    // f64 [k]
    int air_g, air_T, coil, rwen;
    int plant;        // f64 [PL_COUNT]
    // i32
    int run, coolreq;                          // [na]
    int mode, prev_valid, dcmd_set, rcmd_set;  // [nv]
    int ip;                                    // [IP_COUNT]
    int ep;                                    // f32 [EP_COUNT] running episode sums
    int occ_state;                             // u8 [nz * nassign]
    int mt;                                    // u32 [624] occupancy stream (in the image)
    int cmt;                                   // u32 [624 + 4] convection stream and position (after the image; 0: none)
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
    PL_DEV_SUM,          // f64 sum since puf_reset of each step's mean zone deviation from the comfort band
    PL_COUNT
};

enum {
    IP_HWS_REQ = 0,
    IP_HWS_RUN,
    IP_PUMP_RUN,
    IP_STEP_INDEX,       // calendar row of the next step
    IP_STEP,             // steps into the episode
    IP_FIRST_DONE,       // the first episode after puf_vec_create has ended
    IP_MT_IDX,           // occupancy stream position in its block (624: twist before the next draw)
    IP_STEPS_TOTAL,      // env-steps since puf_reset
    IP_EPISODES,         // episodes ended since puf_reset
    IP_COUNT = 12
};

// The reference GPU env's running episode sums, float (complete_port/gpu/
// smart_buildings.cu:118-121, 1965-1971): the reward, the 8 per-step
// diagnostics (productivity term, normalized energy cost, normalized carbon,
// mean zone deviation, worst zone deviation (its sum unused), out-of-band
// fraction, electricity kWh, gas kWh), then the worst deviation as a maximum
enum { EP_RET = 0, EP_PART = 1, EP_WORST = 9, EP_COUNT = 10 };

// Read-only tables of one field scenario (device pointers).
struct Tabs {
    int n_cvs, nz, nv, na, k, n_act, n_dev, n_aux, nassign, n1;
    // zone z's room cells (field cell ids r * cols + c, the room's order) are
    // zcells[zoff[z] .. zoff[z + 1])
    const int* zoff;
    const int* zcells;
    const double* zone_area;      // [nz]
    const double* zm_init;        // [nz] zone means of temp_init (host, the room's order)
    const int* vz_off;            // [nv + 1] VAV -> zones
    const int* vz_idx;
    const int* vav_ahu;           // [nv]
    const int* coupled;           // [k] column -> VAV
    const int* av_off;            // [na + 1] AHU -> its VAVs, ascending
    const int* av_idx;
    const int* ac_off;            // [na + 1] AHU -> the columns of its VAVs, ascending
    const int* ac_idx;
    const int* zc_off;            // [nz + 1] zone -> the columns that heat it, in column order
    const int* zc_idx;
    const double* vav_c;          // [nv * 9]
    const double* ahu_c;          // [na * 9]
    const double* boiler_c;       // [10]
    double pump_head0, pump_eff, header_res, internal_w_m2, standby_frac, occupant_w, cv_area, dt_sec, h;
    double gas_den;               // log(r2 / c6) / c8 + 1 / c4 / r2 (sb_reward.c:19-23)
    // actions: per action its trainer column (continuous block or SB_CONT + d),
    // its target (kind | actuator << 4 | owner index << 8) and whether it is
    // the last action writing that target (the one the sequential apply keeps)
    const int* act_col;
    const int* act_tgt;
    const uint8_t* act_live;
    const uint8_t* act_disc;
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
    // field re-initialisation at an auto-reset
    const double* temp_init;      // [n_cvs]
    const double* mass_init;      // [n]
    int n_solved;
    // stochastic convection (sb_convect.c): rooms [cv_rooms + 1] offsets into
    // the cell list, each cell's field id, its candidate count (u8) and CSR
    // candidates as room-local positions
    int cv_rooms, cv_cells, cv_max_room;
    uint32_t cv_thr_hi, cv_thr_lo;   // swap when the 53-bit draw is <= this (hi:lo); hi = 0xFFFFFFFF: never
    const int* cv_off;
    const int* cv_cell;
    const uint8_t* cv_ncand;
    const int* cv_coff;
    const uint16_t* cv_cidx;
};

// One env of a field group: its index in the vec, its calendar start, episode
// lengths, its occupancy and convection stream seeds.
struct Slot {
    int env;
    int start;
    int max_steps;
    int first_steps;
    uint32_t occ_seed;
    uint32_t conv_seed;
    int pad[2];
};

enum { FE_STEP = 0, FE_RESET = 1 };

struct Args {
    Tabs t;
    StateLayout st;
    unsigned char* state;         // [G][st.record]
    const Slot* slots;            // [G]
    int G;
    int mode;
    // the trainer's buffers (rows of SB_OBS / SB_ACT floats)
    const float* actions;
    float* obs;
    float* rewards;
    float* terminals;
    void* host_env;               // Env array (host-coherent), or null
    int env_stride, log_offset;
    float reward_scale;
    int lds_bytes;                // dynamic LDS of the HVAC kernels (image + scratch)
    // the field step's inputs: per env the heat per room cell of each zone,
    // the ambient temperature, h, per column the air-side conductance and
    // supply temperature
    double* qz;                   // [G][nz]
    double* amb;                  // [G]
    double* hh;                   // [G]
    double* g;                    // [G][k]
    double* airT;                 // [G][k]
    // the group's field: cell p of env b * Gl + l at T[(b * n_cvs + p) * Gl + l]
    double* T;
    double* M;                    // interior mass, [(b * n + q) * Gl + l]
    int Gl;
    double* live;                 // the live-sums kernel adds the totals since puf_reset to live[0..2]
    int live_scen;                //   and the scenario's to live[3 + 3 live_scen ..]
    // convection moves of the step: per env at most cv_cells (convection cell
    // << 32 | source convection cell) words, their count, the gathered values;
    // pair overflow past the plan kernel's LDS
    unsigned long long* cv_moves; // [G][cv_cells]
    int* cv_count;                // [G]
    double* cv_vals;              // [G][cv_cells]
    unsigned int* cv_spill;       // [G][2][cv_max_room]: pairs, then shuffle draws, past the LDS
    int cv_lds_pairs;             // pairs the plan kernel keeps in LDS
    int exact;                    // the field group runs in exact mode (SBX_FDM_EXACT): sums in the reference's order
};

// The host (g++) and the device (hipcc) compile these structs separately and
// exchange them byte for byte: both builds check the same sizes and offsets.
static_assert(sizeof(StateLayout) == 144 && offsetof(StateLayout, cmt) == 140, "StateLayout layout");
static_assert(sizeof(Slot) == 32, "Slot layout");
static_assert(offsetof(Tabs, gas_co2) == 528 && offsetof(Tabs, temp_init) == 536 && offsetof(Tabs, cv_off) == 576
              && sizeof(Tabs) == 616, "Tabs layout");
static_assert(offsetof(Args, st) == 616 && offsetof(Args, state) == 760 && offsetof(Args, qz) == 840
              && offsetof(Args, live) == 904 && sizeof(Args) == 960, "Args layout");

}  // namespace sbe
