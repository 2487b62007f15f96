// Internal layout shared by the host planner (vec.cpp, plan.cpp) and the HIP
// step kernel (step_kernel.hip). Not part of the public ABI.
#pragma once
#include <stddef.h>
#include <stdint.h>

// Read-only device tables live in the constant address space when compiled for
// the device: uniform reads become scalar loads, divergent ones global loads,
// and neither is a flat access (flat loads also hold the LDS wait counter).
#if defined(__HIP_DEVICE_COMPILE__)
#define SBK_C __attribute__((address_space(4)))
#else
#define SBK_C
#endif

#define SBK_MAX_AHU 16
#define SBK_MT_N 624
#define SBK_NAUX_MAX 16
#define SBK_KMAX 16      // terms per lane per pass (matches the planner)
#define SBK_PLAN_DEPTH 4 // pass count multiple and prefetch depth (matches the planner)
#define SBK_NSTAMP 32        // phase stamps per env when phase timing is on
#define SBK_STAMP_HELPER 15  // stamps 15..18 are the env's helper wavefront's
#define SBK_STAMP_ENTRY 19   // the first wavefront's entry into the kernel (20.. finer stamps of its HVAC pre-step)
#define SBK_VPL 4        // VAVs (and coupled columns) per lane: at most 256 per env
#define SBK_RX_RPL 4     // relaxation rows per lane (matches the planner)
#define SBK_RX_ROWS 256  // padded relaxation rows
#define SBK_RX_TERMS 8   // relaxation off-diagonal entries per row
#define SBK_RX_MAXIT 64  // sweep cap (rho <= 1/2 contracts by 2^-64 before it)
#define SBK_RX_TOL 1e-13 // stop when the error bound is below TOL * max |T|
#define SBK_BX_ROWS 3    // block-Jacobi rows per block (matches the planner)
#define SBK_BX_SLOTS 2   // block slots per lane
#define SBK_BX_TERMS 8   // off-block entries per block
#define SBK_CV_WIN 256   // tempered convection words held in LDS at a time
#define SBK_CV_ROOM 64   // cells per convection room (one draw round per wavefront)

namespace sbk {

// Per-env state record, identical in HBM and in LDS (one bulk copy each way).
// Byte offsets are per layout (sizes differ), all 16-byte aligned.
struct StateLayout {
    int bytes;        // size of the bulk-copied image (multiple of 16)
    // f64 arrays
    int T, M;                                   // [n]
    int damper, reheat, ratio, heatsp, coolsp, dcmd, rcmd, sensing;  // [nv]
    int recirc, sat, fan, flow;                 // [na]
    int plant;                                  // f64[PF_COUNT], see PF_*
    int cal, cal_n;                             // f64[2][cal_n]: a step's calendar values (RW_*, then
                                                // the aux-time row), in section (calendar index & 1),
                                                // prefetched by the step before (or the reset)
    // i32 arrays
    int run, coolreq;                           // [na]
    int iplant;                                 // i32[PI_COUNT], see PI_*
    // u8 arrays
    int mode, prev_valid, dcmd_set, rcmd_set;   // [nv]
    int occ_state;                              // [nz * nassign]
    int occV;                                   // [nz]
    // MT19937 words live after the image in HBM (loaded only when drawn from)
    int mt;                                     // u32[624], HBM offset
    int cmt;                                    // u32[624] convection stream, HBM offset (0: no convection tables)
    int record_bytes;                           // image + mt (+ cmt), 256-byte aligned
};

// PF_SWEEPS: relaxation sweeps of the last step; PF_CAPPED: steps that hit the sweep cap;
// PF_DEV_SUM: sum since puf_reset of each step's mean zone deviation from the comfort band
enum { PF_PUMP_HEAD = 0, PF_BOILER_SP, PF_BOILER_RET, PF_BOILER_CUR, PF_BOILER_DSTEP,
       PF_REW_SUM, PF_SWEEPS, PF_CAPPED, PF_DEV_SUM, PF_COUNT };

enum { SOLVER_LU = 0, SOLVER_RELAX = 1 };
// Step-kernel variants, one per field-solver form (each compiles only its own
// solver, which keeps the instruction footprint of a launch small); a launch
// covers the tiles whose layouts use that form.
enum { KV_LU = 0, KV_POINT = 1, KV_BLOCK = 2, KV_COUNT = 3 };
// PI_FIRST_DONE: 1 once the env's first episode after puf_vec_create has
// ended (puf_reset leaves it; the first episode is the one desync truncates).
// PI_EP .. PI_EP + EP_COUNT - 1 (float bits): the episode's running sums that
// fill the Log when it ends (EP_*)
enum { PI_HWS_RUN = 0, PI_PUMP_RUN, PI_HWS_REQ, PI_STEP_INDEX, PI_STEP, PI_MT_IDX,
       PI_STEPS_TOTAL, PI_EPISODES, PI_CONV_IDX, PI_FIRST_DONE, PI_EP, PI_COUNT = 20 };
// The reference GPU env's running episode sums (complete_port/gpu/smart_buildings.cu:
// 118-121, 1965-1971): the float reward, the 8 per-step diagnostics (productivity
// term, normalized energy cost, normalized carbon, mean zone deviation, worst zone
// deviation (its sum unused), out-of-band fraction, electricity kWh, gas kWh),
// then the worst deviation as a maximum
enum { EP_RET = 0, EP_PART = 1, EP_WORST = 9, EP_COUNT = 10 };

// Per-env LDS region (byte offsets from the env's base; a workgroup holds the
// layout image first, then one region per env).
struct LdsLayout {
    int state;        // state image (StateLayout offsets are relative to this)
    int mt;           // u32[624] MT19937 words (filled from HBM when a draw twists the state)
    int scen;         // scenario image (ScenImg offsets are relative to this)
    int act;          // f32[SB_ACT] action row of the step
    int slots;        // f64[n_slots]: 0 zero, 1 sink, LU entries, vector (relaxation: node heat)
    int zq;           // f64[nz] zone heat / zone mean temperature
    int vtmp;         // f64[4 * nv]: unrestricted flow, flow demand, reheat energy, per-AHU list values
    int g;            // f64[k] air-side conductance
    int tair;         // f64[k] supply air temperature
    int atmp;         // f64[8 * na]: wsum, atotal, satv, demand, fd sum, count
    int red;          // f64[64] reduction scratch
    int misc;         // f64[MS_SIZE] scalars
    int obsx;         // f64[OX_AHU + 4 * na] per-step values the observation reads (OX_*)
    int iscr;         // i32[W + 8] scan scratch
    int occn;         // u8[nz * nassign + nz] the helper's new chain states and zone counts
    int hzq;          // f64[nz] the helper's zone means
    int sync;         // i32[SY_WORDS] hand-off area of the env's two wavefronts
    int stamps;       // u64[SBK_NSTAMP] phase stamps (phase timing only)
    int prec;         // int4[n_pass] solve pass records (copied at kernel start)
    // convection (layouts with convection tables only): tempered stream words,
    // the step's permutation of the room cells, one room's swap pairs
    int cvwin;        // u32[SBK_CV_WIN]
    int cvsig;        // i32[cv_cells]
    int cvl, cvr;     // i32[cv_max_room]
    int bytes;        // region size, 16-byte multiple
};

// Layout image: every per-layout table the step reads, packed (16-byte aligned
// sections) so a workgroup copies it to LDS in one burst and its envs share it.
struct ImgLayout {
    int bytes;        // 16-byte multiple
    // f64
    int cap, mcoup, mret, mgain, solar_c, rx_diag;          // [n]
    int zone_area;                                          // [nz]
    int vav_area;                                           // [nv]
    int ahu_area;                                           // [na]: its VAVs' areas summed in ascending VAV order
    int vav_c, ahu_c;                                       // [9 nv], [9 na]
    int act_mn, act_mx, act_mnr, act_mxr, act_hi;           // [n_act]
    int f_mean, f_sd;                                       // [n_dev]
    int f_src;                                              // u32 [n_dev], OBS_SRC_*
    // i32
    int rx_air, pos;                                        // [n]
    int zone_cell_off, zone_cells, vz_off, vz_idx, vav_ahu, coupled, zone_col_off, zone_cols;
    int ahu_vav_off, ahu_vavs;     // [na + 1], [nv]: each AHU's VAVs, ascending
    int ahu_col_off, ahu_cols;     // [na + 1], [k]: each AHU's coupled columns, ascending
    int vav_lpos, col_lpos;        // [nv], [k]: each VAV's position in ahu_vavs, each column's in ahu_cols
    int act_src, act_dst, act_aux;                          // [n_act] (dst/aux: ACT_*)
    int air_slot, air_node;                                 // [k]
    // block-Jacobi tables (block form only), chunk-major so lane l reading block
    // b = q * 64 + l takes 16 consecutive bytes per chunk: bx_d double2[9][nb]
    // = a_ii (3), in-block a(p, p2) for (0,1) (0,2) (1,0) (1,2) (2,0) (2,1), the
    // 8 off-block entry values, 0; bx_i int4[3][nb] = row | air << 16 (3, each
    // -1 as 0xffff / -1), 0, then col | row-in-block << 16 of the 8 entries
    int bx_d, bx_i;
    // convection rooms (sb_convect.h): room offsets [cv_rooms + 1] into the
    // cell list, each cell's node [cv_cells], its candidates as CSR over cell
    // positions [cv_cells + 1], [candidates]
    int cv_off, cv_node, cv_coff, cv_cidx;
    // u8
    int is_room;                                            // [n]
    int act_disc, act_flags;                                // [n_act]
};

// Scenario image: per-scenario tables the step reads, staged per env.
struct ScenImg {
    int bytes;        // 16-byte multiple
    int dirx;         // f64[n] dirichlet + exposure(h)
    int elec_wk, elec_we, elec_co2;   // f64[24]
    int gas_price;    // f64[12]
};

// misc scratch (f64[MS_SIZE]): step scalars
enum { MS_FFS = 0, MS_TOTAL_REHEAT, MS_TF, MS_REWARD, MS_COMFORT, MS_AMB, MS_CMIN, MS_CMAX, MS_SIZE };
// Observation field source, resolved on the host: a value at a byte offset of
// the env's LDS region (state image, obsx values) or of the layout image.
#define OBS_SRC_IMG (1u << 31)   // offset into the layout image (else the env region)
#define OBS_SRC_I32 (1u << 30)   // int32 value (else f64)
#define OBS_SRC_OFF 0x3FFFFFFFu
// Action target, resolved on the host (sb_sim.c:220-244 actuator routing): the
// decoded value goes to a byte offset of the env's state image as f64, or as
// int32 (value == 1) when ACT_I32; the aux word optionally also sets a u8 flag
// to 1 (ACT_AUX_U8) or stores the same int32 (ACT_AUX_I32) at its offset.
#define ACT_I32 (1u << 31)
#define ACT_AUX_U8 (1u << 31)
#define ACT_AUX_I32 (1u << 30)
#define ACT_OFF 0x3FFFFFFFu
// act_flags: clamp to [0, act_hi]; divide by the pump head's bar -> m factor
enum { ACT_CLAMP = 1, ACT_PUMP_HEAD = 2 };

// obsx: ambient of the observed row, pump differential pressure, then per AHU
// a at OX_AHU + 4a: static pressure, delivered flow, flow fraction, outside-air flow
enum { OX_AMB = 0, OX_DP = 1, OX_AHU = 2 };

// A step's calendar values (StateLayout::cal): rows kk = the calendar index
// before the step and j = kk + 1 (RW_*), then the aux-time row j.
enum { RW_AMB_K = 0, RW_SOLAR_K, RW_COMF_K, RW_COMF_KM1, RW_HSP_K, RW_CSP_K, RW_AMB_J, RW_HSP_J, RW_CSP_J,
       RW_OCC_HOUR_J, RW_OCC_WORK_J, RW_REW_HOUR_J, RW_REW_MONTH_J, RW_REW_WORK_J, RW_COUNT };

// One layout (building structure): solve plan + HVAC topology + constant tables.
struct DevLayout {
    int n, nz, nv, na, k, n_act, n_cont, n_disc, n_dev, n_aux, nassign;
    int n_slots, vec_base, n_pass, width;
    int max_room_cells;
    int solver;                        // SOLVER_LU or SOLVER_RELAX
    int rx_terms;                      // longest off-diagonal (or off-block) row (relaxation)
    int rx_block;                      // block-Jacobi form with 1 or 2 block slots per lane (bx_*), 0: point form (rx_*)
    int lu_sbase;                      // compact LU terms (a | b << 12 | v << 24): the 1.0 slot before the
                                       // reciprocals, third factor slot[lu_sbase + v]; 0: terms a | b << 16
    double rx_stop;                    // rho / (1 - rho)
    StateLayout st;
    LdsLayout lds;
    ImgLayout img;
    const SBK_C unsigned char* img_src;   // the layout image in HBM
    // relaxation tables, rows padded to SBK_RX_ROWS
    const SBK_C double* rx_diag;       // [SBK_RX_ROWS]
    const SBK_C int* rx_air;           // [SBK_RX_ROWS] air-side column or -1
    const SBK_C double* rx_val;        // [SBK_RX_TERMS * SBK_RX_ROWS]
    const SBK_C int* rx_col;           // [SBK_RX_TERMS * SBK_RX_ROWS]
    int bx_nb;                         // block-Jacobi blocks (tables in the layout image: bx_d, bx_i)
    int cv_rooms, cv_cells, cv_max_room;   // convection rooms and cells (tables in the layout image: cv_*)
    // solve plan
    const SBK_C int* pinfo;            // [n_pass * 4]: hdr_off, word_off, nact | maxcnt << 8 | pivot << 16, 0
    const SBK_C uint64_t* hdr;         // per active lane: target | mul << 16 | inv_target << 32 | count << 48
    const SBK_C uint32_t* words;       // term words a | b << 16, rows of nact words
    const SBK_C double* slot_init;     // [n_slots]
    const SBK_C int* pos;              // [n]
    const SBK_C int* air_slot;         // [k]
    const SBK_C int* air_node;         // [k]
    // field
    const SBK_C double* cap;           // [n]
    const SBK_C double* mcoup;         // [n]
    const SBK_C double* mret;          // [n]
    const SBK_C double* mgain;         // [n]
    const SBK_C double* solar_c;       // [n]
    const SBK_C uint8_t* is_room;      // [n]
    // zones / rooms (rooms flattened to node lists)
    const SBK_C int* zone_cell_off;    // [nz + 1]
    const SBK_C int* zone_cells;       // node ids
    const SBK_C double* zone_area;     // [nz]
    const SBK_C int* vz_off;           // [nv + 1]
    const SBK_C int* vz_idx;
    const SBK_C double* vav_area;      // [nv] (constant: sum of its zones' areas)
    const SBK_C int* vav_ahu;          // [nv]
    const SBK_C int* coupled;          // [k] col -> vav
    const SBK_C int* zone_col_off;     // [nz + 1] coupled columns feeding zone z
    const SBK_C int* zone_cols;
    const SBK_C double* vav_c;         // [nv * 9]
    const SBK_C double* ahu_c;         // [na * 9]
    // actions
    const SBK_C uint8_t* act_kind;
    const SBK_C uint8_t* act_act;
    const SBK_C uint8_t* act_disc;
    const SBK_C int* act_idx;
    const SBK_C int* act_src;          // column in the trainer row (cont block or SB_CONT + d)
    const SBK_C double* act_mn;
    const SBK_C double* act_mx;
    const SBK_C double* act_mnr;
    const SBK_C double* act_mxr;
    // observation map
    const SBK_C uint8_t* f_kind;
    const SBK_C uint8_t* f_id;
    const SBK_C int* f_idx;
    const SBK_C double* f_mean;
    const SBK_C double* f_sd;          // sqrt(var) or 0 when var <= 0
    // bytes of algorithmic traffic per env-step (the persistent state, the
    // action row, the observation prefix, reward and terminal), and what the
    // kernel's record image round trip moves for them
    double bytes_per_step;
    double record_bytes_per_step;
    double solve_flops;
};

// One scenario (blob): calendar, weather, prices, scalar constants.
struct DevScen {
    int layout;
    int n1;                      // calendar rows
    ScenImg img;
    const SBK_C unsigned char* img_src;   // the scenario image in HBM
    const SBK_C double* amb;
    const SBK_C double* solar_i;
    const SBK_C double* comfort;
    const SBK_C double* heat_sp;
    const SBK_C double* cool_sp;
    const SBK_C double* aux_time;      // [n1 * (n_aux - 1)]
    const SBK_C uint8_t* occ_hour;
    const SBK_C uint8_t* occ_work;
    const SBK_C uint8_t* hour_m1;
    const SBK_C uint8_t* work_m1;
    const SBK_C uint8_t* rew_hour;
    const SBK_C uint8_t* rew_month;
    const SBK_C uint8_t* rew_work;
    const SBK_C double* dirx;          // [n] dirichlet + exposure(h)
    const SBK_C double* temp_init;     // [n]
    const SBK_C double* mass_init;     // [n]
    const SBK_C double* elec_wk;       // [24]
    const SBK_C double* elec_we;       // [24]
    const SBK_C double* elec_co2;      // [24]
    const SBK_C double* gas_price;     // [12]
    double gas_co2;
    double rw[8];
    double boiler_c[10];
    double diss_den;             // log(r2/c6)/c8 + 1/c4/r2, host libm
    double pump_eff, pump_head0, header_res;
    double internal_w_m2, standby_frac, occupant_w, cv_area, dt_sec;
    double p_arr, p_dep;
    int ea, la, ed, ld;
    int conv_tmean;              // 1 if some AHU may need the field mean
    int conv_on;                 // stochastic convection: conv_p != 0 and conv_distance != 0
    double conv_p;
    double inv_nz;               // 1 / zones (the per-step comfort diagnostics are zone means)
    double kwh_per_w;            // dt / 3.6e6: one step's energy in kWh per W
};

struct EnvDesc {
    int scen;
    int layout;
    long long state_off;         // byte offset of the env's record
    int start;                   // calendar start offset
    int max_steps;
    // staging burst inputs, copied from the scenario so the burst can be
    // issued from this record alone
    int scn16;                   // scenario image size in 16-byte units
    int first_steps;             // length of the env's first episode after puf_vec_create (desync
                                 // truncates it; = max_steps otherwise)
    const SBK_C unsigned char* scen_src;   // scenario image in HBM
};

enum { KMODE_STEP = 0, KMODE_RESET = 1 };
// Words of an env's hand-off area (LdsLayout::sync): flags posted by the first
// wavefront (state after the HVAC pre-step and boiler update ready, new field
// ready) and by the helper (VAV sensed temperatures ready; AHU return-air
// sums ready; observation
// written, new occupancy committed and reward half ready); the helper's reward
// half (7 f64 from SY_PART); the helper's stores of the record's leading
// arrays complete (SY_STORED); the helper's convection permutation of the
// step (SY_CONV).
enum { SY_PRE = 0, SY_POST = 1, SY_HALF = 2, SY_SENS = 3, SY_PART = 4, SY_RET = 18, SY_CONV = 19,
       SY_STORED = 20, SY_SLOTS = 21, SY_WORDS = 22 };

// A workgroup's envs: order[first .. first + count) all of one layout, with
// the layout's staging burst inputs (copied from its DevLayout) and each
// slot's env index and record (copied from the env table; a slot past count
// repeats the first), so the burst is issued after reading this record alone.
struct Tile {
    int layout, first, count, lds_bytes;   // lds_bytes: one env's LDS region
    int img16, rec16;                      // layout image, record image (+ convection state), 16-byte units
    int lds_state, lds_scen, lds_act;      // LDS offsets within the env region
    int st_iplant;                         // byte offset of the i32 plant counters in the record
    int pad0, pad1;
    const SBK_C unsigned char* img_src;    // layout image in HBM
    long long pad2;
    int env[4];                            // env index of each slot
    EnvDesc desc[4];                       // its env record
};

struct KParams {
    const SBK_C EnvDesc* envs;
    const SBK_C int* order;      // tile slot -> env
    const SBK_C Tile* tiles;     // block -> tile
    const SBK_C DevLayout* layouts;
    const SBK_C DevScen* scens;
    unsigned char* state;
    const float* actions;
    float* obs;
    float* rewards;
    float* terminals;
    void* host_env;              // Env array (host-coherent), or null
    int env_stride;              // sizeof(Env)
    int log_offset;              // offsetof(Env, log)
    int n_envs;
    int mode;
    float reward_scale;
    int img_lds;                 // LDS bytes reserved for the layout image (max over layouts)
    unsigned long long* phase_ts;   // null, or [n_envs * SBK_NSTAMP] wall-clock stamps
    unsigned long long* pass_ts;    // null, or [n_pass + 1] shader-clock stamps of one env
    int pass_ts_env;                // env whose solve passes are stamped
    int air_stride;                 // doubles per env half of air_trace (the largest k)
    double* air_trace;              // null, or [n_envs][2][air_stride]: the step's air_g, then air_T
};

// The host (g++) and the device (hipcc) compile these structs separately and
// exchange them byte for byte: both builds check the same sizes and offsets.
static_assert(sizeof(EnvDesc) == 40 && offsetof(EnvDesc, state_off) == 8 && offsetof(EnvDesc, first_steps) == 28
              && offsetof(EnvDesc, scen_src) == 32, "EnvDesc layout");
static_assert(sizeof(Tile) == 240 && offsetof(Tile, img_src) == 48 && offsetof(Tile, env) == 64
              && offsetof(Tile, desc) == 80, "Tile layout");
static_assert(sizeof(StateLayout) == 120 && sizeof(LdsLayout) == 96 && sizeof(ImgLayout) == 200
              && sizeof(ScenImg) == 24, "table layouts");
static_assert(sizeof(DevLayout) == 896 && offsetof(DevLayout, st) == 88 && offsetof(DevLayout, img_src) == 504
              && offsetof(DevLayout, bytes_per_step) == 872, "DevLayout layout");
static_assert(sizeof(DevScen) == 488 && offsetof(DevScen, img_src) == 32 && offsetof(DevScen, gas_co2) == 200
              && offsetof(DevScen, conv_p) == 464, "DevScen layout");
static_assert(sizeof(KParams) == 144 && offsetof(KParams, host_env) == 80 && offsetof(KParams, phase_ts) == 112
              && offsetof(KParams, pass_ts_env) == 128 && offsetof(KParams, air_trace) == 136, "KParams layout");

}  // namespace sbk
