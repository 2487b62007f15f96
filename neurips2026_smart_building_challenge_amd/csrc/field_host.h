// Host side of the field envs (FDM-scale scenarios behind the PufferLib ABI;
// field_env.h describes the step). The vec (vec.cpp) owns one FieldScen per
// such scenario and drives it through these calls on its bound stream.
#pragma once
#include <hip/hip_runtime_api.h>
#include <stdint.h>

#include <string>
#include <vector>

#include "field_env.h"
#include "sbb_reader.h"

struct FieldScen;

struct FieldCounts {
    int n_act, n_cont, n_disc;
    int n1;                 // calendar rows
    int episode_steps;
    int hour_m1_rows;
    int64_t occ_seed;
    int64_t conv_seed;      // the convection stream's seed (env j of the scenario: + j, as the occupancy one)
    int n_cvs, n_solved, nz;
    int n_obs;              // observation prefix (n_dev + n_aux floats)
};

// A blob the RC step kernel cannot hold: more solved cells than its LDS plans
// take, or an air side other than one unit column per node.
bool field_blob(const sbh::Blob& b);

// Reads and checks the scenario's HVAC, calendar and reward tables (host).
FieldScen* field_open(const sbh::Blob& b, std::string* err);
FieldCounts field_counts(const FieldScen* f);

// Device tables, the field group (sbx_fdm with `flags`, `envs_per_block`) and
// the per-env records of the scenario's envs (slots in vec order), with their
// occupancy and convection streams seeded.
bool field_attach(FieldScen* f, const std::string& path, const std::vector<sbe::Slot>& slots, int flags,
                  int envs_per_block, std::string* err);

struct FieldIo {
    const float* actions;
    float* obs;
    float* rewards;
    float* terminals;
    void* host_env;
    int env_stride, log_offset;
    float reward_scale;
};

// One env-step of every env of the scenario, or (reset) puf_reset of them.
bool field_step(FieldScen* f, const FieldIo& io, bool reset, hipStream_t s, std::string* err);

// The oracle's state order for slot `slot` (synchronous): field, interior
// mass, VAV damper / reheat / ratio / sensing, AHU flow / sat / recirc / fan,
// air_g / air_T, occupancy, boiler current / return / setpoint, pump head,
// calendar index, then the f64 reward sum and the steps since puf_reset.
int field_state(FieldScen* f, int slot, double* out, int cap);

// Adds the scenario's totals since puf_reset (reward sum, env-steps,
// episodes) to out[0..2] and (reward sum, mean zone deviation sum, env-steps)
// to out[3 + 3 scen ..] (device, stream-ordered).
bool field_live(FieldScen* f, double* out, int scen, hipStream_t s);

double field_bytes_per_step(const FieldScen* f);
double field_flops_per_step(const FieldScen* f);
void field_close(FieldScen* f);
