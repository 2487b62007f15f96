// Canonical layout of the policy interface (env kwargs canonical / residual),
// shared by the host (vec.cpp builds one table per layout) and the device
// (canon_kernel.hip). Not part of the public ABI.
//
// The slot layout is the reference's policy interface and is kept as it is
// (complete_port/gpu/sb_gpu_base.inc:31-45, complete_port/submission/
// residual_policy.py:36-44): AHU k < 9 owns zone slots 10 k .. 10 k + 9 (its
// zones in the order their temperature field appears in the observation); the
// observation is 90 zone slots x 9 features, 9 AHU slots x 16, 10 hot-water
// features and 19 global ones (983 floats); the actions are damper and reheat
// per zone slot, supply temperature / static pressure / recirculation / run per
// AHU slot, supply temperature / pump dP / run for the hot water (219 heads).
#pragma once
#include <stdint.h>

#include "sbenv.h"

#define SBC_K 9
#define SBC_ZPA 10
#define SBC_ZS (SBC_K * SBC_ZPA)
#define SBC_FZ 9
#define SBC_FA 16
#define SBC_FH 10
#define SBC_FG 19
#define SBC_OA (SBC_ZS * SBC_FZ)
#define SBC_OH (SBC_OA + SBC_K * SBC_FA)
#define SBC_OG (SBC_OH + SBC_FH)
#define SBC_OBS (SBC_OG + SBC_FG)
#define SBC_AA (2 * SBC_ZS)
#define SBC_AH (SBC_AA + 4 * SBC_K)
#define SBC_ACT (SBC_AH + 3)

namespace sbk {

// One layout's canonical maps: observation field indices, native action
// indices, the schedule band and the fields' normalisation (-1 = absent).
struct CanonTab {
    int K;                     // AHUs
    int n_act;                 // native actions
    int morning, evening;      // comfort hours [morning, evening) on days 0..4
    int zc[SBC_K];             // zones on AHU k
    int zT[SBC_ZS], zH[SBC_ZS], zC[SBC_ZS], zD[SBC_ZS], zR[SBC_ZS];   // zone fields
    int zAd[SBC_ZS], zAr[SBC_ZS];                                     // zone damper / reheat actions
    int aObs[SBC_K][8];        // outside-air temp, static pressure, supply flow, outside-air flow,
                               // supply temp setpoint, recirculation, cooling requests, run command
    int aT[SBC_K], aP[SBC_K], aRec[SBC_K], aRun[SBC_K];               // AHU actions
    int hObs[6];               // supply water temp, its setpoint, dP, dP setpoint, run status, requests
    int hW, hDPa, hRun;        // hot-water actions
    int g[SBC_FG];             // hod sin x4, hod cos x4, dow sin x4, dow cos x4, comfort now, soon, occupants
    int slot_of_action[SB_ACT];   // native action -> canonical action slot
    int act_of_col[SB_ACT];       // column of the env's native action row -> native action
    uint8_t act_disc[SB_ACT];
    float tmean, tstd;            // zone temperature normalisation
    double comfort_lo, comfort_hi, eco_lo, eco_hi;
    float fmean[SB_OBS], fstd[SB_OBS];   // native value of a field: obs * fstd + fmean
};

struct EnvDesc;

// Arguments of the canonical kernels (canon_kernel.hip).
struct CanonArgs {
    const CanonTab* tabs;      // per layout
    const EnvDesc* envs;       // env -> layout
    const float* raw_obs;      // [n][SB_OBS] the env's own observation rows
    float* obs;                // [n][SB_OBS] trainer rows: the canonical observation
    const float* actions;      // [n][SB_ACT] trainer rows: the canonical action heads
    float* native;             // [n][SB_ACT] the env's native action rows
    const float* terminals;    // [n]
    double* pid;               // [n][2 SBC_K] integral, previous error per AHU
    float* base;               // [n][SB_ACT] proposal per native action
    float* trust;              // [n][SB_ACT] guard trust per native action
    float* ainfo;              // [n][2 SBC_K] effort, mean zone temperature per AHU
    int n;
    int reset;                 // puf_reset: every env starts an episode, the rows' padding is zeroed
    int resid;                 // residual decode (else absolute)
    float scale, dscale;       // residual authority of continuous heads / run bits
    int guard;                 // comfort guard on
    float d0, d1;
    int hot;
};

}  // namespace sbk
